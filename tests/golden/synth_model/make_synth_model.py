"""Regenerates the weights of the reference's synthetic tiny Qwen3-MoE model that its
vendored fixtures do not hold, so the whole-model checks (per-layer block outputs,
end-to-end logits) can run.

The reference builds this model in `tools/make_fixtures.py:289-323` (a transformers
`Qwen3MoeForCausalLM` of the SYNTH_TINY config `:66-80`, `torch.manual_seed(0)`, every
1-D norm weight redrawn as `1 + 0.1·N(0,1)`) and bakes the projections, the embedding,
the output head and the expert banks into GGUF Q8_0 (`:327-374`, the quantiser `:117-132`:
d = max|w| / 127, q = roundf(w · (1/d)) with halves away from zero, the scale stored as
f16). This script restates that recipe with the installed transformers (no reference code
is imported or run) and checks what it regenerates against every weight the vendored
fixtures hold:

- the Q8_0 blobs of `l{0,2,3}_attn_q`, the three expert banks of `l{0,2,3}_experts` and the
  output head (`lm_head`) must match byte for byte, but for at most one byte in 10^4 (a
  weight moved by an ulp, below, can move a block's f16 scale by one step: the output head
  differs in one scale byte);
- the f32 norm and router weights must match within a few ulp (torch's normal sampler and
  the `1 + 0.1·x` rounding moved by an ulp between the torch release the reference used and
  this one).

It writes `weights.npz` beside itself with the tensors the fixtures lack: layer 1 whole,
every layer's k/v/output projections, k-norm and ffn-norm weights, the token embedding and
the output norm. Tests take every other weight from the vendored fixtures.

Run: python tests/golden/synth_model/make_synth_model.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = os.path.join(HERE, "..", "ds5_synthetic")
sys.path.insert(0, os.path.join(HERE, "..", "..", ".."))
from oracle.oracle import load_ds5t  # noqa: E402

CFG = dict(n_layers=4, hidden_dim=256, n_q_heads=4, n_kv_heads=2, head_dim=64, n_experts=8, top_k=4,
           expert_ffn_dim=128, vocab_size=512, rms_eps=1e-6, rope_theta=1e6, norm_topk_prob=True, max_ctx=512)


def build_model(seed: int = 0):
    from transformers.models.qwen3_moe import Qwen3MoeConfig, Qwen3MoeForCausalLM
    c = CFG
    hf = Qwen3MoeConfig(
        vocab_size=c["vocab_size"], hidden_size=c["hidden_dim"], intermediate_size=2 * c["expert_ffn_dim"],
        moe_intermediate_size=c["expert_ffn_dim"], num_hidden_layers=c["n_layers"],
        num_attention_heads=c["n_q_heads"], num_key_value_heads=c["n_kv_heads"], head_dim=c["head_dim"],
        num_experts=c["n_experts"], num_experts_per_tok=c["top_k"], norm_topk_prob=c["norm_topk_prob"],
        decoder_sparse_step=1, mlp_only_layers=[], rope_theta=c["rope_theta"], rms_norm_eps=c["rms_eps"],
        max_position_embeddings=c["max_ctx"], tie_word_embeddings=False, attention_bias=False,
        hidden_act="silu", attn_implementation="eager", use_cache=False)
    torch.manual_seed(seed)
    model = Qwen3MoeForCausalLM(hf).eval().float()
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name and p.dim() == 1:
                p.copy_(1.0 + 0.1 * torch.randn_like(p))
    return {k: v.detach().to(torch.float32).contiguous().numpy() for k, v in model.named_parameters()}


def q8_0_bake(w: np.ndarray) -> np.ndarray:
    """GGUF Q8_0 rows [rows, k/32·34] of f32 w [..., k]: per 32-element block d = max|w|/127,
    q = roundf(w · (1/d)) (halves away from zero), scale stored as f16."""
    w = np.asarray(w, np.float32)
    k = w.shape[-1]
    b = w.reshape(-1, k // 32, 32)
    d = np.abs(b).max(axis=-1) / np.float32(127.0)
    safe = np.where(d > 0, d, np.float32(1.0))
    inv = np.where(d > 0, np.float32(1.0) / safe, np.float32(0.0)).astype(np.float32)
    x = (b * inv[..., None]).astype(np.float32)
    q = np.trunc(x + np.copysign(np.float32(0.5), x)).astype(np.int8)
    out = np.empty(b.shape[:2] + (34,), np.uint8)
    out[..., 0:2] = d.astype(np.float16)[..., None].view(np.uint8)
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(b.shape[0], -1)


def max_ulp(a, b) -> int:
    a = np.ascontiguousarray(a, np.float32).reshape(-1).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).reshape(-1).view(np.int32).astype(np.int64)
    return int(np.abs(a - b).max())


def model_tensors(sd: dict) -> dict:
    """GGUF-named tensors (tools/make_fixtures.py:340-374 naming): Q8_0 as uint8 rows,
    norms and router as f32."""
    ffn = CFG["expert_ffn_dim"]
    t = {"token_embd.weight": q8_0_bake(sd["model.embed_tokens.weight"]),
         "output.weight": q8_0_bake(sd["lm_head.weight"]),
         "output_norm.weight": sd["model.norm.weight"]}
    for li in range(CFG["n_layers"]):
        h, g = f"model.layers.{li}.", f"blk.{li}."
        t[g + "attn_norm.weight"] = sd[h + "input_layernorm.weight"]
        t[g + "ffn_norm.weight"] = sd[h + "post_attention_layernorm.weight"]
        t[g + "attn_q_norm.weight"] = sd[h + "self_attn.q_norm.weight"]
        t[g + "attn_k_norm.weight"] = sd[h + "self_attn.k_norm.weight"]
        for proj, gn in (("q_proj", "attn_q"), ("k_proj", "attn_k"), ("v_proj", "attn_v"),
                         ("o_proj", "attn_output")):
            t[g + gn + ".weight"] = q8_0_bake(sd[h + f"self_attn.{proj}.weight"])
        t[g + "ffn_gate_inp.weight"] = sd[h + "mlp.gate.weight"]
        gu, dn = sd[h + "mlp.experts.gate_up_proj"], sd[h + "mlp.experts.down_proj"]
        t[g + "ffn_gate_exps.weight"] = q8_0_bake(gu[:, :ffn, :])
        t[g + "ffn_up_exps.weight"] = q8_0_bake(gu[:, ffn:, :])
        t[g + "ffn_down_exps.weight"] = q8_0_bake(dn)
    return t


# Vendored fixture tensor -> GGUF name, for layers 0, 2 and 3.
def vendored_names(li: int) -> dict:
    g = f"blk.{li}."
    return {f"l{li}_attn_q.weight": (g + "attn_q.weight", "bytes"),
            f"l{li}_experts.gate": (g + "ffn_gate_exps.weight", "bytes"),
            f"l{li}_experts.up": (g + "ffn_up_exps.weight", "bytes"),
            f"l{li}_experts.down": (g + "ffn_down_exps.weight", "bytes"),
            f"l{li}_attn_norm.weight": (g + "attn_norm.weight", "ulp"),
            f"l{li}_q_norm.weight": (g + "attn_q_norm.weight", "ulp"),
            f"l{li}_router.weight": (g + "ffn_gate_inp.weight", "ulp")}


def vendored(fixture: str) -> np.ndarray:
    return load_ds5t(os.path.join(FIXTURES, fixture + ".ds5t")).data


def main() -> None:
    tensors = model_tensors(build_model(0))
    checks = {"lm_head.weight": ("output.weight", "bytes")}
    for li in (0, 2, 3):
        checks.update(vendored_names(li))
    for fx, (name, kind) in checks.items():
        want = vendored(fx)
        got = tensors[name]
        if kind == "bytes":
            diff = np.flatnonzero(np.asarray(want).reshape(-1) != got.reshape(-1))
            print(f"{fx:24s} == {name:28s} bytes differing: {diff.size} of {got.size}")
            # an ulp-moved weight can land a block's f16 scale on the other side of a rounding
            # boundary (one byte); anything more means the recipe is wrong
            assert diff.size <= max(1, got.size // 10000), fx
        else:
            u = max_ulp(want, got)
            print(f"{fx:24s} ~= {name:28s} max {u} ulp")
            # a norm weight near 1 moves by <= 2 ulp; router weights ~N(0, 0.02) by ~1e-7 relative
            assert u <= 2 or np.abs(np.asarray(want).reshape(-1) - got.reshape(-1)).max() < 1e-7, fx
    present = {name for name, _ in checks.values()}
    missing = {k: v for k, v in tensors.items() if k not in present}
    path = os.path.join(HERE, "weights.npz")
    np.savez(path, **missing)
    print(f"wrote {len(missing)} tensors, {os.path.getsize(path)} bytes -> {path}")


if __name__ == "__main__":
    main()
