"""CPU restatement of the reference engine's forward pass (TEST INFRASTRUCTURE ONLY).

Only tests/ import this module: it is the checker the device engine
(qw3_amd/engine.py) is compared against, never the thing measured or shipped.

DS5's engine (src/engine/forward.zig:154-516) runs one decoder layer as a fixed
sequence of kernel-provider calls. `Engine.forward` makes the same calls, in the
same order and on buffers of the same shapes, on the oracle's restatements of
the CPU provider (oracle/ds5_oracle.c via oracle.py):

    x = embed[token]                       forward.zig:310-316, embedRow :503-516
    per layer                              forward.zig:322-471
      h = rmsNorm(x, attn_norm)
      q, k, v = h . Wq^T, h . Wk^T, h . Wv^T
      q, k = rmsNorm per head (q_norm, k_norm); rope(q), rope(k)
      kvAppend(k, v); attn = gqaAttention(q, cache)
      x = x + attn . Wo^T
      h2 = rmsNorm(x, ffn_norm)
      ids, w = routerTopK(h2); proj = 0; proj += experts(h2, pairs)
      x = x + proj                         (trace point "block")
    logits = rmsNorm(x, output_norm) . output^T   forward.zig:473-492

It is pinned by the reference's own whole-model fixtures: the residual stream
after layers 0, 2 and 3 of prompt p0 (`l{0,2,3}_block.output`) and the logits
and greedy tokens of the five manifest prompts (`p*.logits`), the checks of
src/test_forward.zig:192-330.
"""
from __future__ import annotations

import numpy as np

from . import oracle as O


def tensor_dtype(a: np.ndarray) -> int:
    """Q8_0 rows are held as uint8 [rows, k/32*34], everything else as f32."""
    return O.Q8_0 if a.dtype == np.uint8 else O.F32


class Engine:
    """forward.zig's Engine(CpuCtx, cpu_kernels) over GGUF-named weights.

    weights: GGUF tensor name -> numpy array (f32, or uint8 Q8_0 rows);
    cfg: the model config of the fixture manifest (contracts.SYNTH_TINY)."""

    def __init__(self, weights: dict, cfg: dict, context_capacity: int, kv_dtype: int = O.F32):
        self.w, self.cfg = weights, cfg
        self.capacity, self.kv_dtype = context_capacity, kv_dtype
        hkv, hd = cfg["n_kv_heads"], cfg["head_dim"]
        cache_dt = np.float32 if kv_dtype == O.F32 else np.uint16
        self.k_cache = [np.zeros(hkv * context_capacity * hd, cache_dt) for _ in range(cfg["n_layers"])]
        self.v_cache = [np.zeros(hkv * context_capacity * hd, cache_dt) for _ in range(cfg["n_layers"])]
        self.pos = 0

    def reset(self) -> None:
        """forward.zig:288-290: a new sequence starts at position 0 (stale cache rows
        beyond it are never read)."""
        self.pos = 0

    def _w(self, layer: int, suffix: str) -> np.ndarray:
        return self.w[f"blk.{layer}.{suffix}"]

    def embed_row(self, tok: int) -> np.ndarray:
        """forward.zig:503-516: the token's embedding row, dequantised on the host."""
        e = self.w["token_embd.weight"]
        if e.dtype == np.uint8:
            return O.q8_0_dequantize(e[tok:tok + 1], self.cfg["hidden_dim"])[0]
        return np.asarray(e[tok], np.float32)

    def forward(self, tokens, trace=None) -> np.ndarray:
        """Logits [n, vocab] of tokens at positions pos..pos+n-1 (forward.zig:299-500).
        trace(layer, op, array) sees the buffers at forward.zig's trace points."""
        c = self.cfg
        n = len(tokens)
        hidden, hq, hkv, hd = c["hidden_dim"], c["n_q_heads"], c["n_kv_heads"], c["head_dim"]
        q_dim, kv_dim, eps = hq * hd, hkv * hd, c["rms_eps"]
        if n == 0:
            raise ValueError("BatchTooLarge")
        if n > self.capacity or self.pos > self.capacity - n:
            raise ValueError("ContextOverflow")
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
        tr = trace or (lambda layer, op, a: None)

        x = np.stack([self.embed_row(int(t)) for t in tokens]).astype(np.float32)
        tr(-1, "embed", x)
        positions = np.arange(self.pos, self.pos + n, dtype=np.int32)
        for li in range(c["n_layers"]):
            h = O.rms_norm(x, self._w(li, "attn_norm.weight"), eps, n, hidden)
            tr(li, "attn_norm", h)
            q = O.matmul(h, self._w(li, "attn_q.weight"), tensor_dtype(self._w(li, "attn_q.weight")), n, q_dim, hidden)
            k = O.matmul(h, self._w(li, "attn_k.weight"), tensor_dtype(self._w(li, "attn_k.weight")), n, kv_dim, hidden)
            v = O.matmul(h, self._w(li, "attn_v.weight"), tensor_dtype(self._w(li, "attn_v.weight")), n, kv_dim, hidden)
            tr(li, "q_proj", q)
            tr(li, "k_proj", k)
            tr(li, "v_proj", v)
            q = O.rms_norm(q, self._w(li, "attn_q_norm.weight"), eps, n * hq, hd)
            k = O.rms_norm(k, self._w(li, "attn_k_norm.weight"), eps, n * hkv, hd)
            tr(li, "q_norm", q)
            tr(li, "k_norm", k)
            q = O.rope(q.reshape(n, hq, hd), positions, c["rope_theta"])
            k = O.rope(k.reshape(n, hkv, hd), positions, c["rope_theta"])
            tr(li, "rope_q", q)
            tr(li, "rope_k", k)
            O.kv_append(k, v, self.k_cache[li], self.v_cache[li], self.kv_dtype, self.pos, n, hkv, hd, self.capacity)
            attn = O.gqa_attention(q, self.k_cache[li], self.v_cache[li], self.kv_dtype, self.pos, n, hq, hkv, hd,
                                   self.capacity, scale).reshape(n, q_dim)
            tr(li, "attn", attn)
            wo = self._w(li, "attn_output.weight")
            x = O.add(x, O.matmul(attn, wo, tensor_dtype(wo), n, hidden, q_dim))
            tr(li, "attn_resid", x)
            h2 = O.rms_norm(x, self._w(li, "ffn_norm.weight"), eps, n, hidden)
            tr(li, "ffn_norm", h2)
            router = self._w(li, "ffn_gate_inp.weight")
            ids, wts = O.router_topk(h2, router, tensor_dtype(router), n, hidden, c["n_experts"], c["top_k"],
                                     c["norm_topk_prob"])
            gate = self._w(li, "ffn_gate_exps.weight")
            proj = O.expert_mlp_swiglu(h2, gate, self._w(li, "ffn_up_exps.weight"),
                                       self._w(li, "ffn_down_exps.weight"), tensor_dtype(gate),
                                       O.pairs_from_router(ids, wts), n, hidden, c["expert_ffn_dim"], c["n_experts"])
            tr(li, "experts", proj)
            x = O.add(x, proj)
            tr(li, "block", x)
        h = O.rms_norm(x, self.w["output_norm.weight"], eps, n, hidden)
        tr(-1, "output_norm", h)
        out_w = self.w["output.weight"]
        logits = O.matmul(h, out_w, tensor_dtype(out_w), n, c["vocab_size"], hidden)
        tr(-1, "logits", logits)
        self.pos += n
        return logits


def argmax(logits: np.ndarray) -> int:
    """forward.zig:518-528: the first index of the maximum (ties to the lower token id)."""
    return int(np.argmax(logits))


# forward.zig's trace points of one layer, in the order they fire (forward.zig:334-470)
LAYER_TRACE_OPS = ("attn_norm", "q_proj", "k_proj", "v_proj", "q_norm", "k_norm", "rope_q", "rope_k", "attn",
                   "attn_resid", "ffn_norm", "experts", "block")


def trace_order(n_layers: int):
    """Every (layer, op) trace point of a forward pass in firing order."""
    pts = [(-1, "embed")]
    for li in range(n_layers):
        pts += [(li, op) for op in LAYER_TRACE_OPS]
    return pts + [(-1, "output_norm"), (-1, "logits")]


def first_divergence(want: dict, got: dict, n_layers: int, atol: float, rtol: float, logits_tol=None):
    """The first trace point, in firing order, where `got` leaves `want`'s tolerance
    (|a - o| <= atol + rtol |o|, NaN fails) -- test_forward.zig:304-330's firstDivergence
    over every point both traces hold. Returns (layer, op, compare result) or None."""
    for key in trace_order(n_layers):
        if key not in want or key not in got:
            continue
        a, t = (atol, rtol) if key[1] != "logits" or logits_tol is None else logits_tol
        r = O.compare(np.asarray(want[key], np.float32).reshape(-1), np.asarray(got[key], np.float32).reshape(-1), a, t)
        if not r.passed:
            return key[0], key[1], r
    return None
