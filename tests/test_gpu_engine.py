"""The whole synthetic model through the device engine (qw3_amd/engine.py), every kernel on
the MI355X: the reference's end-to-end gates (src/test_forward.zig:192-330,
src/test_gpu_forward.zig:94-360) plus a live diff against the oracle engine.

- per-layer trace diff: the residual stream after layers 0, 2 and 3 of p0's prefill
  against `l{0,2,3}_block.output`, and after every layer against the oracle engine
  (layer tolerance atol 2e-3, rtol 1e-2, as test_gpu_forward.zig:338-341);
- the five prompts: logits within the manifest tolerance and, with an f32 cache, every
  greedy pick exact (p3's first pick is a near-tie an f16 cache flips; see
  test_engine_oracle.py);
- the f16 cache within 0.02 of the f32 engine (test_forward.zig:131-190);
- both modes: the eight provider ops one call each, and the fused decls
  (matmulGroup, attentionStep, matmulAdd, moe).
"""
import numpy as np
import pytest

import synth_model as S

pytestmark = pytest.mark.gpu

LAYER_ATOL, LAYER_RTOL = 2e-3, 1e-2


@pytest.fixture(scope="module")
def model(oracle):
    return S.load()


@pytest.fixture(scope="module")
def weights(ctx, model):
    from qw3_amd import engine as E
    cfg, w, _ = model
    return E.Weights(ctx, w, cfg)


def _engine(ctx, hip, weights, kv, fused, capacity=64):
    from qw3_amd import engine as E
    return E.Engine(ctx, weights, max_batch=capacity, context_capacity=capacity,
                    kv_dtype=hip.DTYPE_F32 if kv == "f32" else hip.DTYPE_F16, fused=fused)


MODES = [("f32", False), ("f16", False), ("f32", True), ("f16", True)]
IDS = ["ops-f32", "ops-f16", "fused-f32", "fused-f16"]


# trace points the fused attention step does not produce (norm and rope run inside it)
FUSED_ONLY_MISSING = {"q_norm", "k_norm", "rope_q", "rope_k"}


@pytest.mark.parametrize("kv,fused", MODES, ids=IDS)
def test_block_trace(ctx, hip, oracle, model, weights, kv, fused):
    """Every trace point of every layer of p0's prefill against the oracle engine, walked
    in firing order for the first divergence (test_forward.zig:304-330); the residual
    after layers 0, 2 and 3 against the reference's block fixtures."""
    from oracle import engine as OE
    cfg, w, prompts = model
    toks = prompts[0]["token_ids"]
    print(f"[engine] trace kv={kv} fused={fused} tokens={len(toks)}", flush=True)
    eng = _engine(ctx, hip, weights, kv, fused)
    got = {}
    eng.trace = lambda layer, op, a: got.__setitem__((layer, op), a)
    eng.forward(toks)
    want = {}
    ref = OE.Engine(w, cfg, 64, oracle.F32 if kv == "f32" else oracle.F16)
    ref.forward(toks, trace=lambda layer, op, a: want.__setitem__((layer, op), a.copy()))
    expected = [p for p in OE.trace_order(cfg["n_layers"]) if not (fused and p[1] in FUSED_ONLY_MISSING)]
    assert sorted(got) == sorted(expected)
    assert np.array_equal(got[(-1, "embed")], want[(-1, "embed")].reshape(-1))
    for layer, x_in, _, x_out, atol, rtol in S.block_cases():
        r = oracle.compare(x_out.reshape(-1), got[(layer, "block")], atol, rtol)
        assert r.passed, ("fixture", layer, r)
    tol = prompts[0]["tolerance"]
    div = OE.first_divergence(want, got, cfg["n_layers"], LAYER_ATOL, LAYER_RTOL, (tol["atol"], tol["rtol"]))
    assert div is None, div


@pytest.mark.parametrize("kv,fused", MODES, ids=IDS)
def test_prompts(ctx, hip, oracle, model, weights, kv, fused):
    from qw3_amd import engine as E
    cfg, w, prompts = model
    eng = _engine(ctx, hip, weights, kv, fused)
    for p in prompts:
        print(f"[engine] prompt {p['name']} kv={kv} fused={fused}", flush=True)
        logits, picks = S.run_prompt(eng, p, E.argmax)
        want = S.prompt_logits(p)
        assert logits.shape == want.shape
        if kv == "f32":
            assert picks == list(p["greedy_tokens"]), (p["name"], picks)
        r = oracle.compare(want.reshape(-1), logits.reshape(-1), p["tolerance"]["atol"], p["tolerance"]["rtol"])
        assert r.passed, (p["name"], r)


@pytest.mark.parametrize("fused", [False, True], ids=["ops", "fused"])
def test_f16_cache_close_to_f32(ctx, hip, oracle, weights, fused):
    from qw3_amd import engine as E
    e32 = _engine(ctx, hip, weights, "f32", fused, capacity=3)
    e16 = _engine(ctx, hip, weights, "f16", fused, capacity=3)
    a, b = e32.forward([1, 2, 3]), e16.forward([1, 2, 3])
    assert oracle.compare(a.reshape(-1), b.reshape(-1), 0.02, 0.02).passed
    assert E.argmax(a[-1]) == E.argmax(b[-1])
    e32.reset(), e16.reset()
    e32.forward([1, 2]), e16.forward([1, 2])
    a, b = e32.forward([3]), e16.forward([3])
    assert oracle.compare(a.reshape(-1), b.reshape(-1), 0.02, 0.02).passed
    assert E.argmax(a[-1]) == E.argmax(b[-1])
    with pytest.raises(ValueError, match="ContextOverflow"):
        e32.forward([4])


def test_fused_matches_ops(ctx, hip, oracle, model, weights):
    """The fused decls against the eight-op engine on p4 (33 tokens, then 4 decode steps)."""
    cfg, w, prompts = model
    p = prompts[4]
    a_eng, b_eng = _engine(ctx, hip, weights, "f16", False), _engine(ctx, hip, weights, "f16", True)
    a, b = a_eng.forward(p["token_ids"]), b_eng.forward(p["token_ids"])
    assert oracle.compare(a.reshape(-1), b.reshape(-1), LAYER_ATOL, LAYER_RTOL).passed
    for t in p["greedy_tokens"][:4]:
        a, b = a_eng.forward([t]), b_eng.forward([t])
        assert oracle.compare(a.reshape(-1), b.reshape(-1), LAYER_ATOL, LAYER_RTOL).passed


def test_engine_rejections(ctx, hip, weights):
    """forward.zig's engine errors: capacity above the model's max_ctx (BadShape,
    test_forward.zig:116-129), an empty or oversized batch, a token id past the
    vocabulary, and a context overflow that leaves pos unchanged (:100-113)."""
    from qw3_amd import engine as E
    with pytest.raises(ValueError, match="BadShape"):
        E.Engine(ctx, weights, max_batch=1, context_capacity=weights.cfg["max_ctx"] + 1)
    eng = _engine(ctx, hip, weights, "f32", False, capacity=2)
    with pytest.raises(ValueError, match="BatchTooLarge"):
        eng.forward([])
    with pytest.raises(ValueError, match="BatchTooLarge"):
        eng.forward([1, 2, 3])
    with pytest.raises(ValueError, match="TokenOutOfRange"):
        eng.forward([weights.cfg["vocab_size"]])
    eng.forward([1, 2])
    assert eng.pos == 2
    with pytest.raises(ValueError, match="ContextOverflow"):
        eng.forward([3])
    assert eng.pos == 2


def test_layer_timing(ctx, hip, model, weights):
    """Per-layer device time of forward passes (kernels/gpu/kernels.zig:442-472
    beginTiming / layerNs, written by main.zig:420-444 as gpu_ns_per_layer_boundary):
    a prefill and a decode step give one positive value per layer each, and they add up
    to no more than the passes' wall time."""
    import time
    from qw3_amd import engine as E
    cfg, _, prompts = model
    eng = _engine(ctx, hip, weights, "f16", True)
    eng.begin_timing()
    t0 = time.perf_counter()
    logits = eng.forward(prompts[0]["token_ids"])
    eng.forward([E.argmax(logits[-1])])
    wall_ns = (time.perf_counter() - t0) * 1e9
    ns = eng.layer_ns()
    print(f"[engine] layer ns: {ns}", flush=True)
    assert len(ns) == 2 * cfg["n_layers"]
    assert all(v > 0 for v in ns)
    assert sum(ns) <= wall_ns
    eng.end_timing()
    eng.forward([1])
    assert eng.layer_ns() == []


def _q8_rows(g, rows, k, scale):
    w = g.integers(0, 256, (rows, k // 32, 34), dtype=np.uint8)
    w[:, :, 0:2] = np.array([scale], np.float16).view(np.uint8)
    return w.reshape(rows, k // 32 * 34)


def _d128_model():
    """A two-layer synthetic model with head_dim 128 (Qwen3's) and Q8_0 weights, so a
    prefill of 16 tokens or more takes the attention block's GEMM-epilogue path."""
    cfg = dict(n_layers=2, hidden_dim=256, n_q_heads=4, n_kv_heads=2, head_dim=128, n_experts=4, top_k=2,
               expert_ffn_dim=128, vocab_size=256, rms_eps=1e-6, rope_theta=1e6, norm_topk_prob=True, max_ctx=64)
    g = np.random.default_rng(31)
    hid, hd, ffn, E = cfg["hidden_dim"], cfg["head_dim"], cfg["expert_ffn_dim"], cfg["n_experts"]
    w = {"token_embd.weight": _q8_rows(g, cfg["vocab_size"], hid, 0.02),
         "output_norm.weight": (1 + 0.02 * g.standard_normal(hid)).astype(np.float32),
         "output.weight": _q8_rows(g, cfg["vocab_size"], hid, 0.002)}
    for li in range(cfg["n_layers"]):
        b = f"blk.{li}."
        w[b + "attn_norm.weight"] = (1 + 0.02 * g.standard_normal(hid)).astype(np.float32)
        w[b + "attn_q.weight"] = _q8_rows(g, cfg["n_q_heads"] * hd, hid, 0.002)
        w[b + "attn_k.weight"] = _q8_rows(g, cfg["n_kv_heads"] * hd, hid, 0.002)
        w[b + "attn_v.weight"] = _q8_rows(g, cfg["n_kv_heads"] * hd, hid, 0.002)
        w[b + "attn_q_norm.weight"] = (1 + 0.02 * g.standard_normal(hd)).astype(np.float32)
        w[b + "attn_k_norm.weight"] = (1 + 0.02 * g.standard_normal(hd)).astype(np.float32)
        w[b + "attn_output.weight"] = _q8_rows(g, hid, cfg["n_q_heads"] * hd, 0.002)
        w[b + "ffn_norm.weight"] = (1 + 0.02 * g.standard_normal(hid)).astype(np.float32)
        w[b + "ffn_gate_inp.weight"] = (0.03 * g.standard_normal((E, hid))).astype(np.float32)
        w[b + "ffn_gate_exps.weight"] = _q8_rows(g, E * ffn, hid, 0.002)
        w[b + "ffn_up_exps.weight"] = _q8_rows(g, E * ffn, hid, 0.002)
        w[b + "ffn_down_exps.weight"] = _q8_rows(g, E * hid, ffn, 0.002)
    return cfg, w


def test_attention_block_inside_engine_d128(ctx, hip):
    """The fused engine at head_dim 128: a 20-token prefill runs the q/k/v projections'
    GEMM with the pre-pass in its epilogue (attentionBlock), then two decode steps at
    pos > 0. With a trace callback the same engine runs matmulGroup then attentionStep
    instead; the ABI says the two are equal bit for bit, so logits and every cache row
    must be."""
    from qw3_amd import engine as E
    cfg, w = _d128_model()
    wts = E.Weights(ctx, w, cfg)
    toks = [int(t) for t in np.random.default_rng(3).integers(0, cfg["vocab_size"], 20)]
    engines = [E.Engine(ctx, wts, max_batch=32, context_capacity=32, kv_dtype=hip.DTYPE_F16, fused=True)
               for _ in range(2)]
    engines[1].trace = lambda layer, op, a: None
    outs = []
    for i, eng in enumerate(engines):
        ctx.set_kernel_timing(True)
        got = [eng.forward(toks)]
        launches = {k: ctx.kernel_time(k)[0] for k in ("matmul_q8_mfma_kernel", "prefill_prep_kernel")}
        ctx.set_kernel_timing(False)
        print(f"[engine] d128 engine {i}: prefill launches {launches}", flush=True)
        if i == 0:  # the block's fused path: the GEMM epilogue, no pre-pass kernel
            assert launches["matmul_q8_mfma_kernel"] >= cfg["n_layers"] and launches["prefill_prep_kernel"] == 0
        else:
            assert launches["prefill_prep_kernel"] == cfg["n_layers"]
        for t in (5, 9):
            got.append(eng.forward([t]))
        caches = [ctx.to_numpy(b, np.uint16) for b in eng.k_cache + eng.v_cache]
        outs.append((got, caches))
    (ga, ca), (gb, cb) = outs
    for a, b in zip(ga, gb):
        assert np.isfinite(a).all()
        assert np.array_equal(a, b)
    for a, b in zip(ca, cb):
        assert np.array_equal(a, b)
