"""ds5_hip_attention_block: the q/k/v projections of the attn_norm output and the
attention step in one call (forward.zig:337-412).

Its contract is ds5_hip_matmul_group(x; wq, wk, wv -> q, k, v) followed by
ds5_hip_attention_step, bit for bit: the attention output and every cache row.
On the fused prefill path (Q8_0 weights on the GEMM path, f16 cache, head_dim
128) the step's pre-pass runs in the projection GEMM's epilogue; the launch
counts show which path ran. The two calls' own parity is pinned elsewhere (the
GEMM against the oracle's matmul, the step against the oracle's step); here the
oracle step also runs on the GPU's projections, so the block's result meets the
step's gates directly.
"""
import numpy as np
import pytest

from conftest import attention_f64
from qw3_amd import synth
from test_gpu_parity import check_cache, check_out

pytestmark = pytest.mark.gpu

KERNELS = ("matmul_x_split_kernel", "matmul_q8_mfma_kernel", "matmul_rows_kernel", "matmul_generic_kernel",
           "prefill_prep_kernel", "prefill_attention_kernel", "decode_split_kernel", "rms_norm_rows_kernel")

# T, pos, n_q_heads, n_kv_heads, head_dim, hidden, weights, fused, oracle check
CASES = {
    "t16": (16, 0, 32, 4, 128, 512, "q8", True, True),
    "t100_pos37": (100, 37, 32, 4, 128, 1024, "q8", True, True),   # ragged row tile, continuation
    "t300_64q": (300, 0, 64, 4, 128, 512, "q8", True, True),       # three row tiles, 16-head groups
    "t130_2group": (130, 3, 8, 4, 128, 256, "q8", True, True),     # 2-head groups
    "c2_hidden2048": (2048, 0, 32, 4, 128, 2048, "q8", True, False),  # the C2 prefill with its projections
    "t8_rows": (8, 0, 32, 4, 128, 512, "q8", False, True),         # row kernel: the two calls
    "t1_decode": (1, 20, 32, 4, 128, 512, "q8", False, True),      # decode: the two calls
    "t1_hidden2048": (1, 40, 32, 4, 128, 2048, "q8", False, True),  # decode at the Qwen3-30B-A3B width
    "f32_weights": (40, 0, 32, 4, 128, 256, "f32", False, True),
    "d64": (64, 0, 32, 4, 64, 256, "q8", False, True),             # head_dim 64: the two calls
}


def _weights(oracle, g, n, k, dt):
    wf = g.standard_normal((n, k)).astype(np.float32) * np.float32(0.05)
    return oracle.q8_0_quantize(wf) if dt == "q8" else wf


class _Inputs:
    def __init__(self, ctx, hip, oracle, case):
        T, pos, hq, hkv, hd, hidden, dt, _, _ = CASES[case]
        self.T, self.pos, self.hq, self.hkv, self.hd, self.hidden = T, pos, hq, hkv, hd, hidden
        self.s = synth.Shape(n_q_heads=hq, n_kv_heads=hkv, head_dim=hd)
        self.cap = pos + T + 5
        g = np.random.default_rng(sum(map(ord, case)))
        self.x = g.standard_normal((T, hidden)).astype(np.float32)
        self.dtype = hip.DTYPE_Q8_0 if dt == "q8" else hip.DTYPE_F32
        self.w = [_weights(oracle, g, n * hd, hidden, dt) for n in (hq, hkv, hkv)]
        _, _, _, self.qn, self.kn = synth.step_inputs(2, T, 1, self.s)
        self.kc, self.vc = synth.cache_f16(2, T, self.s, self.cap, pos)
        self.positions = np.arange(pos, pos + T, dtype=np.int32)
        self.xb = ctx.from_numpy(self.x)
        self.wb = [ctx.from_numpy(w) for w in self.w]
        self.qnb, self.knb, self.pb = ctx.from_numpy(self.qn), ctx.from_numpy(self.kn), ctx.from_numpy(self.positions)

    def step_args(self, ctx, hip):
        """Fresh q/k/v scratch, caches holding the initial rows, output."""
        T, hq, hkv, hd = self.T, self.hq, self.hkv, self.hd
        q, k, v = (ctx.createBuffer(T * h * hd * 4) for h in (hq, hkv, hkv))
        kcb, vcb = ctx.from_numpy(self.kc), ctx.from_numpy(self.vc)
        out = ctx.createBuffer(T * hq * hd * 4)
        s = self.s
        return hip.AttentionStepArgs(q, k, v, self.qnb, self.knb, self.pb, kcb, vcb, out, 1, self.pos, T, hq, hkv,
                                     hd, self.cap, s.eps, s.theta, 1.0, s.scale)

    def results(self, ctx, a):
        out = ctx.to_numpy(a.out, np.float32, (self.T, self.hq, self.hd))
        kc = ctx.to_numpy(a.k_cache, np.uint16, self.kc.shape)
        vc = ctx.to_numpy(a.v_cache, np.uint16, self.vc.shape)
        return out, kc, vc


def _counted(ctx, fn):
    ctx.set_kernel_timing(True)
    try:
        fn()
        ctx.submit()
        return {kn: ctx.kernel_time(kn)[0] for kn in KERNELS}
    finally:
        ctx.set_kernel_timing(False)


@pytest.mark.parametrize("case", list(CASES))
def test_attention_block_equals_the_two_calls(ctx, hip, oracle, case):
    inp = _Inputs(ctx, hip, oracle, case)
    T, hq, hkv, hd, hidden = inp.T, inp.hq, inp.hkv, inp.hd, inp.hidden
    fused, check_oracle = CASES[case][7], CASES[case][8]
    print(f"  case {case}: T={T} pos={inp.pos} {hq}q/{hkv}kv d{hd} hidden={hidden}", flush=True)

    blk = inp.step_args(ctx, hip)
    block = hip.AttentionBlockArgs(inp.xb, *inp.wb, inp.dtype, hidden, blk)
    counts = _counted(ctx, lambda: hip.attentionBlock(ctx, block))
    print(f"  launches: { {k: c for k, c in counts.items() if c} }", flush=True)
    if fused:  # the pre-pass is the GEMM's epilogue: no prep launch, one split and one GEMM
        assert counts["matmul_q8_mfma_kernel"] == 1 and counts["matmul_x_split_kernel"] == 1
        assert counts["prefill_prep_kernel"] == 0 and counts["prefill_attention_kernel"] == 1
    else:
        assert counts["prefill_prep_kernel"] + counts["decode_split_kernel"] + counts["rms_norm_rows_kernel"] >= 1

    two = inp.step_args(ctx, hip)
    hip.matmulGroup(ctx, hip.MatmulGroupArgs.of(inp.xb, inp.dtype, T, hidden,
                                                [(inp.wb[0], two.q, hq * hd), (inp.wb[1], two.k, hkv * hd),
                                                 (inp.wb[2], two.v, hkv * hd)]))
    proj = [ctx.to_numpy(b, np.float32, (T, h, hd)) for b, h in ((two.q, hq), (two.k, hkv), (two.v, hkv))]
    hip.attentionStep(ctx, two)

    got, want = inp.results(ctx, blk), inp.results(ctx, two)
    for name, a, b in zip(("out", "k_cache", "v_cache"), got, want):
        same = a.view(np.uint32 if a.dtype == np.float32 else np.uint16) == \
            b.view(np.uint32 if b.dtype == np.float32 else np.uint16)
        print(f"  {name}: {int((~same).sum())} of {same.size} differ from the two calls", flush=True)
        assert same.all()

    out, gk, gv = got
    if check_oracle:  # the oracle step on the GPU's projections
        kc, vc = inp.kc.copy(), inp.vc.copy()
        wout, _, _ = oracle.attention_step(*proj, inp.qn, inp.kn, inp.positions, kc, vc, kv_dtype=1, pos=inp.pos,
                                           n_tokens=T, n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, max_ctx=inp.cap,
                                           eps=inp.s.eps, theta=inp.s.theta, scale=inp.s.scale)
        check_cache(gk, gv, kc, vc, inp.kc, inp.vc, inp.pos, T)
        check_out(out, wout)
    else:  # full size: every cache row against the oracle's norm + rope + append, four heads in float64
        s = inp.s
        q, k, v = proj
        k_rot = oracle.rope(oracle.rms_norm(k, inp.kn, s.eps), inp.positions, s.theta)
        wk, wv = inp.kc.copy(), inp.vc.copy()
        oracle.kv_append(k_rot, v, wk, wv, 1, inp.pos, T, hkv, hd, inp.cap)
        check_cache(gk, gv, wk, wv, inp.kc, inp.vc, inp.pos, T)
        q_rot = oracle.rope(oracle.rms_norm(q, inp.qn, s.eps), inp.positions, s.theta)
        group = hq // hkv
        for h in (0, 9, 18, 31):
            check_out(out[:, h], attention_f64(q_rot[:, h], wk[h // group][:T], wv[h // group][:T], s.scale))


def test_attention_block_errors(ctx, hip, oracle):
    """Preconditions are the two calls', projections first; nothing runs on a failed check."""
    inp = _Inputs(ctx, hip, oracle, "t16")
    a = inp.step_args(ctx, hip)
    bad_w = inp.wb[1].view(0, inp.wb[1].len - 1)  # wk one byte short
    with pytest.raises(hip.KernelError):
        hip.attentionBlock(ctx, hip.AttentionBlockArgs(inp.xb, inp.wb[0], bad_w, inp.wb[2], inp.dtype, inp.hidden, a))
    a.max_ctx = inp.T - 1  # the step's cache bound
    with pytest.raises(hip.KernelError):
        hip.attentionBlock(ctx, hip.AttentionBlockArgs(inp.xb, *inp.wb, inp.dtype, inp.hidden, a))
    ctx.submit()
    assert np.array_equal(ctx.to_numpy(a.k_cache, np.uint16, inp.kc.shape), inp.kc)
    assert np.array_equal(ctx.to_numpy(a.v_cache, np.uint16, inp.vc.shape), inp.vc)


@pytest.mark.parametrize("case", ["t16", "t300_64q", "c2_hidden2048", "t8_rows", "t1_decode", "f32_weights",
                                  "t130_2group", "d64", "t1_hidden2048"])
def test_attention_block_with_norm(ctx, hip, oracle, case):
    """The block with x_norm (attn_norm applied first) equals ds5_hip_rms_norm(x -> h) then
    the block on h, bit for bit (output and every cache row): the norm inside the row
    kernel (decode), inside the GEMM's x split (prefill), or written to the context's
    second buffer (hidden <= 256: the serial order; the other paths). The raw x has rows
    of widely varying magnitude, so the norm is not the identity."""
    inp = _Inputs(ctx, hip, oracle, case)
    T, hidden = inp.T, inp.hidden
    g = np.random.default_rng(7 + T)
    x = (inp.x * np.exp(g.uniform(-3, 3, (T, 1)))).astype(np.float32)
    nw = (1.0 + 0.05 * g.standard_normal(hidden)).astype(np.float32)
    xb, nwb = ctx.from_numpy(x), ctx.from_numpy(nw)
    eps = 1e-6
    print(f"  case {case}: T={T} hidden={hidden}", flush=True)
    a = inp.step_args(ctx, hip)
    hip.attentionBlock(ctx, hip.AttentionBlockArgs(xb, *inp.wb, inp.dtype, hidden, a, nwb, eps))
    h = ctx.createBuffer(T * hidden * 4)
    hip.rmsNorm(ctx, hip.RmsNormArgs(xb, nwb, h, T, hidden, eps))
    b = inp.step_args(ctx, hip)
    hip.attentionBlock(ctx, hip.AttentionBlockArgs(h, *inp.wb, inp.dtype, hidden, b))
    for name, p, q in zip(("out", "k_cache", "v_cache"), inp.results(ctx, a), inp.results(ctx, b)):
        same = p.view(np.uint8) == q.view(np.uint8)
        print(f"  {name}: {int((~same).sum())} bytes differ", flush=True)
        assert same.all()
    assert np.array_equal(ctx.to_numpy(xb, np.float32, x.shape), x)  # x itself is left as it was
    with pytest.raises(hip.ShapeMismatch):
        hip.attentionBlock(ctx, hip.AttentionBlockArgs(xb, *inp.wb, inp.dtype, hidden, inp.step_args(ctx, hip),
                                                       hip.Buf(nwb.handle, nwb.offset, hidden * 4 - 4), eps))


@pytest.mark.parametrize("case", ["t300_64q", "t8_rows"])
def test_attention_block_graph_replays(ctx, hip, oracle, case):
    """The block captured into a HIP graph (fused prefill path and the two-call path),
    replayed three times with eager work and synchronisations between the replays:
    every replay's output and cache rows equal the eager call's, bit for bit."""
    inp = _Inputs(ctx, hip, oracle, case)
    a = inp.step_args(ctx, hip)
    block = hip.AttentionBlockArgs(inp.xb, *inp.wb, inp.dtype, inp.hidden, a)
    hip.attentionBlock(ctx, block)  # eager; also sizes the workspace before the capture
    want = inp.results(ctx, a)
    other = inp.step_args(ctx, hip)
    g = ctx.capture(lambda: hip.attentionBlock(ctx, block))
    try:
        for r in range(3):
            ctx.upload(a.out, 0, np.zeros(inp.T * inp.hq * inp.hd, np.float32))
            ctx.upload(a.k_cache, 0, inp.kc)  # the replay appends the same rows again
            ctx.upload(a.v_cache, 0, inp.vc)
            hip.attentionBlock(ctx, hip.AttentionBlockArgs(inp.xb, *inp.wb, inp.dtype, inp.hidden, other))
            ctx.submit()
            g.launch()
            ctx.submit()
            got = inp.results(ctx, a)
            same = [np.array_equal(x.view(np.uint8), y.view(np.uint8)) for x, y in zip(got, want)]
            print(f"  replay {r}: out/k/v bit-identical {same}", flush=True)
            assert all(same)
        assert all(np.array_equal(x.view(np.uint8), y.view(np.uint8)) for x, y in zip(inp.results(ctx, other), want))
    finally:
        g.destroy()
