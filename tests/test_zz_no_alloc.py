"""The allocation-free attention step (ds5_hip_attention_step_noalloc) against
ds5_hip_attention_step, through the C ABI: the same kernels run, only the
split-K partials / f16 q operand live in the library's static per-GPU scratch,
so outputs and cache rows must be bit-identical. Two calls in a row, the second
smaller, check that the array keeps nothing that matters between calls; a call
needing more scratch than the array holds is rejected before any device work;
a capture on a fresh context (no workspace ever allocated) replays correctly."""
import numpy as np
import pytest

from qw3_amd import synth

pytestmark = pytest.mark.gpu


def _inputs(config, layer, s, cap, pos, T):
    if T == 1:
        q, k, v, qn, kn = synth.step_inputs(config, layer, 1, s)
    else:
        q, k, v, qn, kn = synth.step_inputs(config, layer, T, s, f16_exact=True)
    kc, vc = synth.cache_f16(config, layer, s, cap, pos)
    return q, k, v, qn, kn, np.arange(pos, pos + T, dtype=np.int32), kc, vc


def _run(ctx, hip, fn, inp, s, pos, T):
    q, k, v, qn, kn, positions, kc, vc = inp
    hq, hd = q.shape[1], q.shape[2]
    hkv, cap = kc.shape[0], kc.shape[1]
    bufs = [ctx.from_numpy(np.ascontiguousarray(a)) for a in (q, k, v, qn, kn, positions, kc, vc)]
    out = ctx.createBuffer(T * hq * hd * 4)
    args = hip.AttentionStepArgs(*bufs, out, hip.DTYPE_F16, pos, T, hq, hkv, hd, cap, s.eps, s.theta, 1.0, s.scale)
    fn(ctx, args)
    return (ctx.to_numpy(out, np.float32), ctx.to_numpy(bufs[6], np.uint16, kc.shape),
            ctx.to_numpy(bufs[7], np.uint16, vc.shape))


def _same(a, b):
    for x, y in zip(a, b):
        assert np.array_equal(x.view(np.uint32) if x.dtype == np.float32 else x,
                              y.view(np.uint32) if y.dtype == np.float32 else y)


# (config of the seeded inputs, shape, cap, pos, T): C1's decode (64 splits, 1.06 MB of
# partials), then smaller calls: a 1000-position decode, a 16-head group and a 64-token prefill
CASES = [
    (1, synth.CONFIGS[1]["shape"], 8192, 8191, 1),
    (1, synth.CONFIGS[1]["shape"], 1024, 999, 1),
    (3, synth.CONFIGS[3]["shape"], 4096, 4000, 1),
    (2, synth.CONFIGS[2]["shape"], 80, 0, 64),
]


@pytest.mark.parametrize("first,second", [(0, 1), (0, 2), (2, 3), (0, 0)])
def test_noalloc_matches_step_two_calls(ctx, hip, first, second):
    for i in (first, second):
        config, s, cap, pos, T = CASES[i]
        inp = _inputs(config, i, s, cap, pos, T)
        want = _run(ctx, hip, hip.attentionStep, inp, s, pos, T)
        got = _run(ctx, hip, hip.attentionStepNoAlloc, inp, s, pos, T)
        print(f"  case {i}: T={T} pos={pos} hq={s.n_q_heads} max|out|={np.abs(want[0]).max():.3f}", flush=True)
        _same(got, want)


def test_noalloc_rejects_oversize_before_device_work(ctx, hip):
    """A fused prefill step of 8193 tokens needs its rope table, 8193 x 128 f32 (just
    over 4 MiB): more than the scratch holds. Nothing runs, nothing is appended."""
    s = synth.CONFIGS[2]["shape"]
    T = cap = 8193
    pos = 0
    assert T * s.head_dim * 4 > hip.NOALLOC_SCRATCH_BYTES
    rng = np.random.default_rng(7)
    q = np.ones((T, s.n_q_heads, s.head_dim), np.float32)
    k = np.ones((T, s.n_kv_heads, s.head_dim), np.float32)
    v = np.ones((T, s.n_kv_heads, s.head_dim), np.float32)
    qn = np.ones(s.head_dim, np.float32)
    kn = np.ones(s.head_dim, np.float32)
    positions = np.arange(T, dtype=np.int32)
    kc = rng.integers(0, 0x7800, (s.n_kv_heads, cap, s.head_dim), dtype=np.uint16)
    vc = kc.copy()
    bufs = [ctx.from_numpy(np.ascontiguousarray(a)) for a in (q, k, v, qn, kn, positions, kc, vc)]
    out = ctx.createBuffer(T * s.n_q_heads * s.head_dim * 4)
    args = hip.AttentionStepArgs(*bufs, out, hip.DTYPE_F16, pos, T, s.n_q_heads, s.n_kv_heads, s.head_dim, cap,
                                 s.eps, s.theta, 1.0, s.scale)
    with pytest.raises(hip.ShapeMismatch, match="scratch"):
        hip.attentionStepNoAlloc(ctx, args)
    assert np.array_equal(ctx.to_numpy(bufs[6], np.uint16, kc.shape), kc)  # nothing appended
    assert not ctx.to_numpy(out, np.float32).any()


def test_noalloc_captured_on_fresh_context(hip):
    """A fresh context has no workspace; the allocation-free call can be captured
    directly (the workspace-backed call would have to grow inside the capture)."""
    config, s, cap, pos, T = CASES[0]
    inp = _inputs(config, 0, s, cap, pos, T)
    ref_ctx = hip.Ctx.init(0)
    try:
        want = _run(ref_ctx, hip, hip.attentionStep, inp, s, pos, T)
    finally:
        ref_ctx.deinit()
    c = hip.Ctx.init(0)
    try:
        q, k, v, qn, kn, positions, kc, vc = inp
        bufs = [c.from_numpy(np.ascontiguousarray(a)) for a in (q, k, v, qn, kn, positions, kc, vc)]
        out = c.createBuffer(s.n_q_heads * s.head_dim * 4)
        args = hip.AttentionStepArgs(*bufs, out, hip.DTYPE_F16, pos, T, s.n_q_heads, s.n_kv_heads, s.head_dim,
                                     cap, s.eps, s.theta, 1.0, s.scale)
        g = c.capture(lambda: hip.attentionStepNoAlloc(c, args))
        try:
            for _ in range(3):
                c.upload(out, 0, np.zeros(s.n_q_heads * s.head_dim, np.float32))  # eager work between replays
                c.submit()
                g.launch()
                c.submit()
                assert np.array_equal(c.to_numpy(out, np.float32).view(np.uint32), want[0].view(np.uint32))
        finally:
            g.destroy()
    finally:
        c.deinit()
