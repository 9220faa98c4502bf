"""Pins the CPU oracle (oracle/ds5_oracle.c) before anything is compared to it.

1. The reference's own golden fixtures (tests/golden/ds5_synthetic, vendored
   from the reference's tests/fixtures/synthetic) under the reference's pass
   rule and tolerances: the fixture tests of kernels_a.zig:281-376 (rmsnorm,
   rope) and kernels_b.zig:164-226 (attention), with the same case counts.
2. Ports of the reference's hand-built semantic tests (kernels_a.zig:455-522,
   :619-701; kernels_b.zig:228-492).
3. Checks fixed by mathematics rather than by retyping the formula: float64
   brute force, closed forms, invariants, and library routines
   (numpy's float16 cast, the C library's correctly rounded powf).
"""
import math

import ctypes as C

import numpy as np
import pytest

from conftest import FIXTURES

# ---------------------------------------------------------------------------
# 1. golden fixtures
# ---------------------------------------------------------------------------


def _cases(O, op):
    m = O.load_manifest(FIXTURES)
    return [c for c in m["cases"] if c["op"] == op]


def _t(O, case, name):
    return O.load_ds5t(f"{FIXTURES}/{case['tensors'][name]}")


def test_fixture_case_counts(oracle):
    # kernels_a.zig:335 (6 rmsnorm), :376 (3 rope), :457 (4 matmul_quant); kernels_b.zig:225 (6 attention)
    assert len(_cases(oracle, "rmsnorm")) == 6
    assert len(_cases(oracle, "rope")) == 3
    assert len(_cases(oracle, "attention")) == 6
    assert len(_cases(oracle, "matmul_quant")) == 4
    assert len(_cases(oracle, "router")) == 3  # kernels_c.zig:317
    assert len(_cases(oracle, "expert_mlp")) == 3  # kernels_c.zig:400


@pytest.mark.parametrize("i", range(4))
def test_matmul_quant_fixtures(oracle, i):
    """kernels_a.zig:395-458: Q8_0 matmul within the case tolerance; the tensors'
    shapes as the reference test checks them (input ne {k, m}, weight {k, n}, output {n, m})."""
    c = _cases(oracle, "matmul_quant")[i]
    p, tol = c["params"], c["tolerance"]
    x, w, want = (_t(oracle, c, n) for n in ("input", "weight", "output"))
    assert x.ne == (p["k"], p["m"]) and w.ne == (p["k"], p["n"]) and want.ne == (p["n"], p["m"])
    assert w.dtype == oracle.Q8_0 and p["w_dtype"] == "q8_0"
    got = oracle.matmul(x.data, w.data, oracle.Q8_0, p["m"], p["n"], p["k"])
    r = oracle.compare(want.data, got, tol["atol"], tol["rtol"])
    assert r.passed, r


@pytest.mark.parametrize("i", range(6))
def test_rmsnorm_fixtures(oracle, i):
    c = _cases(oracle, "rmsnorm")[i]
    p, tol = c["params"], c["tolerance"]
    x, w, want = (_t(oracle, c, n) for n in ("input", "weight", "output"))
    assert x.ne[0] == p["dim"]
    got = oracle.rms_norm(x.data, w.data, p["eps"], p["n_rows"], p["dim"])
    r = oracle.compare(want.data, got, tol["atol"], tol["rtol"])
    assert r.passed, r


@pytest.mark.parametrize("i", range(3))
def test_rope_fixtures(oracle, i):
    c = _cases(oracle, "rope")[i]
    p, tol = c["params"], c["tolerance"]
    x, pos, want = (_t(oracle, c, n) for n in ("input", "positions", "output"))
    assert x.ne[:3] == (p["head_dim"], p["n_heads"], p["n_tokens"])
    assert pos.dtype == oracle.I32
    got = oracle.rope(x.data, pos.data, p["theta"], p["freq_scale"])
    r = oracle.compare(want.data, got, tol["atol"], tol["rtol"])
    assert r.passed, r


@pytest.mark.parametrize("i", range(6))
def test_attention_fixtures(oracle, i):
    c = _cases(oracle, "attention")[i]
    p, tol = c["params"], c["tolerance"]
    q, kc, vc, want = (_t(oracle, c, n) for n in ("q", "k_cache", "v_cache", "output"))
    kv_dtype = p.get("kv_dtype", oracle.F32)  # kernels_b.zig:188 default
    got = oracle.gqa_attention(q.data, kc.data, vc.data, kv_dtype, p["pos"], p["n_tokens"], p["n_q_heads"],
                               p["n_kv_heads"], p["head_dim"], p["max_ctx"], p["scale"])
    r = oracle.compare(want.data, got, tol["atol"], tol["rtol"])
    assert r.passed, r


def test_compare_rule_rejects_nan_and_out_of_tolerance(oracle):
    o = np.array([1.0, 2.0, 0.0], np.float32)
    assert oracle.compare(o, o, 0, 0).passed
    assert not oracle.compare(o, np.array([1.0, np.nan, 0.0], np.float32), 1, 1).passed
    r = oracle.compare(o, np.array([1.0, 2.0 + 2e-4, 0.0], np.float32), 1e-4, 0.0)
    assert not r.passed and r.first_bad == 1
    assert oracle.compare(o, np.array([1.0, 2.0 + 2e-4, 0.0], np.float32), 0.0, 1.5e-4).passed


def test_ds5t_roundtrip(oracle, tmp_path):
    a = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    oracle.write_ds5t(str(tmp_path / "a.ds5t"), a, oracle.F32)
    t = oracle.load_ds5t(str(tmp_path / "a.ds5t"))
    assert t.ne == (4, 3, 2) and np.array_equal(t.data, a)
    raw = bytearray((tmp_path / "a.ds5t").read_bytes())
    raw[0] ^= 1
    (tmp_path / "b.ds5t").write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="BadMagic"):
        oracle.load_ds5t(str(tmp_path / "b.ds5t"))


# ---------------------------------------------------------------------------
# 2. hand-built reference tests
# ---------------------------------------------------------------------------


def test_rmsnorm_hand_case_aliasing(oracle):
    # kernels_a.zig:455-484: rows {3,4}, {-1,1}; w {2, 0.5}; out aliases x.
    x = np.array([3, 4, -1, 1], np.float32)
    w = np.array([2.0, 0.5], np.float32)
    oracle.rms_norm(x, w, 1e-6, 2, 2, out=x)
    inv0 = 1.0 / math.sqrt(12.5 + 1e-6)
    inv1 = 1.0 / math.sqrt(1.0 + 1e-6)
    np.testing.assert_allclose(x, [3 * inv0 * 2, 4 * inv0 * 0.5, -1 * inv1 * 2, 1 * inv1 * 0.5], atol=1e-6)


def test_rope_hand_case(oracle):
    # kernels_a.zig:486-522: pos 0 is the identity; pos 3 closed-form angles.
    x = np.array([1, 2, 3, 4, 1, 0, 0, 1], np.float32).reshape(2, 1, 4)
    y = oracle.rope(x, np.array([0, 3], np.int32), 100.0)
    np.testing.assert_array_equal(y[0], x[0])
    a1 = 3.0 * 100.0 ** -0.5
    np.testing.assert_allclose(y[1, 0], [math.cos(3.0), -math.sin(a1), math.sin(3.0), math.cos(a1)], atol=1e-6)


@pytest.mark.parametrize("kv_dtype", [0, 1])
def test_kv_append_sentinel_roundtrip(oracle, kv_dtype):
    # kernels_a.zig:619-683 (f32) and the same for f16: only slots pos..pos+T-1 change.
    hkv, hd, cap, pos, T = 2, 4, 8, 3, 2
    if kv_dtype == 0:
        kc = -np.arange(hkv * cap * hd, dtype=np.float32)
        vc = -1000.0 - np.arange(hkv * cap * hd, dtype=np.float32)
    else:
        kc = np.arange(hkv * cap * hd, dtype=np.uint16) + 0x3000
        vc = np.arange(hkv * cap * hd, dtype=np.uint16) + 0xB000
    k0, v0 = kc.copy(), vc.copy()
    t, h, d = np.meshgrid(np.arange(T), np.arange(hkv), np.arange(hd), indexing="ij")
    kn = (100 * t + 10 * h + d).astype(np.float32)
    vn = -kn - 0.5
    oracle.kv_append(kn, vn, kc, vc, kv_dtype, pos, T, hkv, hd, cap)
    conv = (lambda a: a) if kv_dtype == 0 else oracle.f32_to_f16_bits
    kc3, vc3 = kc.reshape(hkv, cap, hd), vc.reshape(hkv, cap, hd)
    k03, v03 = k0.reshape(hkv, cap, hd), v0.reshape(hkv, cap, hd)
    for hh in range(hkv):
        for p in range(cap):
            if pos <= p < pos + T:
                np.testing.assert_array_equal(kc3[hh, p], conv(kn[p - pos, hh]))
                np.testing.assert_array_equal(vc3[hh, p], conv(vn[p - pos, hh]))
            else:
                np.testing.assert_array_equal(kc3[hh, p], k03[hh, p])
                np.testing.assert_array_equal(vc3[hh, p], v03[hh, p])


def test_kv_append_rejects_overflow_and_dtype(oracle):
    z = np.zeros(64, np.float32)
    with pytest.raises(oracle.KernelError) as e:   # kernels_a.zig:685-701
        oracle.kv_append(z, z, z, z, 0, 7, 2, 1, 4, 8)
    assert e.value.code == oracle.SHAPE_MISMATCH
    with pytest.raises(oracle.KernelError) as e:
        oracle.kv_append(z, z, z, z, 8, 0, 1, 1, 4, 8)  # q8_0 cache
    assert e.value.code == oracle.UNSUPPORTED_DTYPE


def test_attention_pos0_returns_v0_nan_tail(oracle):
    # kernels_b.zig:228-282: pos 0 -> out == v[kv_head, 0]; NaN beyond proves mask + stride.
    hq, hkv, hd, cap = 4, 2, 4, 3
    g = np.random.default_rng(1)
    q = g.standard_normal(hq * hd).astype(np.float32)
    k = np.full((hkv, cap, hd), np.nan, np.float32)
    v = np.full((hkv, cap, hd), np.nan, np.float32)
    k[:, 0] = g.standard_normal((hkv, hd))
    for kh in range(hkv):
        v[kh, 0] = kh * 100 + np.arange(hd)
    out = oracle.gqa_attention(q, k, v, 0, 0, 1, hq, hkv, hd, cap, 0.5)
    for h in range(hq):
        np.testing.assert_allclose(out[h * hd:(h + 1) * hd], (h // 2) * 100 + np.arange(hd), atol=1e-6)


def test_attention_ragged_pos_packed_equivalence(oracle):
    # kernels_b.zig:284-373: max_ctx stride, causality, bitwise packed == strided.
    hq, hkv, hd, pos, T, big = 4, 2, 8, 2, 2, 8
    valid = pos + T
    g = np.random.default_rng(42)
    q = g.standard_normal((T, hq, hd)).astype(np.float32)
    kp = g.standard_normal((hkv, valid, hd)).astype(np.float32)
    vp = g.standard_normal((hkv, valid, hd)).astype(np.float32)
    kb = np.full((hkv, big, hd), np.nan, np.float32)
    vb = np.full((hkv, big, hd), np.nan, np.float32)
    kb[:, :valid], vb[:, :valid] = kp, vp
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    a = oracle.gqa_attention(q, kp, vp, 0, pos, T, hq, hkv, hd, valid, scale)
    b = oracle.gqa_attention(q, kb, vb, 0, pos, T, hq, hkv, hd, big, scale)
    assert np.array_equal(a, b)
    kb[:, 3] += 1.5
    vb[:, 3] -= 2.0
    c = oracle.gqa_attention(q, kb, vb, 0, pos, T, hq, hkv, hd, big, scale)
    row = hq * hd
    assert np.array_equal(b[:row], c[:row]) and not np.array_equal(b[row:], c[row:])


def test_attention_mha_analytic(oracle):
    # kernels_b.zig:375-422
    q = np.array([1, 0, 0, 1], np.float32)
    k = np.array([1, 0, -1, 0, 0, 0, 0, 2], np.float32)
    v = np.array([10, 20, 30, 40, -1, 1, -3, 3], np.float32)
    out = oracle.gqa_attention(q, k, v, 0, 1, 1, 2, 2, 2, 2, 1.0)
    p0 = math.e / (math.e + math.exp(-1))
    p1 = 1 / (1 + math.exp(2))
    np.testing.assert_allclose(out, [p0 * 10 + (1 - p0) * 30, p0 * 20 + (1 - p0) * 40,
                                     p1 * -1 + (1 - p1) * -3, p1 * 1 + (1 - p1) * 3], atol=1e-5)


def test_attention_softmax_stability(oracle):
    # kernels_b.zig:424-454: scores +-200 stay finite.
    out = oracle.gqa_attention(np.array([100, 0], np.float32), np.array([-2, 0, 2, 0], np.float32),
                               np.array([7, -7, 3.5, -3.5], np.float32), 0, 1, 1, 1, 1, 2, 2, 1.0)
    np.testing.assert_allclose(out, [3.5, -3.5], atol=1e-6)


def test_attention_shape_rejections(oracle):
    # kernels_b.zig:456-492
    mem = np.zeros(64, np.float32)
    base = dict(pos=0, n_tokens=1, n_q_heads=2, n_kv_heads=2, head_dim=4, max_ctx=8, scale=0.5)

    def run(**kw):
        a = {**base, **kw}
        oracle.gqa_attention(mem, mem, mem, 0, a["pos"], a["n_tokens"], a["n_q_heads"], a["n_kv_heads"],
                             a["head_dim"], a["max_ctx"], a["scale"], out=mem)

    for kw in (dict(pos=8), dict(n_q_heads=3, n_kv_heads=2), dict(max_ctx=64)):
        with pytest.raises(oracle.KernelError) as e:
            run(**kw)
        assert e.value.code == oracle.SHAPE_MISMATCH


# ---------------------------------------------------------------------------
# 3. checks fixed by mathematics / library routines
# ---------------------------------------------------------------------------


def test_f16_cast_matches_numpy_rne(oracle):
    g = np.random.default_rng(7)
    bits = g.integers(0, 2 ** 32, size=400_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    edge = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 6.103515625e-05, 6.097555160522461e-05,
                     2.9802322387695312e-08, 2.98023259e-08, 5.960464477539063e-08, 8.940696716308594e-08,
                     1.0009765625, 1.00048828125, 1.00146484375, np.inf, -np.inf], np.float32)
    x = np.concatenate([x, edge, g.standard_normal(100_000).astype(np.float32) * 1e-5])
    finite = ~np.isnan(x)
    with np.errstate(over="ignore"):
        want = x[finite].astype(np.float16).view(np.uint16)
    got = oracle.f32_to_f16_bits(x[finite])
    assert np.array_equal(got, want)
    nan_bits = oracle.f32_to_f16_bits(x[~finite])
    assert np.all((nan_bits & 0x7C00) == 0x7C00) and np.all(nan_bits & 0x3FF)
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    wide = oracle.f16_bits_to_f32(allh)
    ref = allh.view(np.float16).astype(np.float32)
    same = (wide.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(wide) & np.isnan(ref))
    assert same.all()


def test_zig_pow_special_cases_and_accuracy(oracle):
    assert oracle.zig_powf(1e6, 0.0) == 1.0 and oracle.zig_powf(1e6, -0.0) == 1.0
    assert oracle.zig_powf(1.0, -0.3) == 1.0
    assert oracle.zig_powf(7.5, 1.0) == 7.5
    assert oracle.zig_powf(1e6, -0.5) == np.float32(1.0) / np.sqrt(np.float32(1e6))
    assert oracle.zig_powf(2.0, -1.0) == 0.5 and oracle.zig_powf(2.0, 3.0) == 8.0
    # Every rope exponent the configs use, against the exact value: within a few f32 ulp.
    for theta in (1e6, 5e6, 1e4, 100.0):
        for hd in (64, 128):
            for i in range(hd // 2):
                e = np.float32(2 * i) / np.float32(hd)
                got = np.float32(oracle.zig_powf(theta, -e))
                exact = float(np.float32(theta)) ** -float(e)
                ulp = np.spacing(np.float32(exact))
                assert abs(float(got) - exact) <= 8 * ulp, (theta, hd, i)


def test_rmsnorm_matches_float64(oracle):
    g = np.random.default_rng(3)
    x = g.standard_normal((37, 128)).astype(np.float32) * 3
    w = (1 + 0.02 * g.standard_normal(128)).astype(np.float32)
    got = oracle.rms_norm(x, w, 1e-6)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-6)


# rmsNorm in the reference GPU kernel's order (kernels_a.metal:127-165), the order
# ds5_hip_rms_norm uses for rows of more than 256 elements.

def _norm_from_sum(x, w, s, eps):
    """(x * inv) * w with inv = 1 / sqrt(s / dim + eps), each step rounded to f32 (numpy's
    float32 operations round correctly)."""
    dim = np.float32(x.size)
    inv = np.float32(1.0) / np.sqrt(np.float32(s) / dim + np.float32(eps))
    return (x * inv) * w


def test_rmsnorm_tree_reduction_order(oracle):
    """Rows whose f32 sum depends on the order: 4096^2 = 2^24 absorbs a lone 1 (a tie,
    rounded to even) but not a 2. With ones at elements 1 and 3, the kernel's order (thread
    t takes elements t, t + 256, ...; partials halve as p[t] += p[t + s], s = 128 .. 1)
    adds p[3] into p[1] before p[1] meets p[0]: the sum is 2^24 + 2. The serial order, an
    adjacent-pair tree and contiguous per-thread chunks each meet the ones one at a time
    and leave 2^24."""
    dim, eps = 512, 1e-6
    x = np.zeros(dim, np.float32)
    x[0], x[1], x[3] = 4096.0, 1.0, 1.0
    w = np.linspace(0.5, 1.5, dim).astype(np.float32)
    got = oracle.rms_norm_tree(x.copy(), w, eps)
    assert np.array_equal(got, _norm_from_sum(x, w, 2.0 ** 24 + 2, eps))
    serial = oracle.rms_norm(x.copy(), w, eps)
    assert np.array_equal(serial, _norm_from_sum(x, w, 2.0 ** 24, eps))
    assert not np.array_equal(got, serial)


def test_rmsnorm_tree_accumulates_with_fma(oracle):
    """A thread's second element is added with one rounding (s = fma(b, b, a^2)): for
    rows holding only x[0] = 1 and x[256] = b, the sum is f32(1 + b^2) computed exactly
    (b^2 has 48 bits, exact in float64), which differs from f32(f32(b^2) + 1) for these b."""
    dim, eps = 300, 1e-6
    w = np.ones(dim, np.float32)
    n = 0
    for b in np.float32(1.0) + np.arange(1, 4000, dtype=np.float32) * np.float32(2.0 ** -23):
        fused = np.float32(1.0 + float(b) * float(b))
        unfused = np.float32(np.float32(b * b) + np.float32(1.0))
        if fused == unfused:
            continue
        x = np.zeros(dim, np.float32)
        x[0], x[256] = 1.0, b
        got = oracle.rms_norm_tree(x.copy(), w, eps)
        assert np.array_equal(got, _norm_from_sum(x, w, fused, eps)), b
        n += 1
        if n == 8:
            break
    assert n == 8


def test_rmsnorm_tree_exact_sums_equal_serial(oracle):
    """Small-integer rows: every partial sum is an exact integer, so any order gives the
    same sum; the tree must then equal the serial form bit for bit (no element dropped or
    counted twice at dims that are not multiples of 256)."""
    g = np.random.default_rng(17)
    for dim in (257, 300, 511, 1000, 4097):
        x = g.integers(-3, 4, (3, dim)).astype(np.float32)
        w = (1 + 0.02 * g.standard_normal(dim)).astype(np.float32)
        assert np.array_equal(oracle.rms_norm_tree(x, w, 1e-6), oracle.rms_norm(x, w, 1e-6)), dim


def test_rmsnorm_tree_matches_float64(oracle):
    g = np.random.default_rng(5)
    for dim in (300, 2048, 4096, 5000):
        x = (g.standard_normal((5, dim)) * 3).astype(np.float32)
        w = (1 + 0.02 * g.standard_normal(dim)).astype(np.float32)
        got = oracle.rms_norm_tree(x, w, 1e-6)
        xd = x.astype(np.float64)
        want = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-6) * w
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("i", range(6))
def test_rmsnorm_tree_within_fixture_tolerance(oracle, i):
    """The reference's note on its GPU kernel (kernels_a.metal:14-16): the tree order stays
    inside the fixtures' atol 1e-5 / rtol 1e-4."""
    c = _cases(oracle, "rmsnorm")[i]
    p, tol = c["params"], c["tolerance"]
    x, w, want = (oracle.load_ds5t(f"{FIXTURES}/{c['tensors'][n]}").data for n in ("input", "weight", "output"))
    got = oracle.rms_norm_tree(x.copy(), w, p["eps"], p["n_rows"], p["dim"])
    assert oracle.compare(want, got, tol["atol"], tol["rtol"]).passed


def test_rope_is_a_rotation(oracle):
    # Norm of every (i, i+d/2) pair is preserved; composing rotations adds angles.
    g = np.random.default_rng(4)
    x = g.standard_normal((5, 3, 128)).astype(np.float32)
    pos = np.array([0, 1, 17, 4096, 32767], np.int32)
    y = oracle.rope(x, pos, 5e6)
    nx = np.hypot(x[..., :64].astype(np.float64), x[..., 64:])
    ny = np.hypot(y[..., :64].astype(np.float64), y[..., 64:])
    np.testing.assert_allclose(ny, nx, rtol=1e-5, atol=1e-6)
    # The reference forms the angle in f32 (kernels_a.zig:120); cos/sin of that f32 angle in float64.
    inv = np.array([oracle.zig_powf(5e6, -np.float32(2 * i) / np.float32(128)) for i in range(64)], np.float32)
    ang = (pos[:, None].astype(np.float32) * np.float32(1.0) * inv[None, :]).astype(np.float64)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    want0 = x[..., :64] * c - x[..., 64:] * s
    want1 = x[..., :64] * s + x[..., 64:] * c
    np.testing.assert_allclose(y[..., :64], want0, atol=5e-5)
    np.testing.assert_allclose(y[..., 64:], want1, atol=5e-5)


def _attention_f64(q, k, v, pos, hq, hkv):
    T, _, hd = q.shape
    out = np.zeros((T, hq, hd))
    scale = 1.0 / math.sqrt(hd)
    for t in range(T):
        for h in range(hq):
            kh = h // (hq // hkv)
            s = k[kh, :pos + t + 1].astype(np.float64) @ q[t, h].astype(np.float64) * scale
            p = np.exp(s - s.max())
            out[t, h] = p @ v[kh, :pos + t + 1] / p.sum()
    return out.reshape(-1)


@pytest.mark.parametrize("hq,hkv,hd,pos,T", [(8, 2, 16, 5, 3), (4, 4, 8, 0, 6), (16, 1, 32, 40, 1)])
def test_attention_matches_float64_bruteforce(oracle, hq, hkv, hd, pos, T):
    g = np.random.default_rng(hq * 100 + pos)
    q = g.standard_normal((T, hq, hd)).astype(np.float32)
    cap = pos + T + 3
    k = g.standard_normal((hkv, cap, hd)).astype(np.float32)
    v = g.standard_normal((hkv, cap, hd)).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    got = oracle.gqa_attention(q, k, v, 0, pos, T, hq, hkv, hd, cap, scale)
    np.testing.assert_allclose(got, _attention_f64(q, k, v, pos, hq, hkv), atol=2e-6, rtol=1e-5)


def test_f16_cache_equals_f32_cache_of_rounded_values(oracle):
    # kernels_b.zig:96-127 vs :68-95: identical op order, exact widening -> bitwise equal.
    g = np.random.default_rng(5)
    hq, hkv, hd, pos, T, cap = 8, 2, 64, 9, 2, 12
    q = g.standard_normal((T, hq, hd)).astype(np.float32)
    kb = oracle.f32_to_f16_bits(g.standard_normal((hkv, cap, hd)).astype(np.float32))
    vb = oracle.f32_to_f16_bits(g.standard_normal((hkv, cap, hd)).astype(np.float32))
    a = oracle.gqa_attention(q, kb, vb, 1, pos, T, hq, hkv, hd, cap, 0.125)
    b = oracle.gqa_attention(q, oracle.f16_bits_to_f32(kb), oracle.f16_bits_to_f32(vb), 0, pos, T, hq, hkv, hd,
                             cap, 0.125)
    assert np.array_equal(a, b)


def test_attention_step_is_the_op_sequence(oracle):
    # forward.zig:345-412 order, restated from the individual ops.
    g = np.random.default_rng(6)
    hq, hkv, hd, pos, T, cap = 4, 2, 16, 3, 2, 8
    q = g.standard_normal((T, hq, hd)).astype(np.float32)
    k = g.standard_normal((T, hkv, hd)).astype(np.float32)
    v = g.standard_normal((T, hkv, hd)).astype(np.float32)
    qn = (1 + 0.02 * g.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.02 * g.standard_normal(hd)).astype(np.float32)
    positions = np.arange(pos, pos + T, dtype=np.int32)
    kc1 = oracle.f32_to_f16_bits(g.standard_normal((hkv, cap, hd)).astype(np.float32))
    vc1 = oracle.f32_to_f16_bits(g.standard_normal((hkv, cap, hd)).astype(np.float32))
    kc2, vc2 = kc1.copy(), vc1.copy()
    out, q_rot, k_rot = oracle.attention_step(q, k, v, qn, kn, positions, kc1, vc1, kv_dtype=1, pos=pos,
                                              n_tokens=T, n_q_heads=hq, n_kv_heads=hkv, head_dim=hd, max_ctx=cap,
                                              eps=1e-6, theta=1e6)
    q2 = oracle.rope(oracle.rms_norm(q, qn, 1e-6), positions, 1e6)
    k2 = oracle.rope(oracle.rms_norm(k, kn, 1e-6), positions, 1e6)
    oracle.kv_append(k2, v, kc2, vc2, 1, pos, T, hkv, hd, cap)
    out2 = oracle.gqa_attention(q2, kc2, vc2, 1, pos, T, hq, hkv, hd, cap,
                                float(np.float32(1) / np.sqrt(np.float32(hd))))
    assert np.array_equal(q_rot, q2) and np.array_equal(k_rot, k2)
    assert np.array_equal(kc1, kc2) and np.array_equal(vc1, vc2) and np.array_equal(out, out2)


def test_paged_slot_map_and_gather(oracle):
    from qw3_amd import synth
    lay = synth.paged_layout(6, 5, 70, 16, seed=3)
    # every (seq, position) maps to a distinct pool slot, inside the pool
    seen = set()
    for b in range(6):
        for p in range(int(lay.seq_lens[b])):
            s = oracle.paged_slot(lay.page_table[b], 16, p)
            assert s == lay.slot(b, p) == lay.page_table[b, p // 16] * 16 + p % 16
            assert 0 <= s < lay.n_pages * 16 and s not in seen
            seen.add(s)
    assert oracle.paged_slot(lay.page_table[0], 16, lay.max_pages * 16) == -1
    g = np.random.default_rng(8)
    pool = g.integers(0, 2 ** 16, size=(2, lay.n_pages * 16, 8), dtype=np.uint64).astype(np.uint16)
    for b in range(6):
        L = int(lay.seq_lens[b])
        got = oracle.paged_gather_f16(pool, lay.page_table[b], 16, L)
        want = np.stack([pool[:, lay.slot(b, p)] for p in range(L)], axis=1)
        assert np.array_equal(got, want)


def test_config0_golden_vectors_reproduce(oracle):
    """tests/golden/c0 (written by tests/golden/make_c0_golden.py): the oracle and
    the seeded generator still produce exactly the committed vectors."""
    import importlib.util
    import os
    from conftest import GOLDEN
    spec = importlib.util.spec_from_file_location("mk", os.path.join(GOLDEN, "make_c0_golden.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    for name, (arr, dt) in mk.make().items():
        t = oracle.load_ds5t(os.path.join(GOLDEN, "c0", f"{name}.ds5t"))
        assert t.dtype == dt
        assert np.array_equal(t.data.reshape(arr.shape).view(np.uint8), np.ascontiguousarray(arr).view(np.uint8)), name


# ---------------------------------------------------------------------------
# matmul (the projection step before the path): kernels_a.zig:136-163
# ---------------------------------------------------------------------------


def test_matmul_f32_hand_case(oracle):
    """kernels_a.zig:524-553: x [2,3] . W^T with rows {1,0,2} and {0,-1,1}."""
    x = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    w = np.array([[1, 0, 2], [0, -1, 1]], np.float32)
    got = oracle.matmul(x, w, oracle.F32, 2, 2, 3)
    assert np.array_equal(got, np.array([[7, 1], [16, 1]], np.float32))


def test_matmul_q8_0_equals_dequantized_f32(oracle):
    """kernels_a.zig:555-602: the Q8_0 path equals the f32 path on the dequantised
    weights (f32(scale) * q is exact in f32, so the serial sums match bit for bit)."""
    g = np.random.default_rng(3)
    k, n = 64, 3
    rows = np.zeros((n, 2, 34), np.uint8)
    for r in range(n):
        for b in range(2):
            rows[r, b, :2] = np.array([0.005 + 0.01 * (r + b)], np.float16).view(np.uint8)
            rows[r, b, 2:] = g.integers(-127, 128, 32).astype(np.int8).view(np.uint8)
    rows = rows.reshape(n, 68)
    x = g.standard_normal((2, k)).astype(np.float32)
    a = oracle.matmul(x, rows, oracle.Q8_0, 2, n, k)
    b = oracle.matmul(x, oracle.q8_0_dequantize(rows, k), oracle.F32, 2, n, k)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("m,n,k", [(1, 40, 2048), (5, 17, 96), (3, 9, 32)])
def test_matmul_matches_float64(oracle, m, n, k):
    """Q8_0 and f32 weights against a float64 product of the dequantised weights."""
    g = np.random.default_rng(m * 1000 + n)
    rows = oracle.q8_0_quantize(g.standard_normal((n, k)).astype(np.float32) * 0.05)
    wf = oracle.q8_0_dequantize(rows, k)
    x = g.standard_normal((m, k)).astype(np.float32)
    want = x.astype(np.float64) @ wf.astype(np.float64).T
    bound = 1e-6 * k * (np.abs(x).astype(np.float64) @ np.abs(wf).astype(np.float64).T) + 1e-30
    for w, dt in ((rows, oracle.Q8_0), (wf, oracle.F32)):
        got = oracle.matmul(x, w, dt, m, n, k).astype(np.float64)
        assert np.all(np.abs(got - want) <= bound)


def test_q8_0_quantize_roundtrip(oracle):
    """The test helper's quantiser: |w - dequant(quant(w))| <= scale / 2 per element
    (the f16 scale is within 2^-11 of max|w| / 127, so max|w| / scale stays below 127.5)."""
    g = np.random.default_rng(11)
    w = g.standard_normal((7, 128)).astype(np.float32)
    rows = oracle.q8_0_quantize(w)
    back = oracle.q8_0_dequantize(rows, 128)
    d = rows.reshape(7, 4, 34)[:, :, :2].copy().view(np.float16).astype(np.float32)
    assert np.all(np.abs(w - back).reshape(7, 4, 32) <= d * 0.5 * (1 + 1e-6))


def test_matmul_rejections(oracle):
    """kernels_a.zig:138-150 and :604-617: unsupported dtype first, then k and buffer sizes."""
    x, w = np.zeros((1, 64), np.float32), np.zeros((2, 68), np.uint8)
    out = np.zeros(2, np.float32)
    call = lambda xa, wa, dt, m, n, k, o=out: oracle.lib().ds5o_matmul(
        oracle.MatmulArgs(oracle.buf(xa), oracle.buf(wa), dt, oracle.buf(o), m, n, k))
    assert call(x, w, 12, 1, 1, 256) == oracle.UNSUPPORTED_DTYPE  # q4_k
    assert call(x, w, oracle.F16, 1, 2, 64) == oracle.UNSUPPORTED_DTYPE
    assert call(x, w, oracle.Q8_0, 1, 2, 0) == oracle.SHAPE_MISMATCH
    assert call(x, w, oracle.Q8_0, 1, 2, 48) == oracle.SHAPE_MISMATCH  # not a block multiple
    assert call(x, w, oracle.Q8_0, 2, 2, 64) == oracle.SHAPE_MISMATCH  # x too small
    assert call(x, w, oracle.Q8_0, 1, 3, 64) == oracle.SHAPE_MISMATCH  # w too small (and out)
    assert call(x, w, oracle.Q8_0, 1, 2, 64, np.zeros(1, np.float32)) == oracle.SHAPE_MISMATCH
    assert call(x, w, oracle.Q8_0, 1, 2, 64) == oracle.OK


def test_add_matches_ieee_and_aliases(oracle):
    """kernels_a.zig:703-724: out = x + y elementwise (an odd size), out aliasing x
    allowed; f32 addition is exactly numpy's IEEE float32 add, specials included."""
    g = np.random.default_rng(11)
    x = g.standard_normal(97).astype(np.float32)
    y = g.standard_normal(97).astype(np.float32)
    x[:6] = [np.inf, -np.inf, np.nan, 0.0, -0.0, 3.4e38]
    y[:6] = [-np.inf, 1.0, 1.0, -0.0, -0.0, 3.4e38]
    with np.errstate(over="ignore", invalid="ignore"):
        want = x + y
    assert np.array_equal(oracle.add(x, y), want, equal_nan=True)
    xa = x.copy()
    assert oracle.lib().ds5o_add(oracle.AddArgs(oracle.buf(xa), oracle.buf(y), oracle.buf(xa), 97)) == oracle.OK
    assert np.array_equal(xa.view(np.uint32), want.view(np.uint32))


def test_add_rejections(oracle):
    """kernels_a.zig:225-227: x, then y, then out too small."""
    a, b = np.zeros(8, np.float32), np.zeros(7, np.float32)
    call = lambda x, y, o, n: oracle.lib().ds5o_add(oracle.AddArgs(oracle.buf(x), oracle.buf(y), oracle.buf(o), n))
    assert call(a, a, a, 8) == oracle.OK
    assert call(b, a, a, 8) == oracle.SHAPE_MISMATCH
    assert call(a, b, a, 8) == oracle.SHAPE_MISMATCH
    assert call(a, a, b, 8) == oracle.SHAPE_MISMATCH
    assert call(b, b, b, 0) == oracle.OK


# ---------------------------------------------------------------------------
# MoE router and expert MLP (kernels_c.zig)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("i", range(3))
def test_router_fixtures(oracle, i):
    """kernels_c.zig:250-318: expert ids 100% exact, gate weights within the case tolerance."""
    c = _cases(oracle, "router")[i]
    p, tol = c["params"], c["tolerance"]
    x, w = _t(oracle, c, "input"), _t(oracle, c, "weight")
    want_ids, want_w = _t(oracle, c, "expert_ids"), _t(oracle, c, "gate_weights")
    assert want_ids.ne == (p["top_k"], p["n_tokens"]) and p["w_dtype"] == "f32"
    ids, wts = oracle.router_topk(x.data, w.data, oracle.F32, p["n_tokens"], p["dim"], p["n_experts"], p["top_k"],
                                  p["norm_topk_prob"])
    assert np.array_equal(ids.astype(np.int32), want_ids.data.reshape(ids.shape))
    r = oracle.compare(want_w.data.reshape(wts.shape), wts, tol["atol"], tol["rtol"])
    assert r.passed, r


def test_router_raw_probabilities(oracle):
    """kernels_c.zig:403-439: norm_topk_prob = false keeps the softmax over all experts."""
    x = np.array([[1, 0, 0, 0]], np.float32)
    w = np.array([[2, 0, 0, 0], [0, 9, 9, 9], [1, 0, 0, 0], [-1, 0, 0, 0]], np.float32)
    ids, wts = oracle.router_topk(x, w, oracle.F32, 1, 4, 4, 2, False)
    assert ids.tolist() == [[0, 2]]
    denom = sum(np.exp(np.float64(l) - 2.0) for l in (2, 0, 1, -1))
    assert abs(wts[0, 0] - 1.0 / denom) <= 1e-6 and abs(wts[0, 1] - np.exp(-1.0) / denom) <= 1e-6
    assert wts.sum() < 1.0


def test_router_tie_break_lower_id(oracle):
    """kernels_c.zig:441-477: equal probabilities pick the lower expert id."""
    x = np.array([[1, 0, 0, 0]], np.float32)
    w = np.array([[1, 0, 0, 0], [3, 0, 0, 0], [3, 0, 0, 0], [0, 0, 0, 0]], np.float32)
    ids, wts = oracle.router_topk(x, w, oracle.F32, 1, 4, 4, 3, True)
    assert ids.tolist() == [[1, 2, 0]] and wts[0, 0] == wts[0, 1]
    assert abs(wts.sum() - 1.0) <= 1e-6


def test_router_f16_and_q8_0_agree_with_f32(oracle):
    """kernels_c.zig:479-548: f16 and Q8_0 weights give the ids of their dequantised f32 rows
    and weights within 1e-6 (scale * q exact in f16 here)."""
    g = np.random.default_rng(7)
    dim, E = 32, 4
    q8 = np.zeros((E, 34), np.uint8)
    wf = np.zeros((E, dim), np.float32)
    for e in range(E):
        sc = np.float16(0.01 + 0.02 * e)
        q = g.integers(-127, 128, dim).astype(np.int8)
        q8[e, :2] = np.array([sc], np.float16).view(np.uint8)
        q8[e, 2:] = q.view(np.uint8)
        wf[e] = np.float32(sc) * q.astype(np.float32)
    x = g.standard_normal((1, dim)).astype(np.float32)
    i32, w32 = oracle.router_topk(x, wf, oracle.F32, 1, dim, E, 2, True)
    i8, w8 = oracle.router_topk(x, q8, oracle.Q8_0, 1, dim, E, 2, True)
    i16, w16 = oracle.router_topk(x, wf.astype(np.float16).view(np.uint16), oracle.F16, 1, dim, E, 2, True)
    assert np.array_equal(i32, i8) and np.array_equal(i32, i16)
    assert np.all(np.abs(w32 - w8) <= 1e-6) and np.all(np.abs(w32 - w16) <= 1e-6)


def test_router_matches_float64(oracle):
    """Seeded routers against a float64 softmax / top-k of the same logits (ids exact where
    the float64 ranking has no near-ties; weights within 1e-5)."""
    g = np.random.default_rng(3)
    T, dim, E, K = 9, 64, 16, 4
    x = g.standard_normal((T, dim)).astype(np.float32)
    w = g.standard_normal((E, dim)).astype(np.float32)
    for norm in (True, False):
        ids, wts = oracle.router_topk(x, w, oracle.F32, T, dim, E, K, norm)
        lg = x.astype(np.float64) @ w.astype(np.float64).T
        pr = np.exp(lg - lg.max(1, keepdims=True))
        pr /= pr.sum(1, keepdims=True)
        order = np.argsort(-pr, axis=1, kind="stable")[:, :K]
        assert np.array_equal(ids, order)
        top = np.take_along_axis(pr, order, 1)
        if norm:
            top = top / top.sum(1, keepdims=True)
        assert np.all(np.abs(wts - top) <= 1e-5)


def test_router_rejections(oracle):
    """kernels_c.zig:81-95 and :625-655: dtype, then top_k, dim, the two output lengths, x, w."""
    x, w = np.zeros((1, 32), np.float32), np.zeros((2, 32), np.float32)
    ids, wts = np.zeros(1, np.uint16), np.zeros(1, np.float32)

    def call(dt=oracle.F32, T=1, dim=32, E=2, K=1, xa=x, wa=w, nid=1, nw=1):
        return oracle.lib().ds5o_router_topk(oracle.RouterArgs(
            oracle.buf(xa), oracle.buf(wa), dt, T, dim, E, K, 1, ids.ctypes.data_as(C.POINTER(C.c_uint16)), nid,
            wts.ctypes.data_as(C.POINTER(C.c_float)), nw))
    assert call() == oracle.OK
    assert call(dt=12) == oracle.UNSUPPORTED_DTYPE  # q4_k
    assert call(K=0) == oracle.SHAPE_MISMATCH
    assert call(K=3) == oracle.SHAPE_MISMATCH
    assert call(dt=oracle.Q8_0, dim=16) == oracle.SHAPE_MISMATCH
    assert call(nid=2) == oracle.SHAPE_MISMATCH
    assert call(nw=0) == oracle.SHAPE_MISMATCH
    assert call(xa=np.zeros(31, np.float32)) == oracle.SHAPE_MISMATCH
    assert call(wa=np.zeros(63, np.float32)) == oracle.SHAPE_MISMATCH


@pytest.mark.parametrize("i", range(3))
def test_expert_mlp_fixtures(oracle, i):
    """kernels_c.zig:320-401: Q8_0 banks, token-major pairs from the fixture's ids and
    weights, output within the case tolerance."""
    c = _cases(oracle, "expert_mlp")[i]
    p, tol = c["params"], c["tolerance"]
    x = _t(oracle, c, "input")
    gate, up, down = (_t(oracle, c, n) for n in ("gate", "up", "down"))
    assert gate.ne == (p["dim"], p["ffn_dim"], p["n_experts"]) and down.ne == (p["ffn_dim"], p["dim"], p["n_experts"])
    ids = _t(oracle, c, "expert_ids").data.reshape(p["n_tokens"], p["top_k"])
    gw = _t(oracle, c, "gate_weights").data.reshape(p["n_tokens"], p["top_k"])
    pairs = oracle.pairs_from_router(ids, gw)
    got = oracle.expert_mlp_swiglu(x.data, gate.data, up.data, down.data, oracle.Q8_0, pairs, p["n_tokens"], p["dim"],
                                   p["ffn_dim"], p["n_experts"])
    r = oracle.compare(_t(oracle, c, "output").data.reshape(got.shape), got, tol["atol"], tol["rtol"])
    assert r.passed, r


def test_expert_mlp_empty_pairs(oracle):
    """kernels_c.zig:550-572: no pairs leave the output untouched."""
    bank = np.zeros((32, 34), np.uint8)
    out = oracle.expert_mlp_swiglu(np.zeros((2, 32), np.float32), bank, bank, bank, oracle.Q8_0,
                                   np.zeros(0, oracle.PAIR_DTYPE), 2, 32, 32, 1)
    assert np.all(out == 0)


def test_expert_mlp_f32_hand_case(oracle):
    """kernels_c.zig:574-623: two pairs accumulate (identity and swapped down projections)."""
    silu = lambda v: np.float32(v) / (np.float32(1) + np.exp(np.float32(-v)))
    x = np.array([[1.0, -2.0]], np.float32)
    gate = np.array([1, 0, 0, 1, 0, 1, 1, 0], np.float32)
    up = np.array([2, 0, 0, 2, 2, 0, 0, 2], np.float32)
    down = np.array([1, 0, 0, 1, 0, 1, 1, 0], np.float32)
    pairs = np.array([(0, 0, 0.5), (0, 1, 2.0)], oracle.PAIR_DTYPE)
    got = oracle.expert_mlp_swiglu(x, gate, up, down, oracle.F32, pairs, 1, 2, 2, 2)
    s1, s2 = silu(1.0), silu(-2.0)
    want = [0.5 * s1 * 2 + 2.0 * s1 * -4, 0.5 * s2 * -4 + 2.0 * s2 * 2]
    assert np.all(np.abs(got[0] - np.array(want, np.float32)) <= 1e-6)


def test_expert_mlp_matches_float64(oracle):
    """Seeded Q8_0 banks: the oracle against a float64 evaluation of the dequantised weights."""
    g = np.random.default_rng(9)
    T, dim, ffn, E = 3, 64, 96, 4
    bank = lambda rows, k: oracle.q8_0_quantize(g.standard_normal((rows, k)).astype(np.float32) * 0.1)
    gate, up, down = bank(E * ffn, dim), bank(E * ffn, dim), bank(E * dim, ffn)
    x = g.standard_normal((T, dim)).astype(np.float32)
    pairs = np.array([(0, 1, 0.6), (0, 3, 0.4), (2, 0, 1.0), (1, 2, 0.25), (2, 2, 0.5)], oracle.PAIR_DTYPE)
    got = oracle.expert_mlp_swiglu(x, gate, up, down, oracle.Q8_0, pairs, T, dim, ffn, E)
    G, U = oracle.q8_0_dequantize(gate, dim).astype(np.float64), oracle.q8_0_dequantize(up, dim).astype(np.float64)
    D = oracle.q8_0_dequantize(down, ffn).astype(np.float64)
    want = np.zeros((T, dim))
    for t, e, wt in pairs.tolist():
        gv = G[e * ffn:(e + 1) * ffn] @ x[t]
        h = gv / (1 + np.exp(-gv)) * (U[e * ffn:(e + 1) * ffn] @ x[t])
        want[t] += wt * (D[e * dim:(e + 1) * dim] @ h)
    assert np.all(np.abs(got - want) <= 1e-4 * (1 + np.abs(want)))


def test_expert_mlp_rejections(oracle):
    """kernels_c.zig:157-183, :625-655: dtype; zero or unblocked dims; x, out, gate, up, down
    sizes; a pair out of range (reached after the pairs before it were added)."""
    bank = np.zeros((32, 34), np.uint8)
    x, out = np.zeros((1, 32), np.float32), np.zeros((1, 32), np.float32)

    def call(dt=oracle.Q8_0, dim=32, ffn=32, E=1, xa=x, oa=out, ga=bank, ua=bank, da=bank, pairs=None):
        pr = np.zeros(0, oracle.PAIR_DTYPE) if pairs is None else pairs
        return oracle.lib().ds5o_expert_mlp_swiglu(oracle.ExpertMlpArgs(
            oracle.buf(xa), oracle.buf(ga), oracle.buf(ua), oracle.buf(da), dt, pr.ctypes.data if pr.size else None,
            pr.size, oracle.buf(oa), 1, dim, ffn, E))
    assert call() == oracle.OK
    assert call(dt=oracle.F16) == oracle.UNSUPPORTED_DTYPE
    assert call(ffn=0) == oracle.SHAPE_MISMATCH
    assert call(dim=16) == oracle.SHAPE_MISMATCH
    assert call(xa=np.zeros(31, np.float32)) == oracle.SHAPE_MISMATCH
    assert call(oa=np.zeros(31, np.float32)) == oracle.SHAPE_MISMATCH
    assert call(ga=bank[:31]) == oracle.SHAPE_MISMATCH
    assert call(ua=bank[:31]) == oracle.SHAPE_MISMATCH
    assert call(da=bank[:31]) == oracle.SHAPE_MISMATCH
    assert call(pairs=np.array([(0, 1, 1.0)], oracle.PAIR_DTYPE)) == oracle.SHAPE_MISMATCH
    assert call(pairs=np.array([(1, 0, 1.0)], oracle.PAIR_DTYPE)) == oracle.SHAPE_MISMATCH


def test_attention_f64_checker_matches_oracle(oracle):
    """The float64 causal attention the full-size GPU prefill test checks every head
    against agrees with the oracle's f16-cache attention (and fails on a shifted mask)."""
    from conftest import attention_f64
    g = np.random.default_rng(3)
    T, d = 96, 128
    q = g.standard_normal((T, 1, d)).astype(np.float32)
    kc = oracle.f32_to_f16_bits(g.standard_normal((1, T, d)).astype(np.float32))
    vc = oracle.f32_to_f16_bits(g.standard_normal((1, T, d)).astype(np.float32))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    want = oracle.gqa_attention(q, kc, vc, 1, 0, T, 1, 1, d, T, scale).reshape(T, d)
    got = attention_f64(q[:, 0], kc[0], vc[0], scale)
    assert np.max(np.abs(got - want)) < 1e-5
    # a mask one position too wide must not pass
    bad = attention_f64(q[1:, 0], kc[0, 1:], vc[0, 1:], scale)
    assert np.max(np.abs(bad - want[1:])) > 1e-3
