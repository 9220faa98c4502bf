"""The C-ABI library without a GPU: it loads, exports every symbol the header
declares, its structs match the C compiler's layout, and every precondition
the reference checks is rejected with the reference's error before any device
work (a null context stands in for the device; valid shapes then report
DeviceFailure instead of launching)."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "ds5_hip.h")


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|void|uint64_t|const char\*|void\*)\s+\**(ds5_hip_\w+)\(", text, re.M)))


def test_library_exports_every_header_symbol(hip):
    names = header_functions()
    assert len(names) >= 18
    nm = subprocess.run(["nm", "-D", "--defined-only", hip.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r" T (ds5_hip_\w+)", nm.stdout))
    assert set(names) <= exported, set(names) - exported
    assert set(names) == set(hip.SIGNATURES), set(names) ^ set(hip.SIGNATURES)
    for n in names:
        assert getattr(hip.LIB, n) is not None


STRUCTS = {
    "ds5_buf": "Buf", "ds5_rms_norm_args": "RmsNormArgs", "ds5_rope_args": "RopeArgs",
    "ds5_kv_append_args": "KvAppendArgs", "ds5_attn_args": "AttnArgs",
    "ds5_attention_step_args": "AttentionStepArgs", "ds5_paged_decode_args": "PagedDecodeArgs",
    "ds5_attention_block_args": "AttentionBlockArgs",
    "ds5_matmul_args": "MatmulArgs", "ds5_matmul_group_args": "MatmulGroupArgs", "ds5_add_args": "AddArgs",
    "ds5_matmul_add_args": "MatmulAddArgs", "ds5_router_args": "RouterArgs", "ds5_pair": "Pair",
    "ds5_expert_mlp_args": "ExpertMlpArgs", "ds5_moe_args": "MoeArgs",
}


def test_struct_layouts_match_c(hip, tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', 'int main(void) {']
    for cname, pyname in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in getattr(hip, pyname)._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    got = dict(l.rsplit(" ", 1) for l in out if l)
    for cname, pyname in STRUCTS.items():
        py = getattr(hip, pyname)
        assert int(got[f"{cname} size"]) == C.sizeof(py), cname
        for fname, _ in py._fields_:
            assert int(got[f"{cname}.{fname}"]) == getattr(py, fname).offset, (cname, fname)
    assert C.sizeof(hip.Buf) == 24  # contracts.zig:210-214 extern struct


# ---------------------------------------------------------------------------
# Preconditions (no device): null ctx, fake device pointers never dereferenced
# ---------------------------------------------------------------------------
FAKE = 1 << 20  # a non-null handle; nothing is dereferenced before the checks pass


def B(nbytes):
    import qw3_amd.hip as H
    return H.Buf(FAKE, 0, nbytes)


def rc_of(hip, fn, args):
    return getattr(hip.LIB, fn)(None, C.byref(args))


def test_rms_norm_preconditions(hip):
    ok = hip.RmsNormArgs(B(64), B(16), B(64), 4, 4, 1e-6)
    assert rc_of(hip, "ds5_hip_rms_norm", ok) == 3  # valid: only the missing device fails
    for bad in (hip.RmsNormArgs(B(64), B(16), B(64), 4, 0, 1e-6), hip.RmsNormArgs(B(60), B(16), B(64), 4, 4, 1e-6),
                hip.RmsNormArgs(B(64), B(16), B(60), 4, 4, 1e-6), hip.RmsNormArgs(B(64), B(12), B(64), 4, 4, 1e-6)):
        assert rc_of(hip, "ds5_hip_rms_norm", bad) == 1


def test_matmul_preconditions(hip):
    """kernels_a.zig:138-150: unsupported weight dtype, then k, then buffer sizes."""
    M = lambda x, w, dt, out, m, n, k: hip.MatmulArgs(B(x), B(w), dt, B(out), m, n, k)
    q8 = hip.DTYPE_Q8_0
    assert rc_of(hip, "ds5_hip_matmul", M(4 * 64, 2 * 68, q8, 8, 1, 2, 64)) == 3  # valid: no device
    assert rc_of(hip, "ds5_hip_matmul", M(4 * 3, 4 * 6, hip.DTYPE_F32, 8, 1, 2, 3)) == 3  # f32: any k
    assert rc_of(hip, "ds5_hip_matmul", M(0, 0, q8, 0, 0, 0, 64)) == 0  # empty product: nothing to do
    for dt in (hip.DTYPE_F16, 12, 9):  # f16, q4_k, q8_1
        assert rc_of(hip, "ds5_hip_matmul", M(4 * 64, 2 * 68, dt, 8, 1, 2, 64)) == 2
    for bad in (M(4 * 64, 2 * 68, q8, 8, 1, 2, 0), M(4 * 64, 2 * 68, q8, 8, 1, 2, 48),
                M(4 * 64 - 4, 2 * 68, q8, 8, 1, 2, 64), M(4 * 64, 2 * 68 - 1, q8, 8, 1, 2, 64),
                M(4 * 64, 2 * 68, q8, 4, 1, 2, 64), M(4 * 3, 4 * 6 - 4, hip.DTYPE_F32, 8, 1, 2, 3)):
        assert rc_of(hip, "ds5_hip_matmul", bad) == 1


def test_matmul_group_preconditions(hip):
    """count in 1..4, then every entry checked as matmul checks, before anything runs."""
    q8 = hip.DTYPE_Q8_0
    G = lambda x, dt, m, k, entries: hip.MatmulGroupArgs.of(B(x), dt, m, k, [(B(w), B(o), n) for w, o, n in entries])
    ok = (2 * 68, 8, 2)
    assert rc_of(hip, "ds5_hip_matmul_group", G(4 * 64, q8, 1, 64, [ok, ok, ok])) == 3  # valid: no device
    assert rc_of(hip, "ds5_hip_matmul_group", G(4 * 64, q8, 1, 64, [])) == 1
    bad = hip.MatmulGroupArgs.of(B(4 * 64), q8, 1, 64, [])
    bad.count = 5
    assert rc_of(hip, "ds5_hip_matmul_group", bad) == 1
    assert rc_of(hip, "ds5_hip_matmul_group", G(4 * 64, hip.DTYPE_F16, 1, 64, [ok])) == 2
    assert rc_of(hip, "ds5_hip_matmul_group", G(4 * 64, q8, 1, 48, [ok])) == 1
    assert rc_of(hip, "ds5_hip_matmul_group", G(4 * 64, q8, 1, 64, [ok, (2 * 68 - 1, 8, 2)])) == 1  # entry 1's w
    assert rc_of(hip, "ds5_hip_matmul_group", G(4 * 64, q8, 1, 64, [ok, ok, (2 * 68, 4, 2)])) == 1  # entry 2's out
    assert rc_of(hip, "ds5_hip_matmul_group", G(4 * 64 - 4, q8, 1, 64, [ok])) == 1  # x
    assert rc_of(hip, "ds5_hip_matmul_group", G(0, q8, 0, 64, [(5 * 68, 0, 5)])) == 0  # no tokens: nothing to do


def test_add_preconditions(hip):
    """kernels_a.zig:225-227: x, y, out sizes in order."""
    A = lambda x, y, o, n: hip.AddArgs(B(x), B(y), B(o), n)
    assert rc_of(hip, "ds5_hip_add", A(40, 40, 40, 10)) == 3
    assert rc_of(hip, "ds5_hip_add", A(0, 0, 0, 0)) == 0
    for bad in (A(36, 40, 40, 10), A(40, 36, 40, 10), A(40, 40, 36, 10)):
        assert rc_of(hip, "ds5_hip_add", bad) == 1


def test_matmul_add_preconditions(hip):
    """matmul's checks, then the residual's size, then 4-byte aligned residual / out."""
    q8 = hip.DTYPE_Q8_0
    M = lambda x, w, dt, r, o, m, n, k: hip.MatmulAddArgs(B(x), B(w), dt, r if isinstance(r, hip.Buf) else B(r),
                                                          B(o), m, n, k)
    assert rc_of(hip, "ds5_hip_matmul_add", M(4 * 64, 2 * 68, q8, 8, 8, 1, 2, 64)) == 3
    assert rc_of(hip, "ds5_hip_matmul_add", M(4 * 64, 2 * 68, hip.DTYPE_F16, 8, 8, 1, 2, 64)) == 2
    assert rc_of(hip, "ds5_hip_matmul_add", M(4 * 64, 2 * 68, q8, 8, 8, 1, 2, 48)) == 1
    assert rc_of(hip, "ds5_hip_matmul_add", M(4 * 64, 2 * 68, q8, 4, 8, 1, 2, 64)) == 1  # residual
    assert rc_of(hip, "ds5_hip_matmul_add", M(4 * 64, 2 * 68, q8, hip.Buf(FAKE, 2, 8), 8, 1, 2, 64)) == 1  # unaligned


def test_router_preconditions(hip):
    """kernels_c.zig:81-95: dtype, top_k, dim, output lengths, x, w (no device touched)."""
    ids, wts = np.zeros(4, np.uint16), np.zeros(4, np.float32)

    def R(x=4 * 2 * 32, w=4 * 8 * 32, dt=hip.DTYPE_F32, T=2, dim=32, E=8, K=2, nid=4, nw=4):
        return hip.RouterArgs(B(x), B(w), dt, T, dim, E, K, 1, ids.ctypes.data_as(C.POINTER(C.c_uint16)), nid,
                              wts.ctypes.data_as(C.POINTER(C.c_float)), nw)
    assert rc_of(hip, "ds5_hip_router_topk", R()) == 3
    assert rc_of(hip, "ds5_hip_router_topk", R(dt=12)) == 2
    assert rc_of(hip, "ds5_hip_router_topk", R(dt=hip.DTYPE_F16, w=2 * 8 * 32)) == 3
    assert rc_of(hip, "ds5_hip_router_topk", R(E=16385, w=4 * 16385 * 32)) == 1  # n_experts > 16384 (LDS)
    assert rc_of(hip, "ds5_hip_router_topk", R(dim=16416, x=4 * 2 * 16416, w=4 * 8 * 16416)) == 1  # row > 64 KiB
    assert rc_of(hip, "ds5_hip_router_topk", R(dim=16384, x=4 * 2 * 16384, w=4 * 8 * 16384)) == 3
    for bad in (R(K=0), R(K=9), R(dt=hip.DTYPE_Q8_0, dim=16, w=8 * 34), R(nid=3), R(nw=5), R(x=4 * 2 * 32 - 4),
                R(w=4 * 8 * 32 - 1)):
        assert rc_of(hip, "ds5_hip_router_topk", bad) == 1


def test_expert_mlp_preconditions(hip):
    """kernels_c.zig:157-183 and every pair in range, before anything runs."""
    q8 = hip.DTYPE_Q8_0
    bank = 2 * 32 * 34  # 2 experts, ffn = dim = 32

    def E(pairs=(), dt=q8, x=4 * 32, out=4 * 32, g=bank, u=bank, d=bank, dim=32, ffn=32):
        pr = np.array(list(pairs), hip.PAIR_DTYPE)
        return hip.ExpertMlpArgs(B(x), B(g), B(u), B(d), dt, pr.ctypes.data if pr.size else None, pr.size, B(out),
                                 1, dim, ffn, 2), pr
    ok, _keep = E([(0, 1, 0.5)])
    assert rc_of(hip, "ds5_hip_expert_mlp_swiglu", ok) == 3
    empty, _keep2 = E()
    assert rc_of(hip, "ds5_hip_expert_mlp_swiglu", empty) == 0  # nothing to do
    bad_dt, _k = E(dt=hip.DTYPE_F16)
    assert rc_of(hip, "ds5_hip_expert_mlp_swiglu", bad_dt) == 2
    for kw in (dict(ffn=0), dict(dim=16), dict(x=4 * 31), dict(out=4 * 31), dict(g=bank - 1), dict(u=bank - 1),
               dict(d=bank - 1), dict(pairs=[(0, 2, 1.0)]), dict(pairs=[(0, 0, 1.0), (1, 0, 1.0)])):
        args, _k = E(**kw)
        assert rc_of(hip, "ds5_hip_expert_mlp_swiglu", args) == 1, kw


def test_moe_preconditions(hip):
    """The router's checks, then the experts', then the optional outputs' sizes."""
    q8 = hip.DTYPE_Q8_0
    bank = 8 * 32 * 34

    def M(rdt=hip.DTYPE_F32, dt=q8, K=2, ids=0, wts=0, g=bank):
        return hip.MoeArgs(B(4 * 32), B(4 * 8 * 32), rdt, B(g), B(bank), B(bank), dt, B(4 * 32), B(ids), B(wts),
                           1, 32, 32, 8, K, 1)
    assert rc_of(hip, "ds5_hip_moe", M()) == 3
    assert rc_of(hip, "ds5_hip_moe", M(ids=4, wts=8)) == 3
    assert rc_of(hip, "ds5_hip_moe", M(rdt=12)) == 2
    assert rc_of(hip, "ds5_hip_moe", M(dt=hip.DTYPE_F16)) == 2
    for bad in (M(K=0), M(g=bank - 1), M(ids=2), M(wts=4)):
        assert rc_of(hip, "ds5_hip_moe", bad) == 1


def test_rope_preconditions(hip):
    assert rc_of(hip, "ds5_hip_rope", hip.RopeArgs(B(2 * 3 * 8 * 4), B(8), 2, 3, 8, 1e6)) == 3
    for bad in (hip.RopeArgs(B(2 * 3 * 7 * 4), B(8), 2, 3, 7, 1e6), hip.RopeArgs(B(100), B(8), 2, 3, 0, 1e6),
                hip.RopeArgs(B(2 * 3 * 8 * 4 - 1), B(8), 2, 3, 8, 1e6), hip.RopeArgs(B(2 * 3 * 8 * 4), B(4), 2, 3, 8, 1e6),
                hip.RopeArgs(B(1 << 20), B(8), 1, 1, 1024, 1e6)):
        assert rc_of(hip, "ds5_hip_rope", bad) == 1


def test_kv_append_preconditions(hip):
    def args(kv_dtype=1, pos=3, T=2, H=2, hd=4, cap=8, new=None, cache=None):
        eb = 2 if kv_dtype == 1 else 4
        new = T * H * hd * 4 if new is None else new
        cache = H * cap * hd * eb if cache is None else cache
        return hip.KvAppendArgs(B(new), B(new), B(cache), B(cache), kv_dtype, pos, T, H, hd, cap)
    assert rc_of(hip, "ds5_hip_kv_append", args()) == 3
    assert rc_of(hip, "ds5_hip_kv_append", args(kv_dtype=0)) == 3
    assert rc_of(hip, "ds5_hip_kv_append", args(pos=7)) == 1           # kernels_a.zig:176 overflow
    assert rc_of(hip, "ds5_hip_kv_append", args(hd=0)) == 1
    assert rc_of(hip, "ds5_hip_kv_append", args(H=0)) == 1
    assert rc_of(hip, "ds5_hip_kv_append", args(new=10)) == 1
    assert rc_of(hip, "ds5_hip_kv_append", args(cache=10)) == 1
    assert rc_of(hip, "ds5_hip_kv_append", args(kv_dtype=8, cache=1 << 20)) == 2  # q8_0 cache


def test_attention_preconditions(hip):
    def args(kv_dtype=1, pos=0, T=1, hq=2, hkv=2, hd=4, cap=8, q=None, cache=None):
        eb = 2 if kv_dtype == 1 else 4
        q = T * hq * hd * 4 if q is None else q
        cache = hkv * cap * hd * eb if cache is None else cache
        return hip.AttnArgs(B(q), B(cache), B(cache), kv_dtype, B(q), pos, T, hq, hkv, hd, cap, 0.5)
    assert rc_of(hip, "ds5_hip_gqa_attention", args()) == 3
    # kernels_b.zig:456-492 rejections
    assert rc_of(hip, "ds5_hip_gqa_attention", args(pos=8)) == 1
    assert rc_of(hip, "ds5_hip_gqa_attention", args(hq=3, hkv=2)) == 1
    assert rc_of(hip, "ds5_hip_gqa_attention", args(cap=64, cache=2 * 8 * 4 * 2)) == 1
    assert rc_of(hip, "ds5_hip_gqa_attention", args(hq=0)) == 1
    assert rc_of(hip, "ds5_hip_gqa_attention", args(q=8)) == 1
    assert rc_of(hip, "ds5_hip_gqa_attention", args(kv_dtype=30, cache=1 << 20)) == 2  # bf16 cache
    assert rc_of(hip, "ds5_hip_gqa_attention", args(T=0)) == 0                        # nothing to do


def test_step_and_paged_preconditions(hip):
    T, hq, hkv, hd, cap = 1, 8, 2, 64, 16
    f = lambda n: B(n * 4)
    ok = hip.AttentionStepArgs(f(T * hq * hd), f(T * hkv * hd), f(T * hkv * hd), f(hd), f(hd), f(T),
                               B(hkv * cap * hd * 2), B(hkv * cap * hd * 2), f(T * hq * hd),
                               1, 15, T, hq, hkv, hd, cap, 1e-6, 1e6, 1.0, 0.125)
    assert rc_of(hip, "ds5_hip_attention_step", ok) == 3
    bad = hip.AttentionStepArgs.from_buffer_copy(ok)
    bad.pos = 16
    assert rc_of(hip, "ds5_hip_attention_step", bad) == 1
    bad = hip.AttentionStepArgs.from_buffer_copy(ok)
    bad.k_norm = f(hd - 1)
    assert rc_of(hip, "ds5_hip_attention_step", bad) == 1
    n_pages, ps, mp, B_ = 10, 16, 4, 3
    pg = hip.PagedDecodeArgs(f(B_ * hq * hd), f(B_ * hkv * hd), f(B_ * hkv * hd), f(hd), f(hd),
                             B(hkv * n_pages * ps * hd * 2), B(hkv * n_pages * ps * hd * 2), f(B_ * mp), f(B_),
                             f(B_ * hq * hd), B_, hq, hkv, hd, ps, n_pages, mp, 64, 1e-6, 1e6, 1.0, 0.125)
    assert rc_of(hip, "ds5_hip_paged_decode", pg) == 3
    bad = hip.PagedDecodeArgs.from_buffer_copy(pg)
    bad.max_seq_len = 65
    assert rc_of(hip, "ds5_hip_paged_decode", bad) == 1
    bad = hip.PagedDecodeArgs.from_buffer_copy(pg)
    bad.head_dim = 96
    assert rc_of(hip, "ds5_hip_paged_decode", bad) == 1
    bad = hip.PagedDecodeArgs.from_buffer_copy(pg)
    bad.page_size = 8  # a 16-position half tile must not straddle pages
    assert rc_of(hip, "ds5_hip_paged_decode", bad) == 1


def test_rope_table_is_the_oracle_pow(hip, oracle):
    # The kernels' inv_freq table equals the oracle's std.math.pow(f32) restatement bit for bit.
    for theta in (1e6, 5e6, 1e4, 100.0):
        for hd in (4, 64, 128, 256):
            t = hip.rope_table(theta, hd)
            o = np.array([oracle.zig_powf(theta, -np.float32(2 * i) / np.float32(hd)) for i in range(hd // 2)],
                         np.float32)
            assert np.array_equal(t.view(np.uint32), o.view(np.uint32)), (theta, hd)
    with pytest.raises(hip.ShapeMismatch):
        hip.rope_table(1e6, 7)


def test_library_missing_fails_loudly(hip, tmp_path):
    with pytest.raises(ImportError, match="no CPU fallback"):
        hip.load_library(str(tmp_path / "nope.so"))
