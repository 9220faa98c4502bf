"""Python face of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; it is the checker, never the thing measured or shipped.

Wraps oracle/build/libds5oracle.so (the C restatement of the reference CPU
path, see ds5_oracle.c) with numpy-friendly helpers, and restates:
  * the DS5T fixture reader  -- src/shared/fixture.zig:42-63 and
    src/shared/contracts.zig:426-449 (magic 0x54355344, 64-byte header,
    ne[0] fastest-varying, data at byte 64)
  * the frozen pass rule     -- src/shared/fixture.zig:87-110
    (|a - o| <= atol + rtol*|o| for every element, f32, NaN fails)
"""
from __future__ import annotations

import ctypes as C
import json
import os
import struct
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libds5oracle.so")

OK, SHAPE_MISMATCH, UNSUPPORTED_DTYPE, DEVICE_FAILURE, OUT_OF_MEMORY = 0, 1, 2, 3, 4
F32, F16, I32 = 0, 1, 26
Q8_0 = 8  # contracts.zig:29; 32-element blocks of 34 bytes (f16 scale, 32 x int8)
ERRORS = {1: "ShapeMismatch", 2: "UnsupportedDtype", 3: "DeviceFailure", 4: "OutOfMemory"}


class KernelError(Exception):
    def __init__(self, code: int):
        super().__init__(ERRORS.get(code, f"status {code}"))
        self.code = code


class Buf(C.Structure):
    _fields_ = [("handle", C.c_void_p), ("offset", C.c_uint64), ("len", C.c_uint64)]


class MatmulArgs(C.Structure):  # contracts.zig:242-250
    _fields_ = [("x", Buf), ("w", Buf), ("w_dtype", C.c_uint32), ("out", Buf),
                ("m", C.c_uint32), ("n", C.c_uint32), ("k", C.c_uint32)]


class AddArgs(C.Structure):  # contracts.zig:334-339
    _fields_ = [("x", Buf), ("y", Buf), ("out", Buf), ("n_elems", C.c_uint64)]


class RouterArgs(C.Structure):  # contracts.zig:293-304
    _fields_ = [("x", Buf), ("w", Buf), ("w_dtype", C.c_uint32), ("n_tokens", C.c_uint32), ("dim", C.c_uint32),
                ("n_experts", C.c_uint32), ("top_k", C.c_uint32), ("norm_topk_prob", C.c_uint32),
                ("out_ids", C.POINTER(C.c_uint16)), ("out_ids_len", C.c_uint64),
                ("out_weights", C.POINTER(C.c_float)), ("out_weights_len", C.c_uint64)]


class Pair(C.Structure):  # contracts.zig:308-312 PairDispatch
    _fields_ = [("token", C.c_uint32), ("expert", C.c_uint32), ("weight", C.c_float)]


PAIR_DTYPE = np.dtype([("token", np.uint32), ("expert", np.uint32), ("weight", np.float32)])


class ExpertMlpArgs(C.Structure):  # contracts.zig:319-331
    _fields_ = [("x", Buf), ("gate", Buf), ("up", Buf), ("down", Buf), ("w_dtype", C.c_uint32),
                ("pairs", C.c_void_p), ("n_pairs", C.c_uint64), ("out", Buf), ("n_tokens", C.c_uint32),
                ("dim", C.c_uint32), ("ffn_dim", C.c_uint32), ("n_experts", C.c_uint32)]


class RmsNormArgs(C.Structure):
    _fields_ = [("x", Buf), ("weight", Buf), ("out", Buf), ("n_rows", C.c_uint32),
                ("dim", C.c_uint32), ("eps", C.c_float)]


class RopeArgs(C.Structure):
    _fields_ = [("x", Buf), ("positions", Buf), ("n_tokens", C.c_uint32), ("n_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("theta", C.c_float), ("freq_scale", C.c_float)]


class KvAppendArgs(C.Structure):
    _fields_ = [("k_new", Buf), ("v_new", Buf), ("k_cache", Buf), ("v_cache", Buf),
                ("kv_dtype", C.c_uint32), ("pos", C.c_uint32), ("n_tokens", C.c_uint32),
                ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("max_ctx", C.c_uint32)]


class AttnArgs(C.Structure):
    _fields_ = [("q", Buf), ("k_cache", Buf), ("v_cache", Buf), ("kv_dtype", C.c_uint32),
                ("out", Buf), ("pos", C.c_uint32), ("n_tokens", C.c_uint32), ("n_q_heads", C.c_uint32),
                ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("max_ctx", C.c_uint32),
                ("scale", C.c_float)]


class StepArgs(C.Structure):
    _fields_ = [(n, Buf) for n in ("q", "k", "v", "q_norm_w", "k_norm_w", "positions", "k_cache",
                                   "v_cache", "out")] + \
               [(n, C.c_uint32) for n in ("kv_dtype", "pos", "n_tokens", "n_q_heads", "n_kv_heads",
                                          "head_dim", "max_ctx")] + \
               [(n, C.c_float) for n in ("eps", "theta", "freq_scale", "scale")]


_lib = None


def lib() -> C.CDLL:
    """Load the oracle library, building it first if it is not built yet."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            import importlib.util
            spec = importlib.util.spec_from_file_location("_oracle_build", os.path.join(HERE, "build.py"))
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            mod.build()
        L = C.CDLL(LIB_PATH)
        for name, argt in (("ds5o_rms_norm", RmsNormArgs), ("ds5o_rms_norm_tree", RmsNormArgs),
                           ("ds5o_rope", RopeArgs),
                           ("ds5o_kv_append", KvAppendArgs), ("ds5o_gqa_attention", AttnArgs),
                           ("ds5o_attention_step", StepArgs), ("ds5o_matmul", MatmulArgs),
                           ("ds5o_add", AddArgs), ("ds5o_router_topk", RouterArgs),
                           ("ds5o_expert_mlp_swiglu", ExpertMlpArgs)):
            f = getattr(L, name)
            f.argtypes = [C.POINTER(argt)]
            f.restype = C.c_int
        L.ds5o_zig_powf.argtypes = [C.c_float, C.c_float]
        L.ds5o_zig_powf.restype = C.c_float
        L.ds5o_f32_to_f16.argtypes = [C.c_float]
        L.ds5o_f32_to_f16.restype = C.c_uint16
        L.ds5o_f16_to_f32.argtypes = [C.c_uint16]
        L.ds5o_f16_to_f32.restype = C.c_float
        L.ds5o_f32_to_f16_array.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64]
        L.ds5o_f16_to_f32_array.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64]
        L.ds5o_paged_slot.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.ds5o_paged_slot.restype = C.c_int64
        L.ds5o_paged_gather_f16.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint32, C.c_uint32,
                                            C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p]
        L.ds5o_paged_gather_f16.restype = C.c_int
        _lib = L
    return _lib


def buf(a: np.ndarray | None, offset: int = 0, length: int | None = None) -> Buf:
    """A Buf viewing a C-contiguous numpy array (an empty Buf for None)."""
    if a is None:
        return Buf(None, 0, 0)
    assert a.flags["C_CONTIGUOUS"]
    return Buf(a.ctypes.data, offset, a.nbytes - offset if length is None else length)


def _check(rc: int) -> None:
    if rc != OK:
        raise KernelError(rc)


# --------------------------------------------------------------------------
# Op wrappers (reference semantics, f32 numpy in/out, f16 caches as uint16)
# --------------------------------------------------------------------------

def add(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """out = x + y elementwise in f32 (kernels_a.zig:223-233)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.float32)
    out = np.empty_like(x)
    _check(lib().ds5o_add(AddArgs(buf(x), buf(y), buf(out), x.size)))
    return out


def router_topk(x, w, w_dtype: int, n_tokens: int, dim: int, n_experts: int, top_k: int, norm_topk_prob: bool):
    """(ids uint16 [n_tokens, top_k], weights f32 [n_tokens, top_k]) (kernels_c.zig:80-155)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w)
    ids = np.zeros((n_tokens, top_k), np.uint16)
    wts = np.zeros((n_tokens, top_k), np.float32)
    _check(lib().ds5o_router_topk(RouterArgs(
        buf(x), buf(w), w_dtype, n_tokens, dim, n_experts, top_k, int(norm_topk_prob),
        ids.ctypes.data_as(C.POINTER(C.c_uint16)), ids.size, wts.ctypes.data_as(C.POINTER(C.c_float)), wts.size)))
    return ids, wts


def pairs_from_router(ids: np.ndarray, weights: np.ndarray) -> np.ndarray:
    """Token-major dispatch pairs from a router's outputs (kernels_c.zig:361-373)."""
    T, K = ids.shape
    p = np.zeros(T * K, PAIR_DTYPE)
    p["token"] = np.repeat(np.arange(T, dtype=np.uint32), K)
    p["expert"] = ids.reshape(-1)
    p["weight"] = weights.reshape(-1)
    return p


def expert_mlp_swiglu(x, gate, up, down, w_dtype: int, pairs: np.ndarray, n_tokens: int, dim: int, ffn_dim: int,
                      n_experts: int, out=None) -> np.ndarray:
    """out[token] += weight * down(silu(gate(x)) * up(x)) per pair (kernels_c.zig:157-214);
    out starts at zero unless given."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros((n_tokens, dim), np.float32) if out is None else np.array(out, np.float32, copy=True)
    pairs = np.ascontiguousarray(pairs, dtype=PAIR_DTYPE)
    _check(lib().ds5o_expert_mlp_swiglu(ExpertMlpArgs(
        buf(x), buf(np.ascontiguousarray(gate)), buf(np.ascontiguousarray(up)), buf(np.ascontiguousarray(down)),
        w_dtype, pairs.ctypes.data if pairs.size else None, pairs.size, buf(out), n_tokens, dim, ffn_dim, n_experts)))
    return out


def matmul(x: np.ndarray, w: np.ndarray, w_dtype: int, m: int, n: int, k: int) -> np.ndarray:
    """out[m, n] = x[m, k] . W^T (kernels_a.zig:136-163). w: f32 [n, k], or the raw Q8_0
    rows as uint8 [n, k / 32 * 34]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w)
    out = np.empty((m, n), np.float32)
    _check(lib().ds5o_matmul(MatmulArgs(buf(x), buf(w), w_dtype, buf(out), m, n, k)))
    return out


def q8_0_quantize(w: np.ndarray) -> np.ndarray:
    """Q8_0 rows from f32 rows [n, k] (k a multiple of 32): per 32-element block the
    scale d = f16(max|w| / 127) and q = round(w / d) clipped to [-127, 127]. Test-input
    helper (quantising with the stored f16 scale); the reference only dequantises
    (contracts.zig:194)."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    blocks = w.reshape(n, k // 32, 32)
    amax = np.abs(blocks).max(axis=2, keepdims=True)
    d = (amax / 127.0).astype(np.float16).astype(np.float32)
    inv = np.where(d > 0, 1.0 / np.where(d > 0, d, 1.0), 0.0)
    q = np.clip(np.rint(blocks * inv), -127, 127).astype(np.int8)
    out = np.empty((n, k // 32, 34), np.uint8)
    out[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(n, k // 32, 2)
    out[:, :, 2:] = q.view(np.uint8)
    return out.reshape(n, k // 32 * 34)


def q8_0_dequantize(rows: np.ndarray, k: int) -> np.ndarray:
    """f32 [n, k] from Q8_0 rows: f32(f16 scale) * q, exactly (contracts.zig:194)."""
    rows = np.ascontiguousarray(rows, np.uint8)
    n = rows.shape[0]
    blk = rows.reshape(n, k // 32, 34)
    scale = blk[:, :, 0:2].copy().view(np.float16).astype(np.float32)
    q = blk[:, :, 2:].copy().view(np.int8).astype(np.float32)
    return (scale * q).reshape(n, k)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float, n_rows: int | None = None,
             dim: int | None = None, out: np.ndarray | None = None) -> np.ndarray:
    dim = w.size if dim is None else dim
    n_rows = x.size // dim if n_rows is None else n_rows
    out = np.empty_like(x) if out is None else out
    _check(lib().ds5o_rms_norm(RmsNormArgs(buf(x), buf(w), buf(out), n_rows, dim, eps)))
    return out


def rms_norm_tree(x: np.ndarray, w: np.ndarray, eps: float, n_rows: int | None = None,
                  dim: int | None = None, out: np.ndarray | None = None) -> np.ndarray:
    """rmsNorm in the reference GPU kernel's reduction order (kernels_a.metal:127-165)."""
    dim = w.size if dim is None else dim
    n_rows = x.size // dim if n_rows is None else n_rows
    out = np.empty_like(x) if out is None else out
    _check(lib().ds5o_rms_norm_tree(RmsNormArgs(buf(x), buf(w), buf(out), n_rows, dim, eps)))
    return out


def rms_norm_device_order(x: np.ndarray, w: np.ndarray, eps: float, n_rows: int | None = None,
                          dim: int | None = None) -> np.ndarray:
    """The order ds5_hip_rms_norm uses: serial for rows of up to 256 elements, the
    GPU kernel's tree for longer rows."""
    dim = w.size if dim is None else dim
    return (rms_norm if dim <= 256 else rms_norm_tree)(x, w, eps, n_rows, dim)


def rope(x: np.ndarray, positions: np.ndarray, theta: float, freq_scale: float = 1.0,
         n_tokens: int | None = None, n_heads: int | None = None, head_dim: int | None = None) -> np.ndarray:
    """Rotates a copy of x [n_tokens, n_heads, head_dim] and returns it."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    positions = np.ascontiguousarray(positions, dtype=np.int32)
    n_tokens = x.shape[0] if n_tokens is None else n_tokens
    n_heads = x.shape[1] if n_heads is None else n_heads
    head_dim = x.shape[2] if head_dim is None else head_dim
    _check(lib().ds5o_rope(RopeArgs(buf(y), buf(positions), n_tokens, n_heads, head_dim, theta, freq_scale)))
    return y


def kv_append(k_new, v_new, k_cache, v_cache, kv_dtype: int, pos: int, n_tokens: int, n_kv_heads: int,
              head_dim: int, max_ctx: int) -> None:
    """Scatters into k_cache/v_cache in place (f32 arrays, or uint16 for f16)."""
    _check(lib().ds5o_kv_append(KvAppendArgs(buf(k_new), buf(v_new), buf(k_cache), buf(v_cache), kv_dtype,
                                             pos, n_tokens, n_kv_heads, head_dim, max_ctx)))


def gqa_attention(q, k_cache, v_cache, kv_dtype: int, pos: int, n_tokens: int, n_q_heads: int,
                  n_kv_heads: int, head_dim: int, max_ctx: int, scale: float,
                  out: np.ndarray | None = None) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros(n_tokens * n_q_heads * head_dim, np.float32) if out is None else out
    _check(lib().ds5o_gqa_attention(AttnArgs(buf(q), buf(k_cache), buf(v_cache), kv_dtype, buf(out), pos,
                                              n_tokens, n_q_heads, n_kv_heads, head_dim, max_ctx, scale)))
    return out


def attention_step(q, k, v, q_norm_w, k_norm_w, positions, k_cache, v_cache, *, kv_dtype: int, pos: int,
                   n_tokens: int, n_q_heads: int, n_kv_heads: int, head_dim: int, max_ctx: int,
                   eps: float, theta: float, freq_scale: float = 1.0, scale: float | None = None):
    """forward.zig:345-412 in order; q/k/v (copies) and the caches are updated in place.
    Returns (out, q_rot, k_rot)."""
    q = np.array(q, dtype=np.float32, copy=True)
    k = np.array(k, dtype=np.float32, copy=True)
    v = np.array(v, dtype=np.float32, copy=True)
    positions = np.ascontiguousarray(positions, dtype=np.int32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(head_dim))) if scale is None else scale
    out = np.zeros(n_tokens * n_q_heads * head_dim, np.float32)
    a = StepArgs(buf(q), buf(k), buf(v), buf(q_norm_w), buf(k_norm_w), buf(positions), buf(k_cache),
                 buf(v_cache), buf(out), kv_dtype, pos, n_tokens, n_q_heads, n_kv_heads, head_dim, max_ctx,
                 eps, theta, freq_scale, scale)
    _check(lib().ds5o_attention_step(a))
    return out, q, k


def zig_powf(x: float, y: float) -> float:
    return lib().ds5o_zig_powf(x, y)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().ds5o_f32_to_f16_array(x.ctypes.data, out.ctypes.data, x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().ds5o_f16_to_f32_array(h.ctypes.data, out.ctypes.data, h.size)
    return out


def paged_slot(page_table: np.ndarray, page_size: int, p: int) -> int:
    pt = np.ascontiguousarray(page_table, dtype=np.int32)
    return lib().ds5o_paged_slot(pt.ctypes.data, pt.size, page_size, p)


def paged_gather_f16(pool: np.ndarray, page_table: np.ndarray, page_size: int, length: int) -> np.ndarray:
    """pool: uint16 [n_kv_heads, pool_slots, head_dim] -> uint16 [n_kv_heads, length, head_dim]."""
    hkv, slots, hd = pool.shape
    pt = np.ascontiguousarray(page_table, dtype=np.int32)
    out = np.empty((hkv, length, hd), np.uint16)
    _check(lib().ds5o_paged_gather_f16(np.ascontiguousarray(pool).ctypes.data, slots, pt.ctypes.data,
                                       pt.size, page_size, length, hkv, hd, out.ctypes.data))
    return out


# --------------------------------------------------------------------------
# DS5T fixtures (fixture.zig:42-63) and the pass rule (fixture.zig:87-110)
# --------------------------------------------------------------------------

DS5T_MAGIC = 0x54355344
_NP_DTYPE = {F32: np.float32, F16: np.uint16, I32: np.int32}


@dataclass
class Tensor:
    dtype: int
    ne: tuple
    data: np.ndarray  # numpy shape = reversed(ne[:n_dims])


def load_ds5t(path: str) -> Tensor:
    raw = open(path, "rb").read()
    if len(raw) < 64:
        raise ValueError("SizeMismatch")
    magic, version, dtype, n_dims, ne0, ne1, ne2, ne3, data_bytes, _ = struct.unpack_from("<IIII4QQQ", raw)
    if magic != DS5T_MAGIC:
        raise ValueError("BadMagic")
    if version != 1:
        raise ValueError("BadVersion")
    ne = (ne0, ne1, ne2, ne3)
    if dtype == Q8_0:  # raw rows of 34-byte blocks: uint8 [rows, ne0 / 32 * 34] (3-D banks: rows = ne1 * ne2)
        if ne0 % 32 or n_dims not in (2, 3):
            raise ValueError("SizeMismatch")
        row_bytes = ne0 // 32 * 34
        rows = ne1 * (ne2 if n_dims == 3 else 1)
        if row_bytes * rows != data_bytes or len(raw) < 64 + data_bytes:
            raise ValueError("SizeMismatch")
        arr = np.frombuffer(raw, dtype=np.uint8, count=data_bytes, offset=64).copy()
        return Tensor(dtype, ne[:n_dims], arr.reshape(rows, row_bytes))
    if dtype not in _NP_DTYPE:
        raise ValueError(f"BadDtype {dtype}")
    n = ne0 * ne1 * ne2 * ne3
    itemsize = np.dtype(_NP_DTYPE[dtype]).itemsize
    if n * itemsize != data_bytes or len(raw) < 64 + data_bytes:
        raise ValueError("SizeMismatch")
    arr = np.frombuffer(raw, dtype=_NP_DTYPE[dtype], count=n, offset=64).copy()
    shape = tuple(reversed(ne[:n_dims]))
    return Tensor(dtype, ne[:n_dims], arr.reshape(shape))


def write_ds5t(path: str, data: np.ndarray, dtype: int) -> None:
    data = np.ascontiguousarray(data)
    ne = list(reversed(data.shape)) + [1] * (4 - data.ndim)
    hdr = struct.pack("<IIII4QQQ", DS5T_MAGIC, 1, dtype, data.ndim, *ne, data.nbytes, 0)
    with open(path, "wb") as f:
        f.write(hdr + data.tobytes())


@dataclass
class CompareResult:
    passed: bool
    n: int
    n_bad: int
    first_bad: int
    max_abs_diff: float
    max_rel_diff: float


def compare(oracle: np.ndarray, actual: np.ndarray, atol: float, rtol: float) -> CompareResult:
    """fixture.zig:87-110, evaluated in f32 like the Zig code."""
    o = np.ascontiguousarray(oracle, dtype=np.float32).ravel()
    a = np.ascontiguousarray(actual, dtype=np.float32).ravel()
    assert o.shape == a.shape
    with np.errstate(invalid="ignore", divide="ignore"):
        diff = np.abs(a - o)
        absO = np.abs(o)
        rel = np.where(o != 0, diff / np.where(o != 0, absO, np.float32(1)), np.float32(0)).astype(np.float32)
        bound = np.float32(atol) + np.float32(rtol) * absO
        bad = np.isnan(diff) | (diff > bound)
    n_bad = int(bad.sum())
    first = int(np.argmax(bad)) if n_bad else 0
    return CompareResult(n_bad == 0, o.size, n_bad, first, float(np.nanmax(diff)) if o.size else 0.0,
                         float(np.nanmax(rel)) if o.size else 0.0)


def load_manifest(fixture_dir: str) -> dict:
    with open(os.path.join(fixture_dir, "manifest.json")) as f:
        return json.load(f)
