"""Host-side mirror of DS5's kernel-provider interface over libds5hip.so.

The reference engine (src/engine/forward.zig:154) is generic over a device
context `Ctx` (contracts.assertGpuApi, src/shared/contracts.zig:374-384) and a
kernel namespace `K` (contracts.assertKernelApi, :358-367). This module gives
both the same names, argument meaning and error behaviour, bound to the gfx950
backend through its C ABI (include/ds5_hip.h):

    ctx = Ctx.init()                         # Ctx.init(allocator)
    buf = ctx.createBuffer(n)                # zero-filled device buffer
    ctx.upload(buf, 0, host_bytes); ctx.download(buf, 0, out)
    rmsNorm(ctx, RmsNormArgs(...)); rope(ctx, RopeArgs(...))
    kvAppend(ctx, KvAppendArgs(...)); gqaAttention(ctx, AttnArgs(...))
    ctx.begin(); ...; ctx.submit(); ctx.gpuElapsedNs()

Failures raise the KernelError subclasses named after the reference's error
set (src/shared/contracts.zig:201-206). There is no CPU fallback: when the
shared library is missing, importing this module fails.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libds5hip.so")

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_Q8_0 = 8


# ---------------------------------------------------------------------------
# KernelError (contracts.zig:201-206)
# ---------------------------------------------------------------------------
class KernelError(Exception):
    code = 0


class ShapeMismatch(KernelError):
    code = 1


class UnsupportedDtype(KernelError):
    code = 2


class DeviceFailure(KernelError):
    code = 3


class OutOfMemory(KernelError):
    code = 4


_ERRORS = {c.code: c for c in (ShapeMismatch, UnsupportedDtype, DeviceFailure, OutOfMemory)}


# ---------------------------------------------------------------------------
# ABI structs (include/ds5_hip.h)
# ---------------------------------------------------------------------------
class Buf(C.Structure):
    """contracts.zig:210-214 Buf: device base pointer + byte offset + byte length."""
    _fields_ = [("handle", C.c_void_p), ("offset", C.c_uint64), ("len", C.c_uint64)]

    def view(self, offset: int, length: int) -> "Buf":
        """Sub-view [offset, offset+length) of this view (bytes)."""
        return Buf(self.handle, self.offset + offset, length)


class RmsNormArgs(C.Structure):
    _fields_ = [("x", Buf), ("weight", Buf), ("out", Buf), ("n_rows", C.c_uint32), ("dim", C.c_uint32),
                ("eps", C.c_float)]


class RopeArgs(C.Structure):
    _fields_ = [("x", Buf), ("positions", Buf), ("n_tokens", C.c_uint32), ("n_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("theta", C.c_float), ("freq_scale", C.c_float)]

    def __init__(self, *args, **kw):
        if len(args) < len(self._fields_):
            kw.setdefault("freq_scale", 1.0)  # contracts.zig:237 default
        super().__init__(*args, **kw)


class KvAppendArgs(C.Structure):
    _fields_ = [("k_new", Buf), ("v_new", Buf), ("k_cache", Buf), ("v_cache", Buf), ("kv_dtype", C.c_uint32),
                ("pos", C.c_uint32), ("n_tokens", C.c_uint32), ("n_kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("max_ctx", C.c_uint32)]


class MatmulArgs(C.Structure):
    _fields_ = [("x", Buf), ("w", Buf), ("w_dtype", C.c_uint32), ("out", Buf), ("m", C.c_uint32),
                ("n", C.c_uint32), ("k", C.c_uint32)]


class AddArgs(C.Structure):
    _fields_ = [("x", Buf), ("y", Buf), ("out", Buf), ("n_elems", C.c_uint64)]


class MatmulAddArgs(C.Structure):
    _fields_ = [("x", Buf), ("w", Buf), ("w_dtype", C.c_uint32), ("residual", Buf), ("out", Buf),
                ("m", C.c_uint32), ("n", C.c_uint32), ("k", C.c_uint32)]


class RouterArgs(C.Structure):
    _fields_ = [("x", Buf), ("w", Buf), ("w_dtype", C.c_uint32), ("n_tokens", C.c_uint32), ("dim", C.c_uint32),
                ("n_experts", C.c_uint32), ("top_k", C.c_uint32), ("norm_topk_prob", C.c_uint32),
                ("out_ids", C.POINTER(C.c_uint16)), ("out_ids_len", C.c_uint64),
                ("out_weights", C.POINTER(C.c_float)), ("out_weights_len", C.c_uint64)]


class Pair(C.Structure):  # contracts.zig:308-312 PairDispatch
    _fields_ = [("token", C.c_uint32), ("expert", C.c_uint32), ("weight", C.c_float)]


PAIR_DTYPE = np.dtype([("token", np.uint32), ("expert", np.uint32), ("weight", np.float32)])


class ExpertMlpArgs(C.Structure):
    _fields_ = [("x", Buf), ("gate", Buf), ("up", Buf), ("down", Buf), ("w_dtype", C.c_uint32),
                ("pairs", C.c_void_p), ("n_pairs", C.c_uint64), ("out", Buf), ("n_tokens", C.c_uint32),
                ("dim", C.c_uint32), ("ffn_dim", C.c_uint32), ("n_experts", C.c_uint32)]


class MoeArgs(C.Structure):
    _fields_ = [("x", Buf), ("router_w", Buf), ("router_dtype", C.c_uint32), ("gate", Buf), ("up", Buf),
                ("down", Buf), ("w_dtype", C.c_uint32), ("out", Buf), ("ids", Buf), ("weights", Buf),
                ("n_tokens", C.c_uint32), ("dim", C.c_uint32), ("ffn_dim", C.c_uint32), ("n_experts", C.c_uint32),
                ("top_k", C.c_uint32), ("norm_topk_prob", C.c_uint32), ("residual", Buf), ("x_norm", Buf),
                ("x_norm_eps", C.c_float)]


MATMUL_GROUP_MAX = 4


class MatmulGroupArgs(C.Structure):
    _fields_ = [("x", Buf), ("w_dtype", C.c_uint32), ("m", C.c_uint32), ("k", C.c_uint32), ("count", C.c_uint32),
                ("w", Buf * MATMUL_GROUP_MAX), ("out", Buf * MATMUL_GROUP_MAX), ("n", C.c_uint32 * MATMUL_GROUP_MAX)]

    @classmethod
    def of(cls, x: Buf, w_dtype: int, m: int, k: int, entries) -> "MatmulGroupArgs":
        """entries: (w, out, n) triples, at most MATMUL_GROUP_MAX."""
        a = cls(x=x, w_dtype=w_dtype, m=m, k=k, count=len(entries))
        for e, (w, out, n) in enumerate(entries):
            a.w[e], a.out[e], a.n[e] = w, out, n
        return a


class AttnArgs(C.Structure):
    _fields_ = [("q", Buf), ("k_cache", Buf), ("v_cache", Buf), ("kv_dtype", C.c_uint32), ("out", Buf),
                ("pos", C.c_uint32), ("n_tokens", C.c_uint32), ("n_q_heads", C.c_uint32),
                ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("max_ctx", C.c_uint32),
                ("scale", C.c_float)]


class AttentionStepArgs(C.Structure):
    _fields_ = [(n, Buf) for n in ("q", "k", "v", "q_norm", "k_norm", "positions", "k_cache", "v_cache", "out")] + \
               [(n, C.c_uint32) for n in ("kv_dtype", "pos", "n_tokens", "n_q_heads", "n_kv_heads", "head_dim",
                                          "max_ctx")] + \
               [(n, C.c_float) for n in ("eps", "theta", "freq_scale", "scale")]


class AttentionBlockArgs(C.Structure):
    """ds5_attention_block_args: the q/k/v projections of x then the attention step."""
    _fields_ = [("x", Buf), ("wq", Buf), ("wk", Buf), ("wv", Buf), ("w_dtype", C.c_uint32), ("hidden", C.c_uint32),
                ("step", AttentionStepArgs), ("x_norm", Buf), ("x_norm_eps", C.c_float)]


class PagedDecodeArgs(C.Structure):
    _fields_ = [(n, Buf) for n in ("q", "k", "v", "q_norm", "k_norm", "k_pool", "v_pool", "page_table",
                                   "seq_lens", "out")] + \
               [(n, C.c_uint32) for n in ("n_seqs", "n_q_heads", "n_kv_heads", "head_dim", "page_size", "n_pages",
                                          "max_pages", "max_seq_len")] + \
               [(n, C.c_float) for n in ("eps", "theta", "freq_scale", "scale")]


# Every symbol include/ds5_hip.h declares, with its ctypes signature.
_P = C.c_void_p
SIGNATURES = {
    "ds5_hip_init": ([C.c_int, C.POINTER(C.c_void_p)], C.c_int),
    "ds5_hip_deinit": ([_P], None),
    "ds5_hip_create_buffer": ([_P, C.c_uint64, C.POINTER(Buf)], C.c_int),
    "ds5_hip_buffer_from_bytes": ([_P, C.c_void_p, C.c_uint64, C.POINTER(Buf)], C.c_int),
    "ds5_hip_upload": ([_P, Buf, C.c_uint64, C.c_void_p, C.c_uint64], C.c_int),
    "ds5_hip_download": ([_P, Buf, C.c_uint64, C.c_void_p, C.c_uint64], C.c_int),
    "ds5_hip_begin": ([_P], None),
    "ds5_hip_submit": ([_P], C.c_int),
    "ds5_hip_gpu_elapsed_ns": ([_P], C.c_uint64),
    "ds5_hip_last_error": ([_P], C.c_char_p),
    "ds5_hip_stream": ([_P], C.c_void_p),
    "ds5_hip_capture_begin": ([_P], C.c_int),
    "ds5_hip_capture_end": ([_P, C.POINTER(C.c_void_p)], C.c_int),
    "ds5_hip_graph_launch": ([_P, C.c_void_p], C.c_int),
    "ds5_hip_graph_destroy": ([C.c_void_p], None),
    "ds5_hip_timing_begin": ([_P], C.c_int),
    "ds5_hip_timing_mark": ([_P], C.c_int),
    "ds5_hip_timing_read": ([_P, C.POINTER(C.c_uint64), C.c_uint32, C.POINTER(C.c_uint32)], C.c_int),
    "ds5_hip_set_kernel_timing": ([_P, C.c_int], C.c_int),
    "ds5_hip_kernel_time": ([_P, C.c_char_p, C.POINTER(C.c_uint64), C.POINTER(C.c_double)], C.c_int),
    "ds5_hip_rms_norm": ([_P, C.POINTER(RmsNormArgs)], C.c_int),
    "ds5_hip_rope": ([_P, C.POINTER(RopeArgs)], C.c_int),
    "ds5_hip_kv_append": ([_P, C.POINTER(KvAppendArgs)], C.c_int),
    "ds5_hip_gqa_attention": ([_P, C.POINTER(AttnArgs)], C.c_int),
    "ds5_hip_matmul": ([_P, C.POINTER(MatmulArgs)], C.c_int),
    "ds5_hip_matmul_group": ([_P, C.POINTER(MatmulGroupArgs)], C.c_int),
    "ds5_hip_add": ([_P, C.POINTER(AddArgs)], C.c_int),
    "ds5_hip_matmul_add": ([_P, C.POINTER(MatmulAddArgs)], C.c_int),
    "ds5_hip_router_topk": ([_P, C.POINTER(RouterArgs)], C.c_int),
    "ds5_hip_expert_mlp_swiglu": ([_P, C.POINTER(ExpertMlpArgs)], C.c_int),
    "ds5_hip_moe": ([_P, C.POINTER(MoeArgs)], C.c_int),
    "ds5_hip_attention_step": ([_P, C.POINTER(AttentionStepArgs)], C.c_int),
    "ds5_hip_attention_step_noalloc": ([_P, C.POINTER(AttentionStepArgs)], C.c_int),
    "ds5_hip_attention_block": ([_P, C.POINTER(AttentionBlockArgs)], C.c_int),
    "ds5_hip_paged_decode": ([_P, C.POINTER(PagedDecodeArgs)], C.c_int),
    "ds5_hip_rope_table": ([C.c_float, C.c_uint32, C.c_void_p], C.c_int),
    "ds5_hip_fill_normal_f16": ([_P, Buf, C.c_uint64, C.c_uint64], C.c_int),
    "ds5_hip_copy_device": ([_P, Buf, Buf, C.c_uint64], C.c_int),
    "ds5_hip_zero": ([_P, Buf, C.c_uint64], C.c_int),
    "ds5_hip_stream_read": ([_P, Buf, C.c_uint64, Buf], C.c_int),
    "ds5_hip_empty_launch": ([_P, C.c_uint32], C.c_int),
}


def load_library(path: str = LIB_PATH) -> C.CDLL:
    if not os.path.exists(path):
        raise ImportError(f"{path} is not built: run `python -m qw3_amd.build` "
                          "(the HIP backend has no CPU fallback)")
    lib = C.CDLL(path)
    for name, (argtypes, restype) in SIGNATURES.items():
        f = getattr(lib, name)
        f.argtypes = argtypes
        f.restype = restype
    return lib


LIB = load_library()


def _as_array(x) -> np.ndarray:
    """A C-contiguous numpy view of a host buffer (ndarray, bytes, bytearray, memoryview)."""
    if isinstance(x, np.ndarray):
        if not x.flags["C_CONTIGUOUS"]:
            raise ValueError("host buffer must be C-contiguous")
        return x
    return np.frombuffer(x, dtype=np.uint8)


def _nbytes(x) -> int:
    return _as_array(x).nbytes


def _ptr(x):
    return _as_array(x).ctypes.data


# ---------------------------------------------------------------------------
# Ctx (contracts.assertGpuApi)
# ---------------------------------------------------------------------------
class Ctx:
    def __init__(self, handle: C.c_void_p):
        self._h = handle

    @classmethod
    def init(cls, device_index: int = 0) -> "Ctx":
        h = C.c_void_p()
        rc = LIB.ds5_hip_init(device_index, C.byref(h))
        if rc:
            raise _ERRORS.get(rc, KernelError)(f"ds5_hip_init failed ({rc})")
        return cls(h)

    def deinit(self) -> None:
        if self._h:
            LIB.ds5_hip_deinit(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.deinit()

    @property
    def handle(self):
        return self._h

    def check(self, rc: int) -> None:
        if rc:
            raise _ERRORS.get(rc, KernelError)(LIB.ds5_hip_last_error(self._h).decode())

    def createBuffer(self, length: int) -> Buf:
        b = Buf()
        self.check(LIB.ds5_hip_create_buffer(self._h, length, C.byref(b)))
        return b

    def bufferFromBytes(self, data) -> Buf:
        b = Buf()
        data = np.ascontiguousarray(data) if isinstance(data, np.ndarray) else data
        self.check(LIB.ds5_hip_buffer_from_bytes(self._h, _ptr(data), _nbytes(data), C.byref(b)))
        return b

    def upload(self, buf: Buf, offset: int, data) -> None:
        data = np.ascontiguousarray(data) if isinstance(data, np.ndarray) else data
        self.check(LIB.ds5_hip_upload(self._h, buf, offset, _ptr(data), _nbytes(data)))

    def download(self, buf: Buf, offset: int, out) -> None:
        self.check(LIB.ds5_hip_download(self._h, buf, offset, _ptr(out), _nbytes(out)))

    def begin(self) -> None:
        LIB.ds5_hip_begin(self._h)

    def submit(self) -> None:
        self.check(LIB.ds5_hip_submit(self._h))

    def gpuElapsedNs(self) -> int:
        return LIB.ds5_hip_gpu_elapsed_ns(self._h)

    # numpy conveniences (tests, bench)
    def from_numpy(self, a: np.ndarray) -> Buf:
        return self.bufferFromBytes(np.ascontiguousarray(a))

    def to_numpy(self, buf: Buf, dtype, shape=None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = (buf.len - offset) // dtype.itemsize if shape is None else int(np.prod(shape))
        out = np.empty(n, dtype)
        self.download(buf, offset, out)
        return out if shape is None else out.reshape(shape)

    def capture(self, fn) -> "Graph":
        """Records the device work `fn()` enqueues into a replayable graph."""
        self.check(LIB.ds5_hip_capture_begin(self._h))
        try:
            fn()
        finally:
            g = C.c_void_p()
            rc = LIB.ds5_hip_capture_end(self._h, C.byref(g))
        self.check(rc)
        return Graph(self, g)

    def timing_begin(self) -> None:
        """Forget earlier device-time marks (kernels/gpu/kernels.zig:446-449 beginTiming)."""
        self.check(LIB.ds5_hip_timing_begin(self._h))

    def timing_mark(self) -> None:
        """Record a device-time mark on the stream (no synchronisation)."""
        self.check(LIB.ds5_hip_timing_mark(self._h))

    def timing_read(self, max_count: int = 4096) -> list[int]:
        """Device ns between consecutive marks (synchronises; kernels.zig:465-467 layerNs)."""
        buf = (C.c_uint64 * max(1, max_count))()
        n = C.c_uint32()
        self.check(LIB.ds5_hip_timing_read(self._h, buf, max_count, C.byref(n)))
        return [int(buf[i]) for i in range(min(n.value, max_count))]

    def set_kernel_timing(self, enable: bool) -> None:
        self.check(LIB.ds5_hip_set_kernel_timing(self._h, int(enable)))

    def kernel_time(self, kernel: str) -> tuple[int, float]:
        """(launches, total device ns) of `kernel` since timing was enabled."""
        n, t = C.c_uint64(), C.c_double()
        self.check(LIB.ds5_hip_kernel_time(self._h, kernel.encode(), C.byref(n), C.byref(t)))
        return n.value, t.value

    def fill_normal_f16(self, buf: Buf, n: int, seed: int) -> None:
        self.check(LIB.ds5_hip_fill_normal_f16(self._h, buf, n, seed))

    def copy_device(self, dst: Buf, src: Buf, length: int) -> None:
        self.check(LIB.ds5_hip_copy_device(self._h, dst, src, length))

    def zero(self, buf: Buf, length: int) -> None:
        """Zero `length` bytes of buf on the context stream (fill kernel, no host copy)."""
        self.check(LIB.ds5_hip_zero(self._h, buf, length))

    def stream_read(self, buf: Buf, length: int, sink: Buf) -> None:
        """One launch reading `length` bytes of buf once (the decode's contiguous K/V access, nothing computed)."""
        self.check(LIB.ds5_hip_stream_read(self._h, buf, length, sink))

    def empty_launch(self, n_workgroups: int = 256) -> None:
        self.check(LIB.ds5_hip_empty_launch(self._h, n_workgroups))


class Graph:
    """An executable HIP graph captured on a context's stream."""

    def __init__(self, ctx: Ctx, handle: C.c_void_p):
        self.ctx, self._g = ctx, handle

    def launch(self) -> None:
        self.ctx.check(LIB.ds5_hip_graph_launch(self.ctx.handle, self._g))

    def destroy(self) -> None:
        if self._g:
            LIB.ds5_hip_graph_destroy(self._g)
            self._g = None


# ---------------------------------------------------------------------------
# Kernel provider (contracts.assertKernelApi: the attention-path ops)
# ---------------------------------------------------------------------------
def rmsNorm(ctx: Ctx, args: RmsNormArgs) -> None:
    ctx.check(LIB.ds5_hip_rms_norm(ctx.handle, C.byref(args)))


def rope(ctx: Ctx, args: RopeArgs) -> None:
    ctx.check(LIB.ds5_hip_rope(ctx.handle, C.byref(args)))


def kvAppend(ctx: Ctx, args: KvAppendArgs) -> None:
    ctx.check(LIB.ds5_hip_kv_append(ctx.handle, C.byref(args)))


def gqaAttention(ctx: Ctx, args: AttnArgs) -> None:
    ctx.check(LIB.ds5_hip_gqa_attention(ctx.handle, C.byref(args)))


def matmul(ctx: Ctx, args: MatmulArgs) -> None:
    """out[m, n] = x[m, k] . W^T, W f32 or Q8_0 rows (kernels_a.zig:136-163)."""
    ctx.check(LIB.ds5_hip_matmul(ctx.handle, C.byref(args)))


def add(ctx: Ctx, args: AddArgs) -> None:
    """out = x + y over n_elems f32 (kernels_a.zig:223-233); out may alias x or y."""
    ctx.check(LIB.ds5_hip_add(ctx.handle, C.byref(args)))


def matmulAdd(ctx: Ctx, args: MatmulAddArgs) -> None:
    """out = residual + x . W^T (forward.zig:416-418's matmul then add, one launch)."""
    ctx.check(LIB.ds5_hip_matmul_add(ctx.handle, C.byref(args)))


def routerTopK(ctx: Ctx, x: Buf, w: Buf, w_dtype: int, n_tokens: int, dim: int, n_experts: int, top_k: int,
               norm_topk_prob: bool):
    """(ids uint16 [n_tokens, top_k], weights f32 [n_tokens, top_k]) on the host
    (kernels_c.zig:80-155; waits for the device)."""
    ids = np.zeros((n_tokens, top_k), np.uint16)
    wts = np.zeros((n_tokens, top_k), np.float32)
    ctx.check(LIB.ds5_hip_router_topk(ctx.handle, C.byref(RouterArgs(
        x, w, w_dtype, n_tokens, dim, n_experts, top_k, int(norm_topk_prob),
        ids.ctypes.data_as(C.POINTER(C.c_uint16)), ids.size, wts.ctypes.data_as(C.POINTER(C.c_float)), wts.size))))
    return ids, wts


def expertMlpSwiglu(ctx: Ctx, x: Buf, gate: Buf, up: Buf, down: Buf, w_dtype: int, pairs: np.ndarray, out: Buf,
                    n_tokens: int, dim: int, ffn_dim: int, n_experts: int) -> None:
    """out[token] += weight * down(silu(gate(x)) * up(x)) per (token, expert, weight)
    pair of the host array `pairs` (PAIR_DTYPE) (kernels_c.zig:157-214)."""
    pairs = np.ascontiguousarray(pairs, dtype=PAIR_DTYPE)
    ctx.check(LIB.ds5_hip_expert_mlp_swiglu(ctx.handle, C.byref(ExpertMlpArgs(
        x, gate, up, down, w_dtype, pairs.ctypes.data if pairs.size else None, pairs.size, out, n_tokens, dim,
        ffn_dim, n_experts))))


def moe(ctx: Ctx, args: MoeArgs) -> None:
    """Router and experts on the device, no host round trip (ds5_hip_moe)."""
    ctx.check(LIB.ds5_hip_moe(ctx.handle, C.byref(args)))


def matmulGroup(ctx: Ctx, args: MatmulGroupArgs) -> None:
    """Up to 4 matmuls on the same x (the engine's q/k/v projections,
    forward.zig:337-339) in one call; each entry equals ds5_hip_matmul bit for bit."""
    ctx.check(LIB.ds5_hip_matmul_group(ctx.handle, C.byref(args)))


def attentionStep(ctx: Ctx, args: AttentionStepArgs) -> None:
    """Fused q/k norm + rope + kvAppend + gqaAttention (one engine layer's attention block)."""
    ctx.check(LIB.ds5_hip_attention_step(ctx.handle, C.byref(args)))


def attentionBlock(ctx: Ctx, args: AttentionBlockArgs) -> None:
    """The q/k/v projections of x then attentionStep, as one call (prefill: the pre-pass
    runs in the projection GEMM's epilogue). No reference counterpart."""
    ctx.check(LIB.ds5_hip_attention_block(ctx.handle, C.byref(args)))


# DS5_NOALLOC_SCRATCH_BYTES (include/ds5_hip.h): the static scratch of the allocation-free entry point
NOALLOC_SCRATCH_BYTES = 4 << 20


def attentionStepNoAlloc(ctx: Ctx, args: AttentionStepArgs) -> None:
    """attentionStep without any device allocation: its split-K partials or f16 q
    operand live in the library's static per-GPU scratch (NOALLOC_SCRATCH_BYTES);
    calls needing more fail with ShapeMismatch. No reference counterpart."""
    ctx.check(LIB.ds5_hip_attention_step_noalloc(ctx.handle, C.byref(args)))


def rope_table(theta: float, head_dim: int) -> np.ndarray:
    """The inv_freq table the rope kernels use (host computation, no device)."""
    out = np.zeros(head_dim // 2, np.float32)
    rc = LIB.ds5_hip_rope_table(theta, head_dim, out.ctypes.data)
    if rc:
        raise _ERRORS.get(rc, KernelError)("ds5_hip_rope_table")
    return out


def pagedDecode(ctx: Ctx, args: PagedDecodeArgs) -> None:
    """Batched decode over a paged f16 pool (one new token per sequence)."""
    ctx.check(LIB.ds5_hip_paged_decode(ctx.handle, C.byref(args)))
