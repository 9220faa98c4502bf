"""The reference engine's forward pass (src/engine/forward.zig:154-516) over the gfx950
kernel provider.

DS5's engine is generic over a device context and a kernel namespace
(`Engine(Ctx, K)`, forward.zig:154); `ds5 run --backend hip` instantiates it with the
hip context and provider. This module is that instantiation on the host side of the C
ABI: the same buffers (forward.zig:209-272), the same calls in the same order, and the
same trace points, with every kernel running on the device through `qw3_amd.hip`.
Only what the reference does on the host stays on the host: the embedding rows are
dequantised there and uploaded (forward.zig:310-316), and in `fused=False` mode the
router's ids and weights come back to build the expert pairs (forward.zig:432-467).

Two modes:
- `fused=False`: exactly the eight provider ops of `assertKernelApi`
  (src/shared/contracts.zig:356-367), one call per reference call;
- `fused=True`: the optional decls the engine takes via `@hasDecl`: attn_norm, the
  q/k/v projections and the q/k norm + rope + append + attention as one
  `attentionBlock` (attn_norm inside the projection kernels as they read x; at a
  prefill the pre-pass runs in the projection GEMM's epilogue, so q, k and v are
  never written in f32; with a trace callback set, the same work as its calls,
  `rmsNorm`, `matmulGroup` then `attentionStep`, which the block equals bit for bit,
  so those trace points exist), Wo and its residual as one `matmulAdd`, and
  ffn_norm, the MoE block and its residual as one `moe` (ffn_norm inside the router's
  logits kernel, router and experts with the pairs kept on the device, x + the
  experts' sum written in the combine; with a trace callback set, `rmsNorm`, `moe`
  into the zeroed accumulator then `add`, which it equals bit for bit, so those trace
  points exist).
Both produce the residual stream of forward.zig within the reference's layer
tolerance; the per-op calls of the fused mode are bit-identical to the separate ones
where the ABI says so (matmulGroup, matmulAdd, moe).
"""
from __future__ import annotations

import numpy as np

from . import hip as H


def _dtype_of(a: np.ndarray) -> int:
    """The GGUF tensor type of a weight as the engine binds it (forward.zig:81-118 takes
    it from the tensor descriptor): Q8_0 rows (uint8 [rows, k/32*34]), f16 or f32."""
    if a.dtype == np.uint8:
        return H.DTYPE_Q8_0
    if a.dtype == np.float16:
        return H.DTYPE_F16
    if a.dtype == np.float32:
        return H.DTYPE_F32
    raise H.UnsupportedDtype(f"weight dtype {a.dtype}: the provider takes f32, f16 or Q8_0")


class Weights:
    """forward.zig:81-118 Weights.fromGguf: every tensor but the embedding uploaded once;
    the embedding stays on the host for embedRow."""

    def __init__(self, ctx: H.Ctx, tensors: dict, cfg: dict):
        self.cfg = cfg
        self.token_embd = np.ascontiguousarray(tensors["token_embd.weight"])
        self.buf, self.dtype = {}, {}
        for name, a in tensors.items():
            if name == "token_embd.weight":
                continue
            a = np.ascontiguousarray(a)
            self.buf[name] = ctx.bufferFromBytes(a)
            self.dtype[name] = _dtype_of(a)

    def layer(self, li: int, suffix: str):
        name = f"blk.{li}.{suffix}"
        return self.buf[name], self.dtype[name]


class Engine:
    def __init__(self, ctx: H.Ctx, weights: Weights, max_batch: int, context_capacity: int,
                 kv_dtype: int = H.DTYPE_F32, fused: bool = False):
        c = weights.cfg
        if max_batch == 0 or context_capacity == 0 or context_capacity > c["max_ctx"]:
            raise ValueError("BadShape")  # forward.zig:216-230
        if kv_dtype not in (H.DTYPE_F32, H.DTYPE_F16):
            raise H.UnsupportedDtype("kv_dtype must be f32 or f16")
        self.ctx, self.w, self.cfg = ctx, weights, c
        self.max_batch, self.capacity, self.kv_dtype, self.fused = max_batch, context_capacity, kv_dtype, fused
        hidden, hq, hkv, hd = c["hidden_dim"], c["n_q_heads"], c["n_kv_heads"], c["head_dim"]
        q_dim, kv_dim = hq * hd, hkv * hd
        f4 = 4
        mk = ctx.createBuffer
        self.x = mk(max_batch * hidden * f4)
        self.h = mk(max_batch * hidden * f4)
        self.h2 = mk(max_batch * hidden * f4)
        self.q = mk(max_batch * q_dim * f4)
        self.k = mk(max_batch * kv_dim * f4)
        self.v = mk(max_batch * kv_dim * f4)
        self.attn = mk(max_batch * q_dim * f4)
        self.proj = mk(max_batch * hidden * f4)
        self.logits = mk(max_batch * c["vocab_size"] * f4)
        self.positions = mk(max_batch * 4)
        esize = 4 if kv_dtype == H.DTYPE_F32 else 2
        cache_bytes = hkv * context_capacity * hd * esize
        self.k_cache = [mk(cache_bytes) for _ in range(c["n_layers"])]
        self.v_cache = [mk(cache_bytes) for _ in range(c["n_layers"])]
        self.zeros = np.zeros(max_batch * hidden, np.float32)
        self.pos = 0
        self.trace = None  # trace(layer, op, numpy array) at forward.zig's trace points
        self.timing = False

    def begin_timing(self) -> None:
        """kernels/gpu/kernels.zig:446-449 beginTiming: forward passes from now on mark
        the device time of every layer."""
        self.ctx.timing_begin()
        self.timing = True

    def layer_ns(self) -> list[int]:
        """kernels/gpu/kernels.zig:465-467 layerNs: the device ns of each layer of the
        forward passes since begin_timing, in order (run metadata's
        gpu_ns_per_layer_boundary, main.zig:420-444). Every layer is bracketed by marks
        on the stream, so entry i is exactly layer i's device time; the reference's
        boundary batch also spans the previous layer's post-router work, because its
        router syncs mid-layer. Synchronises."""
        ns = self.ctx.timing_read()
        # marks: before each pass's first layer and after each layer; a pass's first
        # interval after the previous pass's last mark spans the host gap between passes
        n_layers = self.cfg["n_layers"]
        per_pass = n_layers + 1
        out = []
        for i, v in enumerate(ns):
            if (i + 1) % per_pass != 0:
                out.append(v)
        return out

    def end_timing(self) -> None:
        """kernels/gpu/kernels.zig:469-473 endTiming."""
        self.timing = False
        self.ctx.timing_begin()

    def reset(self) -> None:
        """forward.zig:288-290."""
        self.pos = 0

    def _trace(self, layer: int, op: str, buf: H.Buf, n_elems: int) -> None:
        if self.trace is not None:
            self.trace(layer, op, self.ctx.to_numpy(buf, np.float32, (n_elems,)))

    def embed_row(self, tok: int) -> np.ndarray:
        """forward.zig:503-516: dequantise the token's Q8_0 (or f32) embedding row."""
        hidden = self.cfg["hidden_dim"]
        e = self.w.token_embd
        if e.dtype != np.uint8:
            return np.asarray(e[tok], np.float32)
        blk = e[tok].reshape(hidden // 32, 34)
        scale = blk[:, 0:2].copy().view(np.float16).astype(np.float32)
        return (scale * blk[:, 2:].copy().view(np.int8).astype(np.float32)).reshape(hidden)

    def forward(self, tokens, want_logits: bool = True):
        """Runs tokens at positions pos..pos+n-1 through every layer; returns the logits
        [n, vocab] on the host (forward.zig:299-500)."""
        c, ctx = self.cfg, self.ctx
        n = len(tokens)
        hidden, hq, hkv, hd = c["hidden_dim"], c["n_q_heads"], c["n_kv_heads"], c["head_dim"]
        q_dim, kv_dim, eps, vocab = hq * hd, hkv * hd, c["rms_eps"], c["vocab_size"]
        if n == 0 or n > self.max_batch:
            raise ValueError("BatchTooLarge")
        if n > self.capacity or self.pos > self.capacity - n:
            raise ValueError("ContextOverflow")
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
        for i, tok in enumerate(tokens):
            if tok >= vocab:
                raise ValueError("TokenOutOfRange")
            ctx.upload(self.x, i * hidden * 4, self.embed_row(int(tok)))
        self._trace(-1, "embed", self.x, n * hidden)
        ctx.upload(self.positions, 0, np.arange(self.pos, self.pos + n, dtype=np.int32))

        if self.timing:
            ctx.timing_mark()
        for li in range(c["n_layers"]):
            attn_norm, _ = self.w.layer(li, "attn_norm.weight")
            (wq, dq), (wk, dk), (wv, dv) = (self.w.layer(li, s) for s in
                                            ("attn_q.weight", "attn_k.weight", "attn_v.weight"))
            # the attention block takes attn_norm itself (h never written) when nothing traces h
            block = self.fused and dq == dk == dv and self.trace is None
            if not block:
                H.rmsNorm(ctx, H.RmsNormArgs(self.x, attn_norm, self.h, n, hidden, eps))
                self._trace(li, "attn_norm", self.h, n * hidden)
            q_norm, _ = self.w.layer(li, "attn_q_norm.weight")
            k_norm, _ = self.w.layer(li, "attn_k_norm.weight")
            step = None
            if self.fused:
                step = H.AttentionStepArgs(
                    self.q, self.k, self.v, q_norm, k_norm, self.positions, self.k_cache[li], self.v_cache[li],
                    self.attn, self.kv_dtype, self.pos, n, hq, hkv, hd, self.capacity, eps, c["rope_theta"], 1.0,
                    scale)
            if block:
                H.attentionBlock(ctx, H.AttentionBlockArgs(self.x, wq, wk, wv, dq, hidden, step, attn_norm, eps))
            elif self.fused and dq == dk == dv:
                H.matmulGroup(ctx, H.MatmulGroupArgs.of(self.h, dq, n, hidden, [
                    (wq, self.q, q_dim), (wk, self.k, kv_dim), (wv, self.v, kv_dim)]))
            else:
                H.matmul(ctx, H.MatmulArgs(self.h, wq, dq, self.q, n, q_dim, hidden))
                H.matmul(ctx, H.MatmulArgs(self.h, wk, dk, self.k, n, kv_dim, hidden))
                H.matmul(ctx, H.MatmulArgs(self.h, wv, dv, self.v, n, kv_dim, hidden))
            self._trace(li, "q_proj", self.q, n * q_dim)
            self._trace(li, "k_proj", self.k, n * kv_dim)
            self._trace(li, "v_proj", self.v, n * kv_dim)
            # fused: q_norm, k_norm, rope_q and rope_k happen inside the step (no trace points)
            if self.fused:
                if not block:
                    H.attentionStep(ctx, step)
            else:
                H.rmsNorm(ctx, H.RmsNormArgs(self.q, q_norm, self.q, n * hq, hd, eps))
                H.rmsNorm(ctx, H.RmsNormArgs(self.k, k_norm, self.k, n * hkv, hd, eps))
                self._trace(li, "q_norm", self.q, n * q_dim)
                self._trace(li, "k_norm", self.k, n * kv_dim)
                H.rope(ctx, H.RopeArgs(self.q, self.positions, n, hq, hd, c["rope_theta"]))
                H.rope(ctx, H.RopeArgs(self.k, self.positions, n, hkv, hd, c["rope_theta"]))
                self._trace(li, "rope_q", self.q, n * q_dim)
                self._trace(li, "rope_k", self.k, n * kv_dim)
                H.kvAppend(ctx, H.KvAppendArgs(self.k, self.v, self.k_cache[li], self.v_cache[li], self.kv_dtype,
                                               self.pos, n, hkv, hd, self.capacity))
                H.gqaAttention(ctx, H.AttnArgs(self.q, self.k_cache[li], self.v_cache[li], self.kv_dtype,
                                               self.attn, self.pos, n, hq, hkv, hd, self.capacity, scale))
            self._trace(li, "attn", self.attn, n * q_dim)

            wo, do = self.w.layer(li, "attn_output.weight")
            if self.fused:
                H.matmulAdd(ctx, H.MatmulAddArgs(self.attn, wo, do, self.x, self.x, n, hidden, q_dim))
            else:
                H.matmul(ctx, H.MatmulArgs(self.attn, wo, do, self.proj, n, hidden, q_dim))
                H.add(ctx, H.AddArgs(self.x, self.proj, self.x, n * hidden))
            self._trace(li, "attn_resid", self.x, n * hidden)

            ffn_norm, _ = self.w.layer(li, "ffn_norm.weight")
            router, dr = self.w.layer(li, "ffn_gate_inp.weight")
            gate, dg = self.w.layer(li, "ffn_gate_exps.weight")
            up, _ = self.w.layer(li, "ffn_up_exps.weight")
            down, _ = self.w.layer(li, "ffn_down_exps.weight")
            if self.fused and self.trace is None:
                # x = x + the experts' sum of ffn_norm(x) in one call: the norm inside it,
                # the sum started from zero and the residual added once, as rmsNorm, the
                # zeroed accumulator and the add give them
                H.moe(ctx, H.MoeArgs(self.x, router, dr, gate, up, down, dg, self.x, H.Buf(), H.Buf(), n,
                                     hidden, c["expert_ffn_dim"], c["n_experts"], c["top_k"],
                                     int(c["norm_topk_prob"]), self.x, ffn_norm, eps))
                if self.timing:
                    ctx.timing_mark()
                self._trace(li, "block", self.x, n * hidden)
                continue
            H.rmsNorm(ctx, H.RmsNormArgs(self.x, ffn_norm, self.h2, n, hidden, eps))
            self._trace(li, "ffn_norm", self.h2, n * hidden)
            # proj doubles as the MoE accumulator and must start at zero (forward.zig:452-454):
            # the eight-op mode uploads zeros as the reference does; the fused mode clears it
            # on the device (no host copy or synchronisation inside the layer)
            if self.fused:
                ctx.zero(self.proj, n * hidden * 4)
            else:
                ctx.upload(self.proj, 0, self.zeros[:n * hidden])
            if self.fused:
                H.moe(ctx, H.MoeArgs(self.h2, router, dr, gate, up, down, dg, self.proj, H.Buf(), H.Buf(), n,
                                     hidden, c["expert_ffn_dim"], c["n_experts"], c["top_k"],
                                     int(c["norm_topk_prob"])))
            else:
                ids, wts = H.routerTopK(ctx, self.h2, router, dr, n, hidden, c["n_experts"], c["top_k"],
                                        c["norm_topk_prob"])
                pairs = np.zeros(n * c["top_k"], H.PAIR_DTYPE)
                pairs["token"] = np.repeat(np.arange(n, dtype=np.uint32), c["top_k"])
                pairs["expert"] = ids.reshape(-1)
                pairs["weight"] = wts.reshape(-1)
                H.expertMlpSwiglu(ctx, self.h2, gate, up, down, dg, pairs, self.proj, n, hidden,
                                  c["expert_ffn_dim"], c["n_experts"])
            self._trace(li, "experts", self.proj, n * hidden)
            H.add(ctx, H.AddArgs(self.x, self.proj, self.x, n * hidden))
            if self.timing:
                ctx.timing_mark()
            self._trace(li, "block", self.x, n * hidden)

        out_norm = self.w.buf["output_norm.weight"]
        H.rmsNorm(ctx, H.RmsNormArgs(self.x, out_norm, self.h, n, hidden, eps))
        self._trace(-1, "output_norm", self.h, n * hidden)
        H.matmul(ctx, H.MatmulArgs(self.h, self.w.buf["output.weight"], self.w.dtype["output.weight"], self.logits,
                                   n, vocab, hidden))
        self._trace(-1, "logits", self.logits, n * vocab)
        self.pos += n
        if not want_logits:
            return None
        return ctx.to_numpy(self.logits, np.float32, (n, vocab))


def argmax(logits: np.ndarray) -> int:
    """forward.zig:518-525: the first index of the maximum (ties to the lower token id)."""
    return int(np.argmax(logits))
