#!/usr/bin/env python3
"""Benchmark of the gfx950 attention path on the BASELINE configurations.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--only C1,C2,...]

Prints ONE JSON line. The headline workload is config 1:
one decode token through 48 independent layers' attention, Qwen3-30B-A3B shape
(32 q / 4 kv heads, head_dim 128), f16 KV cache of 8192 tokens per layer. A
"step" is that 48-layer sweep: per layer one fused attention step (q/k
RMSNorm, rope, f16 append of k/v at position 8191, causal GQA attention over
8192 positions). The sweep is captured once into a HIP graph and replayed;
W untimed warmup sweeps precede EXACTLY K timed sweeps, bracketed by stream
synchronisation on both sides and timed with HIP events on the context
stream. Inputs are synthetic and already resident in HBM.

Order of a run: every selected workload is built on the device; then the CPU
legs run (the oracle -- a line-by-line single-threaded C restatement of the
reference's CPU path -- on bounded samples of each configuration, timed on
one core); then the GPU legs, each followed by the comparison of its sampled
layers' GPU outputs with the oracle's (the parity figures of the record).

value  = C1 algorithmic HBM bytes of the K sweeps / elapsed (GB/s)
roofline.achieved = algorithmic bytes of one decode_split_kernel launch (one
         layer) / that kernel's mean duration, from start/stop events attached
         to each launch (hipExtLaunchKernelGGL) on the context stream in an
         eager pass of the same sweep; rocprof_* fields repeat the fraction
         with the committed rocprofv3 kernel-trace average of that kernel
cpu_baseline = the oracle on C1 layers, 1 core (per-config CPU figures are in
         configs.C*.cpu)

configs.C0..C4 hold each BASELINE configuration's GPU figures, CPU figures
and parity; floors holds the measured cost of one dependent launch and of a
bare once-read of a C1 layer's K/V; extra holds the projection / MoE legs
(the rows after the attention path).
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2516.6
BF16_MFMA_PEAK_TFLOPS = 2516.6  # dense bf16 matrix-core peak (same as f16)
QKV_BYTES = 5120 * 64 * 34 + 2048 * 4 + 5120 * 4  # Qwen3-30B-A3B q/k/v weights + x + out per layer
ROCPROF_JSON = os.path.join(ROOT, "profiles", "rocprof_kernel_us.json")
OUT_ATOL, OUT_COS = 2e-3, 0.99999  # BASELINE attention-output gates
LOG = sys.stderr


def log(*a):
    print(*a, file=LOG, flush=True)


def decode_bytes(hq, hkv, d, L):
    """Algorithmic HBM bytes of one decode attention step for one sequence:
    f16 K+V once per GQA group, f32 q in and out, f32 new k/v, two f32 norm
    vectors, one i32 position."""
    return 4 * hkv * L * d + 8 * hq * d + 8 * hkv * d + 8 * d + 4


def prefill_flops(hq, d, S):
    """QK^T and PV over the causal triangle (diagonal included)."""
    return 4 * d * hq * S * (S + 1) // 2


# ---------------------------------------------------------------------------
# Workloads (device side)
# ---------------------------------------------------------------------------

class DecodeSweep:
    """n_layers independent layers of single-token decode on a contiguous cache.
    Each layer has its own cache (filled on the device), inputs and output."""

    def __init__(self, H, synth, ctx, config, repeat=1):
        cfg = synth.CONFIGS[config]
        self.H, self.ctx, self.config, self.repeat = H, ctx, config, repeat
        s = self.s = cfg["shape"]
        self.cap, self.pos, self.layers = cfg["cap"], cfg["pos"], cfg["layers"]
        hkv, d = s.n_kv_heads, s.head_dim
        n = hkv * self.cap * d
        self.args, self.host, self.caches, self.outs = [], [], [], []
        self.pos_buf = ctx.from_numpy(np.array([self.pos], np.int32))
        for layer in range(self.layers):
            kc, vc = ctx.createBuffer(2 * n), ctx.createBuffer(2 * n)
            ctx.fill_normal_f16(kc, n, seed=(config << 20) + 2 * layer + 1)
            ctx.fill_normal_f16(vc, n, seed=(config << 20) + 2 * layer + 2)
            q, k, v, qn, kn = synth.step_inputs(config, layer, 1, s)
            out = ctx.createBuffer(s.n_q_heads * d * 4)
            self.host.append((q, k, v, qn, kn))
            self.caches.append((kc, vc))
            self.outs.append(out)
            self.args.append(H.AttentionStepArgs(ctx.from_numpy(q), ctx.from_numpy(k), ctx.from_numpy(v),
                                                 ctx.from_numpy(qn), ctx.from_numpy(kn), self.pos_buf, kc, vc, out,
                                                 H.DTYPE_F16, self.pos, 1, s.n_q_heads, hkv, d, self.cap, s.eps,
                                                 s.theta, 1.0, s.scale))
        self.bytes_per_layer = decode_bytes(s.n_q_heads, hkv, d, self.pos + 1)

    def cache_host(self, layer):
        """The layer's K/V cache as f16 bits [Hkv, cap, d] (rows < pos are never written by a step)."""
        shape = (self.s.n_kv_heads, self.cap, self.s.head_dim)
        kc, vc = self.caches[layer]
        return self.ctx.to_numpy(kc, np.uint16, shape), self.ctx.to_numpy(vc, np.uint16, shape)

    def sweep(self):
        for _ in range(self.repeat):
            for a in self.args:
                self.H.attentionStep(self.ctx, a)


class SixOpSweep:
    """C1's layers through the engine's six separate ops (forward.zig:345-412) on
    their own q/k/out buffers: part "prep" = rmsNorm q, rmsNorm k, rope q, rope k,
    kvAppend (five launches); part "attn" = gqaAttention; "all" = the six."""

    def __init__(self, H, ctx, dec: DecodeSweep, part: str):
        self.H, self.ctx, self.part, self.layers = H, ctx, part, dec.layers
        s, pos, cap = dec.s, dec.pos, dec.cap
        hq, hkv, d = s.n_q_heads, s.n_kv_heads, s.head_dim
        self.calls = []
        for layer in range(dec.layers):
            q, k, v, qn, kn = dec.host[layer]
            qb, kb, vb, qnb, knb = (ctx.from_numpy(a) for a in (q, k, v, qn, kn))
            kc, vc = dec.caches[layer]
            out = ctx.createBuffer(hq * d * 4)
            prep = [(H.rmsNorm, H.RmsNormArgs(qb, qnb, qb, hq, d, s.eps)),
                    (H.rmsNorm, H.RmsNormArgs(kb, knb, kb, hkv, d, s.eps)),
                    (H.rope, H.RopeArgs(qb, dec.pos_buf, 1, hq, d, s.theta)),
                    (H.rope, H.RopeArgs(kb, dec.pos_buf, 1, hkv, d, s.theta)),
                    (H.kvAppend, H.KvAppendArgs(kb, vb, kc, vc, H.DTYPE_F16, pos, 1, hkv, d, cap))]
            attn = [(H.gqaAttention, H.AttnArgs(qb, kc, vc, H.DTYPE_F16, out, pos, 1, hq, hkv, d, cap, s.scale))]
            self.calls += {"prep": prep, "attn": attn, "all": prep + attn}[part]

    def sweep(self):
        for fn, a in self.calls:
            fn(self.ctx, a)


class PagedSweep:
    """C4: n_layers of batched paged decode (32 sequences, 16-token pages)."""

    def __init__(self, H, synth, ctx, config=4):
        cfg = synth.CONFIGS[config]
        self.H, self.ctx = H, ctx
        s = self.s = cfg["shape"]
        self.layers = cfg["layers"]
        lay = self.lay = synth.paged_layout(cfg["n_seqs"], cfg["lo"], cfg["hi"], cfg["page_size"], seed=0)
        hq, hkv, d = s.n_q_heads, s.n_kv_heads, s.head_dim
        B = self.B = cfg["n_seqs"]
        self.slots = lay.n_pages * lay.page_size
        pt, sl = ctx.from_numpy(lay.page_table), ctx.from_numpy(lay.seq_lens)
        self.args, self.host, self.pools, self.outs = [], [], [], []
        for layer in range(self.layers):
            kp, vp = ctx.createBuffer(2 * hkv * self.slots * d), ctx.createBuffer(2 * hkv * self.slots * d)
            ctx.fill_normal_f16(kp, hkv * self.slots * d, seed=(config << 20) + 2 * layer + 1)
            ctx.fill_normal_f16(vp, hkv * self.slots * d, seed=(config << 20) + 2 * layer + 2)
            q, k, v, qn, kn = synth.step_inputs(config, layer, B, s)
            out = ctx.createBuffer(B * hq * d * 4)
            self.host.append((q, k, v, qn, kn))
            self.pools.append((kp, vp))
            self.outs.append(out)
            self.args.append(H.PagedDecodeArgs(ctx.from_numpy(q), ctx.from_numpy(k), ctx.from_numpy(v),
                                               ctx.from_numpy(qn), ctx.from_numpy(kn), kp, vp, pt, sl, out, B, hq,
                                               hkv, d, lay.page_size, lay.n_pages, lay.max_pages,
                                               int(lay.seq_lens.max()), s.eps, s.theta, 1.0, s.scale))
        pages = ((lay.seq_lens.astype(np.int64) + lay.page_size - 1) // lay.page_size).sum()
        self.bytes_per_layer = int(sum(decode_bytes(hq, hkv, d, int(L)) - 8 * d for L in lay.seq_lens)
                                   + 8 * d + 4 * pages)

    def pool_host(self, layer):
        shape = (self.s.n_kv_heads, self.slots, self.s.head_dim)
        kp, vp = self.pools[layer]
        return self.ctx.to_numpy(kp, np.uint16, shape), self.ctx.to_numpy(vp, np.uint16, shape)

    def sweep(self):
        for a in self.args:
            self.H.pagedDecode(self.ctx, a)


class Prefill:
    """C2: causal prefill of 2048 tokens into an empty f16 cache, one layer
    (fused: the attention step; separate: the six ops)."""

    def __init__(self, H, synth, ctx, config=2, fused=True):
        cfg = synth.CONFIGS[config]
        self.H, self.ctx, self.fused = H, ctx, fused
        s = self.s = cfg["shape"]
        T = self.T = cfg["tokens"]
        hq, hkv, d = s.n_q_heads, s.n_kv_heads, s.head_dim
        self.host = synth.step_inputs(config, 0, T, s, f16_exact=True)
        q, k, v, qn, kn = self.host
        self.kc, self.vc = ctx.createBuffer(2 * hkv * T * d), ctx.createBuffer(2 * hkv * T * d)
        self.out = ctx.createBuffer(T * hq * d * 4)
        qb, kb, vb, qnb, knb = (ctx.from_numpy(a) for a in (q, k, v, qn, kn))
        pb = ctx.from_numpy(np.arange(T, dtype=np.int32))
        self.args = H.AttentionStepArgs(qb, kb, vb, qnb, knb, pb, self.kc, self.vc, self.out, H.DTYPE_F16, 0, T, hq,
                                        hkv, d, T, s.eps, s.theta, 1.0, s.scale)
        self.calls = [(H.rmsNorm, H.RmsNormArgs(qb, qnb, qb, T * hq, d, s.eps)),
                      (H.rmsNorm, H.RmsNormArgs(kb, knb, kb, T * hkv, d, s.eps)),
                      (H.rope, H.RopeArgs(qb, pb, T, hq, d, s.theta)),
                      (H.rope, H.RopeArgs(kb, pb, T, hkv, d, s.theta)),
                      (H.kvAppend, H.KvAppendArgs(kb, vb, self.kc, self.vc, H.DTYPE_F16, 0, T, hkv, d, T)),
                      (H.gqaAttention, H.AttnArgs(qb, self.kc, self.vc, H.DTYPE_F16, self.out, 0, T, hq, hkv, d, T,
                                                  s.scale))]
        self.flops = prefill_flops(hq, d, T)

    def sweep(self):
        if self.fused:
            self.H.attentionStep(self.ctx, self.args)
        else:
            for fn, a in self.calls:
                fn(self.ctx, a)


class FloorSweep:
    """The floors of one decode layer: 48 launches of an empty kernel (one
    dependent launch each), 48 bare once-reads of a distinct 16 MiB buffer (a
    C1 layer's K and V), or both per layer (the launch count of split + merge)."""

    def __init__(self, H, ctx, layers=48, nbytes=16 << 20, mode="read"):
        self.ctx, self.layers, self.mode, self.nbytes = ctx, layers, mode, nbytes
        self.bufs = []
        if mode != "empty":
            for layer in range(layers):
                b = ctx.createBuffer(nbytes)
                ctx.fill_normal_f16(b, nbytes // 2, seed=(9 << 20) + layer)
                self.bufs.append(b)
        self.sink = ctx.createBuffer(16)

    def sweep(self):
        for layer in range(self.layers):
            if self.mode != "empty":
                self.ctx.stream_read(self.bufs[layer], self.nbytes, self.sink)
            if self.mode != "read":
                self.ctx.empty_launch(256)


class ProjSweep:
    """The q/k/v projections of a decode step (the matmuls before the attention path,
    forward.zig:337-339): n_layers of x [1, hidden] . W^T for the three Q8_0 weights
    wq [n_q_heads*d, hidden], wk and wv [n_kv_heads*d, hidden], as one grouped call
    (grouped=True) or as the engine's three matmul calls; distinct random weights per
    layer (the 256 MB MALL cannot hold the sweep)."""

    def __init__(self, H, ctx, layers=48, hidden=2048, hq=32, hkv=4, d=128, seed=7, grouped=True):
        self.H, self.ctx, self.layers, self.grouped = H, ctx, layers, grouped
        self.ns, self.k = (hq * d, hkv * d, hkv * d), hidden
        self.n = sum(self.ns)
        nb = self.k // 32
        g = np.random.default_rng(seed)
        self.args = []
        for _ in range(layers):
            x = ctx.from_numpy(g.standard_normal((1, self.k)).astype(np.float32))
            entries = []
            for n in self.ns:
                w = g.integers(0, 256, (n, nb, 34), dtype=np.uint8)
                w[:, :, 0:2] = np.array([0.02], np.float16).view(np.uint8)
                entries.append((ctx.from_numpy(w.reshape(n, nb * 34)), ctx.createBuffer(n * 4), n))
            if grouped:
                self.args.append(H.MatmulGroupArgs.of(x, H.DTYPE_Q8_0, 1, self.k, entries))
            else:
                self.args.append([H.MatmulArgs(x, w, H.DTYPE_Q8_0, o, 1, n, self.k) for w, o, n in entries])
        self.bytes_per_layer = self.n * nb * 34 + self.k * 4 + self.n * 4

    def sweep(self):
        for a in self.args:
            if self.grouped:
                self.H.matmulGroup(self.ctx, a)
            else:
                for one in a:
                    self.H.matmul(self.ctx, one)


class WoSweep:
    """The output projection and residual of a decode step (forward.zig:416-418):
    n_layers of x[1, hidden] += attn[1, n_q_heads*d] . Wo^T, Wo Q8_0 [hidden, n_q_heads*d],
    as one matmul_add call (fused=True) or as the engine's matmul then add."""

    def __init__(self, H, ctx, layers=48, hidden=2048, hq=32, d=128, seed=5, fused=True):
        self.H, self.ctx, self.layers, self.fused = H, ctx, layers, fused
        self.n, self.k = hidden, hq * d
        nb = self.k // 32
        g = np.random.default_rng(seed)
        self.x = ctx.from_numpy(g.standard_normal((1, hidden)).astype(np.float32))  # the residual stream
        self.args = []
        for _ in range(layers):
            attn = ctx.from_numpy(g.standard_normal((1, self.k)).astype(np.float32))
            w = g.integers(0, 256, (self.n, nb, 34), dtype=np.uint8)
            w[:, :, 0:2] = np.array([0.002], np.float16).view(np.uint8)
            wb = ctx.from_numpy(w.reshape(self.n, nb * 34))
            if fused:
                self.args.append(H.MatmulAddArgs(attn, wb, H.DTYPE_Q8_0, self.x, self.x, 1, self.n, self.k))
            else:
                proj = ctx.createBuffer(self.n * 4)
                self.args.append((H.MatmulArgs(attn, wb, H.DTYPE_Q8_0, proj, 1, self.n, self.k),
                                  H.AddArgs(self.x, proj, self.x, self.n)))
        self.bytes_per_layer = self.n * nb * 34 + self.k * 4 + 2 * self.n * 4

    def sweep(self):
        for a in self.args:
            if self.fused:
                self.H.matmulAdd(self.ctx, a)
            else:
                self.H.matmul(self.ctx, a[0])
                self.H.add(self.ctx, a[1])


class MoeSweep:
    """The MoE block of a decode step (forward.zig after the attention block): n_layers of
    router top-8 of 128 experts (f32 router weights [128 x 2048]) and the SwiGLU experts
    (Q8_0 banks: gate/up [128, 768, 2048], down [128, 2048, 768]) for one token, on the
    device (ds5_hip_moe: no host round trip). Every layer has its own banks (642 MB) and
    its own x, so its 8 experts differ; the 16 layers' 640 MB of touched experts exceed the
    256 MB MALL. Bank bytes are random with small scales (one random template per shape)."""

    def __init__(self, H, ctx, layers=16, dim=2048, ffn=768, E=128, K=8, seed=13):
        self.H, self.ctx, self.layers = H, ctx, layers
        g = np.random.default_rng(seed)

        def template(rows, k):
            w = g.integers(0, 256, (rows, k // 32, 34), dtype=np.uint8)
            w[:, :, 0:2] = np.array([0.002], np.float16).view(np.uint8)
            return w.reshape(rows, k // 32 * 34)
        gu, dn = template(E * ffn, dim), template(E * dim, ffn)
        empty = H.Buf(None, 0, 0)
        self.args = []
        for _ in range(layers):
            x = ctx.from_numpy(g.standard_normal((1, dim)).astype(np.float32))
            rw = ctx.from_numpy((g.standard_normal((E, dim)) * 0.03).astype(np.float32))
            self.args.append(H.MoeArgs(x, rw, H.DTYPE_F32, ctx.from_numpy(gu), ctx.from_numpy(gu), ctx.from_numpy(dn),
                                       H.DTYPE_Q8_0, ctx.createBuffer(dim * 4), empty, empty, 1, dim, ffn, E, K, 1))
        # bytes one token moves: router weights, its 8 experts' three matrices, x, out (read and written)
        self.bytes_per_layer = E * dim * 4 + K * 3 * ffn * (dim // 32) * 34 + 3 * dim * 4

    def sweep(self):
        for a in self.args:
            self.H.moe(self.ctx, a)


class MoePrefill:
    """The MoE block over T prompt tokens (Qwen3-30B-A3B shape: dim 2048, 128 experts top 8,
    ffn 768, Q8_0 banks, f32 router): ds5_hip_moe with the logits in tiles and the
    experts grouped by expert on the matrix cores. Synthetic x, router and banks (one
    random template per shape, small scales)."""

    def __init__(self, H, ctx, T=2048, dim=2048, ffn=768, E=128, K=8, seed=17):
        self.H, self.ctx, self.T = H, ctx, T
        g = np.random.default_rng(seed)

        def template(rows, k):
            w = g.integers(0, 256, (rows, k // 32, 34), dtype=np.uint8)
            w[:, :, 0:2] = np.array([0.002], np.float16).view(np.uint8)
            return w.reshape(rows, k // 32 * 34)
        gu, dn = template(E * ffn, dim), template(E * dim, ffn)
        x = ctx.from_numpy(g.standard_normal((T, dim)).astype(np.float32))
        rw = ctx.from_numpy((g.standard_normal((E, dim)) * 0.03).astype(np.float32))
        empty = H.Buf(None, 0, 0)
        self.args = H.MoeArgs(x, rw, H.DTYPE_F32, ctx.from_numpy(gu), ctx.from_numpy(gu), ctx.from_numpy(dn),
                              H.DTYPE_Q8_0, ctx.createBuffer(T * dim * 4), empty, empty, T, dim, ffn, E, K, 1)
        # the experts' useful products: gate and up (2 x ffn x dim) and down (dim x ffn) per pair
        self.expert_flops = 2 * T * K * 3 * dim * ffn
        self.router_flops = 2 * T * E * dim

    def sweep(self):
        self.H.moe(self.ctx, self.args)


class DecodeLayerSweep:
    """One decode token through n_layers whole layers at the Qwen3-30B-A3B shape, in the
    engine's fused order (forward.zig:322-494; qw3_amd/engine.py fused mode): the
    attention block (attn_norm, q/k/v projections + the fused step over an 8K f16 cache), Wo
    and the residual, the MoE block on the device with ffn_norm and the residual. Distinct
    weights, caches and expert banks per layer (synthetic; the banks are device copies
    of one random template, 642 MB per layer, 30.8 GB for 48 layers), the residual
    stream x shared and reset from x0 at the start of each sweep (an 8 KB copy)."""

    def __init__(self, H, ctx, layers=48, hidden=2048, hq=32, hkv=4, d=128, ctx_len=8192, E=128, K=8, ffn=768,
                 seed=21):
        self.H, self.ctx, self.layers = H, ctx, layers
        g = np.random.default_rng(seed)
        nb = hidden // 32
        eps, theta = 1e-6, 1e6

        def q8(rows, k, scale):
            w = g.integers(0, 256, (rows, k // 32, 34), dtype=np.uint8)
            w[:, :, 0:2] = np.array([scale], np.float16).view(np.uint8)
            return w.reshape(rows, k // 32 * 34)

        def norm_w(n):
            return ctx.from_numpy((1 + 0.02 * g.standard_normal(n)).astype(np.float32))

        f4 = 4
        mk = ctx.createBuffer
        self.x0 = ctx.from_numpy(g.standard_normal((1, hidden)).astype(np.float32))
        self.x = mk(hidden * f4)
        q, k, v = mk(hq * d * f4), mk(hkv * d * f4), mk(hkv * d * f4)
        attn = mk(hq * d * f4)
        pos = ctx_len - 1
        positions = ctx.from_numpy(np.array([pos], np.int32))
        gu_t, dn_t = ctx.from_numpy(q8(E * ffn, hidden, 0.002)), ctx.from_numpy(q8(E * hidden, ffn, 0.002))
        gu_bytes, dn_bytes = E * ffn * nb * 34, E * hidden * (ffn // 32) * 34
        empty = H.Buf(None, 0, 0)
        scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
        self.layer_args = []
        cache_elems = hkv * ctx_len * d
        for li in range(layers):
            wq, wk, wv = (ctx.from_numpy(q8(n, hidden, 0.002)) for n in (hq * d, hkv * d, hkv * d))
            wo = ctx.from_numpy(q8(hidden, hq * d, 0.002))
            kc, vc = mk(2 * cache_elems), mk(2 * cache_elems)
            ctx.fill_normal_f16(kc, cache_elems, 1000 + 2 * li)
            ctx.fill_normal_f16(vc, cache_elems, 1001 + 2 * li)
            gate, up, down = mk(gu_bytes), mk(gu_bytes), mk(dn_bytes)
            ctx.copy_device(gate, gu_t, gu_bytes)
            ctx.copy_device(up, gu_t, gu_bytes)
            ctx.copy_device(down, dn_t, dn_bytes)
            router = ctx.from_numpy((0.03 * g.standard_normal((E, hidden))).astype(np.float32))
            an, fn, qn, kn = norm_w(hidden), norm_w(hidden), norm_w(d), norm_w(d)
            step = H.AttentionStepArgs(q, k, v, qn, kn, positions, kc, vc, attn, H.DTYPE_F16, pos, 1, hq, hkv, d,
                                       ctx_len, eps, theta, 1.0, scale)
            self.layer_args.append((
                None,
                H.AttentionBlockArgs(self.x, wq, wk, wv, H.DTYPE_Q8_0, hidden, step, an, eps),
                H.MatmulAddArgs(attn, wo, H.DTYPE_Q8_0, self.x, self.x, 1, hidden, hq * d),
                None,
                H.MoeArgs(self.x, router, H.DTYPE_F32, gate, up, down, H.DTYPE_Q8_0, self.x, empty, empty, 1,
                          hidden, ffn, E, K, 1, self.x, fn, eps)))
        del gu_t, dn_t
        self.hidden = hidden
        self.marks = False

    def layer(self, a):
        H, ctx = self.H, self.ctx
        H.attentionBlock(ctx, a[1])  # attn_norm inside
        H.matmulAdd(ctx, a[2])
        H.moe(ctx, a[4])  # ffn_norm inside, x + the experts' sum (the engine's fused order)

    def sweep(self):
        self.ctx.copy_device(self.x, self.x0, self.hidden * 4)
        if self.marks:
            self.ctx.timing_mark()
        for a in self.layer_args:
            self.layer(a)
            if self.marks:
                self.ctx.timing_mark()


class ProjPrefill:
    """The q/k/v projections of a 2048-token prefill (forward.zig:337-339 at m = T):
    x [T, hidden] f32 . W^T for wq [n_q_heads*d, hidden], wk and wv [n_kv_heads*d,
    hidden], Q8_0, in one grouped call."""

    def __init__(self, H, ctx, T=2048, hidden=2048, hq=32, hkv=4, d=128, seed=11):
        self.H, self.ctx = H, ctx
        self.m, self.k = T, hidden
        ns = (hq * d, hkv * d, hkv * d)
        self.n = sum(ns)
        nb = self.k // 32
        g = np.random.default_rng(seed)
        x = ctx.from_numpy(g.standard_normal((T, self.k)).astype(np.float32))
        entries = []
        for n in ns:
            w = g.integers(0, 256, (n, nb, 34), dtype=np.uint8)
            w[:, :, 0:2] = np.array([0.02], np.float16).view(np.uint8)
            entries.append((ctx.from_numpy(w.reshape(n, nb * 34)), ctx.createBuffer(T * n * 4), n))
        self.args = H.MatmulGroupArgs.of(x, H.DTYPE_Q8_0, T, self.k, entries)
        self.flops = 2 * self.m * self.n * self.k

    def sweep(self):
        self.H.matmulGroup(self.ctx, self.args)


class BlockPrefill:
    """The attention block of a 2048-token prefill (forward.zig:337-412): x [T, hidden]
    f32 through the Q8_0 q/k/v projections, then the attention step into an empty f16
    cache. fused: ds5_hip_attention_block (the pre-pass in the projection GEMM's
    epilogue); otherwise ds5_hip_matmul_group then ds5_hip_attention_step."""

    def __init__(self, H, synth, ctx, fused=True, hidden=2048, seed=12):
        self.H, self.ctx, self.fused = H, ctx, fused
        s = self.s = synth.CONFIGS[2]["shape"]
        T = self.T = synth.CONFIGS[2]["tokens"]
        hq, hkv, d = s.n_q_heads, s.n_kv_heads, s.head_dim
        g = np.random.default_rng(seed)
        nb = hidden // 32
        x = ctx.from_numpy(g.standard_normal((T, hidden)).astype(np.float32))
        ws = []
        for n in (hq * d, hkv * d, hkv * d):
            w = g.integers(0, 256, (n, nb, 34), dtype=np.uint8)
            w[:, :, 0:2] = np.array([0.02], np.float16).view(np.uint8)
            ws.append(ctx.from_numpy(w.reshape(n, nb * 34)))
        _, _, _, qn, kn = synth.step_inputs(2, 0, 1, s)
        q, k, v = (ctx.createBuffer(T * h * d * 4) for h in (hq, hkv, hkv))
        self.kc, self.vc = ctx.createBuffer(2 * hkv * T * d), ctx.createBuffer(2 * hkv * T * d)
        self.out = ctx.createBuffer(T * hq * d * 4)
        pb = ctx.from_numpy(np.arange(T, dtype=np.int32))
        self.step = H.AttentionStepArgs(q, k, v, ctx.from_numpy(qn), ctx.from_numpy(kn), pb, self.kc, self.vc,
                                        self.out, H.DTYPE_F16, 0, T, hq, hkv, d, T, s.eps, s.theta, 1.0, s.scale)
        self.block = H.AttentionBlockArgs(x, *ws, H.DTYPE_Q8_0, hidden, self.step)
        self.group = H.MatmulGroupArgs.of(x, H.DTYPE_Q8_0, T, hidden, [(ws[0], q, hq * d), (ws[1], k, hkv * d),
                                                                        (ws[2], v, hkv * d)])
        self.proj_flops = 2 * T * (hq + 2 * hkv) * d * hidden
        self.attn_flops = prefill_flops(hq, d, T)

    def sweep(self):
        if self.fused:
            self.H.attentionBlock(self.ctx, self.block)
        else:
            self.H.matmulGroup(self.ctx, self.group)
            self.H.attentionStep(self.ctx, self.step)


# ---------------------------------------------------------------------------
# Timing helpers
# ---------------------------------------------------------------------------

USE_GRAPHS = True  # --no-graph: sweeps run eagerly (profiling runs; the profiler's graph interception is unstable)


# Single-layer legs (C2, QKVP, BLK) capture this many back-to-back sweeps per graph: a graph
# launch costs ~5-35 us of device idle per replay here (measured: BLK 228 us per sweep with
# one sweep per graph, 195 with eight, 194 eager), which a multi-layer graph amortises and an
# op inside a real forward graph never pays on its own.
SWEEPS_PER_GRAPH = 8


class Repeat:
    """n back-to-back sweeps of `work` as one sweep (one captured graph holds all n)."""

    def __init__(self, work, n):
        self.work, self.n = work, n

    def sweep(self):
        for _ in range(self.n):
            self.work.sweep()


def time_graph(ctx, work, steps, warmup):
    """Capture work.sweep() once, replay warmup + steps times; returns (device seconds
    of the timed replays from events on the context stream, wall seconds). Without
    graphs (--no-graph) the sweeps are enqueued eagerly instead."""
    work.sweep()                      # eager once: sizes the split-K workspace
    ctx.submit()
    if not USE_GRAPHS:
        for _ in range(warmup):
            work.sweep()
        ctx.submit()
        ctx.begin()
        t0 = time.perf_counter()
        for _ in range(steps):
            work.sweep()
        ctx.submit()
        wall = time.perf_counter() - t0
        return ctx.gpuElapsedNs() * 1e-9, wall
    g = ctx.capture(work.sweep)
    try:
        for _ in range(warmup):
            g.launch()
        ctx.submit()                  # drain (barrier before the timed region)
        ctx.begin()
        t0 = time.perf_counter()
        for _ in range(steps):
            g.launch()
        ctx.submit()                  # records the end event and waits (barrier after)
        wall = time.perf_counter() - t0
        return ctx.gpuElapsedNs() * 1e-9, wall
    finally:
        g.destroy()


def replays_for(seconds_per_step, min_seconds, floor):
    return max(floor, int(min_seconds / max(seconds_per_step, 1e-9)) + 1)


def kernel_stats(ctx, work, kernels, min_seconds=0.3, max_reps=2000):
    """Mean device duration (ns) and launch count of each named kernel over eager
    sweeps (at least min_seconds of them), each launch timed by start/stop events
    attached to its own dispatch."""
    ctx.set_kernel_timing(True)
    try:
        t0, reps = time.perf_counter(), 0
        while reps < max_reps and (reps < 2 or time.perf_counter() - t0 < min_seconds):
            work.sweep()
            reps += 1
            if reps % 4 == 0:
                ctx.kernel_time(kernels[0])  # resolves the pending event pairs (bounded event pool)
        ctx.submit()
        out = {}
        for k in kernels:
            n, total = ctx.kernel_time(k)
            out[k] = (total / n if n else None, n)
    finally:
        ctx.set_kernel_timing(False)
    return out


def rocprof_kernel_us(workload, kernel):
    """The rocprofv3 kernel-trace average (us) of `kernel` in the committed summary
    for `workload` (profiles/rocprof_kernel_us.json), or None."""
    if not os.path.exists(ROCPROF_JSON):
        return None
    with open(ROCPROF_JSON) as f:
        return json.load(f).get(workload, {}).get(kernel, {}).get("avg_us")


def measured_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (profiles/<kernel>_<workload>_traffic.json: FETCH_SIZE and WRITE_SIZE per
    dispatch, scaled by the same counters' reading of a copy of known size),
    or None when no summary is committed."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def ingest_rocprof(stats_csv, workload):
    """Record the per-kernel averages of a rocprofv3 --stats kernel_stats.csv under
    `workload` in profiles/rocprof_kernel_us.json."""
    data = json.load(open(ROCPROF_JSON)) if os.path.exists(ROCPROF_JSON) else {}
    entry = {}
    import subprocess
    with open(stats_csv) as f:
        for row in csv.DictReader(f):
            name = row["Name"]
            if name.startswith("_ZN12_GLOBAL__N_1"):  # (anonymous namespace)::<len><name>...
                rest = name[len("_ZN12_GLOBAL__N_1"):]
                digits = len(rest) - len(rest.lstrip("0123456789"))
                name = rest[digits:digits + int(rest[:digits])]
            elif name.startswith("_Z"):
                name = subprocess.run(["c++filt", name], capture_output=True, text=True).stdout.strip() or name
            name = name.replace("(anonymous namespace)::", "")
            if name.startswith("void "):
                name = name[5:]
            name = name.split("(")[0].split("<")[0].strip().split("::")[-1]
            calls = int(row["Calls"])
            avg = float(row["AverageNs"]) / 1e3
            prev = entry.get(name)
            if prev is None or calls > prev["calls"]:
                entry[name] = dict(avg_us=round(avg, 3), calls=calls, min_us=round(float(row["MinNs"]) / 1e3, 3),
                                   max_us=round(float(row["MaxNs"]) / 1e3, 3))
    data[workload] = entry
    with open(ROCPROF_JSON, "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)
        f.write("\n")
    print(json.dumps({workload: entry}))


# ---------------------------------------------------------------------------
# Parity and the CPU legs (the oracle: tests infrastructure, used here only as
# the checker and the CPU baseline)
# ---------------------------------------------------------------------------

def parity(got, want, got_rows=None, want_rows=None):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    err = float(np.max(np.abs(got - want)))
    cos = float(got @ want / (np.linalg.norm(got) * np.linalg.norm(want)))
    r = dict(max_abs=float(f"{err:.3e}"), cosine=round(cos, 9), ok=bool(err <= OUT_ATOL and cos >= OUT_COS
                                                                         and np.all(np.isfinite(got))))
    if got_rows is not None:
        def mono(x):
            x = np.asarray(x, np.uint16).astype(np.int32)
            return np.where(x & 0x8000, 0x8000 - (x & 0x7FFF), 0x8000 + x)
        ulp = int(np.max(np.abs(mono(got_rows) - mono(want_rows))))
        r["kv_ulp_max"] = ulp
        r["ok"] = r["ok"] and ulp <= 1
    return r


def oracle_decode(O, s, host, kc, vc, pos, cap):
    q, k, v, qn, kn = host
    kc, vc = kc.copy(), vc.copy()
    out, _, _ = O.attention_step(q, k, v, qn, kn, np.array([pos], np.int32), kc, vc, kv_dtype=1, pos=pos,
                                 n_tokens=1, n_q_heads=s.n_q_heads, n_kv_heads=s.n_kv_heads, head_dim=s.head_dim,
                                 max_ctx=cap, eps=s.eps, theta=s.theta, scale=s.scale)
    return out, kc[:, pos], vc[:, pos]


def cpu_decode_leg(O, w, layers, seconds):
    """The oracle on `layers` of a DecodeSweep, cycling until `seconds` have passed
    (at least one pass); returns (us per layer, layer-steps, seconds, {layer: reference})."""
    samples = {layer: w.cache_host(layer) for layer in layers}
    refs, n, t = {}, 0, 0.0
    while n < len(layers) or t < seconds:
        layer = layers[n % len(layers)]
        kc, vc = samples[layer]
        t0 = time.perf_counter()
        r = oracle_decode(O, w.s, w.host[layer], kc, vc, w.pos, w.cap)
        t += time.perf_counter() - t0
        refs[layer] = r
        n += 1
    return t / n * 1e6, n, t, refs


def cpu_paged_leg(O, w, layer=0):
    """The oracle on every sequence of one C4 layer: gather the sequence's pages
    into a contiguous cache, then the decode step (the reduction the parity tests
    use). Returns (us for the layer, seconds, references)."""
    s, lay = w.s, w.lay
    kp, vp = w.pool_host(layer)
    q, k, v, qn, kn = w.host[layer]
    refs, t = [], 0.0
    for b in range(w.B):
        L = int(lay.seq_lens[b])
        kc = O.paged_gather_f16(kp, lay.page_table[b], lay.page_size, L)
        vc = O.paged_gather_f16(vp, lay.page_table[b], lay.page_size, L)
        t0 = time.perf_counter()
        r = oracle_decode(O, s, (q[b:b + 1], k[b:b + 1], v[b:b + 1], qn, kn), kc, vc, L - 1, L)
        t += time.perf_counter() - t0
        refs.append(r)
    return t * 1e6, t, refs


def cpu_prefill_leg(O, p, group=0):
    """The oracle on one GQA group of C2 (q heads of kv head `group`, all 2048
    tokens); the layer's CPU time is that times the number of kv heads."""
    s, T = p.s, p.T
    hg = s.n_q_heads // s.n_kv_heads
    q, k, v, qn, kn = p.host
    qg = np.ascontiguousarray(q[:, group * hg:(group + 1) * hg])
    kg = np.ascontiguousarray(k[:, group:group + 1])
    vg = np.ascontiguousarray(v[:, group:group + 1])
    kc = np.zeros((1, T, s.head_dim), np.uint16)
    vc = np.zeros((1, T, s.head_dim), np.uint16)
    t0 = time.perf_counter()
    out, _, _ = O.attention_step(qg, kg, vg, qn, kn, np.arange(T, dtype=np.int32), kc, vc, kv_dtype=1, pos=0,
                                 n_tokens=T, n_q_heads=hg, n_kv_heads=1, head_dim=s.head_dim, max_ctx=T, eps=s.eps,
                                 theta=s.theta, scale=s.scale)
    t = time.perf_counter() - t0
    return t * 1e6 * s.n_kv_heads, t, (out.reshape(T, hg, s.head_dim), kc[0], vc[0])


# ---------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50, help="timed 48-layer sweeps (C1)")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU legs (and the parity figures)")
    ap.add_argument("--cpu-seconds", type=float, default=3.0, help="CPU time per cycled decode leg (C0, C1)")
    ap.add_argument("--leg-seconds", type=float, default=0.5,
                    help="minimum device time of each secondary timed leg (graph replays / eager kernel timing)")
    ap.add_argument("--only", default="C0,C1,C2,C3,C4,FLOOR,SIX,QKV,WO,MOE,LAYER,QKVP,BLK,MOEP",
                    help="comma list of legs: C0-C4 (BASELINE configs; C1 is the headline), FLOOR (launch and "
                         "bare-read floors), SIX (C1 through the six separate ops), QKV / QKVP (decode / prefill "
                         "q/k/v projections), WO (output projection + residual), MOE (decode MoE block), LAYER (48 whole "
                         "decode layers in the engine's fused order), BLK (prefill attention block: projections + "
                         "step, fused vs the two calls), MOEP (MoE block over 2048 prompt tokens)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="also run one device-to-device copy of MIB MiB (the known-size reference dispatch for "
                         "the FETCH_SIZE / WRITE_SIZE traffic counters)")
    ap.add_argument("--no-graph", action="store_true",
                    help="enqueue the timed sweeps eagerly instead of replaying captured graphs (for profiler runs)")
    ap.add_argument("--ingest-rocprof", nargs=2, metavar=("KERNEL_STATS_CSV", "WORKLOAD"),
                    help="record a rocprofv3 --stats kernel_stats.csv under WORKLOAD in "
                         "profiles/rocprof_kernel_us.json and exit (no GPU)")
    args = ap.parse_args()
    if args.ingest_rocprof:
        ingest_rocprof(*args.ingest_rocprof)
        return
    global USE_GRAPHS
    USE_GRAPHS = not args.no_graph
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(layers/heads/sequences would shard across GPUs; no multi-GPU path is built)", file=sys.stderr)
        sys.exit(2)

    import qw3_amd.hip as H
    from qw3_amd import synth

    only = set(args.only.upper().split(","))
    ctx = H.Ctx.init(0)
    if args.calibrate_copy:
        nb = args.calibrate_copy << 20
        src, dst = ctx.createBuffer(nb), ctx.createBuffer(nb)
        ctx.fill_normal_f16(src, nb // 2, seed=7)
        ctx.copy_device(dst, src, nb)
        ctx.submit()
        log(f"[bench] calibration copy of {args.calibrate_copy} MiB done")

    # ---- 1. build the device workloads
    W = {}
    for c in (0, 1, 3):
        if f"C{c}" in only or (c == 1 and "SIX" in only):
            log(f"[bench] C{c}: building {synth.CONFIGS[c]['layers']} layers")
            # C0 is one layer: a step is replayed 100 times per graph so that the
            # figure is the device's per-step time, not one graph launch's host cost
            W[c] = DecodeSweep(H, synth, ctx, c, repeat=100 if c == 0 else 1)
    if "C4" in only:
        log("[bench] C4: building 48 layers of paged pools (32 sequences)")
        W[4] = PagedSweep(H, synth, ctx)
    if "C2" in only:
        log("[bench] C2: prefill 2048 tokens")
        W[2] = Prefill(H, synth, ctx)
    ctx.submit()

    # ---- 2. CPU legs (before the GPU legs): the oracle, one core, on bounded samples
    cpu, refs = {}, {}
    O = None
    if not args.no_cpu:
        from oracle import oracle as O
        O.lib()
        for c, layers in ((0, [0]), (1, [0, 1, 2]), (3, [0])):
            if c in W and f"C{c}" in only:
                secs = args.cpu_seconds if c != 3 else 0.0
                us, n, t, refs[c] = cpu_decode_leg(O, W[c], layers, secs)
                cpu[c] = dict(us_per_layer=round(us, 1), cores=1, kind="port",
                              sample=f"{n} decode layer-steps over layers {layers} through oracle/ds5_oracle.c "
                                     f"ds5o_attention_step, {t:.1f} s")
                log(f"[bench] CPU C{c}: {us:.1f} us/layer ({n} layer-steps, {t:.1f} s)")
        if 4 in W:
            us, t, refs[4] = cpu_paged_leg(O, W[4])
            cpu[4] = dict(us_per_layer=round(us, 1), cores=1, kind="port",
                          sample=f"layer 0, all {W[4].B} sequences (pages gathered, then ds5o_attention_step), "
                                 f"{t:.1f} s")
            log(f"[bench] CPU C4: {us:.1f} us/layer ({t:.1f} s)")
        if 2 in W:
            us, t, refs[2] = cpu_prefill_leg(O, W[2])
            cpu[2] = dict(us_per_layer=round(us, 1), cores=1, kind="port",
                          sample=f"one GQA group of 4 (kv head 0, 8 q heads, all 2048 tokens) through "
                                 f"ds5o_attention_step in {t:.1f} s, times 4 for the layer")
            log(f"[bench] CPU C2: {us / 1e6:.2f} s/layer (one group {t:.1f} s)")

    # ---- 3. GPU legs; each config's parity (its GPU outputs vs the oracle's) is read
    #         right after its leg, before a later leg can touch its caches
    configs, extra, result = {}, {}, None
    leg = args.leg_seconds

    def parity_decode(c):
        if c not in refs:
            return
        w, pr = W[c], []
        for layer, (wout, wk, wv) in refs[c].items():
            got = ctx.to_numpy(w.outs[layer], np.float32)
            gk, gv = w.cache_host(layer)
            pr.append(parity(got, wout, np.stack([gk[:, w.pos], gv[:, w.pos]]), np.stack([wk, wv])))
        configs[f"C{c}"]["parity"] = dict(layers=sorted(refs[c]), max_abs=max(x["max_abs"] for x in pr),
                                          cosine_min=min(x["cosine"] for x in pr),
                                          kv_ulp_max=max(x["kv_ulp_max"] for x in pr), ok=all(x["ok"] for x in pr))

    def parity_c4():
        if 4 not in refs:
            return
        w = W[4]
        got = ctx.to_numpy(w.outs[0], np.float32).reshape(w.B, -1)
        kp, vp = w.pool_host(0)
        pr = []
        for b, (wout, wk, wv) in enumerate(refs[4]):
            slot = w.lay.slot(b, int(w.lay.seq_lens[b]) - 1)
            pr.append(parity(got[b], wout, np.stack([kp[:, slot], vp[:, slot]]), np.stack([wk, wv])))
        configs["C4"]["parity"] = dict(sequences=w.B, max_abs=max(x["max_abs"] for x in pr),
                                       cosine_min=min(x["cosine"] for x in pr),
                                       kv_ulp_max=max(x["kv_ulp_max"] for x in pr), ok=all(x["ok"] for x in pr))

    def parity_c2():
        if 2 not in refs:
            return
        p = W[2]
        s, T = p.s, p.T
        hg = s.n_q_heads // s.n_kv_heads
        wout, wk, wv = refs[2]
        got = ctx.to_numpy(p.out, np.float32).reshape(T, s.n_q_heads, s.head_dim)[:, :hg]
        shape = (s.n_kv_heads, T, s.head_dim)
        gk, gv = ctx.to_numpy(p.kc, np.uint16, shape)[0], ctx.to_numpy(p.vc, np.uint16, shape)[0]
        configs["C2"]["parity"] = dict(parity(got, wout, np.stack([gk, gv]), np.stack([wk, wv])),
                                       sample="kv head 0: its 8 q heads x 2048 tokens and its 2048 cache rows")

    def decode_leg(c, steps, warmup):
        w = W[c]
        elapsed, wall = time_graph(ctx, w, steps, warmup)
        us = elapsed / (w.layers * getattr(w, "repeat", 1) * steps) * 1e6
        ks = kernel_stats(ctx, w, ("decode_split_kernel", "decode_merge_kernel"), leg)
        split_ns, n_split = ks["decode_split_kernel"]
        merge_ns, _ = ks["decode_merge_kernel"]
        r = dict(us_per_layer=round(us, 3), gbs=round(w.bytes_per_layer / (us * 1e3), 1),
                 frac=round(w.bytes_per_layer / (us * 1e3) / HBM_PEAK_GBS, 4), bytes_per_layer=w.bytes_per_layer,
                 steps=steps, layers=w.layers, kernel_us=dict(decode_split_kernel=round(split_ns / 1e3, 3),
                                                               decode_merge_kernel=None if merge_ns is None
                                                               else round(merge_ns / 1e3, 3)),
                 kernel_frac=round(w.bytes_per_layer / split_ns / HBM_PEAK_GBS, 4), kernel_launches=n_split)
        ru = rocprof_kernel_us(f"C{c}", "decode_split_kernel")
        if ru:
            r["rocprof_kernel_us"] = ru
            r["rocprof_kernel_frac"] = round(w.bytes_per_layer / (ru * 1e3) / HBM_PEAK_GBS, 4)
        return r, elapsed, wall, split_ns

    if 1 in W and "C1" in only:
        w = W[1]
        r, elapsed, wall, split_ns = decode_leg(1, args.steps, args.warmup)
        layers = w.layers * args.steps
        log(f"[bench] C1 graph sweep: {r['us_per_layer']:.3f} us/layer, {r['gbs']:.1f} GB/s "
            f"(wall {wall / layers * 1e6:.3f} us/layer); decode_split_kernel {split_ns / 1e3:.3f} us")
        ctx.submit()
        ctx.begin()
        for _ in range(args.steps):
            w.sweep()
        ctx.submit()
        r["us_per_layer_eager"] = round(ctx.gpuElapsedNs() / (w.layers * args.steps) / 1e3, 3)
        configs["C1"] = dict(workload="decode, 48 layers, 32q/4kv, d128, L 8192, f16 cache, fused step", gpu=r)
        achieved = w.bytes_per_layer / split_ns  # bytes/ns == GB/s
        roof = dict(bound="hbm", achieved=round(achieved, 2), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(achieved / HBM_PEAK_GBS, 4), traffic=measured_traffic("decode_split_kernel", "c1"),
                    kernel="decode_split_kernel", kernel_mean_us=round(split_ns / 1e3, 4),
                    algorithmic_bytes_per_launch=w.bytes_per_layer)
        if "rocprof_kernel_us" in r:
            roof["rocprof_kernel_mean_us"] = r["rocprof_kernel_us"]
            roof["rocprof_frac"] = r["rocprof_kernel_frac"]
        result = dict(
            metric="decode attn µs/layer & HBM GB/s (32q/4kv,d128,8K ctx f16 KV); prefill TFLOP/s",
            value=r["gbs"], unit="GB/s", n_gpus=1, steps=args.steps, warmup=args.warmup,
            ms_per_step=round(elapsed / args.steps * 1e3, 4), higher_is_better=True, scaling="weak",
            vs_baseline=None,
            dtype="f16 KV; f16 MFMA products of hi/lo-split q and p (about 22 significant bits) with f32 "
                  "accumulation; f32 softmax and norms", data="synthetic",
            config=dict(workload="C1: decode 1 token x 48 independent layers, Qwen3-30B-A3B attention "
                                 "(32q/4kv, d128), f16 KV cache 8192 tokens/layer, fused qk-norm+rope+append+attention",
                        layers=w.layers, ctx_len=w.pos + 1, n_q_heads=32, n_kv_heads=4, head_dim=128,
                        parallelism="single GPU"),
            us_per_layer=r["us_per_layer"], us_per_layer_eager=r["us_per_layer_eager"], roofline=roof)
        parity_decode(1)

    if 1 in W and "SIX" in only:
        six = {}
        for part in ("prep", "attn", "all"):
            sw = SixOpSweep(H, ctx, W[1], part)
            el, _ = time_graph(ctx, sw, max(5, args.steps // 2), 2)
            six[part] = round(el / (sw.layers * max(5, args.steps // 2)) * 1e6, 3)
            if part == "all":
                names = ("rms_norm_rows_kernel", "rope_kernel", "kv_append_kernel", "decode_split_kernel",
                         "decode_merge_kernel")
                ks = kernel_stats(ctx, sw, names, leg)
                six["kernel_us"] = {k: round(ks[k][0] / 1e3, 3) for k in names}
            del sw
        fused = configs.get("C1", {}).get("gpu", {}).get("us_per_layer")
        extra["C1_six_ops"] = dict(
            norm_rope_append_us_per_layer=six["prep"], attention_us_per_layer=six["attn"],
            six_ops_us_per_layer=six["all"], fused_step_us_per_layer=fused, six_ops_kernel_us=six["kernel_us"],
            note="(i) rmsNorm q, rmsNorm k, rope q, rope k, kvAppend (five launches); (ii) gqaAttention "
                 "(split + merge); (iii) the fused step (norm/rope/append inside the split kernel)")
        log(f"[bench] C1 six ops: norm/rope/append {six['prep']:.3f}, attention {six['attn']:.3f}, all six "
            f"{six['all']:.3f} us/layer; fused step {fused}; kernels {six['kernel_us']}")

    if "FLOOR" in only:
        fl = {}
        for mode in ("empty", "read", "both"):
            fw = FloorSweep(H, ctx, mode=mode)
            el, _ = time_graph(ctx, fw, max(5, args.steps), 2)
            fl[mode] = round(el / (fw.layers * max(5, args.steps)) * 1e6, 3)
            del fw
        for mode in ("read", "both"):  # C3's K+V per layer: 2 x 4 kv heads x 32768 x 128 f16 = 64 MiB
            fw = FloorSweep(H, ctx, layers=47, nbytes=64 << 20, mode=mode)
            el, _ = time_graph(ctx, fw, max(5, args.steps // 4), 2)
            fl[mode + "64"] = round(el / (fw.layers * max(5, args.steps // 4)) * 1e6, 3)
            del fw
        extra["floors"] = dict(
            empty_launch_us=fl["empty"], read_16MiB_us=fl["read"], read_plus_empty_us=fl["both"],
            read_16MiB_gbs=round((16 << 20) / (fl["read"] * 1e3), 1),
            read_64MiB_us=fl["read64"], read_64MiB_plus_empty_us=fl["both64"],
            read_64MiB_gbs=round((64 << 20) / (fl["read64"] * 1e3), 1),
            note="per layer in a 48-layer graph: one dependent launch of an empty kernel; one launch reading a "
                 "distinct 16 MiB buffer once (C1's K+V per layer) with the decode's 16-byte non-temporal loads; "
                 "both (the split + merge launch count); the same for 64 MiB (C3's K+V per layer) in a 47-layer "
                 "graph")
        log(f"[bench] floors: empty launch {fl['empty']:.3f} us, 16 MiB read {fl['read']:.3f} us, "
            f"read + empty {fl['both']:.3f} us per layer; 64 MiB read {fl['read64']:.3f} us, read + empty "
            f"{fl['both64']:.3f} us per layer")

    if 0 in W and "C0" in only:
        w = W[0]
        el1, _ = time_graph(ctx, w, 2, 1)
        reps = replays_for(el1 / 2, leg, 20)
        r, _, _, _ = decode_leg(0, reps, 5)
        configs["C0"] = dict(workload="decode, 1 layer, 32q/4kv, d128, 31 cached + 1 appended, f16 cache, fused step",
                             gpu=r, note="launch-bound: us per step (100 dependent steps per graph replay) is the "
                                         "figure; GB/s is not meaningful at 103 KB per step")
        log(f"[bench] C0 {r['us_per_layer']:.3f} us/step (graph of 100 steps, {reps} replays)")
        parity_decode(0)

    if 2 in W and "C2" in only:
        p = W[2]
        pr = Repeat(p, SWEEPS_PER_GRAPH)
        el1, _ = time_graph(ctx, pr, 3, 1)
        reps = replays_for(el1 / 3, leg, 5)
        elapsed, _ = time_graph(ctx, pr, reps, 2)
        e2e_us = elapsed / (reps * SWEEPS_PER_GRAPH) * 1e6
        ks = kernel_stats(ctx, p, ("prefill_prep_kernel", "prefill_attention_kernel"), leg)
        ns_pf = ks["prefill_attention_kernel"][0]
        tf = p.flops / ns_pf / 1e3
        sep = Prefill(H, synth, ctx, fused=False)
        n_sep = max(5, reps // 4)
        el_sep, _ = time_graph(ctx, Repeat(sep, SWEEPS_PER_GRAPH), n_sep, 2)
        r = dict(end_to_end_us=round(e2e_us, 3), kernel_us=dict(prefill_prep_kernel=round(ks["prefill_prep_kernel"][0] / 1e3, 3),
                                                               prefill_attention_kernel=round(ns_pf / 1e3, 3)),
                 tflops=round(tf, 2), frac=round(tf / F16_MFMA_PEAK_TFLOPS, 4),
                 tflops_end_to_end=round(p.flops / (e2e_us * 1e3) / 1e3, 2),
                 frac_end_to_end=round(p.flops / (e2e_us * 1e3) / 1e3 / F16_MFMA_PEAK_TFLOPS, 4), flops=p.flops,
                 peak_tflops=F16_MFMA_PEAK_TFLOPS,
                 six_ops_end_to_end_us=round(el_sep / (n_sep * SWEEPS_PER_GRAPH) * 1e6, 3),
                 sweeps_per_graph=SWEEPS_PER_GRAPH)
        ru = rocprof_kernel_us("C2", "prefill_attention_kernel")
        if ru:
            r["rocprof_kernel_us"] = ru
            r["rocprof_frac"] = round(p.flops / (ru * 1e3) / 1e3 / F16_MFMA_PEAK_TFLOPS, 4)
        configs["C2"] = dict(workload="causal prefill 2048 tokens, 32q/4kv, d128, empty f16 cache, fused step",
                             gpu=r)
        extra["C2_prefill"] = dict(kernel="prefill_attention_kernel", kernel_us=round(ns_pf / 1e3, 3),
                                   tflops=r["tflops"], frac=r["frac"], end_to_end_us=r["end_to_end_us"])
        log(f"[bench] C2 prefill_attention_kernel {ns_pf / 1e3:.2f} us -> {tf:.1f} TFLOP/s; end-to-end {e2e_us:.2f} us; "
            f"six ops {r['six_ops_end_to_end_us']:.2f} us")
        del sep
        parity_c2()

    if 3 in W and "C3" in only:
        w = W[3]
        el1, _ = time_graph(ctx, w, 2, 1)
        r, _, _, _ = decode_leg(3, replays_for(el1 / 2, leg, max(5, args.steps // 4)), 2)
        configs["C3"] = dict(workload="decode, 47 layers, 64q/4kv, d128, L 32768, theta 5e6, f16 cache, fused step",
                             gpu=r)
        extra["C3_decode"] = dict(us_per_layer=r["us_per_layer"], gbs=r["gbs"],
                                  kernel_us=r["kernel_us"]["decode_split_kernel"], kernel_frac=r["kernel_frac"])
        log(f"[bench] C3 {r['us_per_layer']:.3f} us/layer; kernel {r['kernel_us']}")
        parity_decode(3)

    if 4 in W and "C4" in only:
        w = W[4]
        el1, _ = time_graph(ctx, w, 1, 1)
        r, _, _, _ = decode_leg(4, replays_for(el1, leg, max(3, args.steps // 10)), 1)
        r["total_tokens"] = int(w.lay.seq_lens.sum())
        configs["C4"] = dict(workload="paged decode, 32 sequences L ~ U[512, 16384], 16-token pages, 48 layers",
                             gpu=r)
        extra["C4_paged_decode"] = dict(us_per_layer=r["us_per_layer"], gbs=r["gbs"],
                                        kernel_us=r["kernel_us"]["decode_split_kernel"], kernel_frac=r["kernel_frac"])
        log(f"[bench] C4 {r['us_per_layer']:.3f} us/layer; kernel {r['kernel_us']}")
        parity_c4()

    if "QKV" in only:
        log("[bench] QKV: decode q/k/v projections, Q8_0 wq [4096 x 2048] + wk, wv [512 x 2048], 48 layers")
        stepsq = max(5, args.steps // 4)
        w = ProjSweep(H, ctx)
        elapsed, _ = time_graph(ctx, w, stepsq, 2)
        us = elapsed / (w.layers * stepsq) * 1e6
        ns_k = kernel_stats(ctx, w, ("matmul_rows_kernel",), leg)["matmul_rows_kernel"][0]
        del w
        w = ProjSweep(H, ctx, grouped=False)
        elapsed, _ = time_graph(ctx, w, stepsq, 2)
        us_sep = elapsed / (w.layers * stepsq) * 1e6
        del w
        extra["qkv_projection_decode"] = dict(
            kernel="matmul_rows_kernel", us_per_layer=round(us, 3), gbs=round(QKV_BYTES / (us * 1e3), 2),
            kernel_us=round(ns_k / 1e3, 3), kernel_frac=round(QKV_BYTES / ns_k / HBM_PEAK_GBS, 4),
            us_per_layer_three_calls=round(us_sep, 3), bytes_per_layer=QKV_BYTES,
            shape="m 1, n 4096 + 512 + 512, k 2048, Q8_0; one grouped call (three matmul calls: us_per_layer_three_calls)")
        log(f"[bench] QKV grouped {us:.3f} us/layer ({QKV_BYTES / (us * 1e3):.1f} GB/s); kernel {ns_k / 1e3:.3f} us; "
            f"three calls {us_sep:.3f} us/layer")

    if "WO" in only:
        log("[bench] WO: decode output projection + residual, Q8_0 wo [2048 x 4096], 48 layers")
        stepsw = max(5, args.steps // 4)
        w = WoSweep(H, ctx)
        elapsed, _ = time_graph(ctx, w, stepsw, 2)
        us = elapsed / (w.layers * stepsw) * 1e6
        ns_k = kernel_stats(ctx, w, ("matmul_rows_kernel",), leg)["matmul_rows_kernel"][0]
        bpl = w.bytes_per_layer
        del w
        w = WoSweep(H, ctx, fused=False)
        elapsed, _ = time_graph(ctx, w, stepsw, 2)
        us_sep = elapsed / (w.layers * stepsw) * 1e6
        del w
        extra["wo_projection_residual_decode"] = dict(
            kernel="matmul_rows_kernel", us_per_layer=round(us, 3), gbs=round(bpl / (us * 1e3), 2),
            kernel_us=round(ns_k / 1e3, 3), kernel_frac=round(bpl / ns_k / HBM_PEAK_GBS, 4),
            us_per_layer_matmul_then_add=round(us_sep, 3), bytes_per_layer=bpl,
            shape="m 1, n 2048, k 4096, Q8_0, residual added in the epilogue (matmul then add: "
                  "us_per_layer_matmul_then_add)")
        log(f"[bench] WO fused {us:.3f} us/layer ({bpl / (us * 1e3):.1f} GB/s); kernel {ns_k / 1e3:.3f} us; "
            f"matmul then add {us_sep:.3f} us/layer")

    if "MOE" in only:
        log("[bench] MOE: decode MoE block (router top-8 of 128, SwiGLU experts 2048 x 768 Q8_0), 16 layers")
        w = MoeSweep(H, ctx)
        stepsm = max(5, args.steps // 4)
        elapsed, _ = time_graph(ctx, w, stepsm, 2)
        us = elapsed / (w.layers * stepsm) * 1e6
        names = ("router_logits_kernel", "router_select_kernel", "moe_gate_up_kernel", "moe_down_combine_kernel")
        ks = kernel_stats(ctx, w, names, leg)
        per = {k: ks[k][0] / 1e3 for k in names}
        extra["moe_block_decode"] = dict(
            us_per_layer=round(us, 3), gbs=round(w.bytes_per_layer / (us * 1e3), 2), bytes_per_layer=w.bytes_per_layer,
            kernel_us={k: round(v, 3) for k, v in per.items()},
            shape="1 token, dim 2048, 128 experts top 8, ffn 768, Q8_0 banks, f32 router; router and experts on the "
                  "device (ds5_hip_moe)")
        log(f"[bench] MOE {us:.3f} us/layer ({w.bytes_per_layer / (us * 1e3):.1f} GB/s); kernels "
            + ", ".join(f"{k} {v:.2f} us" for k, v in per.items()))
        del w

    if "LAYER" in only:
        log("[bench] LAYER: one decode token through 48 whole layers, Qwen3-30B-A3B shape, fused engine order")
        w = DecodeLayerSweep(H, ctx)
        stepsl = max(5, args.steps // 4)
        elapsed, _ = time_graph(ctx, w, stepsl, 2)
        us = elapsed / (w.layers * stepsl) * 1e6
        # per-layer device time of eager sweeps (the engine's timing marks)
        w.marks = True
        ctx.timing_begin()
        for _ in range(3):
            w.sweep()
        ns = np.array(ctx.timing_read(), np.float64)
        w.marks = False
        ns = ns[[i for i in range(len(ns)) if (i + 1) % (w.layers + 1) != 0]] / 1e3  # drop the gaps between sweeps
        names = ("rms_norm_tree_kernel", "rms_norm_rows_kernel", "matmul_rows_kernel", "decode_split_kernel",
                 "decode_merge_kernel", "router_logits_kernel", "router_select_kernel", "moe_gate_up_kernel",
                 "moe_down_combine_kernel", "add_kernel", "zero_words_kernel")
        ks = kernel_stats(ctx, w, names, leg)
        n_layer_runs = max(1, ks["decode_split_kernel"][1])  # one split launch per layer
        per_layer = {k: round(ks[k][0] * ks[k][1] / n_layer_runs / 1e3, 3) for k in names if ks[k][1]}
        parts = {"qkv_projection_decode": "us_per_layer", "wo_projection_residual_decode": "us_per_layer",
                 "moe_block_decode": "us_per_layer"}
        part_us = {k: extra[k][f] for k, f in parts.items() if k in extra}
        if "C1" in configs:
            part_us["attention_step_C1"] = configs["C1"]["gpu"]["us_per_layer"]
        extra["decode_layer"] = dict(
            us_per_layer=round(us, 3), layers=w.layers, steps=stepsl,
            eager_us_per_layer=dict(mean=round(float(ns.mean()), 3), min=round(float(ns.min()), 3),
                                    max=round(float(ns.max()), 3)),
            separate_legs_us=part_us, separate_legs_sum_us=round(sum(part_us.values()), 3) if len(part_us) == 4 else None,
            kernel_us_per_layer=per_layer, kernel_sum_us_per_layer=round(sum(per_layer.values()), 3),
            shape="1 token, hidden 2048, 32q/4kv d128, 8K f16 cache, Q8_0 wq/wk/wv/wo, 128 experts top 8 ffn 768; "
                  "attention block with attn_norm, Wo + residual, MoE with ffn_norm and residual (3 calls per layer)")
        log(f"[bench] LAYER {us:.3f} us/layer (graph of 48 layers); eager per-layer marks mean {ns.mean():.3f} "
            f"min {ns.min():.3f} max {ns.max():.3f} us; separate legs {part_us}; kernels per layer {per_layer}")
        del w

    if "MOEP" in only:
        log("[bench] MOEP: MoE block over 2048 prompt tokens (router top-8 of 128, experts 2048 x 768 Q8_0 grouped "
            "by expert)")
        w = MoePrefill(H, ctx)
        n_rep, per_graph = max(10, args.steps // 5), 4
        elapsed, _ = time_graph(ctx, Repeat(w, per_graph), n_rep, 2)
        us = elapsed / (n_rep * per_graph) * 1e6
        names = ("router_logits_tile_kernel", "router_select_kernel", "moe_sort_kernel", "matmul_x_split_kernel",
                 "matmul_q8_mfma_kernel", "moe_h_split_kernel", "moe_combine_kernel")
        ks = kernel_stats(ctx, w, names, leg)
        calls = max(1, ks["moe_sort_kernel"][1])
        per = {k: round(ks[k][0] * ks[k][1] / calls / 1e3, 3) for k in names if ks[k][1]}
        mfma_us = per.get("matmul_q8_mfma_kernel", 0.0)
        tf = w.expert_flops / (mfma_us * 1e6) if mfma_us else None
        extra["moe_block_prefill"] = dict(
            us=round(us, 3), us_per_token=round(us / w.T, 4), calls_per_graph=per_graph, kernel_us_per_call=per,
            expert_products_tflops=round(tf, 2) if tf else None,
            expert_products_frac=round(tf / BF16_MFMA_PEAK_TFLOPS, 4) if tf else None,
            expert_flops=w.expert_flops,
            shape="2048 tokens, dim 2048, 128 experts top 8 (16,384 pairs), ffn 768, Q8_0 banks, f32 router; logits "
                  "in tiles, experts grouped by expert (x / h split into f16 hi and lo: 2 matrix-core products per "
                  "useful one)")
        log(f"[bench] MOEP {us:.1f} us per call ({us / w.T:.3f} us/token); kernels per call {per}; expert products "
            f"{tf:.1f} TFLOP/s (useful)" if tf else f"[bench] MOEP {us:.1f} us per call; kernels {per}")
        del w

    if "QKVP" in only:
        log("[bench] QKVP: prefill q/k/v projections, 2048 tokens, Q8_0 wq [4096 x 2048] + wk, wv [512 x 2048]")
        p = ProjPrefill(H, ctx)
        n_rep = max(10, args.steps // 3)
        elapsed, _ = time_graph(ctx, Repeat(p, SWEEPS_PER_GRAPH), n_rep, 2)
        elapsed /= SWEEPS_PER_GRAPH
        ks = kernel_stats(ctx, p, ("matmul_q8_mfma_kernel", "matmul_x_split_kernel"), leg)
        ns_k, ns_split = ks["matmul_q8_mfma_kernel"][0], ks["matmul_x_split_kernel"][0]
        tf = p.flops / ns_k / 1e3
        extra["qkv_projection_prefill"] = dict(
            kernel="matmul_q8_mfma_kernel", kernel_us=round(ns_k / 1e3, 3), tflops=round(tf, 2),
            frac=round(tf / BF16_MFMA_PEAK_TFLOPS, 4), end_to_end_us=round(elapsed / n_rep * 1e6, 3),
            flops=p.flops, peak_tflops=BF16_MFMA_PEAK_TFLOPS,
            split_us=round(ns_split / 1e3, 3), sweeps_per_graph=SWEEPS_PER_GRAPH,
            shape="m 2048, n 4096 + 512 + 512, k 2048, Q8_0, one grouped call; x split into f16 hi and lo "
                  "(2 matrix-core products per useful one)")
        log(f"[bench] QKVP matmul_q8_mfma_kernel {ns_k / 1e3:.2f} us -> {tf:.1f} TFLOP/s (useful)")
        del p

    if "BLK" in only:
        log("[bench] BLK: prefill attention block, 2048 tokens: Q8_0 q/k/v projections (hidden 2048) + step")
        legs = {}
        for fused in (True, False):
            p = BlockPrefill(H, synth, ctx, fused=fused)
            n_rep = max(10, args.steps // 3)
            elapsed, _ = time_graph(ctx, Repeat(p, SWEEPS_PER_GRAPH), n_rep, 2)
            elapsed /= SWEEPS_PER_GRAPH
            names = ("matmul_x_split_kernel", "matmul_q8_mfma_kernel", "prefill_prep_kernel",
                     "prefill_attention_kernel")
            ks = kernel_stats(ctx, p, names, leg)
            legs[fused] = dict(end_to_end_us=round(elapsed / n_rep * 1e6, 3), sweeps_per_graph=SWEEPS_PER_GRAPH,
                               kernel_us={k: round(ks[k][0] / 1e3, 3) for k in names if ks[k][1]})
            del p
        extra["attention_block_prefill"] = dict(
            fused=legs[True], two_calls=legs[False],
            shape="T 2048, hidden 2048, wq [4096 x 2048] + wk, wv [512 x 2048] Q8_0, 32q/4kv d128, empty f16 "
                  "cache; fused = ds5_hip_attention_block (norm, rope, f16 append and the q operand in the "
                  "projection GEMM's epilogue), two_calls = ds5_hip_matmul_group + ds5_hip_attention_step")
        log(f"[bench] BLK fused {legs[True]['end_to_end_us']:.2f} us ({legs[True]['kernel_us']}); two calls "
            f"{legs[False]['end_to_end_us']:.2f} us ({legs[False]['kernel_us']})")

    for c, r in cpu.items():
        if f"C{c}" in configs:
            configs[f"C{c}"]["cpu"] = r
            g = configs[f"C{c}"]["gpu"]
            gus = g.get("us_per_layer", g.get("end_to_end_us"))
            if gus:
                r["gpu_speedup"] = round(r["us_per_layer"] / gus, 1)
    for name, cfg in configs.items():
        if "parity" in cfg:
            log(f"[bench] parity {name}: {cfg['parity']}")

    if result is None:
        result = dict(metric="partial run", value=None)
    if "floors" in extra and "roofline" in result:
        # why the 70% target (3.0 us/layer at C1) is out of reach with one dependent launch per layer
        result["roofline"]["floor_us"] = extra["floors"]["read_plus_empty_us"]
        result["roofline"]["floor_note"] = (
            "per layer in a 48-layer graph: one launch reading the layer's 16 MiB of K/V once plus one dependent "
            "empty launch (the split + merge launch count), nothing computed; 70% of HBM peak would be "
            f"{decode_bytes(32, 4, 128, 8192) / (0.7 * HBM_PEAK_GBS) / 1e3:.3f} us per layer")
    result["configs"] = configs
    result["extra"] = extra
    if 1 in cpu:
        bpl = decode_bytes(32, 4, 128, 8192)
        c1 = cpu[1]
        result["cpu_baseline"] = dict(value=round(bpl / (c1["us_per_layer"] * 1e3), 4), unit="GB/s", cores=1,
                                      kind="port", us_per_layer=c1["us_per_layer"], host_nproc=os.cpu_count(),
                                      sample="C1: " + c1["sample"])
    ctx.deinit()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
