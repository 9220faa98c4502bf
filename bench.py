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

value  = C1 algorithmic HBM bytes of the K sweeps / elapsed (GB/s)
roofline.achieved = algorithmic bytes of one decode_split_kernel launch (one
         layer) / that kernel's mean device duration from HIP events around
         each launch on the context stream (a separate, eager pass)
cpu_baseline = the CPU oracle (a line-by-line C restatement of the reference's
         single-threaded CPU path) on a bounded sample of C1 layers, 1 core.

Secondary figures (prefill C2 TFLOP/s, C3 decode, C4 paged decode) are
reported under "extra"; they are not the headline value.
"""
from __future__ import annotations

import argparse
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
# Workloads
# ---------------------------------------------------------------------------

class DecodeSweep:
    """n_layers independent layers of single-token decode on a contiguous cache."""

    def __init__(self, H, synth, ctx, config, verbose=True):
        cfg = synth.CONFIGS[config]
        self.H, self.ctx, self.config = H, ctx, config
        s = self.s = cfg["shape"]
        self.cap, self.pos, self.layers = cfg["cap"], cfg["pos"], cfg["layers"]
        hkv, d = s.n_kv_heads, s.head_dim
        n = hkv * self.cap * d
        self.args = []
        pos_buf = ctx.from_numpy(np.array([self.pos], np.int32))
        for layer in range(self.layers):
            kc, vc = ctx.createBuffer(2 * n), ctx.createBuffer(2 * n)
            ctx.fill_normal_f16(kc, n, seed=(config << 20) + 2 * layer + 1)
            ctx.fill_normal_f16(vc, n, seed=(config << 20) + 2 * layer + 2)
            q, k, v, qn, kn = synth.step_inputs(config, layer, 1, s)
            out = ctx.createBuffer(s.n_q_heads * d * 4)
            self.args.append(H.AttentionStepArgs(ctx.from_numpy(q), ctx.from_numpy(k), ctx.from_numpy(v),
                                                 ctx.from_numpy(qn), ctx.from_numpy(kn), pos_buf, kc, vc, out,
                                                 H.DTYPE_F16, self.pos, 1, s.n_q_heads, hkv, d, self.cap, s.eps,
                                                 s.theta, 1.0, s.scale))
        self.bytes_per_layer = decode_bytes(s.n_q_heads, hkv, d, self.pos + 1)

    def sweep(self):
        for a in self.args:
            self.H.attentionStep(self.ctx, a)


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


class PagedSweep:
    """C4: n_layers of batched paged decode (32 sequences, 16-token pages)."""

    def __init__(self, H, synth, ctx, config=4):
        cfg = synth.CONFIGS[config]
        self.H, self.ctx = H, ctx
        s = self.s = cfg["shape"]
        self.layers = cfg["layers"]
        lay = self.lay = synth.paged_layout(cfg["n_seqs"], cfg["lo"], cfg["hi"], cfg["page_size"], seed=0)
        hq, hkv, d = s.n_q_heads, s.n_kv_heads, s.head_dim
        B = cfg["n_seqs"]
        slots = lay.n_pages * lay.page_size
        pt, sl = ctx.from_numpy(lay.page_table), ctx.from_numpy(lay.seq_lens)
        self.args = []
        for layer in range(self.layers):
            kp, vp = ctx.createBuffer(2 * hkv * slots * d), ctx.createBuffer(2 * hkv * slots * d)
            ctx.fill_normal_f16(kp, hkv * slots * d, seed=(config << 20) + 2 * layer + 1)
            ctx.fill_normal_f16(vp, hkv * slots * d, seed=(config << 20) + 2 * layer + 2)
            q, k, v, qn, kn = synth.step_inputs(config, layer, B, s)
            out = ctx.createBuffer(B * hq * d * 4)
            self.args.append(H.PagedDecodeArgs(ctx.from_numpy(q), ctx.from_numpy(k), ctx.from_numpy(v),
                                               ctx.from_numpy(qn), ctx.from_numpy(kn), kp, vp, pt, sl, out, B, hq,
                                               hkv, d, lay.page_size, lay.n_pages, lay.max_pages,
                                               int(lay.seq_lens.max()), s.eps, s.theta, 1.0, s.scale))
        pages = ((lay.seq_lens.astype(np.int64) + lay.page_size - 1) // lay.page_size).sum()
        self.bytes_per_layer = int(sum(decode_bytes(hq, hkv, d, int(L)) - 8 * d for L in lay.seq_lens)
                                   + 8 * d + 4 * pages)

    def sweep(self):
        for a in self.args:
            self.H.pagedDecode(self.ctx, a)


class Prefill:
    """C2: causal prefill of 2048 tokens into an empty f16 cache, one layer."""

    def __init__(self, H, synth, ctx, config=2):
        cfg = synth.CONFIGS[config]
        self.H, self.ctx = H, ctx
        s = self.s = cfg["shape"]
        T = self.T = cfg["tokens"]
        hq, hkv, d = s.n_q_heads, s.n_kv_heads, s.head_dim
        q, k, v, qn, kn = synth.step_inputs(config, 0, T, s, f16_exact=True)
        kc, vc = ctx.createBuffer(2 * hkv * T * d), ctx.createBuffer(2 * hkv * T * d)
        out = ctx.createBuffer(T * hq * d * 4)
        self.args = H.AttentionStepArgs(ctx.from_numpy(q), ctx.from_numpy(k), ctx.from_numpy(v), ctx.from_numpy(qn),
                                        ctx.from_numpy(kn), ctx.from_numpy(np.arange(T, dtype=np.int32)), kc, vc,
                                        out, H.DTYPE_F16, 0, T, hq, hkv, d, T, s.eps, s.theta, 1.0, s.scale)
        self.flops = prefill_flops(hq, d, T)

    def sweep(self):
        self.H.attentionStep(self.ctx, self.args)


def time_graph(ctx, work, steps, warmup):
    """Capture work.sweep() once, replay warmup + steps times; returns seconds of the timed replays."""
    work.sweep()                      # eager once: sizes the split-K workspace
    ctx.submit()
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


def kernel_mean_ns(ctx, work, kernel, reps):
    """Mean device duration of `kernel` over `reps` eager sweeps, from HIP events
    recorded around each launch on the context stream."""
    ctx.set_kernel_timing(True)
    try:
        for _ in range(reps):
            work.sweep()
        ctx.submit()
        n, total = ctx.kernel_time(kernel)
    finally:
        ctx.set_kernel_timing(False)
    return (total / n if n else float("nan")), n


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


def cpu_baseline_c1(synth, seconds):
    """Oracle (single-threaded C restatement of kernels_a/b.zig) on C1 layers."""
    from oracle import oracle as O
    cfg = synth.CONFIGS[1]
    s, cap, pos = cfg["shape"], cfg["cap"], cfg["pos"]
    data = []
    for layer in range(3):
        q, k, v, qn, kn = synth.step_inputs(1, layer, 1, s)
        kc, vc = synth.cache_f16(1, layer, s, cap, pos)
        data.append((q, k, v, qn, kn, kc, vc))
    n, t_total = 0, 0.0
    while t_total < seconds:
        q, k, v, qn, kn, kc, vc = data[n % len(data)]
        t0 = time.perf_counter()
        O.attention_step(q, k, v, qn, kn, np.array([pos], np.int32), kc, vc, kv_dtype=1, pos=pos, n_tokens=1,
                         n_q_heads=s.n_q_heads, n_kv_heads=s.n_kv_heads, head_dim=s.head_dim, max_ctx=cap,
                         eps=s.eps, theta=s.theta, scale=s.scale)
        t_total += time.perf_counter() - t0
        n += 1
    us = t_total / n * 1e6
    return dict(us_per_layer=us, layers=n, seconds=t_total)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50, help="timed 48-layer sweeps")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--only", default="C1,C2,C3,C4,QKV,WO,MOE,QKVP",
                    help="comma list of configs to run (C1 is the headline; QKV / QKVP: the decode / prefill "
                         "q/k/v projections; WO: the decode output projection and residual; MOE: the decode MoE block)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="also run one device-to-device copy of MIB MiB (the known-size reference dispatch for "
                         "the FETCH_SIZE / WRITE_SIZE traffic counters)")
    args = ap.parse_args()
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
    extra = {}
    result = None

    if "C1" in only:
        log("[bench] C1: building 48 layers (8192-token f16 caches)")
        w = DecodeSweep(H, synth, ctx, 1)
        elapsed, wall = time_graph(ctx, w, args.steps, args.warmup)
        layers = w.layers * args.steps
        us_layer = elapsed / layers * 1e6
        gbs = w.bytes_per_layer * layers / elapsed / 1e9
        log(f"[bench] C1 graph sweep: {us_layer:.3f} us/layer, {gbs:.1f} GB/s (wall {wall / layers * 1e6:.3f} us/layer)")
        ns_split, n_split = kernel_mean_ns(ctx, w, "decode_split_kernel", max(2, args.steps // 10))
        achieved = w.bytes_per_layer / ns_split  # bytes/ns == GB/s
        log(f"[bench] C1 decode_split_kernel mean {ns_split / 1e3:.3f} us over {n_split} launches -> {achieved:.1f} GB/s")
        ctx.submit()
        ctx.begin()
        for _ in range(args.steps):
            w.sweep()
        ctx.submit()
        eager_us = ctx.gpuElapsedNs() / (w.layers * args.steps) / 1e3
        log(f"[bench] C1 eager (no graph) sweep: {eager_us:.3f} us/layer")
        result = dict(
            metric="decode attn µs/layer & HBM GB/s (32q/4kv,d128,8K ctx f16 KV); prefill TFLOP/s",
            value=round(gbs, 2), unit="GB/s", n_gpus=1, steps=args.steps, warmup=args.warmup,
            ms_per_step=round(elapsed / args.steps * 1e3, 4), higher_is_better=True, scaling="weak",
            vs_baseline=None, dtype="f16 KV / f32 compute", data="synthetic",
            config=dict(workload="C1: decode 1 token x 48 independent layers, Qwen3-30B-A3B attention "
                                 "(32q/4kv, d128), f16 KV cache 8192 tokens/layer, fused qk-norm+rope+append+attention",
                        layers=w.layers, ctx_len=w.pos + 1, n_q_heads=32, n_kv_heads=4, head_dim=128,
                        parallelism="single GPU"),
            us_per_layer=round(us_layer, 4),
            us_per_layer_eager=round(eager_us, 4),
            roofline=dict(bound="hbm", achieved=round(achieved, 2), peak=HBM_PEAK_GBS, unit="GB/s",
                          frac=round(achieved / HBM_PEAK_GBS, 4),
                          traffic=measured_traffic("decode_split_kernel", "c1"),
                          kernel="decode_split_kernel", kernel_mean_us=round(ns_split / 1e3, 4),
                          algorithmic_bytes_per_launch=w.bytes_per_layer),
        )
        del w

    if "C2" in only:
        log("[bench] C2: prefill 2048 tokens")
        p = Prefill(H, synth, ctx)
        elapsed, _ = time_graph(ctx, p, max(5, args.steps // 5), 2)
        n_rep = max(5, args.steps // 5)
        e2e_us = elapsed / n_rep * 1e6
        ns_pf, _ = kernel_mean_ns(ctx, p, "prefill_attention_kernel", 5)
        tf = p.flops / ns_pf / 1e3
        extra["C2_prefill"] = dict(kernel="prefill_attention_kernel", kernel_us=round(ns_pf / 1e3, 3), tflops=round(tf, 2),
                                   frac=round(tf / F16_MFMA_PEAK_TFLOPS, 4), end_to_end_us=round(e2e_us, 3),
                                   flops=p.flops, peak_tflops=F16_MFMA_PEAK_TFLOPS)
        log(f"[bench] C2 prefill_attention_kernel {ns_pf / 1e3:.2f} us -> {tf:.1f} TFLOP/s; end-to-end {e2e_us:.2f} us")
        del p

    if "C3" in only:
        log("[bench] C3: building 47 layers (32768-token f16 caches, 64q/4kv)")
        w = DecodeSweep(H, synth, ctx, 3)
        steps3 = max(5, args.steps // 4)
        elapsed, _ = time_graph(ctx, w, steps3, 2)
        us = elapsed / (w.layers * steps3) * 1e6
        ns_k, _ = kernel_mean_ns(ctx, w, "decode_split_kernel", 2)
        extra["C3_decode"] = dict(us_per_layer=round(us, 3), gbs=round(w.bytes_per_layer / (us * 1e3), 2),
                                  kernel_us=round(ns_k / 1e3, 3),
                                  kernel_frac=round(w.bytes_per_layer / ns_k / HBM_PEAK_GBS, 4),
                                  bytes_per_layer=w.bytes_per_layer)
        log(f"[bench] C3 {us:.3f} us/layer; kernel {ns_k / 1e3:.3f} us")
        del w

    if "C4" in only:
        log("[bench] C4: building 48 layers of paged pools (32 sequences)")
        w = PagedSweep(H, synth, ctx)
        steps4 = max(3, args.steps // 10)
        elapsed, _ = time_graph(ctx, w, steps4, 1)
        us = elapsed / (w.layers * steps4) * 1e6
        ns_k, _ = kernel_mean_ns(ctx, w, "decode_split_kernel", 1)
        extra["C4_paged_decode"] = dict(us_per_layer=round(us, 3), gbs=round(w.bytes_per_layer / (us * 1e3), 2),
                                        kernel_us=round(ns_k / 1e3, 3),
                                        kernel_frac=round(w.bytes_per_layer / ns_k / HBM_PEAK_GBS, 4),
                                        bytes_per_layer=w.bytes_per_layer,
                                        total_tokens=int(w.lay.seq_lens.sum()))
        log(f"[bench] C4 {us:.3f} us/layer; kernel {ns_k / 1e3:.3f} us")
        del w

    if "QKV" in only:
        log("[bench] QKV: decode q/k/v projections, Q8_0 wq [4096 x 2048] + wk, wv [512 x 2048], 48 layers")
        stepsq = max(5, args.steps // 4)
        w = ProjSweep(H, ctx)
        elapsed, _ = time_graph(ctx, w, stepsq, 2)
        us = elapsed / (w.layers * stepsq) * 1e6
        ns_k, _ = kernel_mean_ns(ctx, w, "matmul_rows_kernel", 2)
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
        ns_k, _ = kernel_mean_ns(ctx, w, "matmul_rows_kernel", 2)
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
        per = {kn: kernel_mean_ns(ctx, w, kn, 2)[0] / 1e3 for kn in
               ("router_logits_kernel", "router_select_kernel", "moe_gate_up_kernel", "moe_down_combine_kernel")}
        extra["moe_block_decode"] = dict(
            us_per_layer=round(us, 3), gbs=round(w.bytes_per_layer / (us * 1e3), 2), bytes_per_layer=w.bytes_per_layer,
            kernel_us={k: round(v, 3) for k, v in per.items()},
            shape="1 token, dim 2048, 128 experts top 8, ffn 768, Q8_0 banks, f32 router; router and experts on the "
                  "device (ds5_hip_moe)")
        log(f"[bench] MOE {us:.3f} us/layer ({w.bytes_per_layer / (us * 1e3):.1f} GB/s); kernels "
            + ", ".join(f"{k} {v:.2f} us" for k, v in per.items()))
        del w

    if "QKVP" in only:
        log("[bench] QKVP: prefill q/k/v projections, 2048 tokens, Q8_0 wq [4096 x 2048] + wk, wv [512 x 2048]")
        p = ProjPrefill(H, ctx)
        n_rep = max(5, args.steps // 5)
        elapsed, _ = time_graph(ctx, p, n_rep, 2)
        ns_k, _ = kernel_mean_ns(ctx, p, "matmul_q8_mfma_kernel", 5)
        ns_split, _ = kernel_mean_ns(ctx, p, "matmul_x_split_kernel", 5)
        tf = p.flops / ns_k / 1e3
        extra["qkv_projection_prefill"] = dict(
            kernel="matmul_q8_mfma_kernel", kernel_us=round(ns_k / 1e3, 3), tflops=round(tf, 2),
            frac=round(tf / BF16_MFMA_PEAK_TFLOPS, 4), end_to_end_us=round(elapsed / n_rep * 1e6, 3),
            flops=p.flops, peak_tflops=BF16_MFMA_PEAK_TFLOPS,
            split_us=round(ns_split / 1e3, 3),
            shape="m 2048, n 4096 + 512 + 512, k 2048, Q8_0, one grouped call; x split into f16 hi and lo "
                  "(2 matrix-core products per useful one)")
        log(f"[bench] QKVP matmul_q8_mfma_kernel {ns_k / 1e3:.2f} us -> {tf:.1f} TFLOP/s (useful)")
        del p

    if result is None:
        result = dict(metric="partial run", value=None, extra=extra)
    else:
        result["extra"] = extra
        if not args.no_cpu:
            log(f"[bench] CPU baseline: oracle on C1 layers for ~{args.cpu_seconds:.0f} s (1 core)")
            cb = cpu_baseline_c1(synth, args.cpu_seconds)
            bpl = decode_bytes(32, 4, 128, 8192)
            result["cpu_baseline"] = dict(
                value=round(bpl / (cb["us_per_layer"] * 1e3), 4), unit="GB/s", cores=1, kind="port",
                us_per_layer=round(cb["us_per_layer"], 1), host_nproc=os.cpu_count(),
                sample=f"{cb['layers']} C1 decode layer-steps (3 distinct seeded layers, 8192-token f16 cache) "
                       f"through oracle/ds5_oracle.c ds5o_attention_step, {cb['seconds']:.1f} s")
    ctx.deinit()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
