// k_moe.hip -- the MoE step after the attention block: router top-k and the
// SwiGLU expert MLP (kernels_c.zig:80-155 routerTopK, :157-214 expertMlpSwiglu).
//
// Router: workgroups of (token, group of experts). Each expert's logit is the reference's
// serial f32 dot (dotRow, kernels_c.zig:40-68: products and sums rounded one by
// one, in storage order), so logits are bit-identical to the reference. The
// softmax keeps its order too: max, exp(l - max) per expert, the sum in expert
// order, then the reciprocal; the top-k rounds pick the largest probability
// with ties to the lower id (a wavefront argmax under that total order equals
// the reference's ascending scan with a strict >); the k weights are summed in
// pick order and optionally scaled by its reciprocal. exp is the device's expf, so
// probabilities may differ from the reference's in the last bit; ids can then
// differ only where two probabilities are that close.
//
// Experts, per dispatch pair p = (token t, expert e, weight w):
//   h[p][j] = silu(gate_e[j] . x_t) * (up_e[j] . x_t)     (moe_gate_up_kernel)
//   y[p][i] = down_e[i] . h[p]                            (moe_down_kernel)
//   out[t][i] += w * y[p][i] over t's pairs in list order (moe_combine_kernel)
// (the last two in one launch, moe_down_combine_kernel, where the outputs fit
// one grid)
// The GEMVs are weight-bandwidth bound: one wavefront per weight row, lane L
// owning the 32-element blocks L + 64 j, a fixed-order wavefront reduction (so
// they agree with the reference's serial dots to rounding). The combine adds
// each product in the reference's order, rounding as it does.
// Many tokens: the logits in token x expert tiles (router_logits_tile_kernel, the
// same serial sums); from two pairs per expert the experts grouped by expert
// (moe_sort_kernel, then Q8_0 matrix-core products per expert row tile,
// launch_experts_grouped), each expert's weights read once per tile.
#include <type_traits>

#include "ds5_common.hpp"

namespace {

constexpr int kMaxDevices = 64;  // per-device one-time kernel attributes

constexpr int kRouterThreads = 256;
constexpr int kMoeWaves = 8;  // wavefronts (weight rows) per GEMV workgroup

struct OpMinF {
    __device__ __forceinline__ float operator()(float a, float b) const { return fminf(a, b); }
};

// ---------------------------------------------------------------------------
// router
// ---------------------------------------------------------------------------

// Weight element i of a router row, widened exactly as the reference widens it
// (f16 -> f32, and a Q8_0 element's f32(scale) * q, exact in f32). AL: the row
// is aligned to its element size; else it is read bytewise.
template <uint32_t DT, bool AL>
__device__ __forceinline__ float router_w(const uint8_t* row, uint32_t i) {
    if constexpr (DT == DS5_DTYPE_Q8_0) {
        const uint8_t* blk = row + (uint64_t)(i / 32) * kQ8Bytes;
        const float scale = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        return scale * (float)(int8_t)blk[2 + i % 32];
    } else if constexpr (DT == DS5_DTYPE_F32) {
        if constexpr (AL) return ((const float*)row)[i];
        float v;
        __builtin_memcpy(&v, row + 4 * (uint64_t)i, 4);
        return v;
    } else {
        if constexpr (AL) return f16_bits_to_f32(((const uint16_t*)row)[i]);
        uint16_t b;
        __builtin_memcpy(&b, row + 2 * (uint64_t)i, 2);
        return f16_bits_to_f32(b);
    }
}

// Logits (router_logits_kernel): workgroup (token t, expert group g) holds the
// token's x and the raw bytes of R consecutive expert rows in LDS, loaded with
// every load in flight at once (the rows are contiguous); thread r < R then
// sums its row in element order, exactly dotRow (kernels_c.zig:40-68). Many
// workgroups per token spread the weight traffic over the CUs; the serial sum
// (one add per element) bounds each.
constexpr uint32_t kRouterRowBytes = 65536;  // LDS for one group's rows

constexpr uint32_t kRouterGroupBytes = 16384;  // rows per group: about this many bytes (more workgroups load faster)
__host__ __device__ inline uint32_t router_rows_per_group(uint64_t row_bytes) {
    const uint64_t r = kRouterGroupBytes / row_bytes;
    return (uint32_t)(r > 16 ? 16 : (r ? r : 1));
}

// Dynamic LDS: x (dim floats), then R rows of raw weights. CP: the rows are
// copied in 16-byte, 4-byte or 1-byte units (by the source's alignment), every
// thread's loads issued before its stores.
template <int CP>
__device__ __forceinline__ void router_copy_rows(const uint8_t* src, uint8_t* dst, uint64_t nbytes) {
    if constexpr (CP == 1) {
        for (uint64_t i = threadIdx.x; i < nbytes; i += kRouterThreads) dst[i] = src[i];
    } else {
        typedef typename std::conditional<CP == 16, f32x4, uint32_t>::type U;
        constexpr int kN = kRouterRowBytes / CP / kRouterThreads;
        const U* s = (const U*)src;
        U* d = (U*)dst;
        const uint32_t n = (uint32_t)(nbytes / CP);
        U v[kN];
#pragma unroll
        for (int k = 0; k < kN; k++) {
            const uint32_t i = threadIdx.x + kRouterThreads * k;
            if (i < n) v[k] = s[i];
        }
#pragma unroll
        for (int k = 0; k < kN; k++) {
            const uint32_t i = threadIdx.x + kRouterThreads * k;
            if (i < n) d[i] = v[k];
        }
    }
}

// The row's sum of products p4[0 .. 4·n4) in element order (dotRow's adds), reading
// eight 16-byte chunks ahead of the adds in two register sets in turn, so the chain
// of dependent adds never waits for LDS.
__device__ __forceinline__ float router_chain(const f32x4* __restrict__ p4, uint32_t n4) {
#pragma clang fp contract(off)
    constexpr uint32_t B = 8;
    float acc = 0.0f;
    uint32_t j = 0;
    auto read = [&](f32x4* v, uint32_t at) {
#pragma unroll
        for (uint32_t b = 0; b < B; b++) v[b] = p4[at + b];
        __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the adds
    };
    auto sum = [&](const f32x4* v) {
#pragma unroll
        for (uint32_t b = 0; b < B; b++)
#pragma unroll
            for (int c = 0; c < 4; c++) acc += v[b][c];
    };
    if (n4 >= B) {
        f32x4 va[B], vb[B];
        read(va, 0);
        for (j = B; j + 2 * B <= n4; j += 2 * B) {
            read(vb, j);
            sum(va);
            read(va, j + B);
            sum(vb);
        }
        if (j + B <= n4) {
            read(vb, j);
            sum(va);
            sum(vb);
            j += B;
        } else {
            sum(va);
        }
    }
    for (; j < n4; j++) {
        const f32x4 v = p4[j];
#pragma unroll
        for (int c = 0; c < 4; c++) acc += v[c];
    }
    return acc;
}

template <uint32_t DT, int CP>
__global__ __launch_bounds__(kRouterThreads) void router_logits_kernel(const float* __restrict__ x,
                                                                       const uint8_t* __restrict__ w,
                                                                       uint64_t row_bytes, uint32_t dim,
                                                                       uint32_t n_experts, uint32_t rows,
                                                                       float* __restrict__ logits,
                                                                       const float* __restrict__ nw, float eps,
                                                                       float* __restrict__ h_out) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float router_smem[];
    float* xs = router_smem;
    uint8_t* ws = (uint8_t*)(router_smem + ((dim + 3) & ~3u));
    const uint32_t t = blockIdx.x, e0 = blockIdx.y * rows;
    const uint32_t nr = min(rows, n_experts - e0);
    if constexpr (DT == DS5_DTYPE_F32 && CP == 16) {
        if (dim % 4 == 0 && ((uintptr_t)x & 15) == 0) {
            // rows and x read together (one memory latency), the products w[i]·x[i]
            // (each rounded, as dotRow rounds them) stored to LDS, then each row's
            // thread adds them in order
            const uint32_t n4 = dim / 4, total = nr * n4;
            const f32x4* g4 = (const f32x4*)(w + (uint64_t)e0 * row_bytes);
            const f32x4* xg4 = (const f32x4*)(x + (uint64_t)t * dim);
            f32x4* p4s = (f32x4*)ws;
            constexpr int kN = kRouterRowBytes / 16 / kRouterThreads;
            f32x4 wv[kN], xv[kN];
            if (nw) {  // uniform: ffn_norm first, h = (x * inv) * nw, inv in the tree order
                // the rows first, so their latency covers the norm
#pragma unroll
                for (int k = 0; k < kN; k++) {
                    const uint32_t u = threadIdx.x + kRouterThreads * k;
                    if (u < total) wv[k] = g4[u];
                }
                f32x4* xs4 = (f32x4*)xs;
                for (uint32_t c = threadIdx.x; c < n4; c += kRouterThreads) xs4[c] = xg4[c];
                __syncthreads();
                __shared__ float s_part[kTreeParts];
                __shared__ float s_inv;
                float sq = 0.0f;
                for (uint32_t i = threadIdx.x; i < dim; i += kTreeParts) sq = __builtin_fmaf(xs[i], xs[i], sq);
                const float inv = tree_rms_inv(sq, dim, eps, s_part, &s_inv);
                for (uint32_t c = threadIdx.x; c < n4; c += kRouterThreads) {
                    const f32x4 v = xs4[c], ww = ((const f32x4*)nw)[c];
                    const f32x4 hv = f32x4{v[0] * inv * ww[0], v[1] * inv * ww[1], v[2] * inv * ww[2],
                                           v[3] * inv * ww[3]};
                    xs4[c] = hv;
                    if (blockIdx.y == 0) ((f32x4*)(h_out + (uint64_t)t * dim))[c] = hv;  // for the experts
                }
                __syncthreads();
#pragma unroll
                for (int k = 0; k < kN; k++) {
                    const uint32_t u = threadIdx.x + kRouterThreads * k;
                    if (u < total) xv[k] = xs4[u % n4];
                }
            } else {
#pragma unroll
                for (int k = 0; k < kN; k++) {
                    const uint32_t u = threadIdx.x + kRouterThreads * k;
                    if (u < total) {
                        wv[k] = g4[u];
                        xv[k] = xg4[u % n4];
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < kN; k++) {
                const uint32_t u = threadIdx.x + kRouterThreads * k;
                if (u < total) p4s[u] = wv[k] * xv[k];
            }
            __syncthreads();
            if (threadIdx.x < nr)
                logits[(uint64_t)t * n_experts + e0 + threadIdx.x] = router_chain(p4s + (uint64_t)threadIdx.x * n4, n4);
            return;
        }
    }
    router_copy_rows<CP>(w + (uint64_t)e0 * row_bytes, ws, (uint64_t)nr * row_bytes);
    for (uint32_t i = threadIdx.x; i < dim; i += kRouterThreads) xs[i] = x[(uint64_t)t * dim + i];
    __syncthreads();
    if constexpr (DT == DS5_DTYPE_F32) {
        if (dim % 4 == 0) {
            // f32 rows of 4·dim bytes, 16-byte aligned in LDS. Every thread first
            // turns the rows into their products w[i]·x[i] in place (each rounded to
            // f32, as dotRow rounds them); the row's thread then only adds, in
            // element order, reading eight 16-byte chunks ahead of its adds so the
            // chain of dependent adds never waits for LDS.
            const uint32_t n4 = dim / 4;
            f32x4* w4 = (f32x4*)ws;
            const f32x4* x4 = (const f32x4*)xs;
            for (uint32_t u = threadIdx.x; u < nr * n4; u += kRouterThreads) w4[u] = w4[u] * x4[u % n4];
            __syncthreads();
            if (threadIdx.x < nr)
                logits[(uint64_t)t * n_experts + e0 + threadIdx.x] = router_chain(w4 + (uint64_t)threadIdx.x * n4, n4);
            return;
        }
    }
    if (threadIdx.x < nr) {
        const uint8_t* row = ws + (uint64_t)threadIdx.x * row_bytes;
        float acc = 0.0f;
        for (uint32_t i = 0; i < dim; i++) acc += router_w<DT, DT != DS5_DTYPE_Q8_0>(row, i) * xs[i];
        logits[(uint64_t)t * n_experts + e0 + threadIdx.x] = acc;
    }
}

// Logits for many tokens (router_logits_tile_kernel): workgroup (16 RT tokens, 16 RT
// experts) stages chunks of kRtK elements of x and of the expert rows (f16 widened
// to f32 exactly) in LDS, transposed, two chunks in turn; thread (tx, ty) keeps the
// RT x RT logits of tokens RT ty + a and experts RT tx + b, each dotRow's serial sum
// (kernels_c.zig:40-68): the product rounded, then added, in element order. The
// chains of the thread's logits interleave, so the adds' latency is covered; RT 2
// shares each LDS read among more products, RT 1 gives four times the workgroups.
constexpr uint32_t kRtK = 64;

template <uint32_t DT>
__device__ __forceinline__ f32x4 router_tile_w4(const uint8_t* row, uint32_t i) {
    if constexpr (DT == DS5_DTYPE_F32) {
        return *(const f32x4*)(row + 4 * (uint64_t)i);
    } else {
        const uint2 v = *(const uint2*)(row + 2 * (uint64_t)i);
        return f32x4{f16_bits_to_f32(v.x & 0xffffu), f16_bits_to_f32(v.x >> 16), f16_bits_to_f32(v.y & 0xffffu),
                     f16_bits_to_f32(v.y >> 16)};
    }
}

template <uint32_t DT, int RT>
__global__ __launch_bounds__(256) void router_logits_tile_kernel(const float* __restrict__ x,
                                                                 const uint8_t* __restrict__ w, uint64_t row_bytes,
                                                                 uint32_t dim, uint32_t n_tokens, uint32_t n_experts,
                                                                 float* __restrict__ logits) {
#pragma clang fp contract(off)
    constexpr uint32_t TR = 16 * RT, S = TR + 1;  // tile rows; LDS row stride (conflict-free transposed stores)
    static_assert(kRtK == 64, "staging: 16 threads of float4s per row and chunk");
    __shared__ float xs[2][kRtK * S], ws[2][kRtK * S];
    const uint32_t t0 = blockIdx.x * TR, e0 = blockIdx.y * TR;
    const uint32_t tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
    // staging unit s: tile row tid / 16 + 16 s, elements 4 (tid % 16) .. + 3 of the chunk
    const uint32_t c4 = tid % 16;
    const float* xr[RT];
    const uint8_t* wr[RT];
    f32x4 xv[RT], wv[RT];
#pragma unroll
    for (int s = 0; s < RT; s++) {
        const uint32_t r = tid / 16 + 16 * s;
        xr[s] = x + (uint64_t)min(t0 + r, n_tokens - 1) * dim;
        wr[s] = w + (uint64_t)min(e0 + r, n_experts - 1) * row_bytes;
        xv[s] = wv[s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    auto load = [&](uint32_t k0) {
        const uint32_t i = k0 + 4 * c4;
        if (i < dim) {  // dim % 4 == 0: the four elements are all inside
#pragma unroll
            for (int s = 0; s < RT; s++) {
                xv[s] = *(const f32x4*)(xr[s] + i);
                wv[s] = router_tile_w4<DT>(wr[s], i);
            }
        }
    };
    auto store = [&](int b) {
#pragma unroll
        for (int s = 0; s < RT; s++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                xs[b][(4 * c4 + j) * S + tid / 16 + 16 * s] = xv[s][j];
                ws[b][(4 * c4 + j) * S + tid / 16 + 16 * s] = wv[s][j];
            }
    };
    float acc[RT][RT];
#pragma unroll
    for (int a = 0; a < RT; a++)
#pragma unroll
        for (int b = 0; b < RT; b++) acc[a][b] = 0.0f;
    auto step = [&](const float* xb, const float* wb) {
        float xa[RT], wb_[RT];
#pragma unroll
        for (int a = 0; a < RT; a++) {
            xa[a] = xb[a];
            wb_[a] = wb[a];
        }
#pragma unroll
        for (int a = 0; a < RT; a++)
#pragma unroll
            for (int b = 0; b < RT; b++) acc[a][b] += xa[a] * wb_[b];
    };
    load(0);
    store(0);
    __syncthreads();
    const uint32_t nch = (dim + kRtK - 1) / kRtK;
    for (uint32_t c = 0; c < nch; c++) {
        const int b = c & 1;
        if (c + 1 < nch) load((c + 1) * kRtK);
        const float* xb = xs[b] + RT * ty;
        const float* wb = ws[b] + RT * tx;
        const uint32_t kc = min(kRtK, dim - c * kRtK);  // uniform
        if (kc == kRtK) {
#pragma unroll 16
            for (uint32_t i = 0; i < kRtK; i++) step(xb + i * S, wb + i * S);
        } else {
            for (uint32_t i = 0; i < kc; i++) step(xb + i * S, wb + i * S);
        }
        if (c + 1 < nch) store(b ^ 1);  // the buffer read in chunk c - 1, before the last barrier
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < RT; a++)
#pragma unroll
        for (int b = 0; b < RT; b++) {
            const uint32_t t = t0 + RT * ty + a, e = e0 + RT * tx + b;
            if (t < n_tokens && e < n_experts) logits[(uint64_t)t * n_experts + e] = acc[a][b];
        }
}

// Softmax and top-k of one token's logits (router_select_kernel, one wavefront).
__global__ __launch_bounds__(64) void router_select_kernel(const float* __restrict__ logits, uint32_t n_experts,
                                                           uint32_t top_k, uint32_t norm, uint16_t* __restrict__ out_ids,
                                                           float* __restrict__ out_w, ds5_pair* __restrict__ pairs) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float probs[];
    __shared__ float s_inv_sum;
    const uint32_t t = blockIdx.x;
    const int lane = threadIdx.x;
    // max (order-free), exp of each logit (independent), then the sum in expert
    // order by one lane, as the reference sums
    float mx = -__builtin_inff();
    for (uint32_t e = lane; e < n_experts; e += 64) mx = fmaxf(mx, logits[(uint64_t)t * n_experts + e]);
    mx = wave_allreduce(mx, OpMax{});
    for (uint32_t e = lane; e < n_experts; e += 64) probs[e] = expf(logits[(uint64_t)t * n_experts + e] - mx);
    __syncthreads();
    if (lane == 0) {
        // in expert order; 32 values read before their adds, so the adds do not
        // wait for LDS one read at a time
        float sum = 0.0f;
        uint32_t e = 0;
        if (n_experts % 4 == 0) {
            const f32x4* p4 = (const f32x4*)probs;
            for (; e + 32 <= n_experts; e += 32) {
                f32x4 v[8];
#pragma unroll
                for (int b = 0; b < 8; b++) v[b] = p4[e / 4 + b];
#pragma unroll
                for (int b = 0; b < 8; b++)
#pragma unroll
                    for (int c = 0; c < 4; c++) sum += v[b][c];
            }
        }
        for (; e < n_experts; e++) sum += probs[e];
        s_inv_sum = 1.0f / sum;
    }
    __syncthreads();
    for (uint32_t e = lane; e < n_experts; e += 64) probs[e] *= s_inv_sum;
    __syncthreads();

    // top-k: round j takes the largest untaken probability, the lower id on ties
    // (lanes scan their experts in ascending order with a strict >, as the
    // reference does; the cross-lane merge keeps that order). A probability
    // picked is overwritten with -1 (below every probability and the -1 start).
    // Every lane ends a round holding the same pick, so each keeps the running sum
    // (in pick order) and lane j keeps pick j; with top_k <= 64 the outputs are then
    // written by top_k lanes at once, with no global round trip.
    const bool in_regs = top_k <= 64;
    // With at most 256 experts each lane also keeps its probabilities (experts
    // lane, lane + 64, ...) in registers, and a round is two DPP all-reduces: the
    // largest probability, then the lowest id holding it.
    constexpr uint32_t kSelRegs = 4;
    const bool fast = in_regs && n_experts <= 64 * kSelRegs;
    float pv[kSelRegs];
#pragma unroll
    for (uint32_t m = 0; m < kSelRegs; m++) {
        const uint32_t e = lane + 64 * m;
        pv[m] = (fast && e < n_experts) ? probs[e] : -2.0f;  // -2: no expert (never beats the -1 start)
    }
    float picked = 0.0f, my_p = 0.0f;
    uint32_t my_id = 0;
    for (uint32_t j = 0; j < top_k; j++) {
        uint32_t best = 0;
        float best_p = -1.0f;
        if (fast) {
#pragma unroll
            for (uint32_t m = 0; m < kSelRegs; m++)
                if (pv[m] > best_p) {
                    best = lane + 64 * m;
                    best_p = pv[m];
                }
            const float mx = wave_allreduce(best_p, OpMax{});
            best = (uint32_t)wave_allreduce(best_p == mx ? (float)best : 3.0e38f, OpMinF{});
            best_p = mx;
#pragma unroll
            for (uint32_t m = 0; m < kSelRegs; m++)
                if (lane + 64 * m == best) pv[m] = -1.0f;  // taken
        } else {
            for (uint32_t e = lane; e < n_experts; e += 64)
                if (probs[e] > best_p) {
                    best = e;
                    best_p = probs[e];
                }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                const float op = __shfl_xor(best_p, off, 64);
                const uint32_t oe = (uint32_t)__shfl_xor((int)best, off, 64);
                if (op > best_p || (op == best_p && oe < best)) {
                    best_p = op;
                    best = oe;
                }
            }
            if (lane == 0) probs[best] = -1.0f;  // taken
        }
        if (lane == (int)(j & 63)) {
            my_id = best;
            my_p = best_p;
        }
        picked += best_p;
        if (!in_regs && lane == 0) {
            out_ids[(uint64_t)t * top_k + j] = (uint16_t)best;
            out_w[(uint64_t)t * top_k + j] = best_p;
        }
        __builtin_amdgcn_wave_barrier();
    }
    const float inv = norm ? 1.0f / picked : 1.0f;
    if (in_regs) {
        if ((uint32_t)lane < top_k) {
            const uint64_t o = (uint64_t)t * top_k + lane;
            const float wv = norm ? my_p * inv : my_p;
            out_ids[o] = (uint16_t)my_id;
            out_w[o] = wv;
            if (pairs) pairs[o] = ds5_pair{t, my_id, wv};
        }
    } else if (lane == 0) {
        for (uint32_t j = 0; j < top_k; j++) {
            const uint64_t o = (uint64_t)t * top_k + j;
            if (norm) out_w[o] *= inv;
            if (pairs) pairs[o] = ds5_pair{t, out_ids[o], out_w[o]};
        }
    }
}

// ---------------------------------------------------------------------------
// expert GEMVs
// ---------------------------------------------------------------------------

// Block b of x . row added into acc (f32 or Q8_0 rows; a Q8_0 block read as
// nine dwords from its dword floor).
template <bool Q8>
__device__ __forceinline__ float lane_block(float acc, const float* __restrict__ x, const uint8_t* __restrict__ row,
                                            const uint8_t* __restrict__ base, uint32_t b) {
    float xr[32];
    const float4* xs = (const float4*)(x + 32 * b);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 v = xs[i];
        xr[4 * i] = v.x;
        xr[4 * i + 1] = v.y;
        xr[4 * i + 2] = v.z;
        xr[4 * i + 3] = v.w;
    }
    if constexpr (Q8) {
        const uint64_t off = (uint64_t)(row - base) + (uint64_t)b * kQ8Bytes;
        const uint32_t sh = (uint32_t)off & 3u;  // base is 4-byte aligned
        const uint32_t* p = (const uint32_t*)(base + (off - sh));
        uint32_t d[9];
#pragma unroll
        for (int i = 0; i < 9; i++) d[i] = p[i];
        const Q8Block blk = q8_unpack(d, sh);
        return __builtin_fmaf(blk.scale, q8_dot(blk.q, xr), acc);
    } else {
        const float* wr = (const float*)row + 32 * b;
        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 32; i++) s[i & 3] = __builtin_fmaf(wr[i], xr[i], s[i & 3]);
        return acc + ((s[0] + s[1]) + (s[2] + s[3]));
    }
}

// This lane's share of x . row over blocks L, L + 64, ...
template <bool Q8>
__device__ __forceinline__ float lane_dot(const float* __restrict__ x, const uint8_t* __restrict__ row,
                                          const uint8_t* __restrict__ base, uint32_t k, int lane) {
    float acc = 0.0f;
    for (uint32_t b = lane; b < k / 32; b += 64) acc = lane_block<Q8>(acc, x, row, base, b);
    return acc;
}

// One wavefront per (pair, ffn row j); x rows 16-byte aligned (dim % 32 == 0).
// ffn % 32 == 0, so the 8 rows of a workgroup belong to one pair: the token's x
// is staged in LDS once per workgroup, after each lane has asked for its first
// Q8_0 blocks (one memory latency covers both).
template <bool Q8>
__global__ __launch_bounds__(kMoeWaves * 64) void moe_gate_up_kernel(const float* __restrict__ x,
                                                                     const uint8_t* __restrict__ gate,
                                                                     const uint8_t* __restrict__ up,
                                                                     const ds5_pair* __restrict__ pairs,
                                                                     float* __restrict__ h, uint32_t n_pairs,
                                                                     uint32_t dim, uint32_t ffn, uint64_t row_h,
                                                                     uint64_t stride) {
    // the arguments in one scalar round trip (before the first early exit)
    asm volatile("" ::"s"(x), "s"(gate), "s"(up), "s"(pairs), "s"(h), "s"(n_pairs), "s"(dim), "s"(ffn), "s"(row_h),
                 "s"(stride));
    extern __shared__ __attribute__((aligned(16))) float moe_xs[];
    const int lane = threadIdx.x & 63;
    const uint64_t r0 = (uint64_t)blockIdx.x * kMoeWaves, r = r0 + (threadIdx.x >> 6);
    const uint32_t p = (uint32_t)(r0 / ffn), j = (uint32_t)(r % ffn);
    const bool live = r < (uint64_t)n_pairs * ffn;  // wave-uniform
    const ds5_pair pr = pairs[p];
    const uint64_t row = (uint64_t)pr.expert * stride + (uint64_t)j * row_h;
    const uint32_t nb = dim / 32;
    uint32_t dg[9] = {}, du[9] = {};
    uint32_t shg = 0, shu = 0;
    if constexpr (Q8) {
        if (live && (uint32_t)lane < nb) {
            const uint64_t og = row + (uint64_t)lane * kQ8Bytes;  // gate and up share the row offset
            shg = (uint32_t)og & 3u;
            shu = shg;
            const uint32_t* pg = (const uint32_t*)(gate + (og - shg));
            const uint32_t* pu = (const uint32_t*)(up + (og - shu));
#pragma unroll
            for (int i = 0; i < 9; i++) dg[i] = pg[i];
#pragma unroll
            for (int i = 0; i < 9; i++) du[i] = pu[i];
        }
    }
    const f32x4* xg = (const f32x4*)(x + (uint64_t)pr.token * dim);
    f32x4* xs4 = (f32x4*)moe_xs;
    for (uint32_t u = threadIdx.x; u < dim / 4; u += kMoeWaves * 64) xs4[u] = xg[u];
    __syncthreads();
    if (!live) return;
    float g = 0.0f, uacc = 0.0f;
    uint32_t b0 = lane;
    if constexpr (Q8) {
        if ((uint32_t)lane < nb) {
            float xr[32];
            const f32x4* xb = xs4 + 8 * lane;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const f32x4 v = xb[i];
                xr[4 * i] = v[0];
                xr[4 * i + 1] = v[1];
                xr[4 * i + 2] = v[2];
                xr[4 * i + 3] = v[3];
            }
            const Q8Block bg = q8_unpack(dg, shg);
            g = __builtin_fmaf(bg.scale, q8_dot(bg.q, xr), g);
            const Q8Block bu = q8_unpack(du, shu);
            uacc = __builtin_fmaf(bu.scale, q8_dot(bu.q, xr), uacc);
        }
        b0 = lane + 64;
    }
    // the remaining blocks (all of them for f32 rows), in lane_dot's order
    for (uint32_t b = b0; b < nb; b += 64) {
        g = lane_block<Q8>(g, moe_xs, gate + row, gate, b);
        uacc = lane_block<Q8>(uacc, moe_xs, up + row, up, b);
    }
    g = wave_allreduce(g, OpAdd{});
    const float u = wave_allreduce(uacc, OpAdd{});
    if (lane == 0) h[r] = g / (1.0f + expf(-g)) * u;  // silu(g) * u, kernels_c.zig:70-72
}

// Q8_0 down rows, 8 per wavefront: lane (r, s) = (lane / 8, lane % 8) takes row r of
// `rows` (row_f bytes apart) and the blocks s, s + 8, s + 16, ... of the pair's h
// (hp), adding scale * (q . h) per block in that order with every load of a batch of
// kPer blocks in flight; then the row's 8 slots add in a fixed tree (xor 1, xor 2,
// the two quads): every lane of row r returns the row's dot product. All 64 lanes
// run the DPP moves (the loop ends uniformly after the batches).
constexpr uint32_t kDownRows = 8;
__device__ __forceinline__ float down_rows8_q8(const float* __restrict__ hp, const uint8_t* rows,
                                               const uint8_t* __restrict__ down, uint64_t row_f, uint32_t nb,
                                               int lane) {
#pragma clang fp contract(off)
    const int r = lane >> 3, s = lane & 7;
    float a = 0.0f;
    constexpr int kPer = 3;
    for (uint32_t b0 = s; b0 < nb; b0 += 8 * kPer) {
        uint32_t d[kPer][9], sh[kPer];
        float4 xv[kPer][8];
#pragma unroll
        for (int j = 0; j < kPer; j++) {
            const uint32_t bb = min(b0 + 8 * j, nb - 1);  // past the row: a valid block, not added
            const uint64_t off = (uint64_t)(rows - down) + (uint64_t)r * row_f + (uint64_t)bb * kQ8Bytes;
            sh[j] = (uint32_t)off & 3u;
            const uint32_t* pw = (const uint32_t*)(down + (off - sh[j]));
#pragma unroll
            for (int k = 0; k < 9; k++) d[j][k] = pw[k];
            const float4* xs = (const float4*)(hp + 32 * bb);
#pragma unroll
            for (int k = 0; k < 8; k++) xv[j][k] = xs[k];
        }
#pragma unroll
        for (int j = 0; j < kPer; j++) {
            if (b0 + 8 * j < nb) {
                float xr[32];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    xr[4 * k] = xv[j][k].x;
                    xr[4 * k + 1] = xv[j][k].y;
                    xr[4 * k + 2] = xv[j][k].z;
                    xr[4 * k + 3] = xv[j][k].w;
                }
                const Q8Block blk = q8_unpack(d[j], sh[j]);
                a = __builtin_fmaf(blk.scale, q8_dot(blk.q, xr), a);
            }
        }
    }
    float o = dpp_mov<0xB1>(a);  // quad_perm [1, 0, 3, 2]
    asm volatile("" : "+v"(o));
    a += o;
    o = dpp_mov<0x4E>(a);  // quad_perm [2, 3, 0, 1]
    asm volatile("" : "+v"(o));
    a += o;
    o = dpp_mov<0x141>(a);  // row_half_mirror: the other quad of the 8 lanes
    asm volatile("" : "+v"(o));
    return a + o;
}

// One wavefront per (pair, output row i); h rows 16-byte aligned (ffn % 32 == 0).
// Q8_0: one wavefront per (pair, 8 output rows), down_rows8_q8's lanes and order.
template <bool Q8>
__global__ __launch_bounds__(kMoeWaves * 64) void moe_down_kernel(const float* __restrict__ h,
                                                                  const uint8_t* __restrict__ down,
                                                                  const ds5_pair* __restrict__ pairs,
                                                                  float* __restrict__ y, uint32_t n_pairs, uint32_t dim,
                                                                  uint32_t ffn, uint64_t row_f, uint64_t stride) {
    // the arguments in one scalar round trip (before the first early exit)
    asm volatile("" ::"s"(h), "s"(down), "s"(pairs), "s"(y), "s"(n_pairs), "s"(dim), "s"(ffn), "s"(row_f),
                 "s"(stride));
    const int lane = threadIdx.x & 63;
    const uint64_t r = (uint64_t)blockIdx.x * kMoeWaves + (threadIdx.x >> 6);
    if constexpr (Q8) {  // wavefront r: rows 8 (r % (dim / 8)) .. + 7 of pair r / (dim / 8)
        const uint32_t groups = dim / kDownRows;
        if (r >= (uint64_t)n_pairs * groups) return;  // wave-uniform
        const uint32_t p = (uint32_t)(r / groups), i0 = (uint32_t)(r % groups) * kDownRows;
        const uint8_t* rows = down + (uint64_t)pairs[p].expert * stride + (uint64_t)i0 * row_f;
        const float v = down_rows8_q8(h + (uint64_t)p * ffn, rows, down, row_f, ffn / 32, lane);
        if ((lane & 7) == 0) y[(uint64_t)p * dim + i0 + (lane >> 3)] = v;
    } else {
        if (r >= (uint64_t)n_pairs * dim) return;  // wave-uniform
        const uint32_t p = (uint32_t)(r / dim), i = (uint32_t)(r % dim);
        const uint64_t row = (uint64_t)pairs[p].expert * stride + (uint64_t)i * row_f;
        const float v = wave_allreduce(lane_dot<Q8>(h + (uint64_t)p * ffn, down + row, down, ffn, lane), OpAdd{});
        if (lane == 0) y[r] = v;
    }
}

// The down GEMV and the combine in one launch: workgroup (token t, output rows
// i0 .. i0 + 7), wavefront w computing y[p][i] of those 8 rows for the token's
// pair q0 + w (+ 8, ...) with moe_down_kernel's lane layout and order (Q8_0:
// down_rows8_q8, all 64 lanes busy even when a row has fewer than 64 blocks; f32:
// one block per lane and step, the h block read once for the 8 rows), then thread
// r adding w_p * y[p][i0 + r] into out[t][i0 + r] in list order, as
// moe_combine_kernel does: bit-identical to the two launches, without the y round
// trip through memory. dim % 8 == 0.
template <bool Q8>
__global__ __launch_bounds__(kMoeWaves * 64) void moe_down_combine_kernel(
    const float* __restrict__ h, const uint8_t* __restrict__ down, const ds5_pair* __restrict__ pairs,
    const uint32_t* __restrict__ order, const uint32_t* __restrict__ offsets, uint32_t top_k, float* out,
    const float* res, uint32_t dim, uint32_t ffn, uint64_t row_f, uint64_t stride) {
#pragma clang fp contract(off)
    // the arguments in one scalar round trip (before the first early exit)
    asm volatile("" ::"s"(h), "s"(down), "s"(pairs), "s"(order), "s"(offsets), "s"(top_k), "s"(out), "s"(res),
                 "s"(dim), "s"(ffn), "s"(row_f), "s"(stride));
    __shared__ float ys[kMoeWaves][kDownRows], wts[kMoeWaves];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t groups = dim / kDownRows;
    const uint32_t t = blockIdx.x / groups, i0 = (blockIdx.x % groups) * kDownRows;
    const uint32_t q0 = offsets ? offsets[t] : t * top_k, q1 = offsets ? offsets[t + 1] : (t + 1) * top_k;
    const uint64_t o = (uint64_t)t * dim + i0 + threadIdx.x;
    if (q0 == q1) {  // no pairs (workgroup-uniform): out stays as it is, or residual + 0
        if (res && threadIdx.x < kDownRows) out[o] = res[o] + 0.0f;
        return;
    }
    const uint32_t nb = ffn / 32;
    // the sum starts from out, or from zero when the residual is added at the end
    float acc = 0.0f;
    if (!res && threadIdx.x < kDownRows) acc = out[o];
    for (uint32_t qb = q0; qb < q1; qb += kMoeWaves) {
        const uint32_t q = qb + wv;
        if (q < q1) {  // wave-uniform
            const uint32_t p = order ? order[q] : q;
            const ds5_pair pr = pairs[p];
            const uint8_t* rows = down + (uint64_t)pr.expert * stride + (uint64_t)i0 * row_f;
            const float* hp = h + (uint64_t)p * ffn;
            if constexpr (Q8) {
                const float v = down_rows8_q8(hp, rows, down, row_f, nb, lane);
                if ((lane & 7) == 0) ys[wv][lane >> 3] = v;
            } else {
                float a[kDownRows];
#pragma unroll
                for (uint32_t r = 0; r < kDownRows; r++) a[r] = 0.0f;
                for (uint32_t b = lane; b < nb; b += 64) {
                    float xr[32];
                    const float4* xs = (const float4*)(hp + 32 * b);
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        const float4 v = xs[k];
                        xr[4 * k] = v.x;
                        xr[4 * k + 1] = v.y;
                        xr[4 * k + 2] = v.z;
                        xr[4 * k + 3] = v.w;
                    }
#pragma unroll
                    for (uint32_t r = 0; r < kDownRows; r++) {
                        const float* wr = (const float*)(rows + r * row_f) + 32 * b;
                        float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int k = 0; k < 32; k++) s4[k & 3] = __builtin_fmaf(wr[k], xr[k], s4[k & 3]);
                        a[r] = a[r] + ((s4[0] + s4[1]) + (s4[2] + s4[3]));
                    }
                }
#pragma unroll
                for (uint32_t r = 0; r < kDownRows; r++) {
                    const float v = wave_allreduce(a[r], OpAdd{});
                    if (lane == 0) ys[wv][r] = v;
                }
            }
            if (lane == 0) wts[wv] = pr.weight;
        }
        __syncthreads();
        if (threadIdx.x < kDownRows) {
            const uint32_t n = min((uint32_t)kMoeWaves, q1 - qb);
            for (uint32_t w = 0; w < n; w++) acc += wts[w] * ys[w][threadIdx.x];
        }
        __syncthreads();
    }
    if (threadIdx.x < kDownRows) out[o] = res ? res[o] + acc : acc;
}

// out[t][i] += w_p * y[p][i] over token t's pairs in list order: pair q of the
// token is order[offsets[t] + q] (or t * top_k + q when offsets is null). With
// res: out = res + that sum started from zero.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ y,
                                                          const ds5_pair* __restrict__ pairs,
                                                          const uint32_t* __restrict__ order,
                                                          const uint32_t* __restrict__ offsets, uint32_t top_k,
                                                          float* out, const float* res, uint32_t n_tokens,
                                                          uint32_t dim) {
#pragma clang fp contract(off)
    // the arguments in one scalar round trip (before the first early exit)
    asm volatile("" ::"s"(y), "s"(pairs), "s"(order), "s"(offsets), "s"(top_k), "s"(out), "s"(res), "s"(n_tokens),
                 "s"(dim));
    const uint64_t id = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= (uint64_t)n_tokens * dim) return;
    const uint32_t t = (uint32_t)(id / dim), i = (uint32_t)(id % dim);
    const uint32_t q0 = offsets ? offsets[t] : t * top_k, q1 = offsets ? offsets[t + 1] : (t + 1) * top_k;
    float acc = res ? 0.0f : out[id];
    for (uint32_t q = q0; q < q1; q++) {
        const uint32_t p = order ? order[q] : q;
        acc += pairs[p].weight * y[(uint64_t)p * dim + i];
    }
    out[id] = res ? res[id] + acc : acc;
}

// moe_combine_kernel over four consecutive outputs per thread (dim % 4 == 0, y, out and
// res 16-byte aligned): the same products and adds per output, in the same order; the
// token's pair weights and product rows loaded eight pairs at a time.
__global__ __launch_bounds__(256) void moe_combine4_kernel(const float* __restrict__ y,
                                                           const ds5_pair* __restrict__ pairs,
                                                           const uint32_t* __restrict__ order,
                                                           const uint32_t* __restrict__ offsets, uint32_t top_k,
                                                           float* out, const float* res, uint32_t n_tokens,
                                                           uint32_t dim) {
#pragma clang fp contract(off)
    asm volatile("" ::"s"(y), "s"(pairs), "s"(order), "s"(offsets), "s"(top_k), "s"(out), "s"(res), "s"(n_tokens),
                 "s"(dim));
    constexpr uint32_t B = 8;
    const uint64_t id = (uint64_t)blockIdx.x * 256 + threadIdx.x;  // float4 index
    const uint32_t d4 = dim / 4;
    if (id >= (uint64_t)n_tokens * d4) return;
    const uint32_t t = (uint32_t)(id / d4), i = (uint32_t)(id % d4) * 4;
    const uint32_t q0 = offsets ? offsets[t] : t * top_k, q1 = offsets ? offsets[t + 1] : (t + 1) * top_k;
    f32x4 acc = res ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : *(const f32x4*)(out + 4 * id);
    for (uint32_t qb = q0; qb < q1; qb += B) {
        float wv[B];
        f32x4 yv[B];
#pragma unroll
        for (uint32_t u = 0; u < B; u++) {
            const uint32_t q = min(qb + u, q1 - 1);
            const uint32_t p = order ? order[q] : q;
            wv[u] = pairs[p].weight;
            yv[u] = *(const f32x4*)(y + (uint64_t)p * dim + i);
        }
#pragma unroll
        for (uint32_t u = 0; u < B; u++)
            if (qb + u < q1)
#pragma unroll
                for (int c = 0; c < 4; c++) acc[c] += wv[u] * yv[u][c];
    }
    if (res) {
        const f32x4 r = *(const f32x4*)(res + 4 * id);
#pragma unroll
        for (int c = 0; c < 4; c++) acc[c] = r[c] + acc[c];
    }
    *(f32x4*)(out + 4 * id) = acc;
}

// Serial fallback for banks the GEMV kernels cannot read (a Q8_0 view that is
// not 4-byte aligned, or that ends 2 bytes short of the dword past its last
// block): one thread per (pair, row), dotRow's order.
__device__ float serial_row_dot(const float* x, const uint8_t* row, bool q8, uint32_t k) {
#pragma clang fp contract(off)
    float acc = 0.0f;
    if (q8) {
        for (uint32_t b = 0; b < k / 32; b++) {
            const uint8_t* blk = row + (uint64_t)b * kQ8Bytes;
            const float scale = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
            for (int i = 0; i < 32; i++) acc += (scale * (float)(int8_t)blk[2 + i]) * x[32 * b + i];
        }
    } else {
        for (uint32_t i = 0; i < k; i++) {
            float wv;
            __builtin_memcpy(&wv, row + 4 * (uint64_t)i, 4);
            acc += wv * x[i];
        }
    }
    return acc;
}

__global__ __launch_bounds__(256) void moe_gate_up_serial_kernel(const float* x, const uint8_t* gate,
                                                                 const uint8_t* up, const ds5_pair* pairs, float* h,
                                                                 uint32_t n_pairs, uint32_t dim, uint32_t ffn,
                                                                 uint32_t q8, uint64_t row_h, uint64_t stride) {
#pragma clang fp contract(off)
    const uint64_t r = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= (uint64_t)n_pairs * ffn) return;
    const uint32_t p = (uint32_t)(r / ffn), j = (uint32_t)(r % ffn);
    const ds5_pair pr = pairs[p];
    const float* xr = x + (uint64_t)pr.token * dim;
    const uint64_t row = (uint64_t)pr.expert * stride + (uint64_t)j * row_h;
    const float g = serial_row_dot(xr, gate + row, q8, dim), u = serial_row_dot(xr, up + row, q8, dim);
    h[r] = g / (1.0f + expf(-g)) * u;
}

__global__ __launch_bounds__(256) void moe_down_serial_kernel(const float* h, const uint8_t* down,
                                                              const ds5_pair* pairs, float* y, uint32_t n_pairs,
                                                              uint32_t dim, uint32_t ffn, uint32_t q8, uint64_t row_f,
                                                              uint64_t stride) {
    const uint64_t r = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= (uint64_t)n_pairs * dim) return;
    const uint32_t p = (uint32_t)(r / dim), i = (uint32_t)(r % dim);
    const uint64_t row = (uint64_t)pairs[p].expert * stride + (uint64_t)i * row_f;
    y[r] = serial_row_dot(h + (uint64_t)p * ffn, down + row, q8, ffn);
}

}  // namespace

template <uint32_t DT, int CP>
static int launch_router_t(ds5_hip_ctx* ctx, const RouterLaunch& a) {
    const uint32_t rows = router_rows_per_group(a.row_bytes);
    const size_t smem = ((size_t)((a.dim + 3) & ~3u)) * sizeof(float) + (size_t)rows * a.row_bytes;
    if (smem > 131072)  // nothing is enqueued yet: the router is the first launch of its calls
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "router: dim %u needs %zu bytes of LDS (131072 at most)", a.dim, smem);
    static bool big_lds[kMaxDevices] = {};  // allow the 64 KiB of rows plus x (up to 128 KiB), once per device
    if (ctx->device >= kMaxDevices) return ds5_fail(ctx, DS5_DEVICE_FAILURE, "router: device index %d", ctx->device);
    if (!big_lds[ctx->device]) {
        if (int rc = ds5_hip_status(ctx, hipFuncSetAttribute((const void*)router_logits_kernel<DT, CP>,
                                                             hipFuncAttributeMaxDynamicSharedMemorySize, 131072),
                                    "router lds"))
            return rc;
        big_lds[ctx->device] = true;
    }
    const dim3 grid(a.n_tokens, (a.n_experts + rows - 1) / rows);
    DS5_TIMED_LAUNCH(ctx, "router_logits_kernel", (router_logits_kernel<DT, CP>), grid, dim3(kRouterThreads), smem,
                     ctx->stream, a.x, a.w, a.row_bytes, a.dim, a.n_experts, rows, a.logits, a.x_norm_w,
                     a.x_norm_eps, a.h_out);
    return ds5_after_launch(ctx, "router_logits_kernel");
}

template <uint32_t DT>
static int launch_router_dt(ds5_hip_ctx* ctx, const RouterLaunch& a) {
    const uintptr_t w = (uintptr_t)a.w;
    if ((w & 15u) == 0 && a.row_bytes % 16 == 0) return launch_router_t<DT, 16>(ctx, a);
    if ((w & 3u) == 0 && a.row_bytes % 4 == 0) return launch_router_t<DT, 4>(ctx, a);
    return launch_router_t<DT, 1>(ctx, a);
}

bool router_tiled(uint32_t w_dtype, uint32_t n_tokens, uint32_t dim, const void* x, const void* w) {
    const uintptr_t wa = (uintptr_t)w;
    return n_tokens >= kRouterTileMinTokens && dim % 4 == 0 && ((uintptr_t)x & 15u) == 0 &&
           ((w_dtype == DS5_DTYPE_F32 && (wa & 15u) == 0) || (w_dtype == DS5_DTYPE_F16 && (wa & 7u) == 0));
}

template <uint32_t DT>
static int launch_router_tile(ds5_hip_ctx* ctx, const RouterLaunch& a) {
    // RT 2 (32 x 32 tiles) once those fill the chip; else RT 1 (16 x 16), four times the workgroups
    const uint64_t wg2 = (uint64_t)((a.n_tokens + 31) / 32) * ((a.n_experts + 31) / 32);
    if (wg2 >= 256) {
        DS5_TIMED_LAUNCH(ctx, "router_logits_tile_kernel", (router_logits_tile_kernel<DT, 2>),
                         dim3((a.n_tokens + 31) / 32, (a.n_experts + 31) / 32), dim3(256), 0, ctx->stream, a.x, a.w,
                         a.row_bytes, a.dim, a.n_tokens, a.n_experts, a.logits);
    } else {
        DS5_TIMED_LAUNCH(ctx, "router_logits_tile_kernel", (router_logits_tile_kernel<DT, 1>),
                         dim3((a.n_tokens + 15) / 16, (a.n_experts + 15) / 16), dim3(256), 0, ctx->stream, a.x, a.w,
                         a.row_bytes, a.dim, a.n_tokens, a.n_experts, a.logits);
    }
    return ds5_after_launch(ctx, "router_logits_tile_kernel");
}

int launch_router(ds5_hip_ctx* ctx, const RouterLaunch& a) {
    if (a.n_tokens == 0) return DS5_OK;
    int rc;
    if (!a.x_norm_w && router_tiled(a.w_dtype, a.n_tokens, a.dim, a.x, a.w))
        rc = a.w_dtype == DS5_DTYPE_F32 ? launch_router_tile<DS5_DTYPE_F32>(ctx, a)
                                        : launch_router_tile<DS5_DTYPE_F16>(ctx, a);
    else
        rc = a.w_dtype == DS5_DTYPE_F32   ? launch_router_dt<DS5_DTYPE_F32>(ctx, a)
             : a.w_dtype == DS5_DTYPE_F16 ? launch_router_dt<DS5_DTYPE_F16>(ctx, a)
                                          : launch_router_dt<DS5_DTYPE_Q8_0>(ctx, a);
    if (rc) return rc;
    // the token's probabilities in dynamic LDS: n_experts * 4 bytes, up to 64 KiB (16384 experts)
    static bool select_lds[kMaxDevices] = {};
    if (!select_lds[ctx->device]) {
        if (int rc2 = ds5_hip_status(ctx, hipFuncSetAttribute((const void*)router_select_kernel,
                                                              hipFuncAttributeMaxDynamicSharedMemorySize, 65536),
                                     "router select lds"))
            return rc2;
        select_lds[ctx->device] = true;
    }
    DS5_TIMED_LAUNCH(ctx, "router_select_kernel", router_select_kernel, dim3(a.n_tokens), dim3(64),
                     (size_t)a.n_experts * sizeof(float), ctx->stream, a.logits, a.n_experts, a.top_k, (uint32_t)a.norm,
                     a.ids, a.weights, a.pairs);
    return ds5_after_launch(ctx, "router_select_kernel");
}

// Pairs sorted by expert, for the grouped products (one workgroup): each expert's
// pair count (LDS atomics), the exclusive scans of the counts and of their row
// tiles (tile_rows rows each), the tile table (first row, end row, expert), then every pair scattered to
// its expert's rows: perm[row] = pair, xrow[row] = its token. Rows of one expert
// land in any order (the atomics), which no result depends on: each product row
// is computed from its own x row and its expert's weights alone.
constexpr int kSortThreads = 1024;
constexpr int kSortBatch = 8;  // pairs per thread whose loads are in flight together
__global__ __launch_bounds__(kSortThreads) void moe_sort_kernel(const ds5_pair* __restrict__ pairs, uint32_t n_pairs,
                                                                uint32_t n_experts, uint32_t* __restrict__ perm,
                                                                uint32_t* __restrict__ xrow, uint4* __restrict__ tiles,
                                                                uint32_t* __restrict__ n_tiles, uint32_t tile_rows) {
    extern __shared__ uint32_t sort_smem[];
    const uint32_t E = n_experts, tid = threadIdx.x;
    uint32_t* cnt = sort_smem;           // [E]
    uint32_t* fill = cnt + E;            // [E]
    uint32_t* off = fill + E;            // [E + 1] first row of each expert
    uint32_t* toff = off + E + 1;        // [E + 1] first tile of each expert
    uint32_t* scan = toff + E + 1;       // [2 * kSortThreads]
    for (uint32_t e = tid; e < E; e += kSortThreads) cnt[e] = fill[e] = 0;
    __syncthreads();
    for (uint32_t p0 = 0; p0 < n_pairs; p0 += kSortThreads * kSortBatch) {
        uint32_t ex[kSortBatch];
#pragma unroll
        for (int u = 0; u < kSortBatch; u++) {
            const uint32_t p = p0 + tid + kSortThreads * u;
            ex[u] = p < n_pairs ? pairs[p].expert : E;
        }
#pragma unroll
        for (int u = 0; u < kSortBatch; u++)
            if (ex[u] < E) atomicAdd(&cnt[ex[u]], 1u);
    }
    __syncthreads();
    // thread tid owns experts [c0, c1): its totals, a block scan of them, then its offsets
    const uint32_t per = (E + kSortThreads - 1) / kSortThreads, c0 = min(tid * per, E), c1 = min(c0 + per, E);
    uint32_t rows = 0, tl = 0;
    for (uint32_t e = c0; e < c1; e++) {
        rows += cnt[e];
        tl += (cnt[e] + tile_rows - 1) / tile_rows;
    }
    scan[tid] = rows;
    scan[kSortThreads + tid] = tl;
    __syncthreads();
    for (uint32_t d = 1; d < kSortThreads; d <<= 1) {  // inclusive Hillis-Steele scan of both
        const uint32_t a = tid >= d ? scan[tid - d] : 0u, b = tid >= d ? scan[kSortThreads + tid - d] : 0u;
        __syncthreads();
        scan[tid] += a;
        scan[kSortThreads + tid] += b;
        __syncthreads();
    }
    uint32_t r0 = scan[tid] - rows, t0 = scan[kSortThreads + tid] - tl;
    for (uint32_t e = c0; e < c1; e++) {
        off[e] = r0;
        toff[e] = t0;
        const uint32_t nt = (cnt[e] + tile_rows - 1) / tile_rows;
        for (uint32_t t = 0; t < nt; t++) tiles[t0 + t] = uint4{r0 + tile_rows * t, r0 + cnt[e], e, 0u};
        r0 += cnt[e];
        t0 += nt;
    }
    if (tid == kSortThreads - 1) {
        off[E] = scan[tid];
        n_tiles[0] = scan[kSortThreads + tid];
    }
    __syncthreads();
    for (uint32_t p0 = 0; p0 < n_pairs; p0 += kSortThreads * kSortBatch) {
        uint32_t ex[kSortBatch], tok[kSortBatch];
#pragma unroll
        for (int u = 0; u < kSortBatch; u++) {
            const uint32_t p = p0 + tid + kSortThreads * u;
            ex[u] = p < n_pairs ? pairs[p].expert : E;
            tok[u] = p < n_pairs ? pairs[p].token : 0u;
        }
#pragma unroll
        for (int u = 0; u < kSortBatch; u++)
            if (ex[u] < E) {
                const uint32_t row = off[ex[u]] + atomicAdd(&fill[ex[u]], 1u);
                perm[row] = p0 + tid + kSortThreads * u;
                xrow[row] = tok[u];
            }
    }
}

// The combine (timed as moe_combine_kernel in either form): four outputs per thread
// where dim and the views allow it.
static int launch_combine(ds5_hip_ctx* ctx, const ExpertLaunch& a) {
    const uint64_t outs = (uint64_t)a.n_tokens * a.dim;
    const bool v4 = a.dim % 4 == 0 && (((uintptr_t)a.y | (uintptr_t)a.out | (uintptr_t)a.res) & 15u) == 0;
    if (v4) {
        DS5_TIMED_LAUNCH(ctx, "moe_combine_kernel", moe_combine4_kernel, dim3((unsigned)((outs / 4 + 255) / 256)),
                         dim3(256), 0, ctx->stream, a.y, a.pairs, a.order, a.offsets, a.top_k, a.out, a.res,
                         a.n_tokens, a.dim);
    } else {
        DS5_TIMED_LAUNCH(ctx, "moe_combine_kernel", moe_combine_kernel, dim3((unsigned)((outs + 255) / 256)),
                         dim3(256), 0, ctx->stream, a.y, a.pairs, a.order, a.offsets, a.top_k, a.out, a.res,
                         a.n_tokens, a.dim);
    }
    return ds5_after_launch(ctx, "moe_combine_kernel");
}

// The grouped experts: sort, the tokens' x rows split, gate and up products (each
// sorted row reading its token's plane row), h = silu(g) * u split, down products
// into pair order, the combine.
static int launch_experts_grouped(ds5_hip_ctx* ctx, const ExpertLaunch& a) {
    const size_t smem = ((size_t)4 * a.n_experts + 2 + 2 * kSortThreads) * sizeof(uint32_t);
    DS5_TIMED_LAUNCH(ctx, "moe_sort_kernel", moe_sort_kernel, dim3(1), dim3(kSortThreads), smem, ctx->stream,
                     a.pairs, a.n_pairs, a.n_experts, a.perm, a.xrow, a.tiles, a.n_tiles, a.tile_rows);
    if (int rc = ds5_after_launch(ctx, "moe_sort_kernel")) return rc;
    if (int rc = launch_x_split_rows(ctx, a.x, a.n_tokens, a.dim, a.xhi, a.xlo, a.xexp)) return rc;
    {
        const uint8_t* w[2] = {a.gate, a.up};
        float* out[2] = {a.h, a.u};
        const uint32_t n[2] = {a.ffn, a.ffn};
        if (int rc = launch_q8_gemm_grouped(ctx, a.xhi, a.xlo, a.xexp, a.dim, w, out, n, 2, a.tiles, a.n_tiles,
                                            a.max_tiles, a.tile_rows, a.stride_gu, a.xrow, nullptr))
            return rc;
    }
    if (int rc = launch_moe_h_split(ctx, a.h, a.u, a.n_pairs, a.ffn, a.hhi, a.hlo, a.hexp)) return rc;
    {
        const uint8_t* w[1] = {a.down};
        float* out[1] = {a.y};
        const uint32_t n[1] = {a.dim};
        if (int rc = launch_q8_gemm_grouped(ctx, a.hhi, a.hlo, a.hexp, a.ffn, w, out, n, 1, a.tiles, a.n_tiles,
                                            a.max_tiles, a.tile_rows, a.stride_d, nullptr, a.perm))
            return rc;
    }
    return launch_combine(ctx, a);
}

int launch_experts(ds5_hip_ctx* ctx, const ExpertLaunch& a) {
    if (a.n_pairs == 0 || a.n_tokens == 0) return DS5_OK;
    if (a.grouped) return launch_experts_grouped(ctx, a);
    const uint64_t gu_rows = (uint64_t)a.n_pairs * a.ffn, dn_rows = (uint64_t)a.n_pairs * a.dim;
    if (a.fast) {
        const dim3 blk(kMoeWaves * 64);
        const size_t xs_bytes = (size_t)a.dim * sizeof(float);  // the token's x, staged per gate/up workgroup
        const uint64_t dn_waves = a.q8 ? dn_rows / kDownRows : dn_rows;  // Q8_0: 8 rows per wavefront (dim % 32 == 0)
        const dim3 g1((unsigned)((gu_rows + kMoeWaves - 1) / kMoeWaves)), g2((unsigned)((dn_waves + kMoeWaves - 1) / kMoeWaves));
        const uint64_t outs = (uint64_t)a.n_tokens * a.dim;
        if (outs > 0x7fffffffu || ctx->moe_two_launch) {  // more outputs than one grid holds workgroups: down, then the combine
            if (a.q8) {
                DS5_TIMED_LAUNCH(ctx, "moe_gate_up_kernel", moe_gate_up_kernel<true>, g1, blk, xs_bytes, ctx->stream, a.x,
                                 a.gate, a.up, a.pairs, a.h, a.n_pairs, a.dim, a.ffn, a.row_h, a.stride_gu);
                if (int rc = ds5_after_launch(ctx, "moe_gate_up_kernel")) return rc;
                DS5_TIMED_LAUNCH(ctx, "moe_down_kernel", moe_down_kernel<true>, g2, blk, 0, ctx->stream, a.h, a.down,
                                 a.pairs, a.y, a.n_pairs, a.dim, a.ffn, a.row_f, a.stride_d);
            } else {
                DS5_TIMED_LAUNCH(ctx, "moe_gate_up_kernel", moe_gate_up_kernel<false>, g1, blk, xs_bytes, ctx->stream, a.x,
                                 a.gate, a.up, a.pairs, a.h, a.n_pairs, a.dim, a.ffn, a.row_h, a.stride_gu);
                if (int rc = ds5_after_launch(ctx, "moe_gate_up_kernel")) return rc;
                DS5_TIMED_LAUNCH(ctx, "moe_down_kernel", moe_down_kernel<false>, g2, blk, 0, ctx->stream, a.h, a.down,
                                 a.pairs, a.y, a.n_pairs, a.dim, a.ffn, a.row_f, a.stride_d);
            }
            if (int rc = ds5_after_launch(ctx, "moe_down_kernel")) return rc;
            return launch_combine(ctx, a);
        }
        const dim3 g3((unsigned)(outs / kDownRows));  // dim % 32 == 0 on this path
        if (a.q8) {
            DS5_TIMED_LAUNCH(ctx, "moe_gate_up_kernel", moe_gate_up_kernel<true>, g1, blk, xs_bytes, ctx->stream, a.x, a.gate,
                             a.up, a.pairs, a.h, a.n_pairs, a.dim, a.ffn, a.row_h, a.stride_gu);
            if (int rc = ds5_after_launch(ctx, "moe_gate_up_kernel")) return rc;
            DS5_TIMED_LAUNCH(ctx, "moe_down_combine_kernel", moe_down_combine_kernel<true>, g3, blk, 0, ctx->stream,
                             a.h, a.down, a.pairs, a.order, a.offsets, a.top_k, a.out, a.res, a.dim, a.ffn,
                             a.row_f, a.stride_d);
        } else {
            DS5_TIMED_LAUNCH(ctx, "moe_gate_up_kernel", moe_gate_up_kernel<false>, g1, blk, xs_bytes, ctx->stream, a.x, a.gate,
                             a.up, a.pairs, a.h, a.n_pairs, a.dim, a.ffn, a.row_h, a.stride_gu);
            if (int rc = ds5_after_launch(ctx, "moe_gate_up_kernel")) return rc;
            DS5_TIMED_LAUNCH(ctx, "moe_down_combine_kernel", moe_down_combine_kernel<false>, g3, blk, 0, ctx->stream,
                             a.h, a.down, a.pairs, a.order, a.offsets, a.top_k, a.out, a.res, a.dim, a.ffn,
                             a.row_f, a.stride_d);
        }
        return ds5_after_launch(ctx, "moe_down_combine_kernel");
    } else {
        DS5_TIMED_LAUNCH(ctx, "moe_gate_up_serial_kernel", moe_gate_up_serial_kernel,
                         dim3((unsigned)((gu_rows + 255) / 256)), dim3(256), 0, ctx->stream, a.x, a.gate, a.up, a.pairs,
                         a.h, a.n_pairs, a.dim, a.ffn, (uint32_t)a.q8, a.row_h, a.stride_gu);
        if (int rc = ds5_after_launch(ctx, "moe_gate_up_serial_kernel")) return rc;
        DS5_TIMED_LAUNCH(ctx, "moe_down_serial_kernel", moe_down_serial_kernel, dim3((unsigned)((dn_rows + 255) / 256)),
                         dim3(256), 0, ctx->stream, a.h, a.down, a.pairs, a.y, a.n_pairs, a.dim, a.ffn, (uint32_t)a.q8,
                         a.row_f, a.stride_d);
        if (int rc = ds5_after_launch(ctx, "moe_down_serial_kernel")) return rc;
    }
    return launch_combine(ctx, a);
}
