// k_norm_rope.hip -- rmsNorm, rope and kvAppend on gfx950 (the separate ops).
//
// Arithmetic follows the reference operation for operation so that results are
// bit-exact where the operations are IEEE-exact:
//   rmsNorm  kernels_a.zig:84-89 for rows of up to 256 elements: sumsq is a
//            serial f32 sum in element order, inv = 1/sqrt(sumsq/dim + eps)
//            (correctly rounded div and sqrt), o = (v*inv)*w -- one thread owns
//            a row for the sum. Longer rows: the reference GPU kernel's order
//            (kernels_a.metal:127-165), 256 strided fma partials and a halving
//            tree, then the same inv and o.
//   rope     kernels_a.zig:117-126: angle = (pos*freq_scale)*inv_freq[i] with
//            the host-built inv_freq table (std.math.pow(f32) evaluation);
//            x0' = x0*c - x1*s, x1' = x0*s + x1*c, never fused into fma.
//   kvAppend kernels_a.zig:196-211: dst = (h*max_ctx + pos + t)*head_dim, f16
//            by round-to-nearest-even conversion.
// cosf/sinf are the device library's full-range versions; they may differ
// from the host C library by an ulp.
#pragma clang fp contract(off)

#include "ds5_common.hpp"

namespace {

constexpr int kNormThreads = 256;
constexpr int kNormTile = 4096;  // floats of a block's rows staged in LDS
// Rows of at most kSerialMaxDim elements (the per-head q/k norms) take the
// reference CPU path's serial sum; longer rows (the hidden-state norms) the
// reference GPU kernel's reduction order (rms_norm_tree_kernel).
constexpr uint32_t kSerialMaxDim = kRmsSerialMaxDim;

// Rows of at most kSerialMaxDim elements: R = min(64, kNormTile / dim) rows per
// block. The block loads its R rows (contiguous in memory) with every load
// in flight, and stages each element's square (rounded on its own, as the
// reference's acc += v * v rounds the product) in LDS at a row stride of
// dim + 4 floats: rows start on 16-byte boundaries, 4 banks apart. Thread r then
// adds row r's squares in element order -- the reference's serial sum -- reading
// four at a time with the reads running ahead of the dependent adds (one LDS word
// per dependent step had made a 2048-wide row take ~25 us); then the block writes
// (v * inv) * w.
__global__ __launch_bounds__(kNormThreads) void rms_norm_rows_kernel(const float* x, const float* __restrict__ w,
                                                                     float* out, uint32_t n_rows, uint32_t dim,
                                                                     uint32_t rows_per_block, float eps) {
    __shared__ __attribute__((aligned(16))) float s_sq[kNormTile + 4 * 64];
    __shared__ float s_inv[64];
    const uint32_t row0 = blockIdx.x * rows_per_block;
    const uint32_t nr = min(rows_per_block, n_rows - row0);
    const uint32_t n = nr * dim;
    const uint32_t stride = dim + 4;
    const float* src = x + (uint64_t)row0 * dim;
    constexpr int kPer = kNormTile / kNormThreads;  // elements per thread
    float v[kPer];
#pragma unroll
    for (int k = 0; k < kPer; k++) {
        const uint32_t i = threadIdx.x + k * kNormThreads;
        v[k] = src[i < n ? i : n - 1];
    }
#pragma unroll
    for (int k = 0; k < kPer; k++) {
        const uint32_t i = threadIdx.x + k * kNormThreads;
        if (i < n) s_sq[(i / dim) * stride + i % dim] = v[k] * v[k];
    }
    __syncthreads();
    if (threadIdx.x < nr) {
        const float* row = s_sq + threadIdx.x * stride;
        float sumsq = 0.0f;
        // 32 squares per batch in two alternating register sets: a batch's reads are
        // issued before the previous batch's adds (the scheduling fences keep them
        // there), so the dependent chain never waits for LDS
        constexpr int B = 8;  // float4 per batch
        const uint32_t nb = dim / (4 * B), db = nb * 4 * B;
        float4 ba[B], bb[B];
        auto rd = [&](float4(&d)[B], uint32_t batch) {
#pragma unroll
            for (int b = 0; b < B; b++) d[b] = *(const float4*)(row + 4 * B * batch + 4 * b);
        };
        auto add = [&](const float4(&d)[B]) {
#pragma unroll
            for (int b = 0; b < B; b++) {
                sumsq += d[b].x;
                sumsq += d[b].y;
                sumsq += d[b].z;
                sumsq += d[b].w;
            }
        };
        // pairs of batches, every read unconditional (a read under a branch makes the
        // compiler's wait at the join count it as outstanding on both paths)
        const uint32_t np = nb / 2;
        if (np) rd(ba, 0);
        for (uint32_t i = 0; i < np; i++) {
            rd(bb, 2 * i + 1);
            __builtin_amdgcn_sched_barrier(0);
            add(ba);
            __builtin_amdgcn_sched_barrier(0);
            rd(ba, min(2 * i + 2, 2 * np - 1));
            __builtin_amdgcn_sched_barrier(0);
            add(bb);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (nb & 1) {
            rd(ba, nb - 1);
            add(ba);
        }
        for (uint32_t j = db; j < dim; j++) sumsq += row[j];
        s_inv[threadIdx.x] = rms_inv(sumsq, (float)dim, eps);
    }
    __syncthreads();
    // out may alias x: every element of the block's rows was read above.
    float* dst = out + (uint64_t)row0 * dim;
#pragma unroll
    for (int k = 0; k < kPer; k++) {
        const uint32_t i = threadIdx.x + k * kNormThreads;
        if (i < n) {
            const uint32_t r = i / dim, c = i % dim;
            dst[i] = v[k] * s_inv[r] * w[c];
        }
    }
}

// Rows of more than kSerialMaxDim elements: the reduction order of the reference's
// GPU kernel (kernels_a.metal:127-165), whose serial CPU sum is latency-bound on a
// long row (a 2048-wide row took ~12.6 us as a chain of dependent adds). One
// workgroup of 256 threads per row: thread t accumulates the squares of elements
// t, t + 256, t + 512, ... with fused multiply-adds, then the 256 partials add in
// a halving tree, partial[t] += partial[t + s] for s = 128, 64, ..., 1 (the two
// strides that cross wavefronts through LDS, the rest by lane shifts within
// wavefront 0; tree_rms_inv, shared with the kernels that normalise a row as they
// stage it); inv = 1/sqrt(sum/dim + eps) correctly rounded, o = (v*inv)*w.
// A thread loads its elements eight at a time, every load of a batch in flight;
// the batch's last loads may fall past the row and are clamped and zeroed, and
// fma(0, 0, s) = s for the non-negative s. out may alias x: a thread writes only
// the elements it read.
constexpr int kTreeThreads = 256;
__global__ __launch_bounds__(kTreeThreads) void rms_norm_tree_kernel(const float* x, const float* __restrict__ w,
                                                                     float* out, uint32_t dim, float eps) {
    __shared__ float s_part[kTreeParts];
    __shared__ float s_inv;
    static_assert(kTreeThreads == kTreeParts, "one partial per thread");
    constexpr int B = 8;
    const uint32_t t = threadIdx.x;
    const float* xr = x + (uint64_t)blockIdx.x * dim;
    float s = 0.0f;
    for (uint32_t i0 = t; i0 < dim; i0 += B * kTreeThreads) {
        float v[B];
#pragma unroll
        for (int j = 0; j < B; j++) {
            const uint32_t i = i0 + j * kTreeThreads;
            v[j] = xr[i < dim ? i : dim - 1];
            v[j] = i < dim ? v[j] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < B; j++) s = __builtin_fmaf(v[j], v[j], s);
    }
    const float inv = tree_rms_inv(s, dim, eps, s_part, &s_inv);
    float* orow = out + (uint64_t)blockIdx.x * dim;
    for (uint32_t i = t; i < dim; i += kTreeThreads) orow[i] = xr[i] * inv * w[i];
}

// One block per token group: the token's cos/sin (one per pair index, shared by
// all heads) go to LDS first, then every head's pairs rotate.
constexpr int kRopeThreads = 256;
constexpr int kRopeHalfMax = DS5_MAX_ROPE_HALF;

__global__ __launch_bounds__(kRopeThreads) void rope_kernel(float* x, const int32_t* __restrict__ positions,
                                                            uint32_t n_tokens, uint32_t n_heads, uint32_t head_dim,
                                                            float freq_scale, RopeTable table) {
    // the arguments in one scalar round trip (before the first early exit)
    asm volatile("" ::"s"(x), "s"(positions), "s"(n_tokens), "s"(n_heads), "s"(head_dim), "s"(freq_scale));
    __shared__ float s_cos[kRopeHalfMax], s_sin[kRopeHalfMax];
    const uint32_t half = head_dim / 2;
    for (uint32_t t = blockIdx.x; t < n_tokens; t += gridDim.x) {
        const float pos = (float)positions[t];
        for (uint32_t i = threadIdx.x; i < half; i += kRopeThreads) {
            const float angle = pos * freq_scale * table.inv[i];
            s_cos[i] = cosf(angle);
            s_sin[i] = sinf(angle);
        }
        __syncthreads();
        float* tok = x + (uint64_t)t * n_heads * head_dim;
        for (uint32_t j = threadIdx.x; j < n_heads * half; j += kRopeThreads) {
            const uint32_t h = j / half, i = j % half;
            float* head = tok + (uint64_t)h * head_dim;
            const float c = s_cos[i], s = s_sin[i];
            const float x0 = head[i];
            const float x1 = head[i + half];
            head[i] = x0 * c - x1 * s;
            head[i + half] = x0 * s + x1 * c;
        }
        __syncthreads();
    }
}

template <typename T>
__device__ inline T to_cache(float v);
template <>
__device__ inline float to_cache<float>(float v) {
    return v;
}
template <>
__device__ inline f16 to_cache<f16>(float v) {
    return (f16)v;  // v_cvt_f16_f32: round to nearest even
}

template <typename T>
__global__ __launch_bounds__(256) void kv_append_kernel(const float* __restrict__ k_new,
                                                        const float* __restrict__ v_new, T* k_cache, T* v_cache,
                                                        uint32_t pos, uint32_t n_tokens, uint32_t n_kv_heads,
                                                        uint32_t head_dim, uint32_t max_ctx) {
    // the arguments in one scalar round trip (before the first early exit)
    asm volatile("" ::"s"(k_new), "s"(v_new), "s"(k_cache), "s"(v_cache), "s"(pos), "s"(n_tokens), "s"(n_kv_heads),
                 "s"(head_dim), "s"(max_ctx), "s"(gridDim.x));
    const uint64_t total = (uint64_t)n_tokens * n_kv_heads * head_dim;
    for (uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (uint64_t)gridDim.x * 256) {
        const uint32_t d = idx % head_dim;
        const uint64_t th = idx / head_dim;
        const uint32_t h = th % n_kv_heads;
        const uint32_t t = th / n_kv_heads;
        const uint64_t dst = ((uint64_t)h * max_ctx + pos + t) * head_dim + d;
        k_cache[dst] = to_cache<T>(k_new[idx]);
        v_cache[dst] = to_cache<T>(v_new[idx]);
    }
}

inline uint32_t grid_for(uint64_t total, uint32_t block) {
    const uint64_t g = (total + block - 1) / block;
    return (uint32_t)(g > 65535u * 16u ? 65535u * 16u : (g ? g : 1));
}

}  // namespace

int launch_rms_norm(ds5_hip_ctx* ctx, const RmsNormLaunch& a) {
    if (a.n_rows == 0) return DS5_OK;
    if (a.dim <= kSerialMaxDim) {
        const uint32_t rpb = std::min<uint32_t>(64, kNormTile / a.dim);
        const uint32_t blocks = (a.n_rows + rpb - 1) / rpb;
        DS5_TIMED_LAUNCH(ctx, "rms_norm_rows_kernel", rms_norm_rows_kernel, dim3(blocks), dim3(kNormThreads), 0,
                         ctx->stream, a.x, a.w, a.out, a.n_rows, a.dim, rpb, a.eps);
        return ds5_after_launch(ctx, "rms_norm_rows_kernel");
    }
    DS5_TIMED_LAUNCH(ctx, "rms_norm_tree_kernel", rms_norm_tree_kernel, dim3(a.n_rows), dim3(kTreeThreads), 0,
                     ctx->stream, a.x, a.w, a.out, a.dim, a.eps);
    return ds5_after_launch(ctx, "rms_norm_tree_kernel");
}

int launch_rope(ds5_hip_ctx* ctx, const RopeLaunch& a) {
    const uint64_t total = (uint64_t)a.n_tokens * a.n_heads * (a.head_dim / 2);
    if (total == 0) return DS5_OK;
    const uint32_t blocks = std::min<uint32_t>(a.n_tokens, 65535u * 16u);
    DS5_TIMED_LAUNCH(ctx, "rope_kernel", rope_kernel, dim3(blocks), dim3(kRopeThreads), 0, ctx->stream, a.x, a.positions,
                     a.n_tokens, a.n_heads, a.head_dim, a.freq_scale, *a.table);
    return ds5_after_launch(ctx, "rope_kernel");
}

int launch_kv_append(ds5_hip_ctx* ctx, const KvAppendLaunch& a) {
    const uint64_t total = (uint64_t)a.n_tokens * a.n_kv_heads * a.head_dim;
    if (total == 0) return DS5_OK;
    const dim3 grid(grid_for(total, 256));
    if (a.kv_dtype == DS5_DTYPE_F16) {
        DS5_TIMED_LAUNCH(ctx, "kv_append_kernel", kv_append_kernel<f16>, grid, dim3(256), 0, ctx->stream, a.k_new, a.v_new,
                           (f16*)a.k_cache, (f16*)a.v_cache, a.pos, a.n_tokens, a.n_kv_heads, a.head_dim,
                           a.max_ctx);
    } else {
        DS5_TIMED_LAUNCH(ctx, "kv_append_kernel", kv_append_kernel<float>, grid, dim3(256), 0, ctx->stream, a.k_new, a.v_new,
                           (float*)a.k_cache, (float*)a.v_cache, a.pos, a.n_tokens, a.n_kv_heads, a.head_dim,
                           a.max_ctx);
    }
    return ds5_after_launch(ctx, "kv_append_kernel");
}
