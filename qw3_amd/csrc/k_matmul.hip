// k_matmul.hip -- the projection matmul of the step before the attention path:
// out[m, n] = x[m, k] . W^T, W a GGUF-layout weight of n rows of k elements in
// f32 or Q8_0 (34-byte blocks: an f16 scale, then 32 int8; value = f32(scale) * q).
//
// Semantics: kernels_a.zig:136-163 (matmul) and :39-62 (dotRow). The reference
// sums each output serially in k order; here each output is a fixed-order tree
// of per-block partial sums (scale * sum_i q_i x_i per block, then a wavefront
// reduction), so results agree to rounding, not bit for bit.
//
// Decode-shaped products (m = a few tokens) are weight-bandwidth bound: every
// weight byte is read once per pass of up to MT tokens. matmul_rows_kernel
// gives each wavefront one weight row: lane L owns the 32-element blocks
// b = L + 64 j of the row (a 2048-wide Q8_0 row, 64 blocks, is one load sweep),
// and the wavefront reduces the row's partial sums. The workgroup (8 rows)
// stages the pass's x once in LDS: read per wavefront from L2 instead, x costs
// as many bytes as the weights themselves. Q8_0 blocks are only 2-byte aligned:
// a lane reads the nine dwords covering its block from the dword boundary below
// it and realigns the bytes in registers.
#include "ds5_common.hpp"

namespace {

constexpr int kMmThreads = 512;  // 8 wavefronts, one weight row each
constexpr int kQ8Bytes = 34;     // Q8_0 block: f16 scale + 32 x int8

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// The 32 int8 of a Q8_0 block as 8 dwords plus its f32 scale, from the nine
// dwords d[0..8] read at (block offset & ~3); sh = block offset & 3 (0 or 2).
// Both cases run the same instructions: a per-lane byte-permute selector picks
// bytes 2..5 (sh = 0) or 4..7 (sh = 2) of each dword pair.
struct Q8Block {
    uint32_t q[8];
    float scale;
};

__device__ __forceinline__ Q8Block q8_unpack(const uint32_t (&d)[9], uint32_t sh) {
    Q8Block r;
    r.scale = f16_bits_to_f32((d[0] >> (8 * sh)) & 0xffffu);
    const uint32_t sel = sh ? 0x07060504u : 0x05040302u;
#pragma unroll
    for (int i = 0; i < 8; i++) r.q[i] = __builtin_amdgcn_perm(d[i + 1], d[i], sel);
    return r;
}

// sum_i q_i * x_i over one block (four interleaved partial sums)
__device__ __forceinline__ float q8_dot(const uint32_t (&q)[8], const float (&x)[32]) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int v = (int)(int8_t)(q[i] >> (8 * e));  // sign-extended byte e
            s[e] = __builtin_fmaf((float)v, x[4 * i + e], s[e]);
        }
    return (s[0] + s[1]) + (s[2] + s[3]);
}

// MT tokens per pass, JB blocks per lane (k <= 2048 * JB).
// Launch: grid.x = ceil(n / 8), one pass of tokens m0..m0+MT-1. Rows past n
// (last workgroup) load row n - 1 and store nothing: every wavefront reaches
// the barrier.
template <int MT, int JB, bool Q8>
__global__ __launch_bounds__(kMmThreads) void matmul_rows_kernel(const float* __restrict__ x, const uint8_t* __restrict__ w,
                                                                 float* __restrict__ out, uint32_t m, uint32_t n,
                                                                 uint32_t k, uint32_t m0) {
    // x in LDS: float4 chunk i of block b of token t at t * kXChunks + 8 b + (i ^ (b & 7)),
    // so the 16-byte reads of 8 consecutive lanes (one block each) hit distinct banks
    constexpr int kXChunks = JB * 512;                                  // float4 chunks of one token's x
    constexpr int kXPer = (kXChunks + kMmThreads - 1) / kMmThreads;     // chunks each thread stages
    __shared__ float4 xs[MT * kXChunks];

    const int lane = threadIdx.x & 63;
    const uint32_t row = min(blockIdx.x * (kMmThreads / 64) + (threadIdx.x >> 6), n - 1);
    const uint32_t nb = k / 32, kc = k / 4;
    const uint64_t row_bytes = Q8 ? (uint64_t)nb * kQ8Bytes : (uint64_t)k * 4;
    const uint32_t mt = min((uint32_t)MT, m - m0);

    // 1. this thread's share of x (tokens past mt re-read token mt - 1; never stored)
    float4 xv[MT][kXPer];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int u = 0; u < kXPer; u++) {
            const uint32_t e = min(threadIdx.x + (uint32_t)kMmThreads * u, kc - 1);
            xv[t][u] = ((const float4*)x)[(uint64_t)(m0 + min((uint32_t)t, mt - 1)) * kc + e];
        }

    // 2. the row's weights, all in flight before x is needed (loads complete in
    //    issue order, so staging x waits for x alone)
    constexpr int kWDw = Q8 ? 9 : 32;  // dwords per lane and block
    uint32_t d[JB][kWDw];
    uint32_t sh[JB];
#pragma unroll
    for (int j = 0; j < JB; j++) {
        const uint32_t b = min(lane + 64u * j, nb - 1);
        if constexpr (Q8) {
            // byte offset from w (w is 4-byte aligned, so offset & 3 is the block's)
            const uint64_t off = row * row_bytes + (uint64_t)b * kQ8Bytes;
            sh[j] = (uint32_t)off & 3u;
            const uint32_t* p = (const uint32_t*)(w + (off - sh[j]));
#pragma unroll
            for (int i = 0; i < 9; i++) d[j][i] = p[i];
        } else {
            const uint4* p = (const uint4*)(w + row * row_bytes + (uint64_t)b * 128);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint4 v = p[i];
                d[j][4 * i] = v.x;
                d[j][4 * i + 1] = v.y;
                d[j][4 * i + 2] = v.z;
                d[j][4 * i + 3] = v.w;
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 3. stage x, then each lane takes the x of its blocks
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int u = 0; u < kXPer; u++) {
            const uint32_t e = threadIdx.x + (uint32_t)kMmThreads * u;
            if (e < kc) xs[t * kXChunks + (e & ~7u) + ((e & 7u) ^ ((e >> 3) & 7u))] = xv[t][u];
        }
    __syncthreads();

    // 4. per-block partial sums (x of the lane's block read from LDS just before
    //    use), then the wavefront's fixed-order reduction
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = 0.0f;
#pragma unroll
    for (int j = 0; j < JB; j++) {
        const uint32_t b = min(lane + 64u * j, nb - 1);
        float xr[MT][32];
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 v = xs[t * kXChunks + 8 * b + (i ^ (b & 7))];
                xr[t][4 * i] = v.x;
                xr[t][4 * i + 1] = v.y;
                xr[t][4 * i + 2] = v.z;
                xr[t][4 * i + 3] = v.w;
            }
        if (lane + 64u * j >= nb) continue;
        if constexpr (Q8) {
            const Q8Block blk = q8_unpack(d[j], sh[j]);
#pragma unroll
            for (int t = 0; t < MT; t++) acc[t] = __builtin_fmaf(blk.scale, q8_dot(blk.q, xr[t]), acc[t]);
        } else {
#pragma unroll
            for (int t = 0; t < MT; t++) {
                float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int i = 0; i < 32; i++)
                    s[i & 3] = __builtin_fmaf(__builtin_bit_cast(float, d[j][i]), xr[t][i], s[i & 3]);
                acc[t] += (s[0] + s[1]) + (s[2] + s[3]);
            }
        }
    }
    const bool live = blockIdx.x * (kMmThreads / 64) + (threadIdx.x >> 6) < n;
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const float v = wave_allreduce(acc[t], OpAdd{});
        if (lane == 0 && live && (uint32_t)t < mt) out[(uint64_t)(m0 + t) * n + row] = v;
    }
}

// Any shape or alignment: one thread per output in the reference's serial order
// with every product and sum rounded on its own (bit-identical to dotRow).
__global__ __launch_bounds__(kMmThreads) void matmul_generic_kernel(const float* __restrict__ x, const uint8_t* __restrict__ w,
                                                                    uint32_t q8, float* __restrict__ out, uint32_t m,
                                                                    uint32_t n, uint32_t k) {
#pragma clang fp contract(off)
    const uint64_t i = (uint64_t)blockIdx.x * kMmThreads + threadIdx.x;
    if (i >= (uint64_t)m * n) return;
    const uint64_t mi = i / n, ni = i % n;
    const float* xr = x + mi * k;
    float acc = 0.0f;
    if (q8) {
        const uint8_t* row = w + ni * ((uint64_t)k / 32 * kQ8Bytes);
        for (uint32_t b = 0; b < k / 32; b++) {
            const uint8_t* blk = row + (uint64_t)b * kQ8Bytes;
            const float scale = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
            for (int e = 0; e < 32; e++) acc += (scale * (float)(int8_t)blk[2 + e]) * xr[32 * b + e];
        }
    } else {
        const float* row = (const float*)w + ni * k;
        for (uint32_t e = 0; e < k; e++) acc += row[e] * xr[e];
    }
    out[i] = acc;
}

template <int MT, int JB, bool Q8>
int launch_rows(ds5_hip_ctx* ctx, const MatmulLaunch& a, uint32_t m0) {
    const uint32_t rows_per_block = kMmThreads / 64;
    const dim3 grid((a.n + rows_per_block - 1) / rows_per_block);
    DS5_TIMED_LAUNCH(ctx, "matmul_rows_kernel", (matmul_rows_kernel<MT, JB, Q8>), grid, dim3(kMmThreads), 0, ctx->stream,
                     a.x, a.w, a.out, a.m, a.n, a.k, m0);
    return ds5_after_launch(ctx, "matmul_rows_kernel");
}

// Tokens per pass: up to 4 / JB (the x registers hold MT * JB * 32 floats per lane),
// and no more than the tokens there are (a 1-token decode runs MT = 1).
template <int JB, bool Q8>
int launch_passes(ds5_hip_ctx* ctx, const MatmulLaunch& a) {
    constexpr uint32_t kMaxMt = 4 / JB;
    const uint32_t mt = a.m >= kMaxMt ? kMaxMt : (a.m >= 2 ? 2 : 1);
    for (uint32_t m0 = 0; m0 < a.m; m0 += mt) {
        int rc;
        if (mt == 4)
            rc = launch_rows<(kMaxMt >= 4 ? 4 : 1), JB, Q8>(ctx, a, m0);
        else if (mt == 2)
            rc = launch_rows<(kMaxMt >= 2 ? 2 : 1), JB, Q8>(ctx, a, m0);
        else
            rc = launch_rows<1, JB, Q8>(ctx, a, m0);
        if (rc) return rc;
    }
    return DS5_OK;
}

template <bool Q8>
int launch_rows_q(ds5_hip_ctx* ctx, const MatmulLaunch& a) {
    const uint32_t nb = a.k / 32;
    if (nb <= 64) return launch_passes<1, Q8>(ctx, a);
    if (nb <= 128) return launch_passes<2, Q8>(ctx, a);
    return launch_passes<4, Q8>(ctx, a);
}

}  // namespace

// The row kernel needs x and out 16-byte aligned, k <= 8192, and f32 weights 16-byte
// aligned or Q8_0 weights 4-byte aligned. A Q8_0 block is read as the nine dwords
// from the dword boundary at or below it, which ends 2 bytes past the block when
// the block starts on a dword boundary; for the last block that stays inside the
// view only if the weights end on a dword boundary or the view has 2 more bytes.
bool matmul_rows_supported(const MatmulLaunch& a, uintptr_t x_addr, uintptr_t out_addr, uintptr_t w_addr,
                           uint64_t w_len) {
    if (a.k % 32 != 0 || a.k / 32 > 256 || (x_addr & 15u) || (out_addr & 15u)) return false;
    if (!a.q8) return (w_addr & 15u) == 0;
    const uint64_t end = (uint64_t)a.n * (a.k / 32) * kQ8Bytes;
    return (w_addr & 3u) == 0 && ((w_addr + end) % 4 == 0 || w_len >= end + 2);
}

int launch_matmul(ds5_hip_ctx* ctx, const MatmulLaunch& a, bool rows_path) {
    if (a.m == 0 || a.n == 0) return DS5_OK;
    if (rows_path) return a.q8 ? launch_rows_q<true>(ctx, a) : launch_rows_q<false>(ctx, a);
    const uint64_t total = (uint64_t)a.m * a.n;
    const dim3 grid((unsigned)((total + kMmThreads - 1) / kMmThreads));
    DS5_TIMED_LAUNCH(ctx, "matmul_generic_kernel", matmul_generic_kernel, grid, dim3(kMmThreads), 0, ctx->stream, a.x,
                     a.w, (uint32_t)a.q8, a.out, a.m, a.n, a.k);
    return ds5_after_launch(ctx, "matmul_generic_kernel");
}
