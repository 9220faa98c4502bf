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
// streams whole weight rows: lane L of a wavefront owns the 32-element blocks
// b = L + 64 j of every row (so a 2048-wide Q8_0 row, 64 blocks, is one load
// sweep of the wavefront), keeps the x values of its blocks in registers for
// all rows, and the wavefront reduces each row's partial sums. Q8_0 blocks are
// only 2-byte aligned: a lane reads the nine dwords covering its block from
// the dword boundary below it and realigns the bytes in registers.
#include "ds5_common.hpp"

namespace {

constexpr int kMmThreads = 256;  // 4 wavefronts
constexpr int kQ8Bytes = 34;     // Q8_0 block: f16 scale + 32 x int8

// Rows one wavefront streams, all loads of a row group issued before use.
template <bool Q8>
constexpr int rows_per_wave() { return Q8 ? 2 : 1; }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// The 32 int8 of a Q8_0 block as 8 dwords plus its f32 scale, from the nine
// dwords d[0..8] read at (block address & ~3); sh = block address & 3 (0 or 2).
struct Q8Block {
    uint32_t q[8];
    float scale;
};

__device__ __forceinline__ Q8Block q8_unpack(const uint32_t (&d)[9], uint32_t sh) {
    Q8Block r;
    if (sh == 0) {  // scale in d[0] bits 0-15, q bytes start at byte 2
        r.scale = f16_bits_to_f32(d[0] & 0xffffu);
#pragma unroll
        for (int i = 0; i < 8; i++) r.q[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], 2);
    } else {        // scale in d[0] bits 16-31, q bytes are d[1..8]
        r.scale = f16_bits_to_f32(d[0] >> 16);
#pragma unroll
        for (int i = 0; i < 8; i++) r.q[i] = d[i + 1];
    }
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

// MT tokens per pass (x in registers), JB blocks per lane (k <= 2048 * JB).
// Launch: grid.x = ceil(n / (4 * rows_per_wave)), one pass of tokens m0..m0+MT-1.
template <int MT, int JB, bool Q8>
__global__ __launch_bounds__(kMmThreads) void matmul_rows_kernel(const float* __restrict__ x, const uint8_t* __restrict__ w,
                                                                 float* __restrict__ out, uint32_t m, uint32_t n,
                                                                 uint32_t k, uint32_t m0) {
    constexpr int RPW = rows_per_wave<Q8>();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nb = k / 32;
    const uint64_t row_bytes = Q8 ? (uint64_t)nb * kQ8Bytes : (uint64_t)k * 4;
    const uint32_t mt = min((uint32_t)MT, m - m0);

    // x of this lane's blocks for the pass's tokens (zero past the block count)
    float xr[JB][MT][32];
#pragma unroll
    for (int j = 0; j < JB; j++) {
        const uint32_t b = lane + 64 * j;
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const bool ok = b < nb && (uint32_t)t < mt;
            const float4* src = (const float4*)(x + (uint64_t)(m0 + (ok ? t : 0)) * k + 32 * (ok ? b : 0));
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 v = ok ? src[i] : float4{0.f, 0.f, 0.f, 0.f};
                xr[j][t][4 * i] = v.x;
                xr[j][t][4 * i + 1] = v.y;
                xr[j][t][4 * i + 2] = v.z;
                xr[j][t][4 * i + 3] = v.w;
            }
        }
    }

    const uint32_t row0 = (blockIdx.x * (kMmThreads / 64) + wave) * RPW;
    if (row0 >= n) return;  // wave-uniform
    float acc[RPW][MT];
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int t = 0; t < MT; t++) acc[r][t] = 0.0f;

    if constexpr (Q8) {
        // all loads of the row group first: nine dwords per (row, block)
        uint32_t d[RPW][JB][9];
        uint32_t sh[RPW][JB];
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int j = 0; j < JB; j++) {
                const uint32_t row = min(row0 + r, n - 1);
                const uint32_t b = min(lane + 64u * j, nb - 1);
                const uintptr_t addr = (uintptr_t)(w + row * row_bytes + (uint64_t)b * kQ8Bytes);
                sh[r][j] = (uint32_t)(addr & 3u);
                const uint32_t* p = (const uint32_t*)(addr - sh[r][j]);
#pragma unroll
                for (int i = 0; i < 9; i++) d[r][j][i] = p[i];
            }
#pragma unroll
        for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int j = 0; j < JB; j++) {
                if (lane + 64u * j >= nb) continue;
                const Q8Block blk = q8_unpack(d[r][j], sh[r][j]);
#pragma unroll
                for (int t = 0; t < MT; t++) acc[r][t] = __builtin_fmaf(blk.scale, q8_dot(blk.q, xr[j][t]), acc[r][t]);
            }
    } else {
        float4 wv[JB][8];
#pragma unroll
        for (int j = 0; j < JB; j++) {
            const uint32_t b = min(lane + 64u * j, nb - 1);
            const float4* p = (const float4*)(w + row0 * row_bytes + (uint64_t)b * 128);
#pragma unroll
            for (int i = 0; i < 8; i++) wv[j][i] = p[i];
        }
#pragma unroll
        for (int j = 0; j < JB; j++) {
            if (lane + 64u * j >= nb) continue;
#pragma unroll
            for (int t = 0; t < MT; t++) {
                float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    s[0] = __builtin_fmaf(wv[j][i].x, xr[j][t][4 * i], s[0]);
                    s[1] = __builtin_fmaf(wv[j][i].y, xr[j][t][4 * i + 1], s[1]);
                    s[2] = __builtin_fmaf(wv[j][i].z, xr[j][t][4 * i + 2], s[2]);
                    s[3] = __builtin_fmaf(wv[j][i].w, xr[j][t][4 * i + 3], s[3]);
                }
                acc[0][t] += (s[0] + s[1]) + (s[2] + s[3]);
            }
        }
    }

#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const uint32_t row = row0 + r;
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const float v = wave_allreduce(acc[r][t], OpAdd{});
            if (lane == 0 && row < n && (uint32_t)t < mt) out[(uint64_t)(m0 + t) * n + row] = v;
        }
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
    const uint32_t rows_per_block = (kMmThreads / 64) * rows_per_wave<Q8>();
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
