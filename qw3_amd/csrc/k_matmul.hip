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


// Up to kMatmulGroupMax weight matrices sharing x, in one launch: entry e owns
// the workgroups (row kernel) or column tiles (GEMM) [wg0[e], wg0[e + 1]).
struct WeightGroup {
    const uint8_t* w[kMatmulGroupMax];
    float* out[kMatmulGroupMax];
    const float* res[kMatmulGroupMax];  // residual added to out (nullptr: none)
    uint32_t n[kMatmulGroupMax];
    uint32_t wg0[kMatmulGroupMax];
    uint32_t count;
};

// Every field of a group in one scalar round trip: the entry selection below
// would otherwise load each entry's fields only after testing the previous
// entry (a chain of dependent argument loads before the first memory access).
#define DS5_GROUP_ARGS(g) \
    "s"((g).w[0]), "s"((g).w[1]), "s"((g).w[2]), "s"((g).w[3]), "s"((g).out[0]), "s"((g).out[1]), "s"((g).out[2]), \
        "s"((g).out[3]), "s"((g).res[0]), "s"((g).res[1]), "s"((g).res[2]), "s"((g).res[3]), "s"((g).n[0]), \
        "s"((g).n[1]), "s"((g).n[2]), "s"((g).n[3]), "s"((g).wg0[0]), "s"((g).wg0[1]), "s"((g).wg0[2]), \
        "s"((g).wg0[3]), "s"((g).count)
static_assert(kMatmulGroupMax == 4, "DS5_GROUP_ARGS lists four entries");

// MT tokens per pass, JB blocks per lane (k <= 2048 * JB).
// Launch: grid.x = sum of ceil(n[e] / 8), one pass of tokens m0..m0+MT-1. Rows
// past n (an entry's last workgroup) load row n - 1 and store nothing: every
// wavefront reaches the barrier.
// NORM: x is first normalised, x' = (x * inv) * nw with inv of the reference GPU
// kernel's tree order (tree_rms_inv; rows of more than 256 elements), as the
// workgroup stages it: ds5_hip_rms_norm then the product, bit for bit, with the
// norm worked out while the weights are in flight.
template <int MT, int JB, bool Q8, bool NORM>
__global__ __launch_bounds__(kMmThreads) void matmul_rows_kernel(const float* __restrict__ x, const WeightGroup g,
                                                                 uint32_t m, uint32_t k, uint32_t m0,
                                                                 const float* __restrict__ nw, float eps) {
    // this workgroup's entry (uniform; selected without indexing the argument arrays,
    // with selects rather than branches so that every field loads in one round trip)
    // (out may be the residual itself: each output is read, then written, by one lane)
    const uint8_t* __restrict__ w = g.w[0];
    float* out = g.out[0];
    const float* res = g.res[0];
    uint32_t n = g.n[0], wg = blockIdx.x;
#pragma unroll
    for (int e = 1; e < kMatmulGroupMax; e++) {
        const bool take = (uint32_t)e < g.count && blockIdx.x >= g.wg0[e];
        w = take ? g.w[e] : w;
        out = take ? g.out[e] : out;
        res = take ? g.res[e] : res;
        n = take ? g.n[e] : n;
        wg = take ? blockIdx.x - g.wg0[e] : wg;
    }

    // x in LDS: float4 chunk i of block b of token t at t * kXChunks + 8 b + (i ^ (b & 7)),
    // so the 16-byte reads of 8 consecutive lanes (one block each) hit distinct banks
    constexpr int kXChunks = JB * 512;                                  // float4 chunks of one token's x
    constexpr int kXPer = (kXChunks + kMmThreads - 1) / kMmThreads;     // chunks each thread stages
    __shared__ float4 xs[MT * kXChunks];

    const int lane = threadIdx.x & 63;
    const uint32_t row = min(wg * (kMmThreads / 64) + (threadIdx.x >> 6), n - 1);
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
    float4 wn[NORM ? kXPer : 1];
    if constexpr (NORM) {
#pragma unroll
        for (int u = 0; u < kXPer; u++) wn[u] = ((const float4*)nw)[min(threadIdx.x + (uint32_t)kMmThreads * u, kc - 1)];
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
    auto slot = [&](int t, uint32_t e) { return t * kXChunks + (e & ~7u) + ((e & 7u) ^ ((e >> 3) & 7u)); };
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int u = 0; u < kXPer; u++) {
            const uint32_t e = threadIdx.x + (uint32_t)kMmThreads * u;
            if (e < kc) xs[slot(t, e)] = xv[t][u];
        }
    __syncthreads();
    if constexpr (NORM) {
        // each token's partials from the staged row (element i: chunk i / 4, lane i % 4),
        // the tree, then the staged row rewritten as (x * inv) * nw
        __shared__ float s_part[kTreeParts];
        __shared__ float s_inv;
        const float* xf = (const float*)xs;
#pragma unroll
        for (int t = 0; t < MT; t++) {
            float sq = 0.0f;
            if (threadIdx.x < kTreeParts)
                for (uint32_t i = threadIdx.x; i < k; i += kTreeParts) {
                    const float v = xf[4 * slot(t, i >> 2) + (i & 3)];
                    sq = __builtin_fmaf(v, v, sq);
                }
            const float inv = tree_rms_inv(sq, k, eps, s_part, &s_inv);
#pragma unroll
            for (int u = 0; u < kXPer; u++) {
                const uint32_t e = threadIdx.x + (uint32_t)kMmThreads * u;
                const float4 v = xv[t][u], ww = wn[u];
                if (e < kc)
                    xs[slot(t, e)] = float4{v.x * inv * ww.x, v.y * inv * ww.y, v.z * inv * ww.z, v.w * inv * ww.w};
            }
        }
        __syncthreads();
    }

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
    const bool live = wg * (kMmThreads / 64) + (threadIdx.x >> 6) < n;
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const float v = wave_allreduce(acc[t], OpAdd{});
        if (lane == 0 && live && (uint32_t)t < mt) {
            const uint64_t o = (uint64_t)(m0 + t) * n + row;
            out[o] = res ? res[o] + v : v;  // the reference's add(residual, proj)
        }
    }
}

// ---------------------------------------------------------------------------
// Prefill-shaped products (many tokens): Q8_0 GEMM on the f16 matrix cores.
//
// out[m, n] = sum_b scale[n, b] * sum_{e < 32} x[m, 32 b + e] * q[n, 32 b + e].
// The int8 q are exact in f16. Each x row is first scaled by a power of two,
// x' = x * 2^(14 - E) with 2^E <= max |x row| < 2^(E+1), so |x'| < 2^15 fits
// f16, and split into two f16 parts, x' = hi + lo (lo the f16 rounding of
// x' - hi): 22 significant bits, and no overflow or loss of range whatever
// the row's magnitude. Per 32-element block and 16 x 16 output tile, two
// v_mfma_f32_16x16x32_f16 (lo, then hi) into a zeroed temporary, then
// acc += scale * tmp in f32 (the scale belongs to the weight row: one per lane
// in the result layout); the epilogue undoes the row's power of two exactly.
//
// matmul_x_split_kernel writes the two planes and the row exponents into the
// context workspace; matmul_q8_mfma_kernel then only copies x tiles.
//
// GEMM workgroup: BM tokens x BN weight rows, WM x WN wavefronts, each with
// TM x TN tiles of 16 x 16. Per block the workgroup stages x (hi and lo
// planes), q (as f16) and the BN scales in LDS. The loop is bound by memory
// latency, not by the matrix cores: every load is issued two blocks before the
// block is multiplied. x goes HBM/L2 -> LDS with direct-to-LDS loads into a
// ring of three stages; each thread's 8-byte q run and its row's scale go to
// registers (three sets) and are converted to f16 into LDS one block ahead.
// One workgroup barrier per block. The loads are inline asm with explicit
// vmcnt waits (the compiler's waits would cover the later blocks' loads too).
// LDS rows are 32 halves (four 16-byte chunks) with chunk c of row r stored at
// c ^ ((r >> 2) & 3), so a 16-lane group reading one chunk of 16 rows hits 16
// distinct bank groups.
//
// MFMA operand layout (16x16x32): lane l supplies row / column l % 16 and the
// eight k of chunk l / 16; result element (4 (l / 16) + i, l % 16) is in
// register i of lane l.
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kSplitThreads = 256;
constexpr int kXExpBias = 14;  // scaled rows have max |x'| in [2^14, 2^15)

// Workspace bytes of the split x: hi and lo planes of m x k halves, m exponents.
inline size_t x_split_bytes(uint32_t m, uint32_t k) { return (size_t)m * k * 4 + (size_t)m * 4; }

// The rope angles of a prefill's tokens, made by the x split of the attention
// block's projection (one workgroup per token): cs[t] holds cos then sin of
// (pos_t * freq_scale) * inv_freq[i], i < half.
struct XSplitRope {
    const int32_t* positions;
    float* cs;
    uint32_t half;
    float freq_scale;
};

// Row `row` of the split planes from load(c) (float4 chunk c of the row's k values):
// max |v|, its exponent E, then hi / lo of v * 2^(14 - E). A row of zeros (or with a
// non-finite maximum) keeps E = 0. red: kSplitThreads / 64 floats of LDS.
template <class F>
__device__ __forceinline__ void split_row(F load, uint64_t row, uint32_t k, uint16_t* __restrict__ hi,
                                          uint16_t* __restrict__ lo, int* __restrict__ row_exp, float* red) {
    const uint32_t kc = k / 4;
    float mx = 0.0f;
    for (uint32_t c = threadIdx.x; c < kc; c += kSplitThreads) {
        const float4 v = load(c);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    mx = wave_allreduce(mx, OpMax{});
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // floor(log2 mx): frexp gives mx = f * 2^x with f in [0.5, 1)
    const int e = (mx > 0.0f && mx <= 3.4028235e38f) ? __builtin_amdgcn_frexp_expf(mx) - 1 : 0;
    const int sh = kXExpBias - e;
    if (threadIdx.x == 0) row_exp[row] = e;
    uint2* h2 = (uint2*)(hi + row * k);
    uint2* l2 = (uint2*)(lo + row * k);
    for (uint32_t c = threadIdx.x; c < kc; c += kSplitThreads) {
        const float4 v = load(c);
        const float f[4] = {v.x, v.y, v.z, v.w};
        uint32_t hb[4], lb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float s = __builtin_ldexpf(f[i], sh);
            const _Float16 h = (_Float16)s;
            hb[i] = __builtin_bit_cast(uint16_t, h);
            lb[i] = __builtin_bit_cast(uint16_t, (_Float16)(s - (float)h));
        }
        h2[c] = uint2{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16)};
        l2[c] = uint2{lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16)};
    }
}

// One workgroup per x row: split_row of x. ROPE: also the
// row's token's rope cos / sin. nw (if not null): the row is first normalised,
// x' = (x * inv) * nw with inv in the reference GPU kernel's tree order
// (tree_rms_inv), exactly as ds5_hip_rms_norm writes rows of more than 256
// elements.
template <bool ROPE>
__global__ __launch_bounds__(kSplitThreads) void matmul_x_split_kernel(const float* __restrict__ x,
                                                                       uint16_t* __restrict__ hi,
                                                                       uint16_t* __restrict__ lo,
                                                                       int* __restrict__ row_exp, uint32_t k,
                                                                       XSplitRope rope, RopeTable table,
                                                                       const float* __restrict__ nw, float eps) {
    static_assert(kSplitThreads >= kTreeParts, "one tree partial per thread");
    __shared__ float red[kSplitThreads / 64];
    __shared__ float s_part[kTreeParts];
    __shared__ float s_inv;
    const uint64_t row = blockIdx.x;
    if constexpr (ROPE) {
        const float pos = (float)rope.positions[row];
        for (uint32_t i = threadIdx.x; i < rope.half; i += kSplitThreads) {
            const float ang = qk_rope_angle(pos, rope.freq_scale, table.inv[i]);
            rope.cs[row * 2 * rope.half + i] = cosf(ang);
            rope.cs[row * 2 * rope.half + rope.half + i] = sinf(ang);
        }
    }
    const float4* xr = (const float4*)(x + row * k);
    float inv = 1.0f;
    if (nw) {  // uniform
        float sq = 0.0f;
        for (uint32_t i = threadIdx.x; i < k; i += kTreeParts) {
            const float v = x[row * k + i];
            sq = __builtin_fmaf(v, v, sq);
        }
        inv = tree_rms_inv(sq, k, eps, s_part, &s_inv);
    }
    auto load = [&](uint32_t c) {
        const float4 v = xr[c];
        if (!nw) return v;
        const float4 w = ((const float4*)nw)[c];
        return float4{v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w};
    };
    split_row(load, row, k, hi, lo, row_exp, red);
}

// The planes of a MoE layer's expert products, for rows sorted by expert: row r of
// h = silu(g) * u (kernels_c.zig:70-72, silu(v) = v / (1 + exp(-v))) from the gate
// and up products g, u [rows, k] f32, split as matmul_x_split_kernel splits x.
__global__ __launch_bounds__(kSplitThreads) void moe_h_split_kernel(const float* __restrict__ g,
                                                                   const float* __restrict__ u,
                                                                   uint16_t* __restrict__ hi,
                                                                   uint16_t* __restrict__ lo,
                                                                   int* __restrict__ row_exp, uint32_t k) {
#pragma clang fp contract(off)
    __shared__ float red[kSplitThreads / 64];
    const uint64_t row = blockIdx.x;
    const float4* gr = (const float4*)(g + row * k);
    const float4* ur = (const float4*)(u + row * k);
    auto load = [&](uint32_t c) {
        const float4 a = gr[c], b = ur[c];
        return float4{a.x / (1.0f + expf(-a.x)) * b.x, a.y / (1.0f + expf(-a.y)) * b.y,
                      a.z / (1.0f + expf(-a.z)) * b.z, a.w / (1.0f + expf(-a.w)) * b.w};
    };
    split_row(load, row, k, hi, lo, row_exp, red);
}

// The same planes, one wavefront per row (rows of k <= 256 R elements): the row's h stays
// in registers between its maximum and its split, no barrier; the arithmetic of
// split_row operation for operation.
template <int R>
__global__ __launch_bounds__(256) void moe_h_split_rows_kernel(const float* __restrict__ g,
                                                               const float* __restrict__ u,
                                                               uint16_t* __restrict__ hi, uint16_t* __restrict__ lo,
                                                               int* __restrict__ row_exp, uint32_t k, uint32_t rows) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t row = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // wavefront-uniform; the kernel has no barrier
    const uint32_t kc = k / 4;
    const float4* gr = (const float4*)(g + row * k);
    const float4* ur = (const float4*)(u + row * k);
    float4 h[R];
    float mx = 0.0f;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t c = lane + 64 * r;
        h[r] = float4{0.0f, 0.0f, 0.0f, 0.0f};
        if (c < kc) {
            const float4 a = gr[c], b = ur[c];
            h[r] = float4{a.x / (1.0f + expf(-a.x)) * b.x, a.y / (1.0f + expf(-a.y)) * b.y,
                          a.z / (1.0f + expf(-a.z)) * b.z, a.w / (1.0f + expf(-a.w)) * b.w};
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(h[r].x), fabsf(h[r].y)), fmaxf(fabsf(h[r].z), fabsf(h[r].w))));
        }
    }
    mx = wave_allreduce(mx, OpMax{});
    const int e = (mx > 0.0f && mx <= 3.4028235e38f) ? __builtin_amdgcn_frexp_expf(mx) - 1 : 0;
    const int sh = kXExpBias - e;
    if (lane == 0) row_exp[row] = e;
    uint2* h2 = (uint2*)(hi + row * k);
    uint2* l2 = (uint2*)(lo + row * k);
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t c = lane + 64 * r;
        if (c < kc) {
            const float f[4] = {h[r].x, h[r].y, h[r].z, h[r].w};
            uint32_t hb[4], lb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float s = __builtin_ldexpf(f[i], sh);
                const _Float16 hv = (_Float16)s;
                hb[i] = __builtin_bit_cast(uint16_t, hv);
                lb[i] = __builtin_bit_cast(uint16_t, (_Float16)(s - (float)hv));
            }
            h2[c] = uint2{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16)};
            l2[c] = uint2{lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16)};
        }
    }
}

// Four int8 (one dword) as four f16: bytes biased to q + 128, placed under the
// f16 pattern 0x64 (1024 + q + 128, exact), then 1152 subtracted in f16.
__device__ __forceinline__ uint2 i8x4_to_f16x4(uint32_t u) {
    const uint32_t v = u ^ 0x80808080u;
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    const h2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const h2_t a = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u)) - bias;
    const h2_t b = __builtin_bit_cast(h2_t, __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u)) - bias;
    return uint2{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)};
}

// Workgroup barrier that orders LDS only: global loads stay in flight across it.
__device__ __forceinline__ void gemm_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ uint32_t gemm_lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)p;
}

// Wave-uniform 64-bit value made explicitly scalar (an asm "s" operand).
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    return ((uint64_t)hi << 32) | (uint64_t)lo;
}

// Wait until at most N vector-memory operations of this wavefront are
// outstanding (the compiler does not count inline-asm loads).
template <int N>
__device__ __forceinline__ void wait_vm_only() {
    static_assert(N >= 0 && N < 16, "vmcnt field");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Direct-to-LDS load: 16 (DW = 4) or 4 (DW = 1) bytes per lane from base + off
// to LDS address lds + lane * 4 DW.
template <int DW>
__device__ __forceinline__ void lds_dma(uint32_t off, uint64_t base, uint32_t lds) {
    if constexpr (DW == 4)
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
                     : "m0", "memory");
    else
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(lds)
                     : "m0", "memory");
}

// EPI = 1: the attention block's q / k / v projections (entries 0, 1, 2 of the
// group), 128 x 128 tiles: a tile is 128 tokens of one head's 128 dims, and
// the epilogue turns it into what the prefill attention reads -- k: RMSNorm
// (serial sum) and rotation, f16 into the cache row pos + t of its kv head; v:
// f16 into the cache; q: RMSNorm, rotation, times q_scale, f16 into the q
// operand [t, n_q_heads, 128] -- with the arithmetic of the pre-pass (k) and of
// the attention kernel's own q operand (q) (the qk_* helpers), so the results
// equal the separate projection and step.
struct AttnPrepEpi {
    const float* q_norm;
    const float* k_norm;
    const float* cs;  // [m, 128]: cos of pairs 0..63, then sin
    f16* q16;
    f16* k_cache;
    f16* v_cache;
    uint32_t pos, n_q_heads, max_ctx;
    float eps, q_scale;
};

// GRP: the experts' products of a MoE layer over rows sorted by expert.
// Workgroup row tile y is tiles[y] = (first row, end row, expert): its rows are the
// sorted rows [first, end) (rows past the end read end - 1, a row of the same
// expert, and store nothing), its weights the expert's matrix, w + expert *
// w_stride; tiles past *count stop at once. Sorted row r reads plane row x_rows[r]
// (null: r) and its output goes to row out_rows[r] (null: r).
struct MoeGemmTiles {
    const uint4* tiles;
    const uint32_t* count;
    uint64_t w_stride;
    const uint32_t* x_rows;
    const uint32_t* out_rows;
};

template <int BM, int BN, int WM, int WN, int EPI, bool GRP = false>
__global__ __launch_bounds__(WM * WN * 64) void matmul_q8_mfma_kernel(const uint16_t* __restrict__ xhi,
                                                                      const uint16_t* __restrict__ xlo,
                                                                      const int* __restrict__ row_exp,
                                                                      const WeightGroup g, uint32_t m, uint32_t k,
                                                                      const AttnPrepEpi ep,
                                                                      const MoeGemmTiles mt) {
    asm volatile("" ::DS5_GROUP_ARGS(g), "s"(xhi), "s"(xlo), "s"(row_exp), "s"(m), "s"(k));
    // this workgroup's entry and column tile (uniform); out may be the residual itself
    // Workgroup L = y * gridDim.x + x runs on XCD L % 8. With gridDim.y a multiple of 8
    // (the launchers pad 8 or more row tiles to one), XCD q takes the row tiles q, q + 8,
    // ... with all their column tiles in a row, so a row tile's x rows come into one L2
    // (every (column, row tile) once; padding row tiles return at once).
    uint32_t bx = blockIdx.x, by = blockIdx.y;
    if (gridDim.y % 8 == 0) {
        const uint32_t L = blockIdx.y * gridDim.x + blockIdx.x, li = L / 8;
        bx = li % gridDim.x;
        by = L % 8 + 8 * (li / gridDim.x);
    }
    if (!GRP && by * BM >= m) return;  // workgroup-uniform, before any barrier
    const uint8_t* __restrict__ w = g.w[0];
    float* out = g.out[0];
    const float* res = g.res[0];
    uint32_t n = g.n[0], tile = bx;
    int entry = 0;
#pragma unroll
    for (int e = 1; e < kMatmulGroupMax; e++)
        if ((uint32_t)e < g.count && bx >= g.wg0[e]) {
            w = g.w[e];
            out = g.out[e];
            res = g.res[e];
            n = g.n[e];
            tile = bx - g.wg0[e];
            entry = e;
        }
    uint32_t m0 = by * BM;
    if constexpr (GRP) {
        if (by >= *mt.count) return;  // workgroup-uniform, before any barrier
        const uint4 te = mt.tiles[by];
        m0 = te.x;
        m = te.y;
        w += (uint64_t)te.z * mt.w_stride;
    }
    constexpr int kThreads = WM * WN * 64;
    constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
    static_assert(TM * WM * 16 == BM && TN * WN * 16 == BN, "tile split");
    constexpr int kBPer = BN * 4 / kThreads;  // 8-byte q runs per thread and block
    static_assert(kBPer >= 1, "at least one q run per thread");

    // LDS: As [stage][hi, lo][row * 4 + swizzled chunk], raw q [stage][wavefront][rows of
    // 9 dwords], Bs [buffer][row * 4 + swizzled chunk], Ss [buffer][row]; EPI 1 reuses
    // the bytes for the f32 tile
    constexpr int kRawBytes = 2 * WM * WN * ((16 * (BN * 4 / (WM * WN * 64)) * 9 + 63) / 64) * 256;
    constexpr int kAsBytes = 3 * 2 * BM * 4 * 16, kBsBytes = 2 * BN * 4 * 16, kSsBytes = 2 * BN * 4;
    constexpr int kMainBytes = kAsBytes + kRawBytes + kBsBytes + kSsBytes;
    constexpr int kTileRow = BN + 4;  // EPI 1 tile row stride in floats (16-byte rows, rows 4 banks apart)
    constexpr int kLdsBytes = EPI == 1 && BM * kTileRow * 4 > kMainBytes ? BM * kTileRow * 4 : kMainBytes;
    __shared__ __attribute__((aligned(16))) unsigned char smem[kLdsBytes];
    auto& As = *reinterpret_cast<u32x4_t(*)[3][2][BM * 4]>(smem);
    auto& Bs = *reinterpret_cast<u32x4_t(*)[2][BN * 4]>(smem + kAsBytes + kRawBytes);
    auto& Ss = *reinterpret_cast<float(*)[2][BN]>(smem + kAsBytes + kRawBytes + kBsBytes);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t n0 = tile * BN;
    const uint32_t nb = k / 32;
    const uint64_t row_bytes = (uint64_t)nb * kQ8Bytes;

    // ---- staging ------------------------------------------------------------------
    // All global loads are direct-to-LDS, issued two blocks ahead and awaited
    // explicitly. Iteration b issues x and the raw q of block b + 2 (one group of
    // loads), multiplies block b, waits until only that group is outstanding
    // (block b + 1 has landed), converts block b + 1's raw q to f16 and meets
    // the barrier. Each wavefront loads the raw rows its own threads convert, so
    // the conversion needs only the wavefront's own wait. Block j uses x stage
    // j % 3, raw q stage j % 2 and f16 q buffer j % 2.
    constexpr int kXStage = 2 * BM * 64;  // bytes: hi plane rows, then lo plane rows
    constexpr int kRowDw = 9;             // raw q row: the 9 dwords covering a 34-byte block
    constexpr int W = WM * WN;
    constexpr int NX = kXStage / 1024 / W;  // x loads per wavefront and block
    static_assert(NX >= 1 && NX * 1024 * W == kXStage, "whole 1 KB x loads per wavefront");
    static_assert((BM * 64) % 1024 == 0, "an x load stays inside one plane");
    constexpr int kWRows = 16 * kBPer;                   // tile rows whose runs a wavefront converts
    constexpr int NQ = (kWRows * kRowDw + 63) / 64;      // raw q loads (256 bytes) per wavefront and block
    constexpr int kQWave = NQ * 256;                     // a wavefront's raw q area in a stage
    constexpr int kQStage = W * kQWave;
    constexpr int kVmPerBlock = NX + NQ;
    const uint32_t wave_u = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
    const uint32_t smem_lds = gemm_lds_addr(smem);

    // x: load i of this wavefront fills stage bytes [1024 (wave + W i), +1024), lane L
    // the 16 bytes at +16 L: plane, row r, slot L % 4 holding chunk (L % 4) ^ ((r >> 2) & 3).
    uint32_t xoff[NX];  // byte offset in the plane: row min(m0 + r, m - 1), chunk c, block 0
#pragma unroll
    for (int i = 0; i < NX; i++) {
        const uint32_t o = 1024u * (wave_u + W * i) + 16u * lane;
        if (GRP && mt.x_rows) {  // uniform
            const uint32_t r = ds5idx::gemm_x_tile_row(o, BM);
            xoff[i] = ds5idx::gemm_x_off_row(r, (uint32_t)lane, mt.x_rows[min(m0 + r, m - 1)], k);
        } else {
            xoff[i] = ds5idx::gemm_x_off(o, (uint32_t)lane, BM, m0, m, k);
        }
    }
    auto issue_x = [&](uint32_t b, int stage) {
#pragma unroll
        for (int i = 0; i < NX; i++) {
            const uint32_t blk = wave_u + W * i;  // uniform
            const uint16_t* plane = blk * 1024 < BM * 64 ? xhi : xlo;
            lds_dma<4>(xoff[i], uniform_u64((uint64_t)(uintptr_t)plane + 64ull * b),
                       (uint32_t)__builtin_amdgcn_readfirstlane(smem_lds + stage * kXStage + 1024 * blk));
        }
    };

    // raw q: the wavefront's local row lr < 16 kBPer is tile row 16 wave + (threads / 4)
    // (lr / 16) + lr % 16 (the rows of its threads' runs). Dword d = 64 i + lane of its
    // area (clamped to the last, d < 9 * 16 kBPer) is dword d % 9 of local row d / 9, from
    // the dword boundary at or below the row's block: weight row wr = min(n0 + row,
    // n - 1), rb = wr * row_bytes, block b at byte rb + 34 b of the weights. 34 b is
    // 0 mod 4 for even b and 2 mod 4 for odd b, so the dwords start at 34 b + (rb & ~3)
    // (even) or 34 b - 2 + ((rb + 2) & ~3) (odd): scalar base w + 34 b or w + 34 b - 2,
    // lane offsets per parity (both sums of non-negative terms: no unsigned wrap).
    uint32_t qoff_e[NQ], qoff_o[NQ];
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        const uint32_t d = ds5idx::gemm_q_dword(i, (uint32_t)lane, kWRows, kRowDw);
        const uint32_t row = ds5idx::gemm_q_row(d, wave_u, kThreads, kRowDw);
        ds5idx::gemm_q_off(d, row, n0, n, (uint32_t)row_bytes, kRowDw, qoff_e[i], qoff_o[i]);
    }
    const uint32_t q_lds = smem_lds + 3 * kXStage + wave_u * kQWave;
    auto issue_q = [&](uint32_t b, int stage) {
        const bool odd = b & 1;
        const uint64_t base = uniform_u64((uint64_t)(uintptr_t)w + (uint64_t)kQ8Bytes * b - (odd ? 2u : 0u));
#pragma unroll
        for (int i = 0; i < NQ; i++)
            lds_dma<1>(odd ? qoff_o[i] : qoff_e[i], base,
                       (uint32_t)__builtin_amdgcn_readfirstlane(q_lds + stage * kQStage + 256 * i));
    };

    // f16 q: thread c = tid + threads u takes tile row c / 4 (local row 16 u + lane / 4 of
    // its wavefront), bytes 2 + 8 (c % 4) .. + 8 of its block: raw-row bytes (s & 3) + 2
    // + 8 (c % 4) .. + 8, inside the three dwords 2 (c % 4) .. + 3 of the raw row (bytes
    // 2..9 of them when s & 3 = 0, bytes 4..11 when it is 2). Part 0's first dword also
    // holds the scale (bytes s & 3, + 1).
    const unsigned char* qraw = smem + 3 * kXStage + wave_u * kQWave;
    uint32_t rbp[kBPer], qrd[kBPer];  // (weight row * row_bytes) & 3; byte of the lane's dwords in the area
#pragma unroll
    for (int u = 0; u < kBPer; u++) {
        const uint32_t c = threadIdx.x + kThreads * u;
        rbp[u] = (min(n0 + (c >> 2), n - 1) * (uint32_t)row_bytes) & 3u;
        qrd[u] = (16 * u + (lane >> 2)) * (kRowDw * 4) + 8 * (lane & 3);
    }
    auto convert_q = [&](uint32_t b, int stage, int buf) {
#pragma unroll
        for (int u = 0; u < kBPer; u++) {
            const uint32_t c = threadIdx.x + kThreads * u;
            const uint32_t row = c >> 2, part = c & 3;
            const bool s2 = (rbp[u] + 2 * b) & 2u;  // s & 3 == 2
            const uint32_t* rw = (const uint32_t*)(qraw + stage * kQStage + qrd[u]);
            const uint32_t d0 = rw[0], d1 = rw[1], d2 = rw[2];
            const uint32_t sel = s2 ? 0x07060504u : 0x05040302u;
            const uint2 a = i8x4_to_f16x4(__builtin_amdgcn_perm(d1, d0, sel));
            const uint2 bb = i8x4_to_f16x4(__builtin_amdgcn_perm(d2, d1, sel));
            Bs[buf][row * 4 + (part ^ ((row >> 2) & 3))] = u32x4_t{a.x, a.y, bb.x, bb.y};
            if (part == 0) Ss[buf][row] = f16_bits_to_f32(s2 ? d0 >> 16 : d0 & 0xffffu);
        }
    };

    // ---- per-wavefront tiles ---------------------------------------------------
    const int wm0 = (wave / WN) * (BM / WM), wn0 = (wave % WN) * (BN / WN);
    const int r16 = lane & 15, grp = lane >> 4;
    f32x4_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // GRP: the wavefront's 16-row tiles holding rows of the tile (uniform); the rest
    // (an expert's last, partial tile) skip their products
    int live = TM;
    if constexpr (GRP) {
        const int left = (int)m - (int)(m0 + wm0);
        live = __builtin_amdgcn_readfirstlane(left <= 0 ? 0 : min(TM, (left + 15) / 16));
    }
    auto multiply = [&](int stage, int buf) {
        f16x8_t bv[TN];
        float sv[TN];
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int row = wn0 + 16 * j + r16;
            bv[j] = __builtin_bit_cast(f16x8_t, Bs[buf][row * 4 + (grp ^ ((row >> 2) & 3))]);
            sv[j] = Ss[buf][row];
        }
#pragma unroll
        for (int i = 0; i < TM; i++) {
            if (GRP && i >= live) break;
            const int row = wm0 + 16 * i + r16;
            const int slot = row * 4 + (grp ^ ((row >> 2) & 3));
            const f16x8_t ah = __builtin_bit_cast(f16x8_t, As[stage][0][slot]);
            const f16x8_t al = __builtin_bit_cast(f16x8_t, As[stage][1][slot]);
#pragma unroll
            for (int j = 0; j < TN; j++) {
                f32x4_t t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bv[j], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bv[j], t, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; e++) acc[i][j][e] = __builtin_fmaf(sv[j], t[e], acc[i][j][e]);
            }
        }
    };

    // prologue: blocks 0 and 1 in flight; block 0's q converted once its loads have landed
    issue_x(0, 0);
    issue_q(0, 0);
    if (nb > 1) {
        issue_x(1, 1);
        issue_q(1, 1);
        wait_vm_only<kVmPerBlock>();
    } else {
        wait_vm_only<0>();
    }
    convert_q(0, 0, 0);
    gemm_lds_sync();
    // iteration b: x stage b % 3 (uniform)
    uint32_t st = 0;
    for (uint32_t b = 0; b < nb; b++) {
        const uint32_t st1 = st == 2 ? 0 : st + 1, st2 = st == 0 ? 2 : st - 1;  // (b + 1) % 3, (b + 2) % 3
        const bool ahead = b + 2 < nb;  // uniform
        if (ahead) {
            issue_x(b + 2, st2);  // the stage of block b - 1, read before the last barrier
            issue_q(b + 2, b & 1);  // the raw stage of block b, converted before the last barrier
        }
        multiply(st, b & 1);
        if (ahead) wait_vm_only<kVmPerBlock>();  // block b + 1 has landed
        else wait_vm_only<0>();
        if (b + 1 < nb) convert_q(b + 1, (b + 1) & 1, (b + 1) & 1);
        gemm_lds_sync();
        st = st1;
    }

    if constexpr (EPI == 1) {
        // The whole 128 x 128 tile (one head of 128 tokens) goes through LDS once;
        // then thread t takes rows t / 8 and t / 8 + 64, dims k8 + [0, 8) and
        // 64 + k8 + [0, 8) (8 rope pairs), k8 = 8 (t % 8). Its norm weights and
        // rope cos / sin are loaded before the tile is written, so their
        // latency overlaps the tile's LDS round trip.
        static_assert(BM == 128 && BN == 128 && WM == 4 && WN == 2, "one head of 128 dims per tile");
        constexpr int D = 128, HALF = 64, TROW = kTileRow;
        const uint32_t head = tile;  // BN = D: tile j of an entry is head j
        const int r0 = threadIdx.x / 8, k8 = 8 * (threadIdx.x % 8);
        const float* nw = entry == 0 ? ep.q_norm : ep.k_norm;
        float w0[8], w1[8], c[2][8], sn[2][8];
        if (entry != 2) {
            *(float4*)&w0[0] = *(const float4*)(nw + k8);
            *(float4*)&w0[4] = *(const float4*)(nw + k8 + 4);
            *(float4*)&w1[0] = *(const float4*)(nw + HALF + k8);
            *(float4*)&w1[4] = *(const float4*)(nw + HALF + k8 + 4);
#pragma unroll
            for (int rr = 0; rr < 2; rr++) {
                const uint32_t tok = min(m0 + r0 + 64 * rr, m - 1);
                const float* cs = ep.cs + (uint64_t)tok * D;
                *(float4*)&c[rr][0] = *(const float4*)(cs + k8);
                *(float4*)&c[rr][4] = *(const float4*)(cs + k8 + 4);
                *(float4*)&sn[rr][0] = *(const float4*)(cs + HALF + k8);
                *(float4*)&sn[rr][4] = *(const float4*)(cs + HALF + k8 + 4);
            }
        }
        // the main loop ended on a barrier after every wavefront's last LDS read
        float* tl = reinterpret_cast<float*>(smem);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int lr = wm0 + 16 * i + 4 * grp + e;
                const uint32_t row = m0 + lr;
                const int sh = row < m ? row_exp[row] - kXExpBias : 0;
#pragma unroll
                for (int j = 0; j < TN; j++) tl[lr * TROW + wn0 + 16 * j + r16] = __builtin_ldexpf(acc[i][j][e], sh);
            }
        __syncthreads();
#pragma unroll
        for (int rr = 0; rr < 2; rr++) {
            const int r = r0 + 64 * rr;
            const uint32_t tok = m0 + r;
            const bool ok = tok < m;
            const float* trow = tl + r * TROW;
            float x0[8], x1[8];
            *(float4*)&x0[0] = *(const float4*)(trow + k8);
            *(float4*)&x0[4] = *(const float4*)(trow + k8 + 4);
            *(float4*)&x1[0] = *(const float4*)(trow + HALF + k8);
            *(float4*)&x1[4] = *(const float4*)(trow + HALF + k8 + 4);
            f16x8_t y0v, y1v;
            f16* dst;
            if (entry == 2) {  // v: f16 append
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    y0v[j] = (f16)x0[j];
                    y1v[j] = (f16)x1[j];
                }
                dst = ep.v_cache + ((uint64_t)head * ep.max_ctx + ep.pos + tok) * D;
            } else {
                if (entry == 0) {
                    // q: the thread's two quarters (pairs k8 .. k8 + 3 and k8 + 4 .. k8 + 7),
                    // then the head's 8 threads in the balanced tree's order (xor 1, 2, 4)
                    float ss = qk_quarter_sumsq(x0[0], x1[0], x0[1], x1[1], x0[2], x1[2], x0[3], x1[3]) +
                               qk_quarter_sumsq(x0[4], x1[4], x0[5], x1[5], x0[6], x1[6], x0[7], x1[7]);
#pragma unroll
                    for (int mm = 1; mm < 8; mm <<= 1) ss += __shfl_xor(ss, mm, 64);
                    const float r = rms_inv(ss, (float)D, ep.eps) * ep.q_scale;
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        _Float16 o0, o1;
                        qk_q_pair(x0[j], x1[j], w0[j], w1[j], c[rr][j], sn[rr][j], r, o0, o1);
                        y0v[j] = o0;
                        y1v[j] = o1;
                    }
                } else {  // k: the reference's serial sum of the row
                    const float inv = rms_inv(qk_serial_sumsq(trow, D), (float)D, ep.eps);
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        float y0, y1;
                        qk_rotate(qk_norm_mul(x0[j], inv, w0[j]), qk_norm_mul(x1[j], inv, w1[j]), c[rr][j], sn[rr][j],
                                  y0, y1);
                        y0v[j] = (f16)y0;
                        y1v[j] = (f16)y1;
                    }
                }
                dst = entry == 0 ? ep.q16 + ((uint64_t)tok * ep.n_q_heads + head) * D
                                 : ep.k_cache + ((uint64_t)head * ep.max_ctx + ep.pos + tok) * D;
            }
            if (ok) {
                *(f16x8_t*)(dst + k8) = y0v;
                *(f16x8_t*)(dst + HALF + k8) = y1v;
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t row = m0 + wm0 + 16 * i + 4 * grp + e;
            if (row >= m) continue;
            const int sh = row_exp[GRP && mt.x_rows ? mt.x_rows[row] : row] - kXExpBias;
            const uint32_t orow = GRP && mt.out_rows ? mt.out_rows[row] : row;
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint32_t col = n0 + wn0 + 16 * j + r16;
                if (col < n) {
                    const uint64_t o = (uint64_t)orow * n + col;
                    const float v = __builtin_ldexpf(acc[i][j][e], sh);
                    out[o] = res ? res[o] + v : v;
                }
            }
        }
}

// Any shape or alignment: one thread per output in the reference's serial order
// with every product and sum rounded on its own (bit-identical to dotRow).
__global__ __launch_bounds__(kMmThreads) void matmul_generic_kernel(const float* __restrict__ x, const uint8_t* __restrict__ w,
                                                                    uint32_t q8, float* out, const float* res, uint32_t m,
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
    out[i] = res ? res[i] + acc : acc;
}

// out = x + y elementwise (kernels_a.zig:223-233): out may be x or y. Views that
// are not all 4-byte aligned go through byte copies.
__global__ __launch_bounds__(kMmThreads) void add_kernel(const uint8_t* x, const uint8_t* y, uint8_t* out, uint64_t n,
                                                         uint32_t aligned) {
    const uint64_t i = (uint64_t)blockIdx.x * kMmThreads + threadIdx.x;
    if (i >= n) return;
    if (aligned) {
        ((float*)out)[i] = ((const float*)x)[i] + ((const float*)y)[i];
    } else {
        float a, b;
        __builtin_memcpy(&a, x + 4 * i, 4);
        __builtin_memcpy(&b, y + 4 * i, 4);
        const float c = a + b;
        __builtin_memcpy(out + 4 * i, &c, 4);
    }
}

template <int MT, int JB, bool Q8, bool NORM>
int launch_rows(ds5_hip_ctx* ctx, const MatmulGroupLaunch& a, uint32_t m0) {
    constexpr uint32_t kRowsPerBlock = kMmThreads / 64;
    WeightGroup g{};
    uint32_t wgs = 0;
    for (uint32_t e = 0; e < a.count; e++) {
        g.w[g.count] = a.w[e];
        g.out[g.count] = a.out[e];
        g.res[g.count] = a.res[e];
        g.n[g.count] = a.n[e];
        g.wg0[g.count] = wgs;
        wgs += (a.n[e] + kRowsPerBlock - 1) / kRowsPerBlock;
        g.count += a.n[e] ? 1 : 0;  // entries without rows are dropped
    }
    if (wgs == 0) return DS5_OK;
    DS5_TIMED_LAUNCH(ctx, "matmul_rows_kernel", (matmul_rows_kernel<MT, JB, Q8, NORM>), dim3(wgs), dim3(kMmThreads), 0,
                     ctx->stream, a.x, g, a.m, a.k, m0, a.norm_w, a.norm_eps);
    return ds5_after_launch(ctx, "matmul_rows_kernel");
}


// Tokens per pass: up to 4 / JB (the x registers hold MT * JB * 32 floats per lane),
// and no more than the tokens there are (a 1-token decode runs MT = 1).
template <int JB, bool Q8, bool NORM>
int launch_passes(ds5_hip_ctx* ctx, const MatmulGroupLaunch& a) {
    constexpr uint32_t kMaxMt = 4 / JB;
    const uint32_t mt = a.m >= kMaxMt ? kMaxMt : (a.m >= 2 ? 2 : 1);
    for (uint32_t m0 = 0; m0 < a.m; m0 += mt) {
        int rc;
        if (mt == 4)
            rc = launch_rows<(kMaxMt >= 4 ? 4 : 1), JB, Q8, NORM>(ctx, a, m0);
        else if (mt == 2)
            rc = launch_rows<(kMaxMt >= 2 ? 2 : 1), JB, Q8, NORM>(ctx, a, m0);
        else
            rc = launch_rows<1, JB, Q8, NORM>(ctx, a, m0);
        if (rc) return rc;
    }
    return DS5_OK;
}

template <bool Q8, bool NORM>
int launch_rows_n(ds5_hip_ctx* ctx, const MatmulGroupLaunch& a) {
    const uint32_t nb = a.k / 32;
    if (nb <= 64) return launch_passes<1, Q8, NORM>(ctx, a);
    if (nb <= 128) return launch_passes<2, Q8, NORM>(ctx, a);
    return launch_passes<4, Q8, NORM>(ctx, a);
}

template <bool Q8>
int launch_rows_q(ds5_hip_ctx* ctx, const MatmulGroupLaunch& a) {
    return a.norm_w ? launch_rows_n<Q8, true>(ctx, a) : launch_rows_n<Q8, false>(ctx, a);
}

// Row tiles of a launch: 8 or more are padded to a multiple of 8 (the kernel's XCD order).
static uint32_t gemm_row_tiles(uint32_t m, uint32_t bm) {
    const uint32_t t = (m + bm - 1) / bm;
    return t >= 8 ? (t + 7) / 8 * 8 : t;
}

// The split x is made once and shared by the group's products.
template <int BM, int BN, int WM, int WN>
int launch_gemm(ds5_hip_ctx* ctx, const MatmulGroupLaunch& a) {
    void* ws = nullptr;
    if (int rc = ds5_workspace(ctx, x_split_bytes(a.m, a.k), &ws)) return rc;
    uint16_t* hi = (uint16_t*)ws;
    uint16_t* lo = hi + (size_t)a.m * a.k;
    int* row_exp = (int*)(lo + (size_t)a.m * a.k);
    DS5_TIMED_LAUNCH(ctx, "matmul_x_split_kernel", matmul_x_split_kernel<false>, dim3(a.m), dim3(kSplitThreads), 0,
                     ctx->stream, a.x, hi, lo, row_exp, a.k, XSplitRope{}, RopeTable{}, a.norm_w, a.norm_eps);
    if (int rc = ds5_after_launch(ctx, "matmul_x_split_kernel")) return rc;
    WeightGroup g{};
    uint32_t tiles = 0;
    for (uint32_t e = 0; e < a.count; e++) {
        g.w[g.count] = a.w[e];
        g.out[g.count] = a.out[e];
        g.res[g.count] = a.res[e];
        g.n[g.count] = a.n[e];
        g.wg0[g.count] = tiles;
        tiles += (a.n[e] + BN - 1) / BN;
        g.count += a.n[e] ? 1 : 0;  // entries without rows are dropped
    }
    if (tiles == 0) return DS5_OK;
    DS5_TIMED_LAUNCH(ctx, "matmul_q8_mfma_kernel", (matmul_q8_mfma_kernel<BM, BN, WM, WN, 0>),
                     dim3(tiles, gemm_row_tiles(a.m, BM)), dim3(WM * WN * 64), 0, ctx->stream, hi, lo, row_exp, g, a.m, a.k,
                     AttnPrepEpi{}, MoeGemmTiles{});
    return ds5_after_launch(ctx, "matmul_q8_mfma_kernel");
}

}  // namespace

// The MoE experts' matrix-core path (rows sorted by expert): the tokens' x rows split,
// the grouped products (sorted rows gather their token's plane row), h = silu(g) * u
// split.
int launch_x_split_rows(ds5_hip_ctx* ctx, const float* x, uint32_t rows, uint32_t k, uint16_t* hi, uint16_t* lo,
                        int* row_exp) {
    if (rows == 0) return DS5_OK;
    DS5_TIMED_LAUNCH(ctx, "matmul_x_split_kernel", matmul_x_split_kernel<false>, dim3(rows), dim3(kSplitThreads), 0,
                     ctx->stream, x, hi, lo, row_exp, k, XSplitRope{}, RopeTable{}, nullptr, 0.0f);
    return ds5_after_launch(ctx, "matmul_x_split_kernel");
}

int launch_moe_h_split(ds5_hip_ctx* ctx, const float* g, const float* u, uint32_t rows, uint32_t k, uint16_t* hi,
                       uint16_t* lo, int* row_exp) {
    if (rows == 0) return DS5_OK;
    const dim3 g4((rows + 3) / 4);
    if (k <= 1024)
        DS5_TIMED_LAUNCH(ctx, "moe_h_split_kernel", moe_h_split_rows_kernel<4>, g4, dim3(256), 0, ctx->stream, g, u, hi,
                         lo, row_exp, k, rows);
    else if (k <= 2048)
        DS5_TIMED_LAUNCH(ctx, "moe_h_split_kernel", moe_h_split_rows_kernel<8>, g4, dim3(256), 0, ctx->stream, g, u, hi,
                         lo, row_exp, k, rows);
    else
        DS5_TIMED_LAUNCH(ctx, "moe_h_split_kernel", moe_h_split_kernel, dim3(rows), dim3(kSplitThreads), 0, ctx->stream,
                         g, u, hi, lo, row_exp, k);
    return ds5_after_launch(ctx, "moe_h_split_kernel");
}

template <int BM, int BN, int WM, int WN>
static int launch_q8_gemm_grouped_t(ds5_hip_ctx* ctx, const uint16_t* hi, const uint16_t* lo, const int* row_exp,
                                    uint32_t k, const uint8_t* const* w, float* const* out, const uint32_t* n,
                                    uint32_t count, uint32_t max_tiles, const MoeGemmTiles& mt) {
    WeightGroup g{};
    uint32_t nt = 0;
    for (uint32_t e = 0; e < count; e++) {
        g.w[e] = w[e];
        g.out[e] = out[e];
        g.n[e] = n[e];
        g.wg0[e] = nt;
        nt += (n[e] + BN - 1) / BN;
    }
    g.count = count;
    if (nt == 0 || max_tiles == 0) return DS5_OK;
    DS5_TIMED_LAUNCH(ctx, "matmul_q8_mfma_kernel", (matmul_q8_mfma_kernel<BM, BN, WM, WN, 0, true>),
                     dim3(nt, gemm_row_tiles(max_tiles, 1)), dim3(WM * WN * 64), 0, ctx->stream, hi, lo, row_exp, g, 0u, k,
                     AttnPrepEpi{}, mt);
    return ds5_after_launch(ctx, "matmul_q8_mfma_kernel");
}

int launch_q8_gemm_grouped(ds5_hip_ctx* ctx, const uint16_t* hi, const uint16_t* lo, const int* row_exp, uint32_t k,
                           const uint8_t* const* w, float* const* out, const uint32_t* n, uint32_t count,
                           const uint4* tiles, const uint32_t* n_tiles, uint32_t max_tiles, uint32_t tile_rows,
                           uint64_t w_stride, const uint32_t* x_rows, const uint32_t* out_rows) {
    const MoeGemmTiles mt{tiles, n_tiles, w_stride, x_rows, out_rows};
    if (tile_rows == 64)
        return launch_q8_gemm_grouped_t<64, 128, 2, 2>(ctx, hi, lo, row_exp, k, w, out, n, count, max_tiles, mt);
    if (tile_rows == 128)
        return launch_q8_gemm_grouped_t<128, 128, 4, 2>(ctx, hi, lo, row_exp, k, w, out, n, count, max_tiles, mt);
    return ds5_fail(ctx, DS5_DEVICE_FAILURE, "moe: row tiles of %u rows", tile_rows);
}

// The rope table follows the x split at the next 16-byte boundary (the epilogue
// reads it in float4s).
static size_t qkv_prep_cs_offset(uint32_t m, uint32_t k) { return (x_split_bytes(m, k) + 15) & ~(size_t)15; }

size_t qkv_prep_workspace_bytes(uint32_t m, uint32_t k, uint32_t head_dim) {
    return qkv_prep_cs_offset(m, k) + (size_t)m * head_dim * sizeof(float);
}

int launch_qkv_prep(ds5_hip_ctx* ctx, const QkvPrepLaunch& a) {
    constexpr int BM = 128, BN = 128, WM = 4, WN = 2;
    uint16_t* hi = (uint16_t*)a.ws;
    uint16_t* lo = hi + (size_t)a.m * a.k;
    int* row_exp = (int*)(lo + (size_t)a.m * a.k);
    float* cs = (float*)((char*)a.ws + qkv_prep_cs_offset(a.m, a.k));
    XSplitRope rope{a.positions, cs, a.head_dim / 2, a.freq_scale};
    DS5_TIMED_LAUNCH(ctx, "matmul_x_split_kernel", matmul_x_split_kernel<true>, dim3(a.m), dim3(kSplitThreads), 0,
                     ctx->stream, a.x, hi, lo, row_exp, a.k, rope, *a.table, a.norm_w, a.norm_eps);
    if (int rc = ds5_after_launch(ctx, "matmul_x_split_kernel")) return rc;
    WeightGroup g{};
    const uint32_t ns[3] = {a.n_q_heads * a.head_dim, a.n_kv_heads * a.head_dim, a.n_kv_heads * a.head_dim};
    const uint8_t* ws[3] = {a.wq, a.wk, a.wv};
    uint32_t tiles = 0;
    for (int e = 0; e < 3; e++) {
        g.w[e] = ws[e];
        g.n[e] = ns[e];
        g.wg0[e] = tiles;
        tiles += ns[e] / BN;
    }
    g.count = 3;
    AttnPrepEpi ep{a.q_norm, a.k_norm, cs, a.q16, a.k_cache, a.v_cache, a.pos, a.n_q_heads, a.max_ctx, a.eps, a.q_scale};
    DS5_TIMED_LAUNCH(ctx, "matmul_q8_mfma_kernel", (matmul_q8_mfma_kernel<BM, BN, WM, WN, 1>),
                     dim3(tiles, gemm_row_tiles(a.m, BM)), dim3(WM * WN * 64), 0, ctx->stream, hi, lo, row_exp, g, a.m, a.k,
                     ep, MoeGemmTiles{});
    return ds5_after_launch(ctx, "matmul_q8_mfma_kernel");
}

// Tokens from which Q8_0 products run on the matrix cores (below, the row
// kernel's passes of up to 4 tokens re-read the weights less often than the
// GEMM wastes matrix-core work)
constexpr uint32_t kGemmMinM = 16;

// The row kernel needs x and out 16-byte aligned, k <= 8192, and f32 weights 16-byte
// aligned or Q8_0 weights 4-byte aligned. A Q8_0 block is read as the nine dwords
// from the dword boundary at or below it, which ends 2 bytes past the block when
// the block starts on a dword boundary; for the last block that stays inside the
// view only if the weights end on a dword boundary or the view has 2 more bytes.
// The GEMM reads x as float4 (x 16-byte aligned), stores single floats (out
// 4-byte aligned) and reads q in 8-byte runs from the dword boundary at or below
// them, with the same end condition. Its loads address an x plane and the
// weights with 32-bit byte offsets from a scalar base.
static bool gemm_offsets_fit(uint32_t m, uint32_t k, uint64_t w_end) {
    return (uint64_t)m * k * 2 < (1ull << 32) && w_end + 2 < (1ull << 32);
}

MatmulPath matmul_path(const MatmulLaunch& a, uint64_t w_len) {
    const uintptr_t x_addr = (uintptr_t)a.x, out_addr = (uintptr_t)a.out, w_addr = (uintptr_t)a.w;
    if (a.k % 32 != 0 || (x_addr & 15u)) return MatmulPath::Generic;
    if (!a.q8) return (a.k / 32 <= 256 && (out_addr & 15u) == 0 && (w_addr & 15u) == 0) ? MatmulPath::Rows
                                                                                         : MatmulPath::Generic;
    const uint64_t end = (uint64_t)a.n * (a.k / 32) * kQ8Bytes;
    if ((w_addr & 3u) || !((w_addr + end) % 4 == 0 || w_len >= end + 2)) return MatmulPath::Generic;
    const bool gemm = (out_addr & 3u) == 0 && gemm_offsets_fit(a.m, a.k, end);
    if (a.m >= kGemmMinM && gemm) return MatmulPath::Gemm;
    if (a.k / 32 <= 256 && (out_addr & 15u) == 0) return MatmulPath::Rows;
    return gemm ? MatmulPath::Gemm : MatmulPath::Generic;
}

static int launch_generic(ds5_hip_ctx* ctx, const float* x, const uint8_t* w, bool q8, float* out, const float* res,
                          uint32_t m, uint32_t n, uint32_t k) {
    const uint64_t total = (uint64_t)m * n;
    const dim3 grid((unsigned)((total + kMmThreads - 1) / kMmThreads));
    DS5_TIMED_LAUNCH(ctx, "matmul_generic_kernel", matmul_generic_kernel, grid, dim3(kMmThreads), 0, ctx->stream, x, w,
                     (uint32_t)q8, out, res, m, n, k);
    return ds5_after_launch(ctx, "matmul_generic_kernel");
}

static int launch_same_path(ds5_hip_ctx* ctx, const MatmulGroupLaunch& a, MatmulPath path) {
    if (a.norm_w && (path == MatmulPath::Generic || a.k <= kRmsSerialMaxDim))
        return ds5_fail(ctx, DS5_DEVICE_FAILURE, "matmul: an in-kernel norm needs the row or GEMM path and k > %u",
                        kRmsSerialMaxDim);
    if (path == MatmulPath::Rows) return a.q8 ? launch_rows_q<true>(ctx, a) : launch_rows_q<false>(ctx, a);
    if (path == MatmulPath::Gemm)
        return a.m >= 128 ? launch_gemm<128, 128, 4, 2>(ctx, a) : launch_gemm<32, 64, 2, 2>(ctx, a);
    for (uint32_t e = 0; e < a.count; e++)
        if (a.n[e])
            if (int rc = launch_generic(ctx, a.x, a.w[e], a.q8, a.out[e], a.res[e], a.m, a.n[e], a.k)) return rc;
    return DS5_OK;
}

int launch_matmul(ds5_hip_ctx* ctx, const MatmulLaunch& a, MatmulPath path) {
    MatmulGroupLaunch g{};
    g.x = a.x;
    g.q8 = a.q8;
    g.m = a.m;
    g.k = a.k;
    g.count = 1;
    g.w[0] = a.w;
    g.out[0] = a.out;
    g.res[0] = a.res;
    g.n[0] = a.n;
    return launch_matmul_group(ctx, g, &path);
}

int launch_add(ds5_hip_ctx* ctx, const void* x, const void* y, void* out, uint64_t n) {
    if (n == 0) return DS5_OK;
    const uint32_t aligned = (((uintptr_t)x | (uintptr_t)y | (uintptr_t)out) & 3u) == 0;
    const dim3 grid((unsigned)((n + kMmThreads - 1) / kMmThreads));
    DS5_TIMED_LAUNCH(ctx, "add_kernel", add_kernel, grid, dim3(kMmThreads), 0, ctx->stream, (const uint8_t*)x,
                     (const uint8_t*)y, (uint8_t*)out, n, aligned);
    return ds5_after_launch(ctx, "add_kernel");
}

// One launch for the whole group when every entry takes the same kernel;
// otherwise each entry on its own kernel, in order.
int launch_matmul_group(ds5_hip_ctx* ctx, const MatmulGroupLaunch& a, const MatmulPath* paths) {
    if (a.m == 0 || a.count == 0) return DS5_OK;
    bool same = true;
    for (uint32_t e = 1; e < a.count; e++) same = same && paths[e] == paths[0];
    if (same) return launch_same_path(ctx, a, paths[0]);
    for (uint32_t e = 0; e < a.count; e++) {
        MatmulGroupLaunch one{};
        one.x = a.x;
        one.q8 = a.q8;
        one.m = a.m;
        one.k = a.k;
        one.count = 1;
        one.w[0] = a.w[e];
        one.out[0] = a.out[e];
        one.res[0] = a.res[e];
        one.n[0] = a.n[e];
        if (int rc = launch_same_path(ctx, one, paths[e])) return rc;
    }
    return DS5_OK;
}
