// k_prefill.hip -- causal prefill on gfx950: the fused step's pre-pass (k/v
// append with rope) and flash attention on f16 MFMA with f32 accumulation.
//
// Semantics: kernels_b.zig:29-133 for n_tokens > 1 -- query token t (absolute
// position pos + t) of q head h attends cache positions 0..pos+t of kv head
// h / group; softmax(scale * q.k) in f32.
//
// prefill_attention_kernel. A workgroup is 4 wavefronts, one q head each, all
// four heads from the same GQA group, so every K/V byte staged in LDS feeds
// four heads. A wavefront owns 32 query rows of its head. Keys stream in
// 64-position tiles through a double-buffered LDS stage (the next tile's global
// loads are in flight while the current one is consumed):
//   S^T[32 keys x 32 q] = K . Q^T         v_mfma_f32_32x32x16_f16 (x2 per tile)
//   O^T[D x 32 q]      += V^T . P^T       v_mfma_f32_32x32x16_f16
// With S transposed a lane holds 16 scores of one query row, so row max/sum
// need one lane exchange, and the P^T operand is the lane's own scores. V^T
// operands come from LDS through gfx950's transpose read (ds_read_b64_tr_b16).
// q and p are rounded to f16 for the products; softmax state is f32 in the
// log2 domain with a lazy reference max (rescale only on growth > 2^8).
// Causal masking runs only on tiles that cross the diagonal.
//
// Load balance: q tiles are paired heaviest with lightest (tile NQ-1-i with
// tile i) so every workgroup carries the same number of key tiles, and the
// workgroups of one kv head are placed on the same XCD (workgroup b runs on
// XCD b % 8), so each XCD's L2 holds one kv head's K/V.
//
// Fused mode: the pre-pass (prefill_prep_kernel) writes the normalised,
// rotated f16 k rows and the f16 v rows into the cache, and a q rotation table
// per (token, pair) with the q_norm weights folded in; the attention kernel
// takes raw q, applies the per-head RMSNorm scale (the row's sum of squares
// reduced across the two lanes that hold it) and the rotation, and rounds q to
// f16.
#include "ds5_common.hpp"

namespace {

// ---------------------------------------------------------------------------
// Pre-pass: one workgroup per token.
// ---------------------------------------------------------------------------
constexpr int kPrepThreads = 256;
constexpr int kPrepMaxRow = 2048;  // n_kv_heads * head_dim floats staged per token

__device__ __forceinline__ float serial_sumsq(const float* row, int dim) {
#pragma clang fp contract(off)
    float acc = 0.0f;
    for (int i = 0; i < dim; i += 4) {
        const float4 v = *(const float4*)(row + i);
        acc += v.x * v.x;
        acc += v.y * v.y;
        acc += v.z * v.z;
        acc += v.w * v.w;
    }
    return acc;
}

__device__ __forceinline__ float norm_mul(float v, float inv, float w) {
#pragma clang fp contract(off)
    return v * inv * w;
}

__device__ __forceinline__ void rotate(float x0, float x1, float c, float s, float& y0, float& y1) {
#pragma clang fp contract(off)
    y0 = x0 * c - x1 * s;
    y1 = x0 * s + x1 * c;
}

__device__ __forceinline__ float rope_angle(float pos, float freq_scale, float inv) {
#pragma clang fp contract(off)
    return pos * freq_scale * inv;
}

// Token t: cos/sin of its rope angles (kernels_a.zig:119-122), the q rotation
// table with the q_norm weights folded in, then every kv head's k row: serial-order RMSNorm (kernels_a.zig:84-89), NeoX
// rotation (:125-126), f16 append at slot pos + t (:196-210); v rows f16.
__global__ __launch_bounds__(kPrepThreads) void prefill_prep_kernel(KvPrepLaunch a, float4* q_rot, RopeTable table) {
    __shared__ __attribute__((aligned(16))) float s_k[kPrepMaxRow];
    __shared__ float s_cos[DS5_MAX_ROPE_HALF], s_sin[DS5_MAX_ROPE_HALF];
    __shared__ float s_inv[kPrepMaxRow / 64];
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    const uint32_t D = a.head_dim, half = D / 2, H = a.n_kv_heads;
    const float pos = (float)a.positions[t];
    for (uint32_t i = tid; i < half; i += kPrepThreads) {
        const float ang = rope_angle(pos, a.freq_scale, table.inv[i]);
        const float c = cosf(ang), s = sinf(ang);
        s_cos[i] = c;
        s_sin[i] = s;
        // q: norm weights folded into the rotation (see load_q)
        const float w0 = a.q_norm[i], w1 = a.q_norm[i + half];
        q_rot[(uint64_t)t * half + i] = float4{w0 * c, w1 * s, w0 * s, w1 * c};
    }
    const float* krow = a.k + (uint64_t)t * H * D;
    for (uint32_t e = tid; e < H * D; e += kPrepThreads) s_k[e] = krow[e];
    __syncthreads();
    for (uint32_t h = tid; h < H; h += kPrepThreads) s_inv[h] = rms_inv(serial_sumsq(s_k + h * D, (int)D), (float)D, a.eps);
    __syncthreads();
    for (uint32_t e = tid; e < H * half; e += kPrepThreads) {
        const uint32_t h = e / half, i = e % half;
        const float inv = s_inv[h];
        const float x0 = norm_mul(s_k[h * D + i], inv, a.k_norm[i]);
        const float x1 = norm_mul(s_k[h * D + i + half], inv, a.k_norm[i + half]);
        float y0, y1;
        rotate(x0, x1, s_cos[i], s_sin[i], y0, y1);
        f16* dst = a.k_cache + ((uint64_t)h * a.max_ctx + a.pos + t) * D;
        dst[i] = (f16)y0;
        dst[i + half] = (f16)y1;
    }
    const float* vrow = a.v + (uint64_t)t * H * D;
    for (uint32_t e = tid; e < H * D; e += kPrepThreads) {
        const uint32_t h = e / D, i = e % D;
        a.v_cache[((uint64_t)h * a.max_ctx + a.pos + t) * D + i] = (f16)vrow[e];
    }
}

// ---------------------------------------------------------------------------
// Attention.
// ---------------------------------------------------------------------------
constexpr int kWaves = 4;      // q heads per workgroup, one per wavefront
constexpr int kThreads = kWaves * 64;
constexpr int kQRows = 32;     // q rows per wavefront tile (MFMA M)
constexpr int kKTile = 64;     // keys per LDS stage
constexpr float kRescaleLog2 = 8.0f;

struct PrefillParams {
    const float* q;
    const float4* q_rot;    // fused only: [n_tokens, head_dim / 2] (w0 cos, w1 sin, w0 sin, w1 cos)
    const f16* k_cache;
    const f16* v_cache;
    float* out;
    uint32_t pos, n_tokens, n_q_heads, group, max_ctx;
    uint32_t n_qtiles, n_pairs, n_hgroups, n_items, items_per_xcd;
    float scale_log2, eps;
};

template <int D>
struct PGeo {
    static constexpr int KS = D / 16;              // k-steps of the S product
    static constexpr int DT = D / 32;              // 32-row blocks of O^T
    static constexpr int ROW = D + 8;              // LDS row stride in halves (16-byte pad)
    static constexpr int STAGE = kKTile * ROW;     // halves per K (or V) stage
    static constexpr int CPT = kKTile * D / 8 / kThreads;  // 16-byte chunks per thread per K (or V) tile
};

__device__ __forceinline__ f16x4 lds_read_tr16(const f16* lds_ptr) {
    typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 v4h;
    typedef __attribute__((address_space(3))) v4h lds_v4h;
    const v4h r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_v4h*)(lds_ptr));
    return __builtin_bit_cast(f16x4, r);
}

// Global loads of the K and V tile starting at key0 (rows past kv_end are
// clamped to valid memory; their V rows are zeroed when staged).
template <int D>
__device__ __forceinline__ void load_tile(u32x4 (&kr)[PGeo<D>::CPT], u32x4 (&vr)[PGeo<D>::CPT], const f16* kc,
                                          const f16* vc, uint32_t key0, uint32_t kv_end, int tid) {
#pragma unroll
    for (int u = 0; u < PGeo<D>::CPT; u++) {
        const int c = tid + kThreads * u;
        const uint32_t key = min(key0 + (uint32_t)(c / (D / 8)), kv_end - 1);
        const int col = (c % (D / 8)) * 8;
        kr[u] = *(const u32x4*)(kc + (uint64_t)key * D + col);
        vr[u] = *(const u32x4*)(vc + (uint64_t)key * D + col);
    }
}

template <int D>
__device__ __forceinline__ void store_tile(f16* sk, f16* sv, const u32x4 (&kr)[PGeo<D>::CPT],
                                           const u32x4 (&vr)[PGeo<D>::CPT], uint32_t key0, uint32_t kv_end, int tid) {
#pragma unroll
    for (int u = 0; u < PGeo<D>::CPT; u++) {
        const int c = tid + kThreads * u;
        const int row = c / (D / 8), col = (c % (D / 8)) * 8;
        *(u32x4*)(sk + row * PGeo<D>::ROW + col) = kr[u];
        *(u32x4*)(sv + row * PGeo<D>::ROW + col) = key0 + row < kv_end ? vr[u] : u32x4{0u, 0u, 0u, 0u};
    }
}

// q operands of one lane: row t of head hq, dims ks*16 + 8h .. +8 for every k-step.
// Fused: two passes over the row so that few values are live at once -- the
// sum of squares (the two lanes of a row hold complementary halves), then
// each rope pair of 8-dim chunks (ks, ks + KS/2) is reloaded, normalised,
// rotated with the cos/sin table and rounded to f16.
template <int D, bool FUSED>
__device__ __forceinline__ void load_q(const PrefillParams& p, uint32_t t, uint32_t hq, bool live,
                                       int h, f16x8 (&qop)[PGeo<D>::KS]) {
    constexpr int KS = PGeo<D>::KS;
    const uint32_t tc = min(t, p.n_tokens - 1);
    const bool keep = live && t < p.n_tokens;
    const float* row = p.q + ((uint64_t)tc * p.n_q_heads + hq) * D;
    auto chunk = [&](int ks, float (&x)[8]) {
        const float4 a = *(const float4*)(row + ks * 16 + 8 * h);
        const float4 b = *(const float4*)(row + ks * 16 + 8 * h + 4);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    };
    if constexpr (FUSED) {
        float ss = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            float x[8];
            chunk(ks, x);
#pragma unroll
            for (int j = 0; j < 8; j++) ss += x[j] * x[j];
        }
        ss += lane_xor(ss, 32);
        const float inv = rms_inv(ss, (float)D, p.eps);
        // y0 = inv (x0 w0 c - x1 w1 s), y1 = inv (x0 w0 s + x1 w1 c): the RMSNorm weights
        // folded into the rotation table (q only feeds attention; reassociating
        // moves it by a few f32 ulp before the f16 rounding)
        const float4* rot = p.q_rot + (uint64_t)tc * (D / 2);
#pragma unroll
        for (int ks = 0; ks < KS / 2; ks++) {
            float x0[8], x1[8];
            chunk(ks, x0);
            chunk(ks + KS / 2, x1);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float4 r = rot[ks * 16 + 8 * h + j];
                const float y0 = inv * (x0[j] * r.x - x1[j] * r.y);
                const float y1 = inv * (x0[j] * r.z + x1[j] * r.w);
                qop[ks][j] = (f16)(keep ? y0 : 0.0f);
                qop[ks + KS / 2][j] = (f16)(keep ? y1 : 0.0f);
            }
        }
    } else {
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            float x[8];
            chunk(ks, x);
#pragma unroll
            for (int j = 0; j < 8; j++) qop[ks][j] = (f16)(keep ? x[j] : 0.0f);
        }
    }
}

template <int D, bool FUSED>
__global__ __launch_bounds__(kThreads) void prefill_attention_kernel(PrefillParams p) {
    using G = PGeo<D>;
    constexpr int KS = G::KS, DT = G::DT, CPT = G::CPT;
    __shared__ __attribute__((aligned(16))) f16 s_k[2 * G::STAGE];
    __shared__ __attribute__((aligned(16))) f16 s_v[2 * G::STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r32 = lane & 31, h = lane >> 5, g16 = lane >> 4, i16 = lane & 15;

    // workgroup -> (kv head, head group, q-tile pair); one kv head per XCD where possible
    uint32_t item = blockIdx.x;
    if (p.items_per_xcd) item = (blockIdx.x % 8) * p.items_per_xcd + blockIdx.x / 8;
    const uint32_t pair = item % p.n_pairs;
    const uint32_t hg = (item / p.n_pairs) % p.n_hgroups;
    const uint32_t kvh = item / (p.n_pairs * p.n_hgroups);
    const uint32_t hin = hg * kWaves + wave;  // head index inside the group
    const bool live = hin < p.group;
    const uint32_t hq = kvh * p.group + (live ? hin : 0);
    const f16* kc = p.k_cache + (uint64_t)kvh * p.max_ctx * D;
    const f16* vc = p.v_cache + (uint64_t)kvh * p.max_ctx * D;


    u32x4 kr[CPT], vr[CPT];
    const uint32_t heavy = p.n_qtiles - 1 - pair;
    for (int sel = 0; sel < 2; sel++) {
        const uint32_t qt = sel == 0 ? heavy : pair;
        if (sel == 1 && qt >= heavy) break;  // the middle tile of an odd count is processed once
        const uint32_t q0 = qt * kQRows;
        const uint32_t t = q0 + r32;
        const uint64_t t_abs = (uint64_t)p.pos + t;
        const uint32_t kv_end = p.pos + min(p.n_tokens, q0 + kQRows);  // keys this tile needs (exclusive)
        const uint32_t n_kt = (kv_end + kKTile - 1) / kKTile;

        f16x8 qop[KS];
        load_q<D, FUSED>(p, t, hq, live, h, qop);

        f32x16 O[DT];
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int i = 0; i < 16; i++) O[dt][i] = 0.0f;
        float m_ref = -INFINITY, l_sum = 0.0f;

        load_tile<D>(kr, vr, kc, vc, 0, kv_end, tid);
        store_tile<D>(s_k, s_v, kr, vr, 0, kv_end, tid);
        __syncthreads();

        for (uint32_t j = 0; j < n_kt; j++) {
            const uint32_t key0 = j * kKTile;
            const bool more = j + 1 < n_kt;
            if (more) load_tile<D>(kr, vr, kc, vc, key0 + kKTile, kv_end, tid);
            const f16* sk = s_k + (j & 1) * G::STAGE;
            const f16* sv = s_v + (j & 1) * G::STAGE;

            // S^T for the two 32-key halves of the tile
            f32x16 S[2];
#pragma unroll
            for (int kh = 0; kh < 2; kh++) {
                f32x16 acc;
#pragma unroll
                for (int i = 0; i < 16; i++) acc[i] = 0.0f;
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    const f16x8 a = *(const f16x8*)(sk + (32 * kh + r32) * G::ROW + ks * 16 + 8 * h);
                    acc = mfma_32x32x16(a, qop[ks], acc);
                }
                S[kh] = acc;
            }
            // lane: query row t; score r of half kh is key key0 + 32kh + 8(r/4) + 4h + r%4.
            // Softmax in place on the accumulators (log2 domain).
#pragma unroll
            for (int kh = 0; kh < 2; kh++) S[kh] *= p.scale_log2;
            if (key0 + kKTile - 1 > (uint64_t)p.pos + q0) {  // tile crosses the diagonal (uniform)
#pragma unroll
                for (int kh = 0; kh < 2; kh++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const uint64_t key = key0 + 32 * kh + 8 * (r / 4) + 4 * h + (r % 4);
                        if (key > t_abs) S[kh][r] = -INFINITY;
                    }
            }
            float mx = S[0][0];
#pragma unroll
            for (int kh = 0; kh < 2; kh++)
#pragma unroll
                for (int r = 0; r < 16; r++) mx = fmaxf(mx, S[kh][r]);
            mx = fmaxf(mx, lane_xor(mx, 32));
            if (j == 0) {
                m_ref = mx;  // key 0 is always visible, so mx is finite
            } else if (__ballot(mx > m_ref + kRescaleLog2) != 0) {
                const float m_new = mx > m_ref + kRescaleLog2 ? mx : m_ref;
                const float alpha = fast_exp2(m_ref - m_new);
                l_sum *= alpha;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) O[dt] *= alpha;
                m_ref = m_new;
            }
            f16x8 pop[4];  // P^T operand of key step m: scores r = 8(m%2) + jj of half m/2
            float psum = 0.0f;
#pragma unroll
            for (int m = 0; m < 4; m++)
#pragma unroll
                for (int jj = 0; jj < 8; jj++) {
                    const float pv = fast_exp2(S[m / 2][8 * (m % 2) + jj] - m_ref);
                    psum += pv;
                    pop[m][jj] = (f16)pv;
                }
            l_sum += psum;

            // O^T += V^T . P^T; k-slot (h, jj) of step m is key 16m + 8(jj/4) + 4h + jj%4.
            // Transpose read: lane i of a 16-lane group addresses row base + i/4, columns
            // c0 + 4(i%4); lane j receives column c0 + j of the 4 rows.
#pragma unroll
            for (int m = 0; m < 4; m++)
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    const int col = dt * 32 + 16 * (g16 & 1) + 4 * (i16 & 3);
                    const int hh = g16 >> 1;
                    const f16x4 lo = lds_read_tr16(sv + (16 * m + 4 * hh + (i16 >> 2)) * G::ROW + col);
                    const f16x4 hi = lds_read_tr16(sv + (16 * m + 8 + 4 * hh + (i16 >> 2)) * G::ROW + col);
                    const f16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    O[dt] = mfma_32x32x16(a, pop[m], O[dt]);
                }

            if (more) store_tile<D>(s_k + ((j + 1) & 1) * G::STAGE, s_v + ((j + 1) & 1) * G::STAGE, kr, vr,
                                    key0 + kKTile, kv_end, tid);
            __syncthreads();
        }

        if (live && t < p.n_tokens) {
            float l = l_sum + lane_xor(l_sum, 32);
            const float inv_l = 1.0f / l;
            float* out = p.out + ((uint64_t)t * p.n_q_heads + hq) * D;
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int i4 = 0; i4 < 4; i4++) {
                    const int d = dt * 32 + 8 * i4 + 4 * h;
                    *(float4*)(out + d) = float4{O[dt][i4 * 4 + 0] * inv_l, O[dt][i4 * 4 + 1] * inv_l,
                                                 O[dt][i4 * 4 + 2] * inv_l, O[dt][i4 * 4 + 3] * inv_l};
                }
        }
    }
}

}  // namespace

bool prefill_prep_supported(uint32_t n_kv_heads, uint32_t head_dim) {
    return (uint64_t)n_kv_heads * head_dim <= kPrepMaxRow && head_dim % 4 == 0;
}

int launch_kv_prep(ds5_hip_ctx* ctx, const KvPrepLaunch& a, float4* q_rot) {
    if (a.n_tokens == 0) return DS5_OK;
    DS5_TIMED_LAUNCH(ctx, "prefill_prep_kernel", prefill_prep_kernel, dim3(a.n_tokens), dim3(kPrepThreads), 0, ctx->stream, a,
                     q_rot, *a.table);
    return ds5_after_launch(ctx, "prefill_prep_kernel");
}

int launch_prefill(ds5_hip_ctx* ctx, const PrefillLaunch& a) {
    if (a.n_tokens == 0) return DS5_OK;
    PrefillParams p{};
    p.q = a.q;
    p.q_rot = a.q_rot;
    p.k_cache = a.k_cache;
    p.v_cache = a.v_cache;
    p.out = a.out;
    p.pos = a.pos;
    p.n_tokens = a.n_tokens;
    p.n_q_heads = a.n_q_heads;
    p.group = a.n_q_heads / a.n_kv_heads;
    p.max_ctx = a.max_ctx;
    p.n_qtiles = (a.n_tokens + kQRows - 1) / kQRows;
    p.n_pairs = (p.n_qtiles + 1) / 2;
    p.n_hgroups = (p.group + kWaves - 1) / kWaves;
    p.n_items = a.n_kv_heads * p.n_hgroups * p.n_pairs;
    p.items_per_xcd = p.n_items % 8 == 0 ? p.n_items / 8 : 0;
    p.scale_log2 = a.scale * 1.4426950408889634f;
    p.eps = a.eps;
    const dim3 grid(p.n_items);
    const bool fused = a.q_rot != nullptr;
    if (a.head_dim == 128) {
        if (fused)
            DS5_TIMED_LAUNCH(ctx, "prefill_attention_kernel", (prefill_attention_kernel<128, true>), grid, dim3(kThreads), 0,
                             ctx->stream, p);
        else
            DS5_TIMED_LAUNCH(ctx, "prefill_attention_kernel", (prefill_attention_kernel<128, false>), grid, dim3(kThreads), 0,
                             ctx->stream, p);
    } else {
        if (fused)
            DS5_TIMED_LAUNCH(ctx, "prefill_attention_kernel", (prefill_attention_kernel<64, true>), grid, dim3(kThreads), 0,
                             ctx->stream, p);
        else
            DS5_TIMED_LAUNCH(ctx, "prefill_attention_kernel", (prefill_attention_kernel<64, false>), grid, dim3(kThreads), 0,
                             ctx->stream, p);
    }
    return ds5_after_launch(ctx, "prefill_attention_kernel");
}
