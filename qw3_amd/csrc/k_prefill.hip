// k_prefill.hip -- causal flash-attention prefill on gfx950 f16 MFMA with f32
// accumulation, over the f16 KV cache.
//
// Semantics: kernels_b.zig:29-133 for n_tokens > 1 -- query token t (absolute
// position pos + t) of q head h attends cache positions 0..pos+t of kv head
// h / group; softmax(scale * q.k) in f32.
//
// Decomposition: one workgroup = 4 wavefronts = 128 query rows of one q head;
// each wavefront owns 32 rows. Workgroups run heaviest-first (the last query
// tiles see the most keys). K/V are streamed in 32-position tiles through
// LDS, shared by the 4 wavefronts:
//   S^T[32 pos x 32 q] = K[32 x D] . Q^T        v_mfma_f32_32x32x16_f16
//   O^T[D x 32 q]     += V^T[D x 32] . P^T      v_mfma_f32_32x32x16_f16
// With S^T (positions as rows) a lane holds 16 scores of ONE query row, so
// row max / sum need one lane exchange. Q^T operands stay in registers for
// the whole key loop. P is rounded to f16 for the P.V product; softmax state
// (running max and sum, log2 domain) is f32.
//
// With q_norm set the kernel takes raw q projections and applies the step's
// per-head RMSNorm and NeoX rope itself (serial-order sum, (v*inv)*w, unfused
// rotation: kernels_a.zig:84-89, :117-126) before rounding q to f16.
#include "ds5_common.hpp"

namespace {

constexpr int kQRows = 128;  // query rows per workgroup
constexpr int kKTile = 32;   // key positions per LDS tile

struct PrefillParams {
    const float* q;
    const float* q_norm;
    const int32_t* positions;
    const f16* k_cache;
    const f16* v_cache;
    float* out;
    uint32_t pos, n_tokens, n_q_heads, group, max_ctx, n_qtiles;
    float scale_log2, eps, freq_scale;
};

template <bool FUSED_Q, int D>
__device__ __forceinline__ void load_q_operands(const PrefillParams& p, const RopeTable& table, uint32_t t,
                                                uint32_t hq, int half_id, f16x8 (&qop)[D / 16]) {
#pragma clang fp contract(off)
    constexpr int KS = D / 16;
    float x[KS][8];
    if (t >= p.n_tokens) {
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
#pragma unroll
            for (int j = 0; j < 8; j++) qop[ks][j] = (f16)0.0f;
        return;
    }
    const float* row = p.q + ((uint64_t)t * p.n_q_heads + hq) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const float4 a = *(const float4*)(row + ks * 16 + 8 * half_id);
        const float4 c = *(const float4*)(row + ks * 16 + 8 * half_id + 4);
        x[ks][0] = a.x; x[ks][1] = a.y; x[ks][2] = a.z; x[ks][3] = a.w;
        x[ks][4] = c.x; x[ks][5] = c.y; x[ks][6] = c.z; x[ks][7] = c.w;
    }
    if constexpr (FUSED_Q) {
        // 1/rms of the full row, summed serially in element order.
        float sumsq = 0.0f;
        for (int i = 0; i < D; i += 4) {
            const float4 v = *(const float4*)(row + i);
            sumsq += v.x * v.x;
            sumsq += v.y * v.y;
            sumsq += v.z * v.z;
            sumsq += v.w * v.w;
        }
        const float inv = rms_inv(sumsq, (float)D, p.eps);
        const float tpos = (float)p.positions[t];
        // This lane holds dims ks*16 + 8*half_id + j; the rope partner of a
        // dim d < D/2 is d + D/2, which is k-step ks + D/32 of the same lane.
#pragma unroll
        for (int ks = 0; ks < KS / 2; ks++) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int d = ks * 16 + 8 * half_id + j;
                const float x0 = x[ks][j] * inv * p.q_norm[d];
                const float x1 = x[ks + KS / 2][j] * inv * p.q_norm[d + D / 2];
                const float angle = tpos * p.freq_scale * table.inv[d];
                const float c = cosf(angle);
                const float s = sinf(angle);
                x[ks][j] = x0 * c - x1 * s;
                x[ks + KS / 2][j] = x0 * s + x1 * c;
            }
        }
    }
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
#pragma unroll
        for (int j = 0; j < 8; j++) qop[ks][j] = (f16)x[ks][j];
}

template <int D, bool FUSED_Q>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillParams p, RopeTable table) {
    constexpr int KS = D / 16;               // k-steps of the Q.K product
    constexpr int DT = D / 32;               // 32-row tiles of O^T
    constexpr int ROW = D + 8;               // LDS row stride in halves (16-byte pad)
    constexpr int CHUNKS = kKTile * D / 8;   // 16-byte chunks per K (or V) tile
    __shared__ __attribute__((aligned(16))) f16 s_k[kKTile * ROW];
    __shared__ __attribute__((aligned(16))) f16 s_v[kKTile * ROW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, half_id = lane >> 5;
    const uint32_t qtile = p.n_qtiles - 1 - blockIdx.x;  // heaviest first
    const uint32_t hq = blockIdx.y;
    const uint32_t kvh = hq / p.group;
    const uint32_t q0 = qtile * kQRows;
    const uint32_t t = q0 + wave * 32 + r32;       // this lane's query row
    const uint64_t t_abs = (uint64_t)p.pos + t;    // its absolute position
    const uint32_t last_row = min(p.n_tokens, q0 + kQRows);             // exclusive
    const uint64_t kv_end = (uint64_t)p.pos + last_row;                 // keys this WG needs
    const uint64_t wave_last = (uint64_t)p.pos + min(p.n_tokens, q0 + wave * 32 + 32);  // exclusive

    const f16* kc = p.k_cache + (uint64_t)kvh * p.max_ctx * D;
    const f16* vc = p.v_cache + (uint64_t)kvh * p.max_ctx * D;

    f16x8 qop[KS];
    load_q_operands<FUSED_Q, D>(p, table, t, hq, half_id, qop);

    f32x16 O[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int i = 0; i < 16; i++) O[dt][i] = 0.0f;
    float m_run = -INFINITY, l_lane = 0.0f;

    for (uint64_t kv0 = 0; kv0 < kv_end; kv0 += kKTile) {
        __syncthreads();
        for (int c = tid; c < CHUNKS; c += 256) {
            const int r = c / (D / 8), col = (c % (D / 8)) * 8;
            const uint64_t kp = kv0 + r;
            u32x4 kv = u32x4{0u, 0u, 0u, 0u}, vv = u32x4{0u, 0u, 0u, 0u};
            if (kp < kv_end) {
                kv = *(const u32x4*)(kc + kp * D + col);
                vv = *(const u32x4*)(vc + kp * D + col);
            }
            *(u32x4*)(s_k + r * ROW + col) = kv;
            *(u32x4*)(s_v + r * ROW + col) = vv;
        }
        __syncthreads();
        if (kv0 >= wave_last) continue;  // every row of this wavefront is before the tile

        // S^T = K . Q^T
        f32x16 S;
#pragma unroll
        for (int i = 0; i < 16; i++) S[i] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const f16x8 a = *(const f16x8*)(s_k + r32 * ROW + ks * 16 + 8 * half_id);
            S = mfma_32x32x16(a, qop[ks], S);
        }
        // lane: query row t, key rows 8*(i/4) + 4*half_id + i%4
        float sc[16];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint64_t kp = kv0 + 8 * (i / 4) + 4 * half_id + (i % 4);
            const float s = (kp <= t_abs && kp < kv_end) ? S[i] * p.scale_log2 : -INFINITY;
            sc[i] = s;
            mx = fmaxf(mx, s);
        }
        mx = fmaxf(mx, lane_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = (m_new == -INFINITY) ? 1.0f : fast_exp2(m_run - m_new);
        float psum = 0.0f;
        f16x8 pop[2];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float pi = (m_new == -INFINITY) ? 0.0f : fast_exp2(sc[i] - m_new);
            psum += pi;
            pop[i / 8][i % 8] = (f16)pi;
        }
        m_run = m_new;
        l_lane = l_lane * alpha + psum;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) O[dt] *= alpha;

        // O^T += V^T . P^T ; k-slot (half_id, jj) of step m <-> key row
        // 16m + 8*(jj/4) + 4*half_id + jj%4 (the lane's own score order).
#pragma unroll
        for (int m = 0; m < 2; m++) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                f16x8 a;
#pragma unroll
                for (int jj = 0; jj < 8; jj++) {
                    const int r = 16 * m + 8 * (jj / 4) + 4 * half_id + (jj % 4);
                    a[jj] = s_v[r * ROW + dt * 32 + r32];
                }
                O[dt] = mfma_32x32x16(a, pop[m], O[dt]);
            }
        }
    }

    if (t >= p.n_tokens) return;
    float l = l_lane + lane_xor(l_lane, 32);
    const float inv_l = 1.0f / l;
    float* out = p.out + ((uint64_t)t * p.n_q_heads + hq) * D;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int i4 = 0; i4 < 4; i4++) {
            const int d = dt * 32 + 8 * i4 + 4 * half_id;
            float4 v;
            v.x = O[dt][i4 * 4 + 0] * inv_l;
            v.y = O[dt][i4 * 4 + 1] * inv_l;
            v.z = O[dt][i4 * 4 + 2] * inv_l;
            v.w = O[dt][i4 * 4 + 3] * inv_l;
            *(float4*)(out + d) = v;
        }
}

}  // namespace

int launch_prefill(ds5_hip_ctx* ctx, const PrefillLaunch& a) {
    if (a.n_tokens == 0) return DS5_OK;
    PrefillParams p{};
    p.q = a.q;
    p.q_norm = a.q_norm;
    p.positions = a.positions;
    p.k_cache = a.k_cache;
    p.v_cache = a.v_cache;
    p.out = a.out;
    p.pos = a.pos;
    p.n_tokens = a.n_tokens;
    p.n_q_heads = a.n_q_heads;
    p.group = a.n_q_heads / a.n_kv_heads;
    p.max_ctx = a.max_ctx;
    p.n_qtiles = (a.n_tokens + kQRows - 1) / kQRows;
    p.scale_log2 = a.scale * 1.4426950408889634f;
    p.eps = a.eps;
    p.freq_scale = a.freq_scale;
    const dim3 grid(p.n_qtiles, a.n_q_heads);
    const bool fused = a.q_norm != nullptr;
    const RopeTable table = fused ? *a.table : RopeTable{};
    if (a.head_dim == 128) {
        if (fused)
            DS5_TIMED_LAUNCH(ctx, "prefill_kernel", (prefill_kernel<128, true>), grid, dim3(256), 0, ctx->stream, p, table);
        else
            DS5_TIMED_LAUNCH(ctx, "prefill_kernel", (prefill_kernel<128, false>), grid, dim3(256), 0, ctx->stream, p, table);
    } else {
        if (fused)
            DS5_TIMED_LAUNCH(ctx, "prefill_kernel", (prefill_kernel<64, true>), grid, dim3(256), 0, ctx->stream, p, table);
        else
            DS5_TIMED_LAUNCH(ctx, "prefill_kernel", (prefill_kernel<64, false>), grid, dim3(256), 0, ctx->stream, p, table);
    }
    return ds5_after_launch(ctx, "prefill_kernel");
}
