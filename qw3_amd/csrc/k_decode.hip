// k_decode.hip -- split-K flash-decoding on gfx950 MFMA for one query token
// per sequence over an f16 KV cache (contiguous or paged).
//
// Semantics: kernels_b.zig:29-133 with n_tokens == 1 -- q head h attends
// positions 0..L-1 of kv head h/group with softmax(scale * q.k) in f32.
//
// Work decomposition. One workgroup serves ALL q heads of one kv head (up to
// 16 per workgroup; larger groups use several head subgroups) for one range
// ("split") of `chunk` positions, so each K/V byte is read from HBM once per
// GQA group. A workgroup is WAVES wavefronts; each wavefront takes 32-position
// tiles of the split in turn:
//   S^T[32 pos x 16 heads] = K[32 pos x D] . Q^T      v_mfma_f32_16x16x32_f16
//   O^T[D x 16 heads]     += V^T[D x 32 pos] . P^T    v_mfma_f32_16x16x32_f16
// K goes from HBM straight into MFMA A-operand registers (16-byte loads, a
// lane owns one position row and 8 consecutive dims per k-step). V is staged
// through LDS (coalesced 16-byte loads, padded rows) and read back transposed
// as the A operand of the P.V product. q and p are split into f16 hi + lo
// parts (x = hi + lo exactly to ~22 bits), and both halves are accumulated
// into the same f32 accumulator, so the products keep ~f32 accuracy while
// K/V stay f16. Softmax runs in the log2 domain with running max / sum per
// head; row reductions are lane exchanges inside the 16-lane groups.
// Workgroup partials (max, sum, unnormalised O) go to a workspace and a merge
// kernel combines the splits, unless one split covers the whole context.
//
// Fused mode adds the step's prologue (forward.zig:345-396 order): the
// workgroup normalises and rotates its q heads itself, and the workgroup whose
// split holds the new position normalises and rotates k, appends k and v (f16)
// to the cache, and feeds the new row to the tile from LDS. All of that uses
// the reference's operation order (serial norm sum, (v*inv)*w, unfused rope).
#include "ds5_common.hpp"

namespace {

constexpr int kTile = 32;  // positions per wavefront tile

struct DecodeParams {
    const float* q;
    const float* k_new;
    const float* v_new;
    const float* q_norm;
    const float* k_norm;
    const int32_t* positions;
    f16* k_cache;
    f16* v_cache;
    uint64_t cache_stride;
    const int32_t* page_table;
    const int32_t* seq_lens;
    float* out;
    float* part_o;   // [n_seqs, n_q_heads, n_splits, D]
    float* part_ml;  // [n_seqs, n_q_heads, n_splits, 2]
    uint32_t page_size, max_pages, n_pages;
    uint32_t ctx_len, max_len, chunk, n_splits;
    uint32_t n_q_heads, n_kv_heads, group, n_sub;
    float scale_log2, eps, freq_scale;
};

template <int D>
struct Geometry {
    static constexpr int KK = D / 32;                  // k-steps of the Q.K product
    static constexpr int DT = D / 16;                  // 16-row tiles of O^T
    static constexpr int ROW_BYTES = D * 2 + 8;        // LDS V row, padded: conflict-free transposed reads
    static constexpr int ROW_CHUNKS = D / 8;           // 16-byte chunks per cache row
    static constexpr int V_CHUNKS = kTile * ROW_CHUNKS / 64;  // 16-byte V loads per lane per tile
};

__device__ __forceinline__ u32x4 load16(const f16* p) { return *(const u32x4*)p; }

template <bool PAGED>
__device__ __forceinline__ int64_t cache_row(const DecodeParams& p, uint32_t b, uint32_t pos) {
    if (!PAGED) return pos;
    const int32_t page = p.page_table[(uint64_t)b * p.max_pages + pos / p.page_size];
    if (page < 0 || (uint32_t)page >= p.n_pages) return -1;
    return (int64_t)page * p.page_size + pos % p.page_size;
}

// Serial-order f32 row norm + NeoX rope of one row held in LDS (in place);
// row_inv is the row's 1/rms computed by one thread.
__device__ __forceinline__ void rope_pair(float x0, float x1, float angle, float& y0, float& y1) {
#pragma clang fp contract(off)
    const float c = cosf(angle);
    const float s = sinf(angle);
    y0 = x0 * c - x1 * s;
    y1 = x0 * s + x1 * c;
}

__device__ __forceinline__ float row_inv_rms(const float* row, int dim, float eps) {
#pragma clang fp contract(off)
    float sumsq = 0.0f;
    for (int i = 0; i < dim; i++) sumsq += row[i] * row[i];
    return rms_inv(sumsq, (float)dim, eps);
}

__device__ __forceinline__ float norm_mul(float v, float inv, float w) {
#pragma clang fp contract(off)
    return v * inv * w;
}

__device__ __forceinline__ float rope_angle(float pos, float freq_scale, float inv) {
#pragma clang fp contract(off)
    return pos * freq_scale * inv;
}

template <int D, int WAVES, bool FUSED, bool PAGED>
__global__ __launch_bounds__(WAVES * 64) void decode_splitk_kernel(DecodeParams p, RopeTable table) {
    using Gm = Geometry<D>;
    constexpr int KK = Gm::KK, DT = Gm::DT, VC = Gm::V_CHUNKS, RC = Gm::ROW_CHUNKS;
    constexpr int NT = WAVES * 64;

    // LDS: V staging per wavefront, reused for the cross-wave reduction.
    constexpr int V_BYTES = WAVES * kTile * Gm::ROW_BYTES;
    constexpr int O_STRIDE = D + 4;  // padded row of the cross-wave O buffer
    constexpr int O_BYTES = WAVES * 16 * O_STRIDE * 4;
    __shared__ __attribute__((aligned(16))) char s_raw[V_BYTES > O_BYTES ? V_BYTES : O_BYTES];
    __shared__ float s_m[WAVES][16], s_l[WAVES][16];
    __shared__ float s_q[FUSED ? 16 : 1][FUSED ? D : 1];
    __shared__ float s_krow[FUSED ? D : 1];
    __shared__ float s_inv[17];
    __shared__ __attribute__((aligned(16))) f16 s_knew[FUSED ? D : 8];
    __shared__ __attribute__((aligned(16))) f16 s_vnew[FUSED ? D : 8];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const uint32_t split = blockIdx.x;
    const uint32_t kvh = blockIdx.y / p.n_sub, sub = blockIdx.y % p.n_sub;
    const uint32_t b = blockIdx.z;
    const uint32_t n0 = sub * 16;
    const int NS = (int)min(16u, p.group - n0);
    const uint32_t hq0 = kvh * p.group + n0;  // first q head of this workgroup

    uint32_t L = p.ctx_len;
    if (PAGED) {
        const int32_t len = p.seq_lens[b];
        if (len < 1 || (uint32_t)len > p.max_len) {
            // Out-of-range sequence: poison its output (written once) and skip it.
            if (split == 0)
                for (int i = tid; i < NS * D; i += NT)
                    p.out[((uint64_t)b * p.n_q_heads + hq0) * D + i] = __builtin_nanf("");
            return;
        }
        L = (uint32_t)len;
    }
    const uint32_t start = split * p.chunk;
    if (start >= L) return;  // whole workgroup idle (uniform)
    const uint32_t end = min(L, start + p.chunk);
    const uint32_t n_tiles = (end - start + kTile - 1) / kTile;
    const uint32_t newpos = L - 1;
    const bool has_new = FUSED && newpos >= start && newpos < end;

    const uint64_t head_base = (uint64_t)kvh * p.cache_stride;  // in rows
    const f16* kbase = p.k_cache + head_base * D;
    const f16* vbase = p.v_cache + head_base * D;

    // ---------------- fused prologue: q/k norm + rope, k/v append ----------
    if constexpr (FUSED) {
        const float* qsrc = p.q + ((uint64_t)b * p.n_q_heads + hq0) * D;
        for (int i = tid; i < NS * D; i += NT) s_q[i / D][i % D] = qsrc[i];
        const uint64_t kv_off = ((uint64_t)b * p.n_kv_heads + kvh) * D;
        if (has_new)
            for (int i = tid; i < D; i += NT) s_krow[i] = p.k_new[kv_off + i];
        __syncthreads();
        if (tid < NS) s_inv[tid] = row_inv_rms(s_q[tid], D, p.eps);
        if (has_new && tid == 16) s_inv[16] = row_inv_rms(s_krow, D, p.eps);
        __syncthreads();
        const float qpos = PAGED ? (float)newpos : (float)p.positions[0];
        for (int i = tid; i < NS * (D / 2); i += NT) {
            const int n = i / (D / 2), j = i % (D / 2);
            const float inv = s_inv[n];
            const float x0 = norm_mul(s_q[n][j], inv, p.q_norm[j]);
            const float x1 = norm_mul(s_q[n][j + D / 2], inv, p.q_norm[j + D / 2]);
            float y0, y1;
            rope_pair(x0, x1, rope_angle(qpos, p.freq_scale, table.inv[j]), y0, y1);
            s_q[n][j] = y0;
            s_q[n][j + D / 2] = y1;
        }
        if (has_new) {
            const int64_t row = cache_row<PAGED>(p, b, newpos);
            f16* kdst = row >= 0 ? p.k_cache + (head_base + row) * D : nullptr;
            f16* vdst = row >= 0 ? p.v_cache + (head_base + row) * D : nullptr;
            for (int j = tid; j < D / 2; j += NT) {
                const float inv = s_inv[16];
                const float x0 = norm_mul(s_krow[j], inv, p.k_norm[j]);
                const float x1 = norm_mul(s_krow[j + D / 2], inv, p.k_norm[j + D / 2]);
                float y0, y1;
                rope_pair(x0, x1, rope_angle(qpos, p.freq_scale, table.inv[j]), y0, y1);
                const f16 h0 = (f16)y0, h1 = (f16)y1;
                s_knew[j] = h0;
                s_knew[j + D / 2] = h1;
                if (kdst) {
                    kdst[j] = h0;
                    kdst[j + D / 2] = h1;
                }
            }
            for (int j = tid; j < D; j += NT) {
                const f16 hv = (f16)p.v_new[kv_off + j];
                s_vnew[j] = hv;
                if (vdst) vdst[j] = hv;
            }
        }
        __syncthreads();
    }

    // ---------------- Q^T operands (B of the S product), hi + lo ------------
    f16x8 qh[KK], ql[KK];
    {
        const bool valid = c16 < NS;
        const float* qrow = p.q + ((uint64_t)b * p.n_q_heads + hq0 + (valid ? c16 : 0)) * D;
#pragma unroll
        for (int kk = 0; kk < KK; kk++) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int d = kk * 32 + 8 * g + j;
                float x = 0.0f;
                if (valid) {
                    if constexpr (FUSED)
                        x = s_q[c16][d];
                    else
                        x = qrow[d];
                }
                const f16 hi = (f16)x;
                qh[kk][j] = hi;
                ql[kk][j] = (f16)(x - (float)hi);
            }
        }
    }

    // ---------------- main loop over this wavefront's tiles -----------------
    char* vlds = s_raw + wave * kTile * Gm::ROW_BYTES;
    f32x4 O[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) O[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_lane = 0.0f;

    for (uint32_t it = wave; it < n_tiles; it += WAVES) {
        const uint32_t p0 = start + it * kTile;
        // K rows straight into A operands: lane row c16 of each 16-row half.
        u32x4 kop[2][KK];
#pragma unroll
        for (int st = 0; st < 2; st++) {
            const uint32_t pos = p0 + 16 * st + c16;
            const int64_t row = pos < end ? cache_row<PAGED>(p, b, pos) : -1;
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                u32x4 v = u32x4{0u, 0u, 0u, 0u};
                if (row >= 0) {
                    if (FUSED && pos == newpos)
                        v = *(const u32x4*)(s_knew + kk * 32 + 8 * g);
                    else
                        v = load16(kbase + (uint64_t)row * D + kk * 32 + 8 * g);
                }
                kop[st][kk] = v;
            }
        }
        // V tile -> LDS (row-major, padded). Rows past the split end are zero.
        u32x4 vreg[VC];
#pragma unroll
        for (int r = 0; r < VC; r++) {
            const int c = lane + 64 * r;
            const uint32_t pos = p0 + c / RC;
            const int64_t row = pos < end ? cache_row<PAGED>(p, b, pos) : -1;
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (row >= 0) {
                if (FUSED && pos == newpos)
                    v = *(const u32x4*)(s_vnew + (c % RC) * 8);
                else
                    v = load16(vbase + (uint64_t)row * D + (c % RC) * 8);
            }
            vreg[r] = v;
        }
#pragma unroll
        for (int r = 0; r < VC; r++) {
            const int c = lane + 64 * r;
            uint32_t* dst = (uint32_t*)(vlds + (c / RC) * Gm::ROW_BYTES + (c % RC) * 16);
            *(uint2*)dst = uint2{vreg[r][0], vreg[r][1]};
            *(uint2*)(dst + 2) = uint2{vreg[r][2], vreg[r][3]};
        }

        // S^T = K . Q^T (hi and lo halves into one accumulator)
        f32x4 S[2];
#pragma unroll
        for (int st = 0; st < 2; st++) {
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                const f16x8 a = __builtin_bit_cast(f16x8, kop[st][kk]);
                acc = mfma_16x16x32(a, qh[kk], acc);
                acc = mfma_16x16x32(a, ql[kk], acc);
            }
            S[st] = acc;
        }
        // Scores of this lane: head c16, positions p0 + 16*st + 4*g + i.
        float sc[8];
        float mx = -INFINITY;
#pragma unroll
        for (int st = 0; st < 2; st++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t pos = p0 + 16 * st + 4 * g + i;
                const float s = pos < end ? S[st][i] * p.scale_log2 : -INFINITY;
                sc[st * 4 + i] = s;
                mx = fmaxf(mx, s);
            }
        mx = fmaxf(mx, lane_xor(mx, 16));
        mx = fmaxf(mx, lane_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2(m_run - m_new);
        m_run = m_new;
        f16x8 ph, pl;
        float psum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float pj = fast_exp2(sc[j] - m_new);
            psum += pj;
            const f16 hi = (f16)pj;
            ph[j] = hi;
            pl[j] = (f16)(pj - (float)hi);
        }
        l_lane = l_lane * alpha + psum;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) O[dt] *= alpha;

        // O^T += V^T . P^T. k-slot (g, j) <-> tile row 4g+j (j<4), 16+4g+j-4.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const f16* vl = (const f16*)vlds;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            f16x8 a;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int r = (j < 4) ? 4 * g + j : 16 + 4 * g + (j - 4);
                a[j] = vl[r * (Gm::ROW_BYTES / 2) + dt * 16 + c16];
            }
            O[dt] = mfma_16x16x32(a, ph, O[dt]);
            O[dt] = mfma_16x16x32(a, pl, O[dt]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // ---------------- combine wavefronts, emit partial or output ------------
    float l_w = l_lane + lane_xor(l_lane, 16);
    l_w += lane_xor(l_w, 32);
    __syncthreads();  // every wavefront is done with its V staging area
    float* s_o = (float*)s_raw;  // [WAVES][16][O_STRIDE]
    if (g == 0) {
        s_m[wave][c16] = m_run;
        s_l[wave][c16] = l_w;
    }
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int i = 0; i < 4; i++) s_o[(wave * 16 + c16) * O_STRIDE + dt * 16 + 4 * g + i] = O[dt][i];
    __syncthreads();

    const bool single = p.n_splits == 1;
    for (int idx = tid; idx < NS * D; idx += NT) {
        const int n = idx / D, d = idx % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < WAVES; w++) M = fmaxf(M, s_m[w][n]);
        float acc = 0.0f, lt = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; w++) {
            const float f = fast_exp2(s_m[w][n] - M);
            acc += s_o[(w * 16 + n) * O_STRIDE + d] * f;
            lt += s_l[w][n] * f;
        }
        const uint64_t qh_idx = (uint64_t)b * p.n_q_heads + hq0 + n;
        if (single) {
            p.out[qh_idx * D + d] = acc / lt;
        } else {
            p.part_o[(qh_idx * p.n_splits + split) * D + d] = acc;
            if (d == 0) {
                p.part_ml[(qh_idx * p.n_splits + split) * 2 + 0] = M;
                p.part_ml[(qh_idx * p.n_splits + split) * 2 + 1] = lt;
            }
        }
    }
}

// Merge of the split partials: one workgroup per (sequence, q head), one
// thread per output dim.
template <int D>
__global__ __launch_bounds__(D) void decode_merge_kernel(DecodeParams p) {
    const uint32_t b = blockIdx.x / p.n_q_heads;
    const uint64_t qh_idx = blockIdx.x;
    uint32_t L = p.ctx_len;
    if (p.seq_lens) {
        const int32_t len = p.seq_lens[b];
        if (len < 1 || (uint32_t)len > p.max_len) return;  // poisoned by the split kernel
        L = (uint32_t)len;
    }
    const uint32_t ns = (L + p.chunk - 1) / p.chunk;
    const float* ml = p.part_ml + qh_idx * p.n_splits * 2;
    float M = -INFINITY;
    for (uint32_t s = 0; s < ns; s++) M = fmaxf(M, ml[2 * s]);
    float acc = 0.0f, lt = 0.0f;
    const float* po = p.part_o + qh_idx * p.n_splits * D + threadIdx.x;
    for (uint32_t s = 0; s < ns; s++) {
        const float f = fast_exp2(ml[2 * s] - M);
        acc += po[(uint64_t)s * D] * f;
        lt += ml[2 * s + 1] * f;
    }
    p.out[qh_idx * D + threadIdx.x] = acc / lt;
}

template <int D, int WAVES>
int launch_decode_d(ds5_hip_ctx* ctx, const DecodeLaunch& a, const DecodeParams& prm, dim3 grid) {
    const dim3 block(WAVES * 64);
    const bool paged = a.page_table != nullptr;
    if (a.fused && paged)
        DS5_TIMED_LAUNCH(ctx, "decode_splitk_kernel", (decode_splitk_kernel<D, WAVES, true, true>), grid, block, 0, ctx->stream, prm, *a.table);
    else if (a.fused)
        DS5_TIMED_LAUNCH(ctx, "decode_splitk_kernel", (decode_splitk_kernel<D, WAVES, true, false>), grid, block, 0, ctx->stream, prm, *a.table);
    else if (paged)
        DS5_TIMED_LAUNCH(ctx, "decode_splitk_kernel", (decode_splitk_kernel<D, WAVES, false, true>), grid, block, 0, ctx->stream, prm, RopeTable{});
    else
        DS5_TIMED_LAUNCH(ctx, "decode_splitk_kernel", (decode_splitk_kernel<D, WAVES, false, false>), grid, block, 0, ctx->stream, prm, RopeTable{});
    int rc = ds5_after_launch(ctx, "decode_splitk_kernel");
    if (rc || prm.n_splits == 1) return rc;
    DS5_TIMED_LAUNCH(ctx, "decode_merge_kernel", decode_merge_kernel<D>, dim3(a.n_seqs * a.n_q_heads), dim3(D), 0, ctx->stream, prm);
    return ds5_after_launch(ctx, "decode_merge_kernel");
}

}  // namespace

int launch_decode(ds5_hip_ctx* ctx, const DecodeLaunch& a) {
    constexpr int WAVES = 4;
    const uint32_t group = a.n_q_heads / a.n_kv_heads;
    const uint32_t n_sub = (group + 15) / 16;
    const uint32_t max_len = a.max_len;
    if (a.n_seqs == 0 || max_len == 0) return DS5_OK;

    // Positions per split: enough workgroups to cover the CUs about twice,
    // never fewer than one 32-position tile per wavefront.
    uint32_t chunk = ctx->decode_chunk;
    if (chunk == 0) {
        const uint64_t units = (uint64_t)a.n_seqs * a.n_kv_heads * n_sub;
        const uint64_t target = 2ull * (ctx->cu_count > 0 ? ctx->cu_count : 256);
        const uint64_t per_unit = (target + units - 1) / units;  // splits wanted per (seq, kv head)
        uint64_t c = (max_len + per_unit - 1) / per_unit;
        c = c < 128 ? 128 : c;
        chunk = (uint32_t)c;
    }
    chunk = (chunk + kTile - 1) / kTile * kTile;
    const uint32_t n_splits = (max_len + chunk - 1) / chunk;

    DecodeParams prm{};
    prm.q = a.q;
    prm.k_new = a.k_new;
    prm.v_new = a.v_new;
    prm.q_norm = a.q_norm;
    prm.k_norm = a.k_norm;
    prm.positions = a.positions;
    prm.k_cache = a.k_cache;
    prm.v_cache = a.v_cache;
    prm.cache_stride = a.cache_stride;
    prm.page_table = a.page_table;
    prm.seq_lens = a.seq_lens;
    prm.out = a.out;
    prm.page_size = a.page_size;
    prm.max_pages = a.max_pages;
    prm.n_pages = a.page_table ? (uint32_t)(a.cache_stride / a.page_size) : 0;
    prm.ctx_len = a.ctx_len;
    prm.max_len = max_len;
    prm.chunk = chunk;
    prm.n_splits = n_splits;
    prm.n_q_heads = a.n_q_heads;
    prm.n_kv_heads = a.n_kv_heads;
    prm.group = group;
    prm.n_sub = n_sub;
    prm.scale_log2 = a.scale * 1.4426950408889634f;
    prm.eps = a.eps;
    prm.freq_scale = a.freq_scale;
    if (n_splits > 1) {
        const size_t n_part = (size_t)a.n_seqs * a.n_q_heads * n_splits;
        void* ws = nullptr;
        int rc = ds5_workspace(ctx, n_part * ((size_t)a.head_dim + 2) * sizeof(float), &ws);
        if (rc) return rc;
        prm.part_o = (float*)ws;
        prm.part_ml = prm.part_o + n_part * a.head_dim;
    }
    const dim3 grid(n_splits, a.n_kv_heads * n_sub, a.n_seqs);
    if (a.head_dim == 128) return launch_decode_d<128, WAVES>(ctx, a, prm, grid);
    return launch_decode_d<64, WAVES>(ctx, a, prm, grid);
}
