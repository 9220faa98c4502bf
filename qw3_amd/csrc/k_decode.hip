// k_decode.hip -- split-K flash decoding on gfx950 MFMA: one query token per
// sequence over an f16 KV cache (contiguous or paged).
//
// Semantics: kernels_b.zig:29-133 with n_tokens == 1 -- q head h attends
// positions 0..L-1 of kv head h/group with softmax(scale * q.k) in f32.
//
// Work decomposition. A workgroup (4 wavefronts) serves up to 16 q heads of one
// kv head -- the whole GQA group for the Qwen3 shapes -- over one range
// ("split") of `chunk` positions, so each K/V byte is read from HBM once per
// group. Each wavefront owns 32-position tiles of the split:
//   S^T[32 pos x 16 heads] = K[32 pos x D] . Q^T      v_mfma_f32_16x16x32_f16
//   O^T[D x 16 heads]     += V^T[D x 32 pos] . P^T    v_mfma_f32_16x16x32_f16
// K rows go from HBM straight into MFMA A-operand registers (16-byte loads);
// V rows are staged through a wavefront-private LDS area and read back
// transposed. q and p are split into f16 hi + lo halves accumulated into one
// f32 accumulator, so the products keep ~22 significant bits while K/V stay
// f16. Softmax runs in the log2 domain against a per-head reference that only
// moves when a tile's maximum exceeds it by more than 2^8 (the lazy rescale),
// so the O accumulators are rescaled rarely.
//
// Latency structure (a decode layer is ~2 us of HBM time, so the critical path
// matters): every wavefront issues its first tile's K/V loads before anything
// else, the q prologue (load, norm, rope, scale, hi/lo split) runs while they
// are in flight, and later tiles are prefetched one tile ahead. Workgroup
// barriers before the main loop are LDS-only, so they never wait for the
// outstanding K/V loads. With one wavefront per SIMD every instruction a
// wavefront issues is on the critical path, so the q operands are built once
// per workgroup (not per wavefront) and the wavefront partials are combined
// through LDS.
//
// Splits combine through a workspace: each workgroup writes its unnormalised
// O, its reference max and its sum; decode_merge_kernel combines the splits of
// every (sequence, q head) (one split per lane, or split slots per thread when
// the rows are many). A single split
// writes the output directly. Cross-workgroup combining inside one launch was
// measured to be slower on this part than the second launch.
//
// Fused mode adds the step's prologue in the engine's op order
// (forward.zig:345-396): the workgroup normalises and rotates its q heads
// (serial-order f32 sum of squares, (v*inv)*w, unfused rotation), and the
// workgroup whose split holds the new position normalises and rotates k,
// appends k and v (f16) to the cache and substitutes the new row into its tile.
#include "ds5_common.hpp"

namespace {

constexpr int kTile = ds5idx::kDecTile;    // positions per wavefront tile
constexpr int kWaves = ds5idx::kDecWaves;  // wavefronts per workgroup (one per SIMD)
constexpr int kThreads = kWaves * 64;
constexpr int kHeads = ds5idx::kDecHeads;  // q heads per workgroup (the MFMA N dimension)
constexpr float kRescaleLog2 = 8.0f;       // lazy-rescale threshold (p <= 2^8 between rescales)
constexpr uint32_t kMaxSplits = ds5idx::kDecMaxSplits;  // splits per sequence at most
constexpr uint32_t kPlanMaxSeqs = 4096;  // paged plan: lengths staged in the V staging area

struct DecodeParams {
    const float* q;
    const float* k_new;
    const float* v_new;
    const float* q_norm;
    const float* k_norm;
    const int32_t* positions;
    f16* k_cache;
    f16* v_cache;
    uint64_t cache_stride;  // rows per kv head: max_ctx, or pool slots when paged
    const int32_t* page_table;
    const int32_t* seq_lens;
    float* out;
    float* part_o;   // [n_seqs * n_q_heads, n_splits, D]
    float* part_ml;  // [n_seqs * n_q_heads, n_splits, 2]: reference max (log2), sum
    uint32_t page_size, max_pages, n_pages;
    uint32_t ctx_len, max_len, chunk, n_splits;
    uint32_t n_q_heads, n_kv_heads, group, n_sub;
    float scale_log2, eps, freq_scale;
    // paged plan (see paged_plan): plan != nullptr when the workgroups take their
    // (sequence, split) from it; plan[0] receives the chunk for the merge
    uint32_t* plan;
    uint32_t plan_cap, n_seqs;
};

template <int D>
struct Geo {
    static constexpr int KK = D / 32;            // k-steps of the S product
    static constexpr int DT = D / 16;            // 16-row blocks of O^T
    static constexpr int RC = D / 8;             // 16-byte chunks per cache row
    static constexpr int VC = kTile * RC / 64;   // V chunks per lane per tile
    static constexpr int VROW = D * 2;           // bytes per staged V row (chunks swizzled, see vswz)
    static constexpr int OROW = D + 4;           // floats per row of the cross-wave O buffer
};

template <int D>
struct TileRegs {
    u32x4 k[2][Geo<D>::KK];  // [half-tile][k-step]: row c16 of the half, dims kk*32 + 8g .. +8
    u32x4 v[Geo<D>::VC];     // chunk r: row (lane + 64r) / RC, dims ((lane + 64r) % RC) * 8 .. +8
};

// Barrier for LDS traffic only: outstanding global loads stay in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// K/V rows are read once per step. V is read with non-temporal loads (streaming
// hint to the caches); K too when the cache is contiguous, with plain loads when
// it is paged. A K load takes a 64-byte piece of each of 16 rows, so two loads
// share every 128-byte line, and for scattered pages a streamed line can be gone
// before its second half is read. Measured on gfx950: paged, non-temporal K is
// 12% slower and non-temporal V 3% faster than plain; contiguous, both
// non-temporal is the fastest end to end.
template <bool NT>
__device__ __forceinline__ u32x4 ld16(const f16* ptr) {
    if constexpr (NT) return __builtin_nontemporal_load((const u32x4*)ptr);
    else return *(const u32x4*)ptr;
}

// gfx950 LDS transpose read (ds_read_b64_tr_b16) of 4 halves; see its use below.
__device__ __forceinline__ f16x4 lds_read_tr16(const char* lds_byte_ptr) {
    typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 v4h;
    typedef __attribute__((address_space(3))) v4h lds_v4h;
    const v4h r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_v4h*)(lds_byte_ptr));
    return __builtin_bit_cast(f16x4, r);
}

// Page of sequence b holding position pos; out-of-range entries read page 0
// and raise `bad` (the workgroup then poisons its output).
__device__ __forceinline__ uint64_t page_base(const DecodeParams& p, uint32_t b, uint32_t pos, bool& bad) {
    const int32_t pg = p.page_table[ds5idx::dec_page_index(b, p.max_pages, pos, p.page_size)];
    return ds5idx::dec_page_first(pg, p.n_pages, p.page_size, bad);
}

// Issues the K/V loads of tile [p0, p0 + 32) of a split ending at `end`.
// Rows at or past `end` are redirected to valid memory (clamped for the
// contiguous cache, kept inside the same page when paged); their scores are
// masked and their V rows zeroed before use.
template <int D, bool PAGED>
__device__ __forceinline__ void issue_tile(TileRegs<D>& T, const DecodeParams& p, const f16* kbase, const f16* vbase,
                                           uint32_t b, uint32_t p0, uint32_t end, int g, int c16, int lane,
                                           bool& bad) {
    using G = Geo<D>;
    uint64_t rowA = 0, rowB = 0;  // paged: first slot of each 16-position half-tile
    if constexpr (PAGED) {
        // page_size is a multiple of 16 and p0 a multiple of 32: each half is inside one page
        // (half 1's page is the one holding min(p0 + 16, end - 1), its offset that of p0 + 16)
        rowA = page_base(p, b, ds5idx::dec_half_pos(p0, end, 0), bad) + p0 % p.page_size;
        rowB = page_base(p, b, ds5idx::dec_half_pos(p0, end, 1), bad) + (p0 + 16) % p.page_size;
    }
#pragma unroll
    for (int st = 0; st < 2; st++) {
        uint64_t row;
        if constexpr (PAGED)
            row = ds5idx::dec_k_row_paged(rowA, rowB, st, c16);
        else
            row = ds5idx::dec_k_row(p0, end, st, c16);
#pragma unroll
        for (int kk = 0; kk < G::KK; kk++) T.k[st][kk] = ld16<!PAGED>(kbase + row * D + ds5idx::dec_k_col(kk, g));
    }
#pragma unroll
    for (int r = 0; r < G::VC; r++) {
        const int c = lane + 64 * r;
        const int tr = c / G::RC;  // row within the tile
        uint64_t row;
        if constexpr (PAGED)
            row = ds5idx::dec_v_row_paged(rowA, rowB, r, G::VC, tr);
        else
            row = ds5idx::dec_v_row(p0, end, tr);
        T.v[r] = ld16<true>(vbase + row * D + ds5idx::dec_v_col(c, G::RC));
    }
}

// Staged V rows are unpadded; 16-byte chunk c of row r sits in slot c ^ vswz(r).
// A transpose read serves 32 lanes (256 bytes, all 64 banks) per cycle: 8
// consecutive rows x 2 adjacent chunks; vswz sends them to 16 distinct slots
// (D = 128: one row per bank period; D = 64: two rows per period, so only rows
// of equal parity need distinct offsets).
template <int D>
__device__ __forceinline__ int vswz(int r) {
    if constexpr (D == 128) return 2 * (r & 7);
    else return 2 * ((r >> 1) & 3);
}

// Splits two values into f16 hi + lo pairs (x ~= hi + lo to ~22 significant
// bits): hi rounds to nearest, the residual x - hi is exact in f32 and is
// rounded again. Packed conversions: three instructions per value.
__device__ __forceinline__ void split2_f16(float x0, float x1, f16x2& hi, f16x2& lo) {
    hi = f16x2{(f16)x0, (f16)x1};
    lo = f16x2{(f16)(x0 - (float)hi[0]), (f16)(x1 - (float)hi[1])};
}

// One 32-position tile of a wavefront: scores, softmax update, P.V.
// q operands are pre-scaled by softmax scale * log2(e), so S is in log2 units.
template <int D, bool FUSED, bool PACK>
__device__ __forceinline__ void compute_tile(TileRegs<D>& T, uint32_t p0, uint32_t end, int g, int c16, int lane,
                                             const f16x8 (&qh)[Geo<D>::KK], const f16x8 (&ql)[Geo<D>::KK],
                                             f32x4 (&O)[Geo<D>::DT], float& m_ref, float& l_sum, char* vlds,
                                             int new_row, const f16* s_knew, const f16* s_vnew, bool first) {
    using G = Geo<D>;
    // Fused: the tile holding the new position takes the freshly appended row from LDS.
    if (FUSED && new_row >= 0) {
#pragma unroll
        for (int st = 0; st < 2; st++)
            if (16 * st + c16 == new_row)
#pragma unroll
                for (int kk = 0; kk < G::KK; kk++) T.k[st][kk] = *(const u32x4*)(s_knew + kk * 32 + 8 * g);
#pragma unroll
        for (int r = 0; r < G::VC; r++) {
            const int c = lane + 64 * r;
            if (c / G::RC == new_row) T.v[r] = *(const u32x4*)(s_vnew + (c % G::RC) * 8);
        }
    }
    const bool partial = p0 + kTile > end;  // wave-uniform

    // S^T = K . Q^T with q = hi + lo. Packed (group <= 8): columns 0-7 carry the
    // hi halves of heads 0-7 and columns 8-15 the lo halves, so one product
    // covers both and lanes c16, c16 ^ 8 add their columns (DPP row_ror:8).
    f32x4 S[2];
#pragma unroll
    for (int st = 0; st < 2; st++) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < G::KK; kk++) {
            const f16x8 a = __builtin_bit_cast(f16x8, T.k[st][kk]);
            acc = mfma_16x16x32(a, qh[kk], acc);
            if constexpr (!PACK) acc = mfma_16x16x32(a, ql[kk], acc);
        }
        if constexpr (PACK) {
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] += dpp_mov<0x128>(acc[i]);
        }
        S[st] = acc;
    }
    // this lane: head c16, positions p0 + 16*st + 4g + i (score j = 4*st + i)
    float s[8];
#pragma unroll
    for (int j = 0; j < 8; j++) s[j] = S[j / 4][j % 4];
    if (partial) {
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (p0 + 16 * (j / 4) + 4 * g + (j % 4) >= end) s[j] = -INFINITY;
    }
    float mx = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
    mx = swap32_op(swap16_op(mx, OpMax{}), OpMax{});
    // Lazy rescale: move the reference only when the tile max exceeds it by > 2^8.
    if (first) {
        m_ref = mx;  // O and l are still zero
    } else if (__ballot(mx > m_ref + kRescaleLog2) != 0) {
        const bool move = mx > m_ref + kRescaleLog2;
        const float m_new = move ? mx : m_ref;
        const float alpha = fast_exp2(m_ref - m_new);  // 1 for heads that keep their reference
        l_sum *= alpha;
#pragma unroll
        for (int dt = 0; dt < G::DT; dt++) O[dt] *= alpha;
        m_ref = m_new;
    }
    float pj[8];
#pragma unroll
    for (int j = 0; j < 8; j++) pj[j] = fast_exp2(s[j] - m_ref);
    l_sum += ((pj[0] + pj[1]) + (pj[2] + pj[3])) + ((pj[4] + pj[5]) + (pj[6] + pj[7]));
    // p as f16 hi + lo; packed: hi in columns 0-7, lo in columns 8-15
    f16x8 ph, pl;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        f16x2 hi, lo;
        split2_f16(pj[j], pj[j + 1], hi, lo);
        if constexpr (PACK) {
            const f16x2 sel = c16 >= 8 ? lo : hi;
            ph[j] = sel[0];
            ph[j + 1] = sel[1];
        } else {
            ph[j] = hi[0];
            ph[j + 1] = hi[1];
            pl[j] = lo[0];
            pl[j + 1] = lo[1];
        }
    }

    // V tile -> wavefront LDS area (rows past the split end zeroed: p is 0 there, V may be garbage)
#pragma unroll
    for (int r = 0; r < G::VC; r++) {
        const int c = lane + 64 * r;
        u32x4 v = T.v[r];
        if (partial && p0 + c / G::RC >= end) v = u32x4{0u, 0u, 0u, 0u};
        *(u32x4*)(vlds + (c / G::RC) * G::VROW + ((c % G::RC) ^ vswz<D>(c / G::RC)) * 16) = v;
    }
    __builtin_amdgcn_wave_barrier();
    // O^T += V^T . P^T; k-slot (g, j) <-> tile row 4g + j (j < 4), 16 + 4g + j - 4 (j >= 4).
    // ds_read_b64_tr_b16: within each 16-lane group, lane i reads 4 halves at row
    // base + i/4, columns c0 + 4*(i%4); lane j then holds column c0 + j of those 4 rows.
    // Halves dt*16 + 4 (c16 & 3) are chunk 2 dt + (c16 & 3) / 2, byte 8 (c16 & 1) inside it.
    const int r_lo = 4 * g + (c16 >> 2), r_hi = 16 + r_lo;
#pragma unroll
    for (int dt = 0; dt < G::DT; dt++) {
        const int ch = 2 * dt + ((c16 & 3) >> 1);
        const f16x4 lo4 = lds_read_tr16(vlds + r_lo * G::VROW + (ch ^ vswz<D>(r_lo)) * 16 + 8 * (c16 & 1));
        const f16x4 hi4 = lds_read_tr16(vlds + r_hi * G::VROW + (ch ^ vswz<D>(r_hi)) * 16 + 8 * (c16 & 1));
        const f16x8 a = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
        O[dt] = mfma_16x16x32(a, ph, O[dt]);
        if constexpr (!PACK) O[dt] = mfma_16x16x32(a, pl, O[dt]);
    }
    __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ float sq(float v) {
#pragma clang fp contract(off)
    return v * v;
}

// Sum of the D squares in index order with f32 rounding after each add -- the
// reference's serial sum of squares (kernels_a.zig:85-86), the products having
// been rounded on their own. Every lane reads the same LDS words (broadcast) and
// computes the same sum; reads go in batches of eight 16-byte chunks.
template <int D>
__device__ __forceinline__ float serial_sum(const float* sq_row) {
#pragma clang fp contract(off)
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < D / 32; b++) {
        float4 c[8];
#pragma unroll
        for (int j = 0; j < 8; j++) c[j] = *(const float4*)(sq_row + 32 * b + 4 * j);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            acc += c[j].x;
            acc += c[j].y;
            acc += c[j].z;
            acc += c[j].w;
        }
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

// Sum over the n consecutive lanes of a group (n = 8 or 16, aligned), result
// on every lane of the group: quad xor 1 and 2, then the 8-lane halves
// (row_half_mirror) and, for 16, the rows (row_mirror).
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(N == 8 || N == 16, "group of 8 or 16 lanes");
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    if constexpr (N == 16) v += dpp_mov<0x140>(v);
    return v;
}

// Paged plan. Sequence lengths differ, so splits of one size taken over the
// longest sequence leave most workgroups short or idle and the longest splits
// set the launch time. Every workgroup of a paged launch computes the same plan
// from the device-side lengths (no extra launch, no host round trip): the
// smallest chunk c -- a multiple of 128, at least max_len / kMaxSplits -- whose
// item count sum_b ceil(L_b / c) fits plan_cap items (the grid's x extent);
// workgroup x takes item x. A length outside [1, max_len] counts one item
// (split 0 poisons that sequence's output).
struct PagedItem {
    int32_t b;  // -1: no item for this workgroup
    uint32_t split, chunk;
};


// s_len: n_seqs words of LDS; s_red: kThreads / 64 + 2 words
__device__ PagedItem paged_plan(const DecodeParams& p, uint32_t x, uint32_t* s_len, uint32_t* s_red) {
    constexpr int NW = kThreads / 64;
    constexpr uint32_t kStep = kWaves * kTile;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t n = p.n_seqs;
    for (uint32_t i = tid; i < n; i += kThreads) {
        s_len[i] = ds5idx::plan_len(p.seq_lens[i], p.max_len);
    }
    __syncthreads();
    // thread t owns sequences [b0, b1)
    const uint32_t per = (n + kThreads - 1) / kThreads;
    const uint32_t b0 = min(n, tid * per), b1 = min(n, b0 + per);
    auto count = [&](uint32_t c) {
        uint32_t k = 0;
        for (uint32_t i = b0; i < b1; i++) k += ds5idx::plan_items(s_len[i], c);
        return k;
    };
    auto block_sum = [&](uint32_t v) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        __syncthreads();  // s_red's previous readers are done
        if (lane == 0) s_red[wave] = v;
        __syncthreads();
        uint32_t t = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) t += s_red[w];
        return t;
    };
    // binary search over c = cmin + kStep k: the count does not grow with c, and
    // c = max_len (rounded up) gives one item per sequence, which the cap admits
    const uint32_t cmin = ds5idx::plan_cmin(p.max_len, kStep, kMaxSplits), cmax = ds5idx::plan_cmax(p.max_len, kStep);
    uint32_t lo = 0, hi = (cmax - min(cmin, cmax)) / kStep;
    while (lo < hi) {  // uniform
        const uint32_t mid = (lo + hi) / 2;
        if (block_sum(count(cmin + kStep * mid)) <= p.plan_cap)
            hi = mid;
        else
            lo = mid + 1;
    }
    const uint32_t chunk = cmin + kStep * lo;
    // Item order: every sequence's whole chunks first (in sequence order), then the
    // partial last chunks (and poisoned sequences): consecutive workgroups go to
    // consecutive XCDs, so the equal-sized items spread evenly over the XCDs and
    // start first. Exclusive prefixes of both counts over the owners, then the
    // owner of item x.
    uint32_t mf = 0, mt = 0;
    for (uint32_t i = b0; i < b1; i++) {
        mf += ds5idx::plan_whole(s_len[i], chunk);
        mt += ds5idx::plan_partial(s_len[i], chunk);
    }
    auto block_scan = [&](uint32_t v, uint32_t& total) {
        uint32_t incl = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t y = __shfl_up(incl, o, 64);
            if (lane >= o) incl += y;
        }
        __syncthreads();
        if (lane == 63) s_red[wave] = incl;
        __syncthreads();
        uint32_t base = 0;
        total = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            base += w < wave ? s_red[w] : 0u;
            total += s_red[w];
        }
        return base + incl - v;
    };
    uint32_t F, T;
    const uint32_t ef = block_scan(mf, F);
    const uint32_t et = block_scan(mt, T);
    __syncthreads();  // s_red's scan readers are done
    if (x < F && x >= ef && x < ef + mf) {  // whole chunk
        uint32_t acc = ef;
        for (uint32_t i = b0; i < b1; i++) {
            const uint32_t k = ds5idx::plan_whole(s_len[i], chunk);
            if (x < acc + k) {
                s_red[NW] = i;
                s_red[NW + 1] = x - acc;
                break;
            }
            acc += k;
        }
    } else if (x >= F && x - F >= et && x - F < et + mt) {  // partial last chunk
        uint32_t acc = et;
        for (uint32_t i = b0; i < b1; i++) {
            if (ds5idx::plan_partial(s_len[i], chunk)) {
                if (x - F == acc) {
                    s_red[NW] = i;
                    s_red[NW + 1] = ds5idx::plan_whole(s_len[i], chunk);
                    break;
                }
                acc++;
            }
        }
    }
    __syncthreads();
    return PagedItem{x < F + T ? (int32_t)s_red[NW] : -1, s_red[NW + 1], chunk};
}

// ONE: every wavefront has at most one tile (chunk <= kWaves * kTile). That case
// gets a kernel of its own without the prefetch loop: the loop's four tile
// bodies double the code, and a decode launch is short enough for instruction
// fetch to show in its duration.
//
// The workgroup runs one wavefront per SIMD, so every instruction a wavefront
// issues sits on the critical path: the q operands (norm, rope, scale, hi/lo
// split) are built once per workgroup -- each thread takes 4 rope pairs of one
// head -- and read from LDS, and the wavefront partials are combined through
// LDS without lane shuffles.
template <int D, bool FUSED, bool PAGED, bool PACK, bool ONE>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(DecodeParams p, RopeTable table) {
    using G = Geo<D>;
    constexpr int W = kWaves;
    constexpr int KK = G::KK, DT = G::DT;
    constexpr int TPH = D / 8;   // prologue threads per q head; thread j owns pairs (4j + k, D/2 + 4j + k), k < 4
    constexpr int QROW = D + 8;  // halves per LDS q-operand row (16-byte pad)
    // One area per wavefront: its V staging tile, later its O for the cross-wavefront
    // combine (a wavefront overwrites only its own staging, so no barrier is needed
    // between its last transpose read and its O writes).
    constexpr int V_BYTES = kTile * G::VROW;
    constexpr int O_BYTES = kHeads * G::OROW * 4;
    constexpr int AREA = V_BYTES > O_BYTES ? V_BYTES : O_BYTES;
    __shared__ __attribute__((aligned(16))) char s_big[W * AREA];
    // q operand rows (f16, pre-scaled): packed, rows 0-7 hold the hi halves of heads
    // 0-7 and rows 8-15 their lo halves; otherwise s_qa holds hi and s_qb lo per head.
    __shared__ __attribute__((aligned(16))) f16 s_qa[kHeads * QROW];
    __shared__ __attribute__((aligned(16))) f16 s_qb[PACK ? 8 : kHeads * QROW];
    __shared__ __attribute__((aligned(16))) float s_krow[FUSED ? D : 4];
    __shared__ __attribute__((aligned(16))) float s_ksq[FUSED ? D : 4];  // squares of the new k row
    __shared__ __attribute__((aligned(16))) float s_qn[FUSED ? D : 4];
    __shared__ float s_kn[FUSED ? D : 1];
    __shared__ __attribute__((aligned(16))) float s_cos[FUSED ? D / 2 : 4];
    __shared__ __attribute__((aligned(16))) float s_sin[FUSED ? D / 2 : 4];
    __shared__ __attribute__((aligned(16))) f16 s_knew[FUSED ? D : 8];
    __shared__ __attribute__((aligned(16))) f16 s_vnew[FUSED ? D : 8];
    __shared__ float s_m[W][kHeads], s_l[W][kHeads];
    __shared__ int s_badw[W];

    // Every argument the first loads need, read in one scalar round trip: left to
    // itself the compiler loads only what the first early-exit test needs, waits,
    // and loads the rest after the branch -- a second dependent round trip (~0.9 us
    // on a cold argument buffer) before the first K/V load.
    if constexpr (PAGED)
        asm volatile("" ::"s"(p.k_cache), "s"(p.v_cache), "s"(p.cache_stride), "s"(p.q), "s"(p.chunk), "s"(p.n_sub),
                     "s"(p.group), "s"(p.n_q_heads), "s"(p.n_kv_heads), "s"(p.k_new), "s"(p.v_new), "s"(p.q_norm),
                     "s"(p.k_norm), "s"(p.plan), "s"(p.seq_lens), "s"(p.max_len), "s"(p.page_table), "s"(p.page_size),
                     "s"(p.max_pages), "s"(p.n_pages), "s"(p.plan_cap), "s"(p.n_seqs), "s"(p.out));
    else
        asm volatile("" ::"s"(p.k_cache), "s"(p.v_cache), "s"(p.cache_stride), "s"(p.q), "s"(p.chunk), "s"(p.n_sub),
                     "s"(p.group), "s"(p.n_q_heads), "s"(p.n_kv_heads), "s"(p.k_new), "s"(p.v_new), "s"(p.q_norm),
                     "s"(p.k_norm), "s"(p.ctx_len), "s"(p.positions));
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, c16 = lane & 15;
    uint32_t split = blockIdx.x, b = blockIdx.z, chunk = p.chunk;
    const uint32_t kvh = blockIdx.y / p.n_sub, sub = blockIdx.y % p.n_sub;
    if constexpr (PAGED) {
        if (p.plan) {
            __shared__ uint32_t s_plan[kThreads / 64 + 2];
            static_assert(kPlanMaxSeqs * 4 <= sizeof(s_big), "the plan's lengths fit the staging area");
            const PagedItem it = paged_plan(p, blockIdx.x, (uint32_t*)s_big, s_plan);
            if (blockIdx.x == 0 && blockIdx.y == 0 && tid == 0) p.plan[0] = it.chunk;  // for the merge
            if (it.b < 0) return;  // uniform: no item
            // uniform values read from LDS: scalar registers, so the page-table
            // lookups stay scalar loads (outside the vector loads' issue order)
            b = (uint32_t)__builtin_amdgcn_readfirstlane(it.b);
            split = (uint32_t)__builtin_amdgcn_readfirstlane((int)it.split);
            chunk = (uint32_t)__builtin_amdgcn_readfirstlane((int)it.chunk);
        }
    }
    const uint32_t n0 = sub * kHeads;
    const int NS = (int)min((uint32_t)kHeads, p.group - n0);
    const uint32_t hq0 = kvh * p.group + n0;  // first q head of this workgroup
    const uint64_t qrow0 = (uint64_t)b * p.n_q_heads + hq0;

    uint32_t L = p.ctx_len;
    if constexpr (PAGED) {
        const int32_t len = p.seq_lens[b];
        if (len < 1 || (uint32_t)len > p.max_len) {
            // Out-of-range sequence: poison its output (written once) and skip it.
            if (split == 0)
                for (int i = tid; i < NS * D; i += kThreads) p.out[qrow0 * D + i] = __builtin_nanf("");
            return;
        }
        L = (uint32_t)len;
    }
    const uint32_t start = split * chunk;
    if (start >= L) return;  // uniform: this split is past the sequence
    const uint32_t end = min(L, start + chunk);
    const uint32_t n_tiles = (end - start + kTile - 1) / kTile;
    const uint32_t newpos = L - 1;
    const bool has_new = FUSED && newpos >= start && newpos < end;

    const uint64_t head_base = (uint64_t)kvh * p.cache_stride;  // rows
    f16* const kbase = p.k_cache + head_base * D;
    f16* const vbase = p.v_cache + head_base * D;
    bool bad = false;

    // ---- 1. small loads first: vmcnt retires loads in issue order, so a load
    //         issued after the K/V tile could only be used once the whole tile
    //         has arrived. Every load here is unconditional with a clamped
    //         (valid) address: loads under divergent branches make the compiler
    //         wait for all outstanding loads at the join, which would include the
    //         K/V tile.
    const int qn = tid / TPH, qj = tid % TPH;  // prologue: head qn, pair block qj
    const float* qsrc = p.q + (qrow0 + min(qn, NS - 1)) * D + 4 * qj;
    const float4 xa = *(const float4*)qsrc;
    const float4 xb = *(const float4*)(qsrc + D / 2);
    const uint64_t kv_off = ((uint64_t)b * p.n_kv_heads + kvh) * D;
    float wq = 0.f, wk = 0.f, kr = 0.f, vr = 0.f, inv_freq = 0.f;
    int32_t pos_raw = 0;
    if constexpr (FUSED) {
        const int i = tid % D;
        wq = p.q_norm[i];
        wk = p.k_norm[i];
        kr = p.k_new[kv_off + i];
        vr = p.v_new[kv_off + i];
        inv_freq = table.inv[tid % (D / 2)];
        if (!PAGED) pos_raw = p.positions[0];
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. the first tile's K/V loads
    // Unconditional (a wavefront without a tile loads the split's last tile and
    // drops it): a branch around the loads would make the compiler's wait
    // counts at the join assume nothing was issued.
    TileRegs<D> TA, TB;
    uint32_t it = wave;
    issue_tile<D, PAGED>(TA, p, kbase, vbase, b, start + min(it, n_tiles - 1) * kTile, end, g, c16, lane, bad);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    // ---- 3. q operands, built once per workgroup while the tile is in flight
    // Fused: the wavefront that owns the tile holding the new position
    // normalises, rotates and appends the new k row itself.
    const int new_wave = has_new ? (int)(((newpos - start) / kTile) % W) : -1;
    float x[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    if constexpr (FUSED) {
        const float qpos = PAGED ? (float)newpos : (float)pos_raw;
        if (tid < D) {
            s_qn[tid] = wq;
            if (has_new) {
                s_krow[tid] = kr;
                s_ksq[tid] = sq(kr);
                s_kn[tid] = wk;
            }
        }
        if (tid < D / 2) {
            const float ang = rope_angle(qpos, p.freq_scale, inv_freq);
            s_cos[tid] = cosf(ang);
            s_sin[tid] = sinf(ang);
        }
        if (has_new && tid < D) {
            // v: f16 append (round to nearest even) into the cache and the tile
            bool pbad = false;
            const uint64_t vslot = PAGED ? page_base(p, b, newpos, pbad) + newpos % p.page_size : newpos;
            const f16 hv = (f16)vr;
            s_vnew[tid] = hv;
            if (!pbad) vbase[vslot * D + tid] = hv;
        }
        lds_barrier();
        // q RMSNorm: the head's sum of squares over its TPH threads (q only feeds
        // attention, so the summation order is free), then (v * inv) * w and the rotation.
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) ss += x[j] * x[j];
        const float inv = rms_inv(group_sum<TPH>(ss), (float)D, p.eps);
        const float4 wa = *(const float4*)&s_qn[4 * qj], wb = *(const float4*)&s_qn[D / 2 + 4 * qj];
        const float w8[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
        for (int j = 0; j < 8; j++) x[j] = norm_mul(x[j], inv, w8[j]);
        const float4 cs = *(const float4*)&s_cos[4 * qj], sn = *(const float4*)&s_sin[4 * qj];
        const float c4[4] = {cs.x, cs.y, cs.z, cs.w}, s4[4] = {sn.x, sn.y, sn.z, sn.w};
#pragma unroll
        for (int k = 0; k < 4; k++) rotate(x[k], x[4 + k], c4[k], s4[k], x[k], x[4 + k]);
    }
    // scale into log2 units, split into f16 hi + lo, write the operand rows
    // (heads past NS get zero rows)
    if (qn < (PACK ? kHeads / 2 : kHeads)) {
        f16x2 hi[4], lo[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float v0 = qn < NS ? x[2 * k] * p.scale_log2 : 0.0f;
            const float v1 = qn < NS ? x[2 * k + 1] * p.scale_log2 : 0.0f;
            split2_f16(v0, v1, hi[k], lo[k]);
        }
        f16* const rh = s_qa + qn * QROW + 4 * qj;
        f16* const rl = (PACK ? s_qa + (qn + kHeads / 2) * QROW : s_qb + qn * QROW) + 4 * qj;
        *(f16x4*)rh = f16x4{hi[0][0], hi[0][1], hi[1][0], hi[1][1]};
        *(f16x4*)(rh + D / 2) = f16x4{hi[2][0], hi[2][1], hi[3][0], hi[3][1]};
        *(f16x4*)rl = f16x4{lo[0][0], lo[0][1], lo[1][0], lo[1][1]};
        *(f16x4*)(rl + D / 2) = f16x4{lo[2][0], lo[2][1], lo[3][0], lo[3][1]};
    }
    lds_barrier();
    f16x8 qh[KK], ql[KK];
#pragma unroll
    for (int kk = 0; kk < KK; kk++) {
        qh[kk] = *(const f16x8*)(s_qa + c16 * QROW + kk * 32 + 8 * g);
        if constexpr (!PACK) ql[kk] = *(const f16x8*)(s_qb + c16 * QROW + kk * 32 + 8 * g);
    }
    if constexpr (FUSED) {
        if (wave == new_wave) {
            // k row: serial-order sum of squares (kernels_a.zig:85-86) in one lane,
            // then norm + rope of pair (lane, lane + D/2) and the f16 append.
            bool pbad = false;
            const uint64_t kslot = PAGED ? page_base(p, b, newpos, pbad) + newpos % p.page_size : newpos;
            bad |= pbad;
            const float kinv = rms_inv(serial_sum<D>(s_ksq), (float)D, p.eps);
            for (int i = lane; i < D / 2; i += 64) {
                const float x0 = norm_mul(s_krow[i], kinv, s_kn[i]);
                const float x1 = norm_mul(s_krow[i + D / 2], kinv, s_kn[i + D / 2]);
                float y0, y1;
                rotate(x0, x1, s_cos[i], s_sin[i], y0, y1);
                const f16 h0 = (f16)y0, h1 = (f16)y1;
                s_knew[i] = h0;
                s_knew[i + D / 2] = h1;
                if (!pbad) {
                    kbase[kslot * D + i] = h0;
                    kbase[kslot * D + i + D / 2] = h1;
                }
            }
        }
    }

    // ---- 4. main loop: prefetch one tile ahead, two register sets
    f32x4 O[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) O[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_ref = -INFINITY, l_sum = 0.0f;
    char* vlds = s_big + wave * AREA;
    auto new_row_of = [&](uint32_t p0) -> int {
        return (FUSED && has_new && newpos >= p0 && newpos < p0 + kTile) ? (int)(newpos - p0) : -1;
    };
    // Every compute path sees a fixed set of outstanding loads (the next tile's
    // or none), so the compiler's wait before a tile's first use never covers
    // the prefetch.
    if constexpr (ONE) {
        if (it < n_tiles) {
            const uint32_t p0 = start + it * kTile;
            compute_tile<D, FUSED, PACK>(TA, p0, end, g, c16, lane, qh, ql, O, m_ref, l_sum, vlds, new_row_of(p0), s_knew,
                                         s_vnew, true);
        }
    } else if (it < n_tiles) {
        bool first = true;
        for (;;) {
            uint32_t nx = it + W;
            uint32_t p0 = start + it * kTile;
            if (nx >= n_tiles) {
                compute_tile<D, FUSED, PACK>(TA, p0, end, g, c16, lane, qh, ql, O, m_ref, l_sum, vlds, new_row_of(p0),
                                             s_knew, s_vnew, first);
                break;
            }
            issue_tile<D, PAGED>(TB, p, kbase, vbase, b, start + nx * kTile, end, g, c16, lane, bad);
            compute_tile<D, FUSED, PACK>(TA, p0, end, g, c16, lane, qh, ql, O, m_ref, l_sum, vlds, new_row_of(p0), s_knew,
                                         s_vnew, first);
            first = false;
            it = nx;
            nx = it + W;
            p0 = start + it * kTile;
            if (nx >= n_tiles) {
                compute_tile<D, FUSED, PACK>(TB, p0, end, g, c16, lane, qh, ql, O, m_ref, l_sum, vlds, new_row_of(p0),
                                             s_knew, s_vnew, false);
                break;
            }
            issue_tile<D, PAGED>(TA, p, kbase, vbase, b, start + nx * kTile, end, g, c16, lane, bad);
            compute_tile<D, FUSED, PACK>(TB, p0, end, g, c16, lane, qh, ql, O, m_ref, l_sum, vlds, new_row_of(p0), s_knew,
                                         s_vnew, false);
            it = nx;
        }
    }

    // ---- 5. combine the wavefronts through LDS, then write the partial (or the output)
    // Wavefront w's O^T column c16 goes to row c16 of its area; packed, rows n and
    // n + 8 hold the hi and lo parts of head n and are added here.
    const float l_w = swap32_op(swap16_op(l_sum, OpAdd{}), OpAdd{});
    float* s_o = (float*)s_big;  // wavefront w's O: [w * AREA / 4 + column * OROW + dim]
    if (g == 0) {
        s_m[wave][c16] = m_ref;
        s_l[wave][c16] = l_w;
    }
    if (lane == 0) s_badw[wave] = bad ? 1 : 0;  // page lookups are wave-uniform
#pragma unroll
    for (int dt = 0; dt < DT; dt++) *(f32x4*)&s_o[wave * (AREA / 4) + c16 * G::OROW + dt * 16 + 4 * g] = O[dt];
    __syncthreads();

    bool poison = false;
#pragma unroll
    for (int w = 0; w < W; w++) poison |= s_badw[w] != 0;
    const bool single = L <= chunk;  // the sequence's only split writes the output itself
    for (int q4 = tid; q4 < NS * (D / 4); q4 += kThreads) {
        const int n = q4 / (D / 4), d0 = (q4 % (D / 4)) * 4;
        float M = s_m[0][n];
#pragma unroll
        for (int w = 1; w < W; w++) M = fmaxf(M, s_m[w][n]);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        float lt = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) {
            const float f = fast_exp2(s_m[w][n] - M);  // 0 for a wavefront without tiles
            f32x4 o = *(const f32x4*)&s_o[w * (AREA / 4) + n * G::OROW + d0];
            if constexpr (PACK) o += *(const f32x4*)&s_o[w * (AREA / 4) + (n + kHeads / 2) * G::OROW + d0];
            acc += o * f;
            lt += s_l[w][n] * f;
        }
        if (poison) acc = f32x4{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
        const uint64_t qi = qrow0 + n;
        if (single) {
            *(f32x4*)(p.out + qi * D + d0) = acc / lt;
        } else {
            *(f32x4*)(p.part_o + (qi * p.n_splits + split) * D + d0) = acc;
            if (d0 == 0) *(float2*)(p.part_ml + (qi * p.n_splits + split) * 2) = float2{M, lt};
        }
    }
}

// Split merge, two forms; both fold the splits of one (sequence, q head) in a
// fixed order, so results are deterministic.
//
// Lanes (at most 64 splits; few rows): block = 4 wavefronts = 4 groups of 4
// output dims of one (sequence, q head); lane s holds split s. One load per
// lane, then DPP / permlane reductions (VALU only): the shortest chain, for
// a grid of rows x D/16 workgroups that fills the chip at most a few times.
template <int D>
__device__ __forceinline__ void merge_lanes(const DecodeParams& p) {
    const uint64_t qi = blockIdx.x;  // sequence * n_q_heads + head
    const uint32_t b = (uint32_t)(qi / p.n_q_heads);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d0 = (blockIdx.y * 4 + wave) * 4;
    uint32_t L = p.ctx_len;
    if (p.seq_lens) {
        const int32_t len = p.seq_lens[b];
        if (len < 1 || (uint32_t)len > p.max_len) return;  // poisoned by the split kernel
        L = (uint32_t)len;
    }
    const uint32_t chunk = p.plan ? p.plan[0] : p.chunk;
    const uint32_t ns = (L + chunk - 1) / chunk;
    if (ns <= 1) return;  // written by its split
    float m = -INFINITY, l = 0.0f;
    float4 o = {0.f, 0.f, 0.f, 0.f};
    if ((uint32_t)lane < ns) {
        const float2 ml = *(const float2*)(p.part_ml + (qi * p.n_splits + lane) * 2);
        m = ml.x;
        l = ml.y;
        o = *(const float4*)(p.part_o + (qi * p.n_splits + lane) * D + d0);
    }
    const float M = wave_allreduce(m, OpMax{});
    const float w = (uint32_t)lane < ns ? fast_exp2(m - M) : 0.0f;
    l *= w;
    o.x *= w;
    o.y *= w;
    o.z *= w;
    o.w *= w;
    l = wave_allreduce(l, OpAdd{});
    o.x = wave_allreduce(o.x, OpAdd{});
    o.y = wave_allreduce(o.y, OpAdd{});
    o.z = wave_allreduce(o.z, OpAdd{});
    o.w = wave_allreduce(o.w, OpAdd{});
    if (lane == 0) *(float4*)(p.out + qi * D + d0) = float4{o.x / l, o.y / l, o.z / l, o.w / l};
}

// Slots (any number of splits; many rows): one workgroup per (sequence, q
// head). Thread (slot, column) takes splits slot, slot + SLOTS, ... of one
// float4 column of O, eight loads in flight at a time, and folds them in split
// order with a running maximum; the slots then combine through LDS in slot order.
template <int D>
__device__ __forceinline__ void merge_slots(const DecodeParams& p) {
    constexpr int COLS = D / 4, SLOTS = 256 / COLS, BATCH = 8;
    __shared__ float4 s_o[SLOTS][COLS];
    __shared__ float2 s_ml[SLOTS];
    const uint64_t qi = blockIdx.x;  // sequence * n_q_heads + head
    const uint32_t b = (uint32_t)(qi / p.n_q_heads);
    const int col = threadIdx.x % COLS, slot = threadIdx.x / COLS;
    uint32_t L = p.ctx_len;
    if (p.seq_lens) {
        const int32_t len = p.seq_lens[b];
        if (len < 1 || (uint32_t)len > p.max_len) return;  // poisoned by the split kernel
        L = (uint32_t)len;
    }
    const uint32_t chunk = p.plan ? p.plan[0] : p.chunk;
    const uint32_t ns = (L + chunk - 1) / chunk;
    if (ns <= 1) return;  // written by its split
    const float2* ml_row = (const float2*)p.part_ml + qi * p.n_splits;
    const float* o_row = p.part_o + qi * p.n_splits * D + 4 * col;
    float m = -INFINITY, l = 0.0f;
    float4 o = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t s0 = slot; s0 < ns; s0 += SLOTS * BATCH) {
        float2 ml[BATCH];
        float4 os[BATCH];
#pragma unroll
        for (int k = 0; k < BATCH; k++) {  // unconditional loads, clamped to a valid split
            const uint32_t s = min(s0 + SLOTS * k, ns - 1);
            ml[k] = ml_row[s];
            os[k] = *(const float4*)(o_row + (uint64_t)s * D);
        }
#pragma unroll
        for (int k = 0; k < BATCH; k++) {
            if (s0 + SLOTS * k >= ns) break;
            const float mn = fmaxf(m, ml[k].x);       // every split has a position: ml.x is finite
            const float a = fast_exp2(m - mn), w = fast_exp2(ml[k].x - mn);  // m = -inf: a = 0
            l = l * a + ml[k].y * w;
            o = o * a + os[k] * w;
            m = mn;
        }
    }
    s_o[slot][col] = o;
    if (col == 0) s_ml[slot] = float2{m, l};
    __syncthreads();
    if (slot == 0) {
        float M = s_ml[0].x;
#pragma unroll
        for (int t = 1; t < SLOTS; t++) M = fmaxf(M, s_ml[t].x);  // slot 0 always has split 0
        float lt = 0.0f;
        float4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < SLOTS; t++) {
            const float w = fast_exp2(s_ml[t].x - M);  // an empty slot: -inf - M, weight 0
            lt += s_ml[t].y * w;
            acc += s_o[t][col] * w;
        }
        *(float4*)(p.out + qi * D + 4 * col) = acc / lt;
    }
}

template <int D, bool SLOTS_FORM>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeParams p) {
    // every argument in one scalar round trip (see decode_split_kernel)
    asm volatile("" ::"s"(p.seq_lens), "s"(p.plan), "s"(p.n_q_heads), "s"(p.ctx_len), "s"(p.max_len), "s"(p.chunk),
                 "s"(p.part_ml), "s"(p.part_o), "s"(p.n_splits), "s"(p.out));
    if constexpr (SLOTS_FORM)
        merge_slots<D>(p);
    else
        merge_lanes<D>(p);
}

template <int D, bool FUSED, bool PAGED, bool PACK, bool ONE>
void launch_split_k(ds5_hip_ctx* ctx, const DecodeParams& prm, const RopeTable& tab, dim3 grid) {
    DS5_TIMED_LAUNCH(ctx, "decode_split_kernel", (decode_split_kernel<D, FUSED, PAGED, PACK, ONE>), grid, dim3(kThreads), 0,
                     ctx->stream, prm, tab);
}

template <int D, bool PACK, bool ONE>
void launch_split(ds5_hip_ctx* ctx, bool fused, bool paged, const DecodeParams& prm, const RopeTable& tab, dim3 grid) {
    if (fused && paged)
        launch_split_k<D, true, true, PACK, ONE>(ctx, prm, tab, grid);
    else if (fused)
        launch_split_k<D, true, false, PACK, ONE>(ctx, prm, tab, grid);
    else if (paged)
        launch_split_k<D, false, true, PACK, ONE>(ctx, prm, tab, grid);
    else
        launch_split_k<D, false, false, PACK, ONE>(ctx, prm, tab, grid);
}

template <int D>
int launch_decode_d(ds5_hip_ctx* ctx, const DecodeLaunch& a, const DecodeParams& prm, dim3 grid) {
    const bool paged = a.page_table != nullptr;
    const RopeTable& tab = a.fused ? *a.table : RopeTable{};
    // groups of at most 8 heads use the packed hi/lo columns (half the products)
    // (a planned launch's chunk is chosen on the device: the looping kernel)
    const bool pack = prm.group <= kHeads / 2, one = prm.plan == nullptr && prm.chunk <= kWaves * kTile;
    if (pack && one)
        launch_split<D, true, true>(ctx, a.fused, paged, prm, tab, grid);
    else if (pack)
        launch_split<D, true, false>(ctx, a.fused, paged, prm, tab, grid);
    else if (one)
        launch_split<D, false, true>(ctx, a.fused, paged, prm, tab, grid);
    else
        launch_split<D, false, false>(ctx, a.fused, paged, prm, tab, grid);
    int rc = ds5_after_launch(ctx, "decode_split_kernel");
    if (rc || prm.n_splits == 1) return rc;
    const uint64_t rows = (uint64_t)a.n_seqs * a.n_q_heads;
    if (prm.n_splits <= 64 && rows * (D / 16) <= 4ull * (ctx->cu_count > 0 ? ctx->cu_count : 256))
        DS5_TIMED_LAUNCH(ctx, "decode_merge_kernel", (decode_merge_kernel<D, false>), dim3(rows, D / 16), dim3(256), 0,
                         ctx->stream, prm);
    else
        DS5_TIMED_LAUNCH(ctx, "decode_merge_kernel", (decode_merge_kernel<D, true>), dim3(rows), dim3(256), 0,
                         ctx->stream, prm);
    return ds5_after_launch(ctx, "decode_merge_kernel");
}

}  // namespace

// Positions per split: about four workgroups per CU over the longest sequence,
// whole 128-position steps (one 32-position tile per wavefront), at most
// kMaxSplits splits (bounds the partials).
static DecodeGeometry decode_geometry_of(const ds5_hip_ctx* ctx, uint32_t n_seqs, uint32_t n_kv_heads, uint32_t n_sub,
                                         uint32_t max_len) {
    DecodeGeometry g{};
    ds5idx::dec_geometry(ctx->cu_count, ctx->decode_chunk, n_seqs, n_kv_heads, n_sub, max_len, g.chunk, g.n_splits);
    return g;
}

// The workspace a launch requests for n_part partial rows: O and (m, l) per row,
// then 16 bytes (the paged plan's chunk word).
static size_t decode_request_bytes(size_t n_part, uint32_t head_dim) {
    return n_part * ((size_t)head_dim + 2) * sizeof(float) + 16;
}

// What launch_decode requests for a contiguous cache (it requests nothing when one
// split covers the sequences).
size_t decode_workspace_bytes(const ds5_hip_ctx* ctx, uint32_t n_seqs, uint32_t n_q_heads, uint32_t n_kv_heads,
                              uint32_t head_dim, uint32_t max_len) {
    if (n_seqs == 0 || max_len == 0 || n_kv_heads == 0) return 0;
    const uint32_t group = n_q_heads / n_kv_heads;
    const uint32_t n_sub = (group + kHeads - 1) / kHeads;
    const DecodeGeometry geo = decode_geometry_of(ctx, n_seqs, n_kv_heads, n_sub, max_len);
    if (geo.n_splits <= 1) return 0;
    return decode_request_bytes((size_t)n_seqs * n_q_heads * geo.n_splits, head_dim);
}

int launch_decode(ds5_hip_ctx* ctx, const DecodeLaunch& a) {
    const uint32_t group = a.n_q_heads / a.n_kv_heads;
    const uint32_t n_sub = (group + kHeads - 1) / kHeads;
    const uint32_t max_len = a.max_len;
    if (a.n_seqs == 0 || max_len == 0) return DS5_OK;
    const bool planned = a.page_table != nullptr && a.n_seqs <= kPlanMaxSeqs;
    const uint32_t cu = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const uint32_t units = a.n_kv_heads * n_sub;
    // planned: about two workgroups per CU (measured at C4 against one, three and
    // four: one and two are equal and fastest), at least one item per sequence
    const uint32_t target = ctx->plan_items ? ctx->plan_items : 2 * cu;
    const uint32_t plan_cap = planned ? std::max<uint32_t>((target + units - 1) / units, a.n_seqs) : 0;
    const DecodeGeometry geo = planned ? DecodeGeometry{0, kMaxSplits}
                                       : decode_geometry_of(ctx, a.n_seqs, a.n_kv_heads, n_sub, max_len);
    const uint32_t chunk = geo.chunk;
    // planned: the partials' layout keeps kMaxSplits slots per row; a launch whose
    // smallest chunk covers max_len has one split per sequence
    constexpr uint32_t kStep = kWaves * kTile;
    const bool may_split = planned ? (max_len + kStep - 1) / kStep * kStep >
                                         std::max(kStep, (max_len + kMaxSplits - 1) / kMaxSplits + kStep - 1) / kStep * kStep
                                   : geo.n_splits > 1;
    const uint32_t n_splits = may_split ? geo.n_splits : 1;

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
    prm.scale_log2 = a.scale * kLog2e;
    prm.eps = a.eps;
    prm.freq_scale = a.freq_scale;
    prm.n_seqs = a.n_seqs;
    prm.plan_cap = plan_cap;
    if (n_splits > 1 || planned) {
        const size_t n_part = n_splits > 1 ? (size_t)a.n_seqs * a.n_q_heads * n_splits : 0;
        void* ws = nullptr;
        int rc = ds5_workspace(ctx, decode_request_bytes(n_part, a.head_dim), &ws);
        if (rc) return rc;
        prm.part_o = (float*)ws;
        prm.part_ml = prm.part_o + n_part * a.head_dim;
        if (planned) prm.plan = (uint32_t*)(prm.part_ml + 2 * n_part);
    }
    const dim3 grid = planned ? dim3(plan_cap, units, 1) : dim3(n_splits, units, a.n_seqs);
    if (a.head_dim == 128) return launch_decode_d<128>(ctx, a, prm, grid);
    return launch_decode_d<64>(ctx, a, prm, grid);
}
