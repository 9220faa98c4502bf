// k_prefill.hip -- causal prefill on gfx950: the fused step's pre-pass (k/v
// append with rope) and flash attention on f16 MFMA with f32 accumulation.
//
// Semantics: kernels_b.zig:29-133 for n_tokens > 1 -- query token t (absolute
// position pos + t) of q head h attends cache positions 0..pos+t of kv head
// h / group; softmax(scale * q.k) in f32.
//
// prefill_attention_kernel. A workgroup serves 4 q heads of one GQA group
// and a pair of 32-row q tiles with 8 wavefronts: two sets of four (one head
// each), so each SIMD runs two wavefronts whose MFMA, exponential and LDS
// phases overlap. Set 0 takes the first half of the heavy q tile's key tiles;
// set 1 the light q tile's key tiles, then the rest of the heavy tile's. Each
// set streams 64-position K/V tiles into its own pair of LDS stages with
// gfx950's direct-to-LDS loads (global_load_lds_dwordx4, no register staging);
// the next tile's loads are in flight while the current one is consumed. Per
// tile:
//   S^T[32 keys x 32 q] = K . Q^T         v_mfma_f32_32x32x16_f16 (x2)
//   O^T[D x 32 q]      += V^T . P^T       v_mfma_f32_32x32x16_f16
// With S transposed a lane holds 16 scores of one query row, so row max/sum
// need one lane swap (v_permlane32_swap), and the P^T operand is the lane's
// own scores. V^T operands come from LDS through the transpose read
// (ds_read_b64_tr_b16). LDS rows are unpadded with XOR-swizzled 16-byte
// chunks so both read patterns are bank-conflict free. q (pre-scaled by
// scale * log2 e) and p are rounded to f16 for the products; the softmax state
// is f32 in the log2 domain with a lazy reference max (rescale only on growth
// > 2^8); the row sum adds the f32 weights. Causal masking runs only on tiles
// that cross the diagonal. Set 1 writes the light tile's rows itself; the two
// sets' (max, sum, O) of the heavy tile merge through LDS at the end.
//
// Load balance: q tiles are paired heaviest with lightest (tile NQ-1-i with
// tile i) so every workgroup carries the same number of key tiles, and the
// workgroups of one kv head are placed on the same XCD (workgroup b runs on
// XCD b % 8), so each XCD's L2 holds one kv head's K/V.
//
// Fused mode: the pre-pass (prefill_prep_kernel, one workgroup per token)
// writes the normalised, rotated f16 k rows and the f16 v rows into the cache,
// and the attention kernel's q operand: q normalised, rotated, times softmax
// scale * log2(e), rounded to f16 ([n_tokens, n_q_heads, head_dim]). The
// separate-op path packs an already normalised and rotated q the same way
// (q_pack_kernel). The attention block's projection GEMM can do the pre-pass
// in its epilogue instead (k_matmul.hip).
#include "ds5_common.hpp"

namespace {

// ---------------------------------------------------------------------------
// Pre-pass: one workgroup per token.
// ---------------------------------------------------------------------------
constexpr int kPrepThreads = 256;
constexpr int kPrepMaxRow = 2048;  // n_kv_heads * head_dim floats staged per token

// Elementwise squares (each rounded to f32, as the reference's acc += v * v rounds the
// product before the add).
__device__ __forceinline__ float4 sq4(float4 v) {
#pragma clang fp contract(off)
    return float4{v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w};
}

// Serial-order sum of D squares held in LDS (kernels_a.zig:85-86's order): the reads
// go out four 16-byte chunks at a time ahead of their adds, so the dependent chain
// waits for one LDS round trip per batch rather than per chunk.
template <int D>
__device__ __forceinline__ float serial_sum_sq(const float* sq) {
#pragma clang fp contract(off)
    float acc = 0.0f;
#pragma unroll 1
    for (int b = 0; b < D; b += 16) {
        float4 v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = *(const float4*)(sq + b + 4 * j);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            acc += v[j].x;
            acc += v[j].y;
            acc += v[j].z;
            acc += v[j].w;
        }
    }
    return acc;
}

// Token t: cos/sin of its rope angles (kernels_a.zig:119-122); every kv head's
// k row: serial-order RMSNorm (kernels_a.zig:84-89), NeoX rotation (:125-126),
// f16 append at slot pos + t (:196-210); v rows f16. Then the q rows of every
// head: RMSNorm, rotation, times softmax scale * log2(e), rounded to f16 into
// q16 [n_tokens, n_q_heads, head_dim] (the attention kernel's operand). q only
// feeds the attention products, so its sum of squares is a lane reduction.
template <int D>
__global__ __launch_bounds__(kPrepThreads) void prefill_prep_kernel(KvPrepLaunch a, f16* q16, RopeTable table) {
    __shared__ __attribute__((aligned(16))) float s_k[kPrepMaxRow];
    __shared__ __attribute__((aligned(16))) float s_ksq[kPrepMaxRow];  // the k squares, formed in parallel
    __shared__ float s_cos[D / 2], s_sin[D / 2];
    __shared__ float s_inv[kPrepMaxRow / 64];
    constexpr uint32_t half = D / 2;
    constexpr uint32_t TPH = D / 16;  // q: threads per head, thread k takes dims 8k + [0, 8) and half + 8k + [0, 8)
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    const uint32_t H = a.n_kv_heads, HQ = a.n_q_heads;
    // Every load of the token is issued up front, with no wait in between (this
    // thread's k and v quads, its first q chunk, the position and its inverse
    // frequency; each unconditional with a clamped index, since a load under a
    // branch makes the compiler wait at the join), so one memory round trip covers
    // them all. (Staging k in LDS straight from its loads made every thread wait
    // for k before issuing q and v: three round trips instead of one.)
    const float pos = (float)a.positions[t];
    const float inv_freq = table.inv[min(tid, half - 1)];  // the threads < half use it
    static_assert(D / 2 <= kPrepThreads, "one rope angle per thread");
    static_assert(kPrepMaxRow / 4 <= 2 * kPrepThreads, "k quads: two per thread at most");
    const uint32_t nk4 = H * D / 4;
    const float4* krow = (const float4*)(a.k + (uint64_t)t * H * D);
    const float4 kq0 = krow[min(tid, nk4 - 1)];
    const float4 kq1 = krow[min(tid + kPrepThreads, nk4 - 1)];
    const float* qbase = a.q + (uint64_t)t * HQ * D;
    float x0[8], x1[8];
    {
        const uint32_t e = min(tid, HQ * TPH - 1);
        const float* row = qbase + (e / TPH) * D + 8 * (e % TPH);
        *(float4*)&x0[0] = *(const float4*)(row);
        *(float4*)&x0[4] = *(const float4*)(row + 4);
        *(float4*)&x1[0] = *(const float4*)(row + half);
        *(float4*)&x1[4] = *(const float4*)(row + half + 4);
    }
    const float4* vrow = (const float4*)(a.v + (uint64_t)t * H * D);
    const float4 v0 = vrow[min(tid, nk4 - 1)];
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if (tid < half) {
        const float ang = qk_rope_angle(pos, a.freq_scale, inv_freq);
        s_cos[tid] = cosf(ang);
        s_sin[tid] = sinf(ang);
    }
    if (tid < nk4) {
        ((float4*)s_k)[tid] = kq0;
        ((float4*)s_ksq)[tid] = sq4(kq0);
    }
    if (tid + kPrepThreads < nk4) {
        ((float4*)s_k)[tid + kPrepThreads] = kq1;
        ((float4*)s_ksq)[tid + kPrepThreads] = sq4(kq1);
    }
    __syncthreads();
    for (uint32_t h = tid; h < H; h += kPrepThreads) s_inv[h] = rms_inv(serial_sum_sq<D>(s_ksq + h * D), (float)D, a.eps);
    // v rows: f16 append
    for (uint32_t e = tid; e < nk4; e += kPrepThreads) {
        const float4 v = e == tid ? v0 : vrow[e];
        const uint32_t h = (4 * e) / D, i = (4 * e) % D;
        const f16x4 y = {(f16)v.x, (f16)v.y, (f16)v.z, (f16)v.w};
        *(f16x4*)(a.v_cache + ((uint64_t)h * a.max_ctx + a.pos + t) * D + i) = y;
    }
    // q rows: RMSNorm (lane-reduced sum of squares), rotation, scale, f16
    for (uint32_t e = tid; e < HQ * TPH; e += kPrepThreads) {
        const uint32_t hq = e / TPH, k8 = 8 * (e % TPH);
        if (e != tid) {
            const float* row = qbase + hq * D + k8;
            *(float4*)&x0[0] = *(const float4*)(row);
            *(float4*)&x0[4] = *(const float4*)(row + 4);
            *(float4*)&x1[0] = *(const float4*)(row + half);
            *(float4*)&x1[4] = *(const float4*)(row + half + 4);
        }
        float ss = qk_pairs_sumsq(x0, x1);
#pragma unroll
        for (uint32_t m = 1; m < TPH; m <<= 1) ss += __shfl_xor(ss, (int)m, 64);
        const float inv = rms_inv(ss, (float)D, a.eps);
        f16x8 y0v, y1v;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t i = k8 + j;
            float y0, y1;
            qk_rotate(qk_norm_mul(x0[j], inv, a.q_norm[i]), qk_norm_mul(x1[j], inv, a.q_norm[i + half]), s_cos[i],
                      s_sin[i], y0, y1);
            y0v[j] = qk_scaled_f16(y0, a.q_scale);
            y1v[j] = qk_scaled_f16(y1, a.q_scale);
        }
        f16* dst = q16 + ((uint64_t)t * HQ + hq) * D;
        *(f16x8*)(dst + k8) = y0v;
        *(f16x8*)(dst + half + k8) = y1v;
    }
    __syncthreads();
    // k rows: serial-order RMSNorm, rotation, f16 append
    for (uint32_t e = tid; e < H * half; e += kPrepThreads) {
        const uint32_t h = e / half, i = e % half;
        const float inv = s_inv[h];
        const float y0n = qk_norm_mul(s_k[h * D + i], inv, a.k_norm[i]);
        const float y1n = qk_norm_mul(s_k[h * D + i + half], inv, a.k_norm[i + half]);
        float y0, y1;
        qk_rotate(y0n, y1n, s_cos[i], s_sin[i], y0, y1);
        f16* dst = a.k_cache + ((uint64_t)h * a.max_ctx + a.pos + t) * D;
        dst[i] = (f16)y0;
        dst[i + half] = (f16)y1;
    }
}

// Separate-op path: q already normalised and rotated; q16 = f16(q * q_scale).
__global__ __launch_bounds__(256) void q_pack_kernel(const float* q, f16* q16, uint64_t n8, float q_scale) {
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n8; i += (uint64_t)gridDim.x * 256) {
        const float4 a = *(const float4*)(q + 8 * i), b = *(const float4*)(q + 8 * i + 4);
        const f16x8 y = {qk_scaled_f16(a.x, q_scale), qk_scaled_f16(a.y, q_scale), qk_scaled_f16(a.z, q_scale),
                         qk_scaled_f16(a.w, q_scale), qk_scaled_f16(b.x, q_scale), qk_scaled_f16(b.y, q_scale),
                         qk_scaled_f16(b.z, q_scale), qk_scaled_f16(b.w, q_scale)};
        *(f16x8*)(q16 + 8 * i) = y;
    }
}

// ---------------------------------------------------------------------------
// Attention.
// ---------------------------------------------------------------------------
constexpr int kHeads = 4;      // q heads per workgroup
constexpr int kSets = 2;       // wavefront sets (set 0: heavy q tile's first key tiles; set 1: the rest)
constexpr int kWaves = kHeads * kSets;
constexpr int kThreads = kWaves * 64;
constexpr int kQRows = 32;     // q rows per wavefront tile (MFMA N)
constexpr int kKTile = 64;     // keys per LDS stage
constexpr float kRescaleLog2 = 8.0f;

struct PrefillParams {
    const f16* q16;          // [n_tokens, n_q_heads, head_dim], scaled by softmax scale * log2(e)
    const f16* k_cache;
    const f16* v_cache;
    float* out;
    uint32_t pos, n_tokens, n_q_heads, group, max_ctx;
    uint32_t n_qtiles, n_pairs, n_hgroups, n_items, items_per_xcd;
};

template <int D>
struct PGeo {
    static constexpr int KS = D / 16;              // k-steps of the S product
    static constexpr int DT = D / 32;              // 32-row blocks of O^T
    static constexpr int RB = D * 2;               // data bytes per cache row
    // LDS row strides, padded so the two read patterns are bank-conflict free
    // on the 64-bank LDS (256 bytes = 16 chunk slots per cycle): the S-operand
    // read puts 16 consecutive K rows at one chunk in a cycle, so the K stride
    // is 1 (mod 16) chunks; the V transpose read puts 4 consecutive rows x 4
    // adjacent chunks in a cycle, so the V stride is 4 (mod 16) chunks. Every
    // read address is then a per-lane base plus an immediate.
    static constexpr int RSK = RB + 16;
    static constexpr int RSV = RB + 64;
    static constexpr int KSTAGE = kKTile * RSK;    // bytes per K stage
    static constexpr int VSTAGE = kKTile * RSV;    // bytes per V stage
    static constexpr int NBK = KSTAGE / 1024, NBV = VSTAGE / 1024;  // 1 KiB direct-to-LDS loads per stage
    static_assert(KSTAGE % 1024 == 0 && VSTAGE % 1024 == 0, "stages are whole 1 KiB loads");
    static constexpr int BK = (NBK + kHeads - 1) / kHeads, BV = (NBV + kHeads - 1) / kHeads;  // per wavefront
    static constexpr int SET_BYTES = 2 * (KSTAGE + VSTAGE);  // double-buffered K and V of one wavefront set
};

__device__ __forceinline__ f16x4 lds_read_tr16(const char* lds_ptr) {
    typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 v4h;
    typedef __attribute__((address_space(3))) v4h lds_v4h;
    const v4h r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_v4h*)(lds_ptr));
    return __builtin_bit_cast(f16x4, r);
}

// Workgroup barrier that orders LDS only: global loads stay in flight across it.
__device__ __forceinline__ void lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Wait until at most n vector-memory operations of this wavefront are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// max / sum of v over lanes l and l ^ 32 (one VALU swap, no LDS round trip)
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Direct-to-LDS loads of the 64 K (or V) rows starting at key0 into one stage
// with row stride RS. Load b fills stage bytes [1024 b, +1024), lane L the 16
// bytes at 1024 b + 16 L: row r, chunk slot c of that row, or the row padding
// (such a lane re-reads the row's first chunk; the padding is never read).
// Loads b = wave, wave + 4, ... are this wavefront's. DmaPlan keeps the lane's
// byte offset inside the tile for each of its loads: whole tiles (all 64 rows
// below kv_end) are fetched with a scalar tile base plus that offset; the last
// tile clamps rows past kv_end to kv_end - 1 (valid memory, weighted 0).
template <int D, int RS, int B>
struct DmaPlan {
    uint32_t off[B];
    __device__ __forceinline__ DmaPlan(int wave, int lane) {
#pragma unroll
        for (int i = 0; i < B; i++) {
            const int pos = 1024 * (wave + kHeads * i) + 16 * lane;
            const int r = pos / RS, c = (pos % RS) / 16;
            off[i] = (uint32_t)(r * 2 * D + (c < D / 8 ? 16 * c : 0));
        }
    }
};

template <int D, int RS, int B>
__device__ __forceinline__ void dma_tile(uint32_t stage_lds, const f16* base, uint32_t key0, uint32_t kv_end,
                                         const DmaPlan<D, RS, B>& dp, int wave, int lane) {
    constexpr int NB = kKTile * RS / 1024;
    // wave-uniform operands made explicitly scalar (else the compiler wraps each
    // asm statement in a loop over the distinct lane values)
    // (readfirstlane returns int: each half goes through uint32_t so that the low
    // half is zero-extended, not sign-extended, when the pointer is rebuilt)
    const uint64_t tb = (uint64_t)(base + (uint64_t)key0 * D);
    const uint32_t tb_hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(tb >> 32));
    const uint32_t tb_lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)tb);
    const uint64_t tile = ((uint64_t)tb_hi << 32) | (uint64_t)tb_lo;
    const bool whole = key0 + kKTile <= kv_end;  // uniform
#pragma unroll
    for (int i = 0; i < B; i++) {
        const int b = wave + kHeads * i;
        if (B * kHeads > NB && b >= NB) break;  // uniform: this wavefront has fewer loads
        const uint32_t lds = __builtin_amdgcn_readfirstlane(stage_lds + 1024 * b);
        // Issued as inline asm: the compiler would otherwise make every later
        // LDS read wait for all such loads (it cannot tell the stages apart).
        // Completion is awaited explicitly (wait_vm) before the barrier that
        // publishes a stage.
        if (whole) {
            asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(dp.off[i]), "s"(tile), "s"(lds)
                         : "m0");
        } else {
            const uint32_t r = dp.off[i] / (2 * D), col = dp.off[i] % (2 * D);
            const uint32_t key = min(key0 + r, kv_end - 1);
            const char* src = (const char*)(base + (uint64_t)key * D) + col;
            asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "m0");
        }
    }
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)p;
}

template <int D>
__global__ __launch_bounds__(kThreads) void prefill_attention_kernel(PrefillParams p) {
    using G = PGeo<D>;
    constexpr int KS = G::KS, DT = G::DT, RSK = G::RSK, RSV = G::RSV;
    // LDS: per set, K stages 0 and 1 then V stages 0 and 1; reused by the set merge
    __shared__ __attribute__((aligned(1024))) char s_kv[kSets * G::SET_BYTES];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int set = wave / kHeads, hw = wave % kHeads;  // key-tile set, head slot
    const int r32 = lane & 31, h = lane >> 5, g16 = lane >> 4, i16 = lane & 15;

    // workgroup -> (kv head, head group, q-tile pair); one kv head per XCD where possible
    uint32_t item = blockIdx.x;
    if (p.items_per_xcd) item = (blockIdx.x % 8) * p.items_per_xcd + blockIdx.x / 8;
    const uint32_t pair = item % p.n_pairs;
    const uint32_t hg = (item / p.n_pairs) % p.n_hgroups;
    const uint32_t kvh = item / (p.n_pairs * p.n_hgroups);
    const uint32_t hin = hg * kHeads + hw;  // head index inside the group
    const bool live = hin < p.group;
    const uint32_t hq = kvh * p.group + (live ? hin : 0);
    const f16* kc = p.k_cache + (uint64_t)kvh * p.max_ctx * D;
    const f16* vc = p.v_cache + (uint64_t)kvh * p.max_ctx * D;
    // this set's stages
    char* const k_st = s_kv + set * G::SET_BYTES;
    char* const v_st = k_st + 2 * G::KSTAGE;
    const uint32_t k_lds = lds_addr(k_st), v_lds = lds_addr(v_st);

    // Per-lane LDS byte bases; every read adds an immediate. S operand of
    // (half kh, k-step ks): row 32 kh + r32, bytes 32 ks + 16 h of the row.
    const int kb = r32 * RSK + 16 * h;
    // V transpose read of (key step m, dim block dt, upper half hi): lane i16 of
    // group g16 reads row 16 m + 8 hi + 4 hh + i16 / 4, halves dt*32 + 16 (g16 & 1)
    // + 4 (i16 & 3), i.e. bytes 64 dt + 32 (g16 & 1) + 8 (i16 & 3) of the row.
    const int vb = (4 * (g16 >> 1) + (i16 >> 2)) * RSV + 32 * (g16 & 1) + 8 * (i16 & 3);
    const DmaPlan<D, RSK, G::BK> dk(hw, lane);
    const DmaPlan<D, RSV, G::BV> dv(hw, lane);

    // Key-tile schedule of the q-tile pair (heavy tile NQ-1-i with H key tiles, light
    // tile i with L): set 0 takes the heavy tile's key tiles [0, k0), set 1 the light
    // tile's L key tiles and then the heavy tile's [k0, H), k0 = ceil((H + L) / 2). Both
    // sets run k0 rounds; the light tile's rows are written by set 1 alone and only the
    // heavy tile's two partials merge, when set 1 reaches that tile.
    const uint32_t heavy = p.n_qtiles - 1 - pair;
    const bool has_light = pair < heavy;  // the middle tile of an odd count is processed once
    auto kv_end_of = [&](uint32_t qtile) -> uint32_t {  // keys the q tile needs (exclusive)
        return p.pos + min(p.n_tokens, qtile * kQRows + kQRows);
    };
    const uint32_t H = (kv_end_of(heavy) + kKTile - 1) / kKTile;
    const uint32_t L = has_light ? (kv_end_of(pair) + kKTile - 1) / kKTile : 0;
    const uint32_t k0 = (H + L + 1) / 2;  // rounds; L <= H, so k0 <= H
    const uint32_t n_items = set == 0 ? k0 : L + H - k0;
    const bool merge = H > k0;  // set 1 ends on the heavy tile
    // item i of this set: its q tile and key tile
    auto item_qt = [&](uint32_t i) -> uint32_t { return set == 1 && i < L ? pair : heavy; };
    auto item_kt = [&](uint32_t i) -> uint32_t { return set == 0 ? i : (i < L ? i : k0 + i - L); };

    // the wavefront's q tile: lane (r32, h) holds query row t
    uint32_t qt = item_qt(0);
    uint32_t t = qt * kQRows + r32;
    bool keep = live && t < p.n_tokens;
    uint32_t n_full = (p.pos + qt * kQRows + 1) / kKTile;  // key tiles with no masked key

    // q operand of lane (r32, h): row t, dims 16 ks + 8 h + [0, 8) for every k-step
    f16x8 qop[KS], qnext[KS];
    auto load_q = [&](f16x8(&dst)[KS], uint32_t qtile) {
        const uint32_t tc = min(qtile * kQRows + r32, p.n_tokens - 1);
        const f16* qrow = p.q16 + ((uint64_t)tc * p.n_q_heads + hq) * D + 8 * h;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) dst[ks] = *(const f16x8*)(qrow + 16 * ks);
    };
    // ---- q operand first (vmcnt retires in issue order), then the first tile
    load_q(qop, qt);
    if (n_items > 0) {
        dma_tile(k_lds, kc, item_kt(0) * kKTile, kv_end_of(qt), dk, hw, lane);
        dma_tile(v_lds, vc, item_kt(0) * kKTile, kv_end_of(qt), dv, hw, lane);
    }
    if (!keep) {
#pragma unroll
        for (int ks = 0; ks < KS; ks++) qop[ks] = f16x8{};
    }

    f32x16 O[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int i = 0; i < 16; i++) O[dt][i] = 0.0f;
    float m_ref = -INFINITY, l_sum = 0.0f;

    // The wavefront's rows of its q tile when every key of the tile went through it:
    // O over its own row sum. Wave-uniform call (the row sum crosses lanes).
    auto write_rows = [&]() {
        const float l = sum_xor32(l_sum);
        if (keep) {
            const float inv_l = 1.0f / l;
            float* out = p.out + ((uint64_t)t * p.n_q_heads + hq) * D;
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int i4 = 0; i4 < 4; i4++)
                    *(float4*)(out + dt * 32 + 8 * i4 + 4 * h) =
                        float4{O[dt][4 * i4] * inv_l, O[dt][4 * i4 + 1] * inv_l, O[dt][4 * i4 + 2] * inv_l,
                               O[dt][4 * i4 + 3] * inv_l};
        }
    };

    wait_vm<0>();
    lds_sync();
    // Round r: item r of each set sits in stage r % 2; item r + 1 streams into the other
    // stage meanwhile (that stage was last read in round r - 1, before the previous barrier).
    for (uint32_t r = 0; r < k0; r++) {
        const uint32_t kcur = (r & 1) * G::KSTAGE, knxt = G::KSTAGE - kcur;
        const uint32_t vcur = (r & 1) * G::VSTAGE, vnxt = G::VSTAGE - vcur;
        if (set == 1 && L > 0 && L < n_items) {
            // set 1 moves from the light tile to the heavy one: the heavy q operand loads
            // one round ahead (drained by that round's barrier wait); at round L the light
            // rows are written and the softmax state restarts
            if (r + 1 == L) load_q(qnext, heavy);
            if (r == L) {
                write_rows();
                qt = heavy;
                t = qt * kQRows + r32;
                keep = live && t < p.n_tokens;
                n_full = (p.pos + qt * kQRows + 1) / kKTile;
#pragma unroll
                for (int ks = 0; ks < KS; ks++) qop[ks] = keep ? qnext[ks] : f16x8{};
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
#pragma unroll
                    for (int i = 0; i < 16; i++) O[dt][i] = 0.0f;
                m_ref = -INFINITY;
                l_sum = 0.0f;
            }
        }
        const bool load_next = r + 1 < n_items;
        const uint32_t nkey0 = item_kt(r + 1) * kKTile, nend = kv_end_of(item_qt(r + 1));
        // The next tile's loads are issued in two halves inside the round (a burst from
        // all eight wavefronts right after the barrier would stall their issue).
        if (r < n_items) {
            const uint32_t j = item_kt(r);
            const uint32_t key0 = j * kKTile;
            const uint64_t t_abs = (uint64_t)p.pos + t;
            const char* sk = k_st + kcur + kb;
            f32x16 S[2];  // S^T of the tile's two 32-key halves
#pragma unroll
            for (int kh = 0; kh < 2; kh++) {
#pragma unroll
                for (int i = 0; i < 16; i++) S[kh][i] = 0.0f;
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    const f16x8 a = *(const f16x8*)(sk + 32 * kh * RSK + 32 * ks);
                    S[kh] = mfma_32x32x16(a, qop[ks], S[kh]);
                }
            }
            if (load_next) dma_tile(k_lds + knxt, kc, nkey0, nend, dk, hw, lane);
            // lane: query row t; score r of half kh is key key0 + 32kh + 8(r/4) + 4h + r%4.
            if (j >= n_full) {  // causal mask on tiles that reach past the first row
#pragma unroll
                for (int kh = 0; kh < 2; kh++)
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        const uint64_t key = key0 + 32 * kh + 8 * (i / 4) + 4 * h + (i % 4);
                        if (key > t_abs) S[kh][i] = -INFINITY;
                    }
            }
            float mx = S[0][0];
#pragma unroll
            for (int kh = 0; kh < 2; kh++)
#pragma unroll
                for (int i = 0; i < 16; i++) mx = fmaxf(mx, S[kh][i]);
            mx = max_xor32(mx);
            if (__ballot(mx > m_ref + kRescaleLog2) != 0) {  // lazy rescale (also the first tile)
                const float m_new = mx > m_ref + kRescaleLog2 ? mx : m_ref;
                const float alpha = m_new == m_ref ? 1.0f : fast_exp2(m_ref - m_new);  // -inf - -inf would be NaN
                l_sum *= alpha;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) O[dt] *= alpha;
                m_ref = m_new;
            }
            // A row with every key so far masked (possible in set 1, whose part of the
            // heavy tile starts at key tile k0) keeps m_ref = -inf; its weights are 0.
            const float m_exp = m_ref == -INFINITY ? 0.0f : m_ref;
            f16x8 pop[4];  // P^T operand of key step m: scores i = 8 (m % 2) + jj of half m / 2
            // Row sum in f32 adds of the f32 weights: v_dot2 of the f16 weights would
            // share the matrix core with the other wavefront's products on this SIMD.
            float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int m = 0; m < 4; m++)
#pragma unroll
                for (int jj = 0; jj < 8; jj++) {
                    const float e = fast_exp2(S[m / 2][8 * (m % 2) + jj] - m_exp);
                    pop[m][jj] = (f16)e;
                    ps[m] += e;
                }
            l_sum += (ps[0] + ps[1]) + (ps[2] + ps[3]);
            if (load_next) dma_tile(v_lds + vnxt, vc, nkey0, nend, dv, hw, lane);
            // O^T += V^T . P^T; k-slot (h, jj) of step m is key 16m + 8(jj/4) + 4h + jj%4.
            // Transpose read: lane i of a 16-lane group addresses row base + i/4, columns
            // c0 + 4(i%4); lane j receives column c0 + j of the 4 rows.
            const char* sv = v_st + vcur + vb;
#pragma unroll
            for (int m = 0; m < 4; m++)
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    const f16x4 lo = lds_read_tr16(sv + 16 * m * RSV + 64 * dt);
                    const f16x4 hi = lds_read_tr16(sv + (16 * m + 8) * RSV + 64 * dt);
                    const f16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    O[dt] = mfma_32x32x16(a, pop[m], O[dt]);
                }
        }
        wait_vm<0>();
        lds_sync();
    }

    if (!merge) {
        if (set == 0 || L > 0) write_rows();  // set 0: the heavy tile; set 1: the light tile
        return;
    }
    // ---- merge set 1 (the heavy tile's keys [k0, H)) into set 0 through LDS; every stage
    // is free after the last round. Head slot hw: [float4 index][lane].
    constexpr int NV4 = DT * 4 + 1;  // O as float4s, then (m, l, -, -)
    static_assert(NV4 * 64 * 16 <= G::KSTAGE && G::KSTAGE <= G::VSTAGE, "a merge slot fits a stage");
    char* const slot = s_kv + (hw >> 1) * G::SET_BYTES + ((hw & 1) == 0 ? 0 : 2 * G::KSTAGE);
    float4* mrg = (float4*)slot + lane;
    if (set == 1) {
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int i4 = 0; i4 < 4; i4++)
                mrg[(dt * 4 + i4) * 64] = float4{O[dt][4 * i4], O[dt][4 * i4 + 1], O[dt][4 * i4 + 2], O[dt][4 * i4 + 3]};
        mrg[DT * 4 * 64] = float4{m_ref, l_sum, 0.0f, 0.0f};
    }
    lds_sync();
    if (set == 0) {
        const float4 ml = mrg[DT * 4 * 64];
        const float m = fmaxf(m_ref, ml.x);  // m_ref is finite (key 0 is visible to set 0)
        // a row whose keys in set 1's range were all masked has ml.x = -inf: a1 = 0
        const float a0 = fast_exp2(m_ref - m), a1 = fast_exp2(ml.x - m);
        const float l = sum_xor32(l_sum * a0 + ml.y * a1);
        if (keep) {
            const float inv_l = 1.0f / l;
            float* out = p.out + ((uint64_t)t * p.n_q_heads + hq) * D;
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int i4 = 0; i4 < 4; i4++) {
                    const float4 o1 = mrg[(dt * 4 + i4) * 64];
                    const int d = dt * 32 + 8 * i4 + 4 * h;
                    *(float4*)(out + d) = float4{(O[dt][4 * i4] * a0 + o1.x * a1) * inv_l,
                                                 (O[dt][4 * i4 + 1] * a0 + o1.y * a1) * inv_l,
                                                 (O[dt][4 * i4 + 2] * a0 + o1.z * a1) * inv_l,
                                                 (O[dt][4 * i4 + 3] * a0 + o1.w * a1) * inv_l};
                }
        }
    }
}

}  // namespace

bool prefill_prep_supported(uint32_t n_kv_heads, uint32_t head_dim) {
    return (uint64_t)n_kv_heads * head_dim <= kPrepMaxRow && (head_dim == 64 || head_dim == 128);
}

int launch_kv_prep(ds5_hip_ctx* ctx, const KvPrepLaunch& a, f16* q16) {
    if (a.n_tokens == 0) return DS5_OK;
    if (a.head_dim == 128)
        DS5_TIMED_LAUNCH(ctx, "prefill_prep_kernel", prefill_prep_kernel<128>, dim3(a.n_tokens), dim3(kPrepThreads), 0,
                         ctx->stream, a, q16, *a.table);
    else
        DS5_TIMED_LAUNCH(ctx, "prefill_prep_kernel", prefill_prep_kernel<64>, dim3(a.n_tokens), dim3(kPrepThreads), 0,
                         ctx->stream, a, q16, *a.table);
    return ds5_after_launch(ctx, "prefill_prep_kernel");
}

int launch_q_pack(ds5_hip_ctx* ctx, const float* q, f16* q16, uint64_t n, float q_scale) {
    if (n == 0) return DS5_OK;
    const uint64_t n8 = n / 8;
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((n8 + 255) / 256, 2048);
    DS5_TIMED_LAUNCH(ctx, "q_pack_kernel", q_pack_kernel, dim3(blocks), dim3(256), 0, ctx->stream, q, q16, n8, q_scale);
    return ds5_after_launch(ctx, "q_pack_kernel");
}

int launch_prefill(ds5_hip_ctx* ctx, const PrefillLaunch& a) {
    if (a.n_tokens == 0) return DS5_OK;
    PrefillParams p{};
    p.q16 = a.q16;
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
    p.n_hgroups = (p.group + kHeads - 1) / kHeads;
    p.n_items = a.n_kv_heads * p.n_hgroups * p.n_pairs;
    p.items_per_xcd = p.n_items % 8 == 0 ? p.n_items / 8 : 0;
    const dim3 grid(p.n_items);
    if (a.head_dim == 128)
        DS5_TIMED_LAUNCH(ctx, "prefill_attention_kernel", prefill_attention_kernel<128>, grid, dim3(kThreads), 0,
                         ctx->stream, p);
    else
        DS5_TIMED_LAUNCH(ctx, "prefill_attention_kernel", prefill_attention_kernel<64>, grid, dim3(kThreads), 0,
                         ctx->stream, p);
    return ds5_after_launch(ctx, "prefill_attention_kernel");
}
