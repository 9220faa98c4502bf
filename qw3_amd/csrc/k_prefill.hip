// k_prefill.hip -- causal prefill on gfx950: the fused step's pre-pass (k/v
// append with rope) and flash attention on f16 MFMA with f32 accumulation.
//
// Semantics: kernels_b.zig:29-133 for n_tokens > 1 -- query token t (absolute
// position pos + t) of q head h attends cache positions 0..pos+t of kv head
// h / group; softmax(scale * q.k) in f32.
//
// prefill_attention_kernel. A workgroup serves 4 q heads of one GQA group and a
// pair of 32-row q tiles (the heavy tile NQ-1-i, then the light tile i, so every
// workgroup carries the same number of key tiles) with 5 wavefronts: 4 compute
// wavefronts, one head each, one per SIMD, and a producer wavefront that only
// streams 64-position K/V tiles through a ring of 4 LDS stages with gfx950's
// direct-to-LDS loads (global_load_lds_dwordx4, no register staging), three tiles
// ahead of their use. Per key tile and head, in two 32-key halves:
//   S^T[32 keys x 32 q] = onecol . mneg + K . Q^T    v_mfma_f32_32x32x16_f16 (1 + D/16)
//   O^T[D x 32 q]      += V^T . P^T                  v_mfma_f32_32x32x16_f16 (D/32 per key step)
//   l^T[32 x 32 q]     += ones . P^T                 v_mfma_f32_32x32x16_f16 (1 per key step)
// With S transposed a lane holds 16 scores of one query row, so the row max needs one
// lane swap (v_permlane32_swap), and the P^T operand is the lane's own weights. The
// first product of the scores adds -m (the row's lazy reference max, an f16 value),
// so the weights are exp2 of the products' result; the row sums come from the matrix
// core too. V^T operands come from LDS through the transpose read
// (ds_read_b64_tr_b16). LDS rows are padded (K: +16 bytes, V: +64 bytes) so both read
// patterns are bank-conflict free. q (pre-scaled by scale * log2 e) and p are rounded
// to f16 for the products; the softmax state is f32 in the log2 domain, rescaled only
// when a row's max grows by more than 2^8. Each compute wavefront issues the next
// half's score products beside the current half's exponentials and the PV products
// beside the next half's row max, so its matrix-core and VALU work overlap in one
// instruction stream. Causal masking runs only on the halves that cross the diagonal,
// in rounds of their own; the other rounds run a branch-free form.
//
// Load balance: q tiles are paired heaviest with lightest (tile NQ-1-i with
// tile i) so every workgroup carries the same number of key tiles, and the
// workgroups of one kv head are placed on the same XCD (workgroup b runs on
// XCD b % 8), so each XCD's L2 holds one kv head's K/V.
//
// Fused mode: the pre-pass (prefill_prep_kernel, one workgroup per token)
// writes the normalised, rotated f16 k rows and the f16 v rows into the cache,
// and every token's rope cos/sin ([n_tokens, head_dim] f32). The attention
// kernel builds its q operand from the raw f32 q when it loads a q tile: q
// normalised, rotated with that table, times softmax scale * log2(e), rounded to
// f16 (each (q tile, head) is loaded by one workgroup, so q is read once, as f32,
// and never written back). The attention block's projection GEMM writes a ready
// f16 operand in its epilogue (k_matmul.hip) with the same arithmetic, so the
// fused step and the attention block give the same outputs from the same
// projections. The separate-op path hands the kernel q already normalised (by
// the serial-order rmsNorm) and rotated, which it only scales.
#include <type_traits>

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

// Token t: cos/sin of its rope angles (kernels_a.zig:119-122), into cs[t] (cos of
// pairs 0 .. D/2 - 1, then their sin) for the attention kernel's q rotation; every
// kv head's k row: serial-order RMSNorm (kernels_a.zig:84-89), NeoX rotation
// (:125-126), f16 append at slot pos + t (:196-210); v rows f16.
template <int D>
__global__ __launch_bounds__(kPrepThreads) void prefill_prep_kernel(KvPrepLaunch a, RopeTable table) {
    __shared__ __attribute__((aligned(16))) float s_k[kPrepMaxRow];
    __shared__ __attribute__((aligned(16))) float s_ksq[kPrepMaxRow];  // the k squares, formed in parallel
    __shared__ float s_cos[D / 2], s_sin[D / 2];
    __shared__ float s_inv[kPrepMaxRow / 64];
    constexpr uint32_t half = D / 2;
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    const uint32_t H = a.n_kv_heads;
    // Every load of the token is issued up front, with no wait in between (this
    // thread's k and v quads, the position and its inverse frequency; each
    // unconditional with a clamped index, since a load under a branch makes the
    // compiler wait at the join), so one memory round trip covers them all.
    const float pos = (float)a.positions[t];
    const float inv_freq = table.inv[min(tid, half - 1)];  // the threads < half use it
    static_assert(D / 2 <= kPrepThreads, "one rope angle per thread");
    static_assert(kPrepMaxRow / 4 <= 2 * kPrepThreads, "k quads: two per thread at most");
    const uint32_t nk4 = H * D / 4;
    const float4* krow = (const float4*)(a.k + (uint64_t)t * H * D);
    const float4 kq0 = krow[min(tid, nk4 - 1)];
    const float4 kq1 = krow[min(tid + kPrepThreads, nk4 - 1)];
    const float4* vrow = (const float4*)(a.v + (uint64_t)t * H * D);
    const float4 v0 = vrow[min(tid, nk4 - 1)];
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if (tid < half) {
        const float ang = qk_rope_angle(pos, a.freq_scale, inv_freq);
        const float c = cosf(ang), sn = sinf(ang);
        s_cos[tid] = c;
        s_sin[tid] = sn;
        a.cs[(uint64_t)t * D + tid] = c;
        a.cs[(uint64_t)t * D + half + tid] = sn;
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

// ---------------------------------------------------------------------------
// Attention.
// ---------------------------------------------------------------------------
constexpr int kHeads = ds5idx::kPfHeads;  // q heads per workgroup, one compute wavefront each
constexpr int kThreads = (kHeads + 1) * 64;  // + the producer wavefront
constexpr int kQRows = ds5idx::kPfQRows;  // q rows per wavefront tile (MFMA N)
constexpr int kKTile = ds5idx::kPfKTile;  // keys per LDS stage
constexpr int kStages = 4;     // K/V ring: a stage is refilled three rounds ahead of its use
constexpr int kAhead = kStages - 1;
constexpr int kOpAhead = 5;    // LDS operand reads in flight ahead of their product
constexpr float kRescaleLog2 = 8.0f;

// Where the attention kernel's q operand comes from:
//   kQOperand: a ready f16 operand (the attention block's projection GEMM writes it)
//   kQRotated: f32 q that is already normalised and rotated (the separate ops):
//              f16(q * q_scale)
//   kQRaw:     the raw f32 projection (the fused step): RMSNorm, rotation with the
//              pre-pass's cos/sin table, times q_scale, f16
enum QMode : int { kQOperand = 0, kQRotated = 1, kQRaw = 2 };

struct PrefillParams {
    const f16* q16;          // kQOperand: [n_tokens, n_q_heads, head_dim], scaled by softmax scale * log2(e)
    const float* q;          // kQRotated, kQRaw: [n_tokens, n_q_heads, head_dim] f32
    const float* q_norm;     // kQRaw: [head_dim]
    const float* cs;         // kQRaw: [n_tokens, head_dim], cos of pairs 0 .. head_dim/2 - 1, then sin
    float eps, q_scale;      // q_scale = softmax scale * log2(e)
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
    static constexpr int RSK = ds5idx::pf_rsk(D);
    static constexpr int RSV = ds5idx::pf_rsv(D);
    static constexpr int KSTAGE = kKTile * RSK;    // bytes of K per stage
    static constexpr int VSTAGE = kKTile * RSV;    // bytes of V per stage
    static constexpr int STAGE = KSTAGE + VSTAGE;
    static constexpr int NBK = KSTAGE / 1024, NBV = VSTAGE / 1024;  // 1 KiB direct-to-LDS loads per stage
    static_assert(KSTAGE % 1024 == 0 && VSTAGE % 1024 == 0, "stages are whole 1 KiB loads");
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

// max(a, b, c) as one v_max3_f32. Written as asm so that the chain stays where it
// is issued (between the products) and takes the raw MFMA results: compiled from
// fmaxf the chain is either gathered after the last product or, pinned in place,
// given a canonicalizing v_max per operand. No NaN reaches it. Every caller reads
// scores whose last product was issued at least two products earlier, past the
// matrix core's result latency (an asm statement gets no hazard wait states).
__device__ __forceinline__ float vmax3(float a, float b, float c) {
    float r;
    asm volatile("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// max of v over lanes l and l ^ 32 (one VALU swap, no LDS round trip)
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Direct-to-LDS loads of the 64 K (or V) rows starting at key0 into one stage
// with row stride RS. Load b fills stage bytes [1024 b, +1024), lane L the 16
// bytes at 1024 b + 16 L: row r, chunk slot c of that row, or the row padding
// (such a lane re-reads the row's first chunk; the padding is never read).
// TilePlan keeps the lane's byte offset inside the tile for every load: a load
// takes the scalar tile base plus that offset; on the last tile of a q tile,
// rows past kv_end are clamped to kv_end - 1 (valid memory, weighted 0).
template <int D, int RS>
struct TilePlan {
    static constexpr int NB = kKTile * RS / 1024;
    uint32_t off[NB];
    __device__ __forceinline__ explicit TilePlan(int lane) {
#pragma unroll
        for (int b = 0; b < NB; b++) off[b] = ds5idx::pf_tile_off(b, lane, D, RS);
    }
};

// A wave-uniform pointer made explicitly scalar (readfirstlane returns int: each
// half goes through uint32_t so that the low half is zero-extended when the
// pointer is rebuilt).
__device__ __forceinline__ uint64_t scalar_ptr(const void* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    return ((uint64_t)hi << 32) | (uint64_t)lo;
}

template <int D, int RS>
__device__ __forceinline__ void dma_tile(uint32_t stage_lds, const f16* base, uint32_t key0, uint32_t kv_end,
                                         const TilePlan<D, RS>& tp) {
    constexpr int NB = TilePlan<D, RS>::NB;
    const uint64_t tile = scalar_ptr(base + (uint64_t)key0 * D);
    // Issued as inline asm: the compiler would otherwise make every later LDS read
    // wait for all such loads (it cannot tell the stages apart). Completion is
    // awaited explicitly (wait_vm) before the barrier that publishes a stage.
    // (Two asm forms keep the clamp a real branch: whole tiles run no address
    // arithmetic.)
    if (key0 + kKTile <= kv_end) {  // uniform
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const uint32_t lds = __builtin_amdgcn_readfirstlane(stage_lds + 1024 * b);
            asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(tp.off[b]), "s"(tile),
                         "s"(lds)
                         : "m0");
        }
    } else {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const uint32_t lds = __builtin_amdgcn_readfirstlane(stage_lds + 1024 * b);
            const uint32_t off = ds5idx::pf_clamped_off(tp.off[b], key0, kv_end, D);
            asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(tile), "s"(lds)
                         : "m0");
        }
    }
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)p;
}

// Causal flash attention. A workgroup serves 4 q heads of one GQA group and a pair
// of 32-row q tiles: the heavy tile NQ-1-i, then the light tile i, so every
// workgroup carries the same number of key tiles and nothing is merged. Four
// compute wavefronts (one head each, one per SIMD) and one producer wavefront
// that does nothing but stream key tiles through a ring of four LDS stages with
// direct-to-LDS loads, three tiles ahead of their use: a direct-to-LDS load holds
// up the wavefront that issues it until the CU's load path accepts it (~64 bytes
// per clock per CU), and the producer takes those stalls in place of the compute
// wavefronts. Round r works on item r (a key tile of the current q tile); within
// a round each compute wavefront issues the next half tile's S products beside the
// current half's exponentials and the current PV products beside the next half's
// row max (see step), so its matrix-core and VALU work overlap in one instruction
// stream.
template <int D, int QM>
__global__ __launch_bounds__(kThreads) void prefill_attention_kernel(PrefillParams p) {
    using G = PGeo<D>;
    constexpr int KS = G::KS, DT = G::DT, RSK = G::RSK, RSV = G::RSV;
    __shared__ __attribute__((aligned(1024))) char s_kv[kStages * G::STAGE];  // stage s: K then V

    const int lane = threadIdx.x & 63;
    const int hw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // head slot (kHeads: the producer)
    const int r32 = lane & 31, h = lane >> 5, g16 = lane >> 4, i16 = lane & 15;

    // workgroup -> (kv head, head group, q-tile pair); one kv head per XCD where possible
    uint32_t item = blockIdx.x;
    if (p.items_per_xcd) item = (blockIdx.x % 8) * p.items_per_xcd + blockIdx.x / 8;
    const uint32_t pair = item % p.n_pairs;
    const uint32_t hg = (item / p.n_pairs) % p.n_hgroups;
    const uint32_t kvh = item / (p.n_pairs * p.n_hgroups);

    // Items: the heavy tile's key tiles 0 .. H-1, then the light tile's 0 .. L-1.
    const uint32_t heavy = p.n_qtiles - 1 - pair;
    const bool has_light = pair < heavy;  // the middle tile of an odd count is processed once
    auto kv_end_of = [&](uint32_t qtile) -> uint32_t {  // keys the q tile needs (exclusive)
        return p.pos + min(p.n_tokens, qtile * kQRows + kQRows);
    };
    const uint32_t H = (kv_end_of(heavy) + kKTile - 1) / kKTile;
    const uint32_t L = has_light ? (kv_end_of(pair) + kKTile - 1) / kKTile : 0;
    const uint32_t n_items = H + L;
    auto item_qt = [&](uint32_t i) -> uint32_t { return i < H ? heavy : pair; };
    auto item_kt = [&](uint32_t i) -> uint32_t { return i < H ? i : i - H; };
    auto k_stage = [&](uint32_t i) -> uint32_t { return (i % kStages) * G::STAGE; };

    if (hw == kHeads) {
        // ---- producer: items 0 .. kAhead - 1 before the first barrier, then item
        // r + kAhead in round r, into the stage item r - 1 left (every wavefront passed
        // round r - 1's barrier). At the end of round r every item up to r + kAhead - 1
        // has landed (items r + 1 and r + 2 are read in round r + 1); only item
        // r + kAhead's loads stay in flight.
        const f16* kc = p.k_cache + (uint64_t)kvh * p.max_ctx * D;
        const f16* vc = p.v_cache + (uint64_t)kvh * p.max_ctx * D;
        const uint32_t kv_lds = lds_addr(s_kv);
        const TilePlan<D, RSK> tk(lane);
        const TilePlan<D, RSV> tv(lane);
        auto dma_item = [&](uint32_t i) {
            const uint32_t key0 = item_kt(i) * kKTile, end = kv_end_of(item_qt(i));
            dma_tile(kv_lds + k_stage(i), kc, key0, end, tk);
            dma_tile(kv_lds + k_stage(i) + G::KSTAGE, vc, key0, end, tv);
        };
#pragma unroll
        for (int i = 0; i < kAhead; i++)
            if ((uint32_t)i < n_items) dma_item(i);
        if (n_items >= kAhead)  // round 0 reads items 0 and 1; item 2 may still be in flight
            wait_vm<(kAhead - 2) * (G::NBK + G::NBV)>();
        else
            wait_vm<0>();
        lds_sync();
        for (uint32_t r = 0; r + 1 < n_items; r++) {
            if (r + kAhead < n_items) {
                dma_item(r + kAhead);
                wait_vm<G::NBK + G::NBV>();
            } else {
                wait_vm<0>();
            }
            if (has_light && r + 1 == H) lds_sync();  // the switch's extra barrier
            lds_sync();
        }
        return;
    }

    const uint32_t hin = hg * kHeads + hw;  // head index inside the group
    const bool live = hin < p.group;
    const uint32_t hq = kvh * p.group + (live ? hin : 0);

    // Per-lane LDS byte bases; every read adds an immediate. S operand of
    // (half kh, k-step ks): row 32 kh + r32, bytes 32 ks + 16 h of the row.
    const int kb = r32 * RSK + 16 * h;
    // V transpose read of (key step m, dim block dt, upper half hi): lane i16 of
    // group g16 reads row 16 m + 8 hi + 4 hh + i16 / 4, halves dt*32 + 16 (g16 & 1)
    // + 4 (i16 & 3), i.e. bytes 64 dt + 32 (g16 & 1) + 8 (i16 & 3) of the row.
    const int vb = (4 * (g16 >> 1) + (i16 >> 2)) * RSV + 32 * (g16 & 1) + 8 * (i16 & 3);

    // Staging area of this wavefront inside a K/V stage that no wavefront reads at the
    // time (a quarter stage each): the q operand and the output rows go through it so
    // that their global loads and stores run along rows. In the MFMA layout a lane
    // holds one q row and the 64 lanes of an access span 32 rows, so every load or
    // store instruction would touch 32 cache lines; along rows it touches 8.
    constexpr int QSTR = 2 * D + 16;   // f16 q operand row stride (bank-conflict free reads)
    constexpr int OSTR = 32 * 4 + 16;  // f32 output row stride (one 32-dim block of O)
    static_assert(32 * QSTR <= G::STAGE / 4 && 32 * OSTR <= G::STAGE / 4 && G::STAGE % 64 == 0,
                  "staging fits a quarter stage");
    auto area_of = [&](uint32_t stage_off) -> char* { return s_kv + stage_off + hw * (G::STAGE / 4); };
    // The lane index through an empty asm: address arithmetic of the prologue, the
    // switch and the end is then computed where it is used; otherwise the compiler
    // hoists it out of the round loop and spills it.
    auto lane_here = [&]() -> uint32_t {
        uint32_t l = lane;
        asm volatile("" : "+v"(l));
        return l;
    };

    // q operand of lane (r32, h): row q0 + r32 of the q tile, dims 16 ks + 8 h + [0, 8)
    // for every k-step, read from the staged f16 rows. Rows are staged along rows:
    //   kQOperand: lane (g, m) copies 8 f16 of row RPI it + g, dims 8 m + [0, 8);
    //   f32 q:     lane (g, m) takes dims 4 m + [0, 4) and D/2 + 4 m + [0, 4) of row
    //              RPI it + g: four rope pairs (quarter m of the row). kQRotated:
    //              times q_scale, f16. kQRaw: RMSNorm, rotation with the pre-pass's
    //              cos/sin and the scale (qk_quarter_sumsq, the quarters' balanced
    //              tree, qk_q_pair), operation for operation the arithmetic of the
    //              projection GEMM's q epilogue, so both give the same operand.
    // Rows past the last token and the heads of an unfilled group read clamped, valid
    // rows: their scores stay in their own columns of S and O and are never written.
    f16x8 qop[KS];
    // q_load issues every load of a q tile's rows (q, then with kQRaw the cos/sin rows
    // and the norm weights); q_form builds the operand from them, so that the switch
    // can issue the light tile's loads before it writes the heavy tile's rows.
    constexpr int QLPR = D / 8, QRPI = 64 / QLPR, QNIT = kQRows / QRPI;  // lanes per row, rows per load, loads
    struct QRows {
        f16x8 v[QNIT];                         // kQOperand
        float4 a[QNIT], b[QNIT], c[QNIT], sn[QNIT];  // f32 q: pairs 4 m + [0, 4) and D/2 + 4 m + [0, 4)
        float4 w0, w1;
    };
    auto q_load = [&](QRows& in, uint32_t qtile) {
        const uint32_t q0 = qtile * kQRows, lane = lane_here();
        const uint32_t m = lane % QLPR, g = lane / QLPR;
        auto row_of = [&](uint32_t row) -> uint64_t {
            return (uint64_t)ds5idx::pf_q_token(q0, row, p.n_tokens) * p.n_q_heads + hq;
        };
        if constexpr (QM == kQOperand) {
#pragma unroll
            for (int it = 0; it < QNIT; it++) in.v[it] = *(const f16x8*)(p.q16 + row_of(QRPI * it + g) * D + 8 * m);
        } else {
#pragma unroll
            for (int it = 0; it < QNIT; it++) {
                const float* qr = p.q + row_of(QRPI * it + g) * D;
                in.a[it] = *(const float4*)(qr + 4 * m);
                in.b[it] = *(const float4*)(qr + D / 2 + 4 * m);
            }
            if constexpr (QM == kQRaw) {
#pragma unroll
                for (int it = 0; it < QNIT; it++) {
                    const float* cr = p.cs + (uint64_t)ds5idx::pf_q_token(q0, QRPI * it + g, p.n_tokens) * D;
                    in.c[it] = *(const float4*)(cr + 4 * m);
                    in.sn[it] = *(const float4*)(cr + D / 2 + 4 * m);
                }
                in.w0 = *(const float4*)(p.q_norm + 4 * m);
                in.w1 = *(const float4*)(p.q_norm + D / 2 + 4 * m);
            }
        }
    };
    auto q_form = [&](f16x8(&dst)[KS], const QRows& in, char* area) {
        const uint32_t lane = lane_here();
        if constexpr (QM == kQOperand) {
            constexpr int LPR = QLPR, RPI = QRPI, NIT = QNIT;
            const uint32_t m = lane % LPR, g = lane / LPR;
#pragma unroll
            for (int it = 0; it < NIT; it++) *(f16x8*)(area + (RPI * it + g) * QSTR + 16 * m) = in.v[it];
        } else {
            constexpr int LPR = QLPR, RPI = QRPI, NIT = QNIT;
            const uint32_t m = lane % LPR, g = lane / LPR;
            const float4 *a = in.a, *b = in.b, *c = in.c, *sn = in.sn;
            const float4 w0 = in.w0, w1 = in.w1;
            float r[NIT];  // kQRaw: the row's 1/rms times q_scale
            if constexpr (QM == kQRaw) {
                // lane m of a row holds quarter m (pairs 4m .. 4m + 3); the quarters add
                // in a balanced tree in index order: xor 1 and xor 2 (quad_perm), the
                // quads of 8 lanes (row_half_mirror), the halves of 16 (row_mirror). DPP
                // moves read other lanes, so every lane runs them (the empty asm keeps the
                // compiler from moving them under a lane mask).
                float tot[NIT];
#pragma unroll
                for (int it = 0; it < NIT; it++) {
                    float v = qk_quarter_sumsq(a[it].x, b[it].x, a[it].y, b[it].y, a[it].z, b[it].z, a[it].w, b[it].w);
                    auto tree_add = [&](auto ctrl) {
                        float o = dpp_mov<decltype(ctrl)::value>(v);
                        asm volatile("" : "+v"(o));
                        v += o;
                    };
                    tree_add(std::integral_constant<int, 0xB1>{});
                    tree_add(std::integral_constant<int, 0x4E>{});
                    tree_add(std::integral_constant<int, 0x141>{});
                    if constexpr (LPR == 16) tree_add(std::integral_constant<int, 0x140>{});
                    tot[it] = v;  // the row's sum of squares on each of its lanes
                }
                // one 1/rms per row: lane l takes row l % 32, then every lane its rows'
                const uint32_t rr = lane % kQRows, src = (rr % RPI) * LPR;
                float mine = 0.0f;
#pragma unroll
                for (int it = 0; it < NIT; it++) {
                    const float tv = __shfl(tot[it], (int)src, 64);
                    if (rr / RPI == (uint32_t)it) mine = tv;
                }
                const float rs = rms_inv(mine, (float)D, p.eps) * p.q_scale;
#pragma unroll
                for (int it = 0; it < NIT; it++) r[it] = __shfl(rs, (int)(RPI * it + g), 64);
            }
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                const float x0[4] = {a[it].x, a[it].y, a[it].z, a[it].w}, x1[4] = {b[it].x, b[it].y, b[it].z, b[it].w};
                f16x4 y0v, y1v;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if constexpr (QM == kQRaw) {
                        const float c_[4] = {c[it].x, c[it].y, c[it].z, c[it].w};
                        const float s_[4] = {sn[it].x, sn[it].y, sn[it].z, sn[it].w};
                        const float w0_[4] = {w0.x, w0.y, w0.z, w0.w}, w1_[4] = {w1.x, w1.y, w1.z, w1.w};
                        _Float16 o0, o1;
                        qk_q_pair(x0[e], x1[e], w0_[e], w1_[e], c_[e], s_[e], r[it], o0, o1);
                        y0v[e] = o0;
                        y1v[e] = o1;
                    } else {
                        y0v[e] = qk_scaled_f16(x0[e], p.q_scale);
                        y1v[e] = qk_scaled_f16(x1[e], p.q_scale);
                    }
                }
                char* rowp = area + (RPI * it + g) * QSTR;
                *(f16x4*)(rowp + 8 * m) = y0v;
                *(f16x4*)(rowp + D + 8 * m) = y1v;
            }
        }
        // (one wavefront wrote these rows: its LDS accesses complete in order)
#pragma unroll
        for (int ks = 0; ks < KS; ks++) dst[ks] = *(const f16x8*)(area + r32 * QSTR + 32 * ks + 16 * h);
    };

    f32x16 O[DT];  // zeroed after the prologue's q operand (and after the switch's)
    // The scores are kept relative to the row's reference m (the lazy running max,
    // an f16 value): every score product starts with a 16-deep product whose only
    // nonzero term is 1 x (-m) (onecol . mneg), so the products leave s - m and the
    // weights are exp2(s - m) with no subtraction. thr: the rescale threshold on the
    // relative max (-inf until a q tile has its first reference).
    float m_sh = 0.0f, thr = -INFINITY;
    f16x8 onecol, mneg;
#pragma unroll
    for (int i = 0; i < 8; i++) onecol[i] = mneg[i] = (f16)0.0f;
    onecol[0] = h == 0 ? (f16)1.0f : (f16)0.0f;
    // Row sums of the weights on the matrix core: Lsum^T += ones . P^T after each key
    // step's PV products (every row of Lsum^T is the row-sum vector; element 0 is read).
    // The sum is of the same f16 weights the products take.
    f32x16 Lsum;
    f16x8 ones;
#pragma unroll
    for (int i = 0; i < 8; i++) ones[i] = (f16)1.0f;
    float mx = -INFINITY;  // row max of the scores computed one step ahead

    // Causal mask of half kh of item i's scores, in place: lane (r32, h), score r of
    // the half is key key0 + 32 kh + 8 (r / 4) + 4 h + r % 4; keys past the row's
    // position are -inf. Needed when the half's last key lies past the q tile's first
    // row.
    auto masked_half = [&](uint32_t i, int kh) -> bool {
        return item_kt(i) * kKTile + 32 * kh + 31 > p.pos + item_qt(i) * kQRows;
    };
    auto mask_half = [&](f32x16& s, uint32_t i, int kh) {
        const int lim = (int)(p.pos + item_qt(i) * kQRows + r32) - (int)(item_kt(i) * kKTile + 32 * kh) - 4 * h;
#pragma unroll
        for (int r = 0; r < 16; r++)
            if (8 * (r / 4) + (r % 4) > lim) s[r] = -INFINITY;
    };
    // Row max of a half (lanes l and l ^ 32 hold the two key subsets of a row); a
    // linear chain, which the backend turns into v_max3 on the raw MFMA results.
    auto half_max = [&](const f32x16& s) -> float {
        float a = s[0];
#pragma unroll
        for (int r = 1; r < 16; r++) a = fmaxf(a, s[r]);
        return max_xor32(a);
    };
    // V operand of key step m, dim block dt, from the stage at byte offset `st`. The
    // k-slot (h, jj) of step m is key 16m + 8(jj/4) + 4h + jj%4. Transpose read: lane
    // i of a 16-lane group addresses row base + i/4, columns c0 + 4(i%4); lane j
    // receives column c0 + j of the 4 rows.
    auto vread = [&](uint32_t st, int m, int dt) -> f16x8 {
        const char* sv = s_kv + st + G::KSTAGE + vb;
        const f16x4 lo = lds_read_tr16(sv + 16 * m * RSV + 64 * dt);
        const f16x4 hi = lds_read_tr16(sv + (16 * m + 8) * RSV + 64 * dt);
        return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    // K operands of the scores in flight; the first AHEAD are read one step early.
    constexpr int AHEAD = kOpAhead < KS ? kOpAhead : KS;
    static_assert(8 % KS == 0 && 8 % DT == 0 && KS >= AHEAD && 2 * DT >= AHEAD, "schedule shape");
    f16x8 kop[KS];
    auto kptr = [&](uint32_t kst, int hn) -> const char* { return s_kv + kst + kb + 32 * hn * RSK; };

    // One step = one 32-key half hc of the current item (scores Sc relative to the
    // reference, their row max mx), in issue order:
    //   - the 1 + KS products of the next half's scores Sn = -m + K . Q^T (K at sk)
    //     when NEXT, beside the weights exp2(Sc) of the half's first 8 scores (the P^T
    //     operand of key step 2 hc, rounded to f16);
    //   - the lazy rescale check against mx: it is evaluated here, after those
    //     weights, rather than before them, so the branch never waits for mx. The
    //     weights were computed against the old reference; when the reference moves
    //     (the half's max exceeds it by more than 2^kRescaleLog2, and at the start of
    //     every q tile) O and the row sum are rescaled, Sc and Sn move to the new
    //     reference and those 8 weights are computed again;
    //   - the 2 DT products O^T += V^T . P^T (V tile in stage vst) and a row-sum
    //     product per key step: the first DT (key step 2 hc) beside the weights of the
    //     other 8 scores (key step 2 hc + 1, used by the last DT), the last DT beside
    //     the row max of Sn.
    // LDS operand reads run AHEAD products ahead of their use, across the steps too
    // (the last products of a step read the first K operands of the next step's
    // scores, at sk_after, when PRE), and scheduling fences keep this order, so the
    // matrix cores and the VALU work at once and no product waits for its operand
    // read.
    auto step = [&](f32x16& Sc, f32x16& Sn, int hc, uint32_t vst, const char* sk, const char* sk_after,
                    auto next, auto pre) {
        constexpr bool NEXT = decltype(next)::value, PRE = decltype(pre)::value;
        constexpr int NK = KS, NV = 2 * DT, E0 = 8 / NK, E1 = 8 / DT;
        f16x8 vop[NV], pop[2];
        float e[16];
        auto vr = [&](int n) -> f16x8 { return vread(vst, 2 * hc + n / DT, n % DT); };
        // (The empty asm statements pin each result where it is computed: without them
        // the compiler sinks the weights below the rescale branch, or gathers the max
        // chain after the last product, and nothing overlaps the matrix cores.)
        auto weight = [&](int f) {  // score f of the half
            e[f] = fast_exp2(Sc[f]);
            if (f % 2 == 1) {
                pop[f / 8][f % 8 - 1] = (f16)e[f - 1];
                pop[f / 8][f % 8] = (f16)e[f];
                if (f % 8 == 7) asm volatile("" : "+v"(pop[f / 8]));
            }
        };
        if constexpr (!NEXT) {  // (a step with NEXT finds kop[0, AHEAD) read)
#pragma unroll
            for (int n = 0; n < AHEAD; n++) vop[n] = vr(n);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int n = 0; n < NK; n++) {
            if constexpr (NEXT) {
                if (n + AHEAD < NK)
                    kop[n + AHEAD] = *(const f16x8*)(sk + 32 * (n + AHEAD));
                else
                    vop[n + AHEAD - NK] = vr(n + AHEAD - NK);
                if (n == 0) {
#pragma unroll
                    for (int r = 0; r < 16; r++) Sn[r] = 0.0f;
                    Sn = mfma_32x32x16(onecol, mneg, Sn);
                }
                Sn = mfma_32x32x16(kop[n], qop[n], Sn);
            }
#pragma unroll
            for (int j = 0; j < E0; j++) weight(E0 * n + j);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (__builtin_expect(__ballot(mx > thr) != 0, 0)) {  // rare: the reference moves
            // New reference: the row's max rounded to f16 (the shift operand is f16; the
            // difference of two f16 values is exact in f32). The scores in flight (Sc,
            // and Sn, whose products started from the old reference) move with it.
            const float m_new = mx > thr ? (float)(f16)fminf(fmaxf(mx + m_sh, -65504.0f), 65504.0f) : m_sh;
            const float delta = m_new - m_sh;
            const float alpha = thr == -INFINITY ? 0.0f : fast_exp2(-delta);  // O and l are 0 at a q tile's start
            Lsum[0] *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) O[dt] *= alpha;
            m_sh = m_new;
            thr = kRescaleLog2;
            mneg[0] = h == 0 ? (f16)(-m_sh) : (f16)0.0f;
            Sc -= delta;
            if constexpr (NEXT) Sn -= delta;
#pragma unroll
            for (int f = 0; f < 8; f++) weight(f);
        }
        __builtin_amdgcn_sched_barrier(0);
        float a = NEXT ? Sn[0] : 0.0f;
#pragma unroll
        for (int n = 0; n < NV; n++) {
            if (n + AHEAD < NV)
                vop[n + AHEAD] = vr(n + AHEAD);
            else if constexpr (PRE)
                kop[n + AHEAD - NV] = *(const f16x8*)(sk_after + 32 * (n + AHEAD - NV));
            O[n % DT] = mfma_32x32x16(vop[n], pop[n / DT], O[n % DT]);
            if (n % DT == DT - 1) Lsum = mfma_32x32x16(ones, pop[n / DT], Lsum);
            if (n < DT) {
#pragma unroll
                for (int j = 0; j < E1; j++) weight(8 + E1 * n + j);
            } else if constexpr (NEXT) {
#pragma unroll
                for (int j = 1; j < 16; j += 2)  // Sn's max over the last DT products
                    if ((j - 1) / 2 * DT / 8 == n - DT) a = vmax3(a, Sn[j], j + 1 < 16 ? Sn[j + 1] : Sn[j]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (NEXT) mx = max_xor32(a);
    };

    // The wavefront's rows of q tile `qtile` when every key of the tile went through
    // it: O over its row sum, one 32-dim block at a time through the staging area
    // (lane (r32, h) holds dims 8 i4 + 4 h + [0, 4) of row r32 in O[dt][4 i4 ..]), then
    // stored along rows: lane l, row 8 it + l / 8, dims 4 (l % 8) + [0, 4).
    // Blocks staged per pass: as many as the quarter stage holds.
    constexpr int OBLK = (G::STAGE / 4) / (32 * OSTR) < DT ? (G::STAGE / 4) / (32 * OSTR) : DT;
    static_assert(OBLK >= 1 && DT % OBLK == 0, "whole passes");
    auto write_rows = [&](uint32_t qtile, char* area) {
        const float inv_l = 1.0f / Lsum[0];
        const uint32_t q0 = qtile * kQRows, lane = lane_here();
#pragma unroll
        for (int d0 = 0; d0 < DT; d0 += OBLK) {
#pragma unroll
            for (int u = 0; u < OBLK; u++)
#pragma unroll
                for (int i4 = 0; i4 < 4; i4++)
                    *(float4*)(area + (32 * u + r32) * OSTR + 32 * i4 + 16 * h) =
                        float4{O[d0 + u][4 * i4] * inv_l, O[d0 + u][4 * i4 + 1] * inv_l, O[d0 + u][4 * i4 + 2] * inv_l,
                               O[d0 + u][4 * i4 + 3] * inv_l};
#pragma unroll
            for (int u = 0; u < OBLK; u++)
#pragma unroll
                for (int it = 0; it < kQRows / 8; it++) {
                    const uint32_t row = 8 * it + lane / 8, c4 = lane % 8;
                    const float4 v = *(const float4*)(area + (32 * u + row) * OSTR + 16 * c4);
                    if (live && q0 + row < p.n_tokens)
                        *(float4*)(p.out + ((uint64_t)(q0 + row) * p.n_q_heads + hq) * D + 32 * (d0 + u) + 4 * c4) = v;
                }
        }
    };

    // Half kh of item i on a tile that crosses the diagonal: its causal mask, in place,
    // then its max again.
    auto mask_if_needed = [&](f32x16& s, uint32_t i, int kh) {
        if (__builtin_expect(masked_half(i, kh), 0)) {
            mask_half(s, i, kh);
            mx = half_max(s);
        }
    };

    // Scores of item i's first half from its stage (no shift: the caller's reference
    // is 0), the K operands of its second half read ahead, and their row max.
    auto first_scores = [&](f32x16& S, uint32_t i) {
        const char* sk = s_kv + k_stage(i) + kb;
#pragma unroll
        for (int r = 0; r < 16; r++) S[r] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) S = mfma_32x32x16(*(const f16x8*)(sk + 32 * ks), qop[ks], S);
#pragma unroll
        for (int n = 0; n < AHEAD; n++) kop[n] = *(const f16x8*)(kptr(k_stage(i), 1) + 32 * n);
        mx = half_max(S);  // (a masked half's max is taken again after its mask)
    };

    auto zero_acc = [&]() {
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int i = 0; i < 16; i++) O[dt][i] = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) Lsum[i] = 0.0f;
    };

    // ---- prologue: the heavy tile's q operand, staged in stage kAhead (the producer
    // streams items 0 .. kAhead - 1 into the others meanwhile and fills this one only
    // after the barrier); the scores of item 0's first half and their row max.
    f32x16 Sa, Sb;  // scores of the current item's first and second half
    {
        QRows in;
        q_load(in, heavy);
        q_form(qop, in, area_of(k_stage(kAhead)));
    }
    lds_sync();
    first_scores(Sa, 0);
    zero_acc();

    // Round r (item r): step 0 (weights and PV of its first half; scores of its second
    // half), then step 1 (weights and PV of its second half; scores of item r + 1's
    // first half, from stage (r + 1) % kStages), then the round's barrier. A special
    // round also masks the halves that cross the diagonal or switches to the light
    // tile; the others run the plain form, so the loop over a run of plain rounds has
    // no branch but the rare rescale.
    // The switch (round H - 1): step 1 forms item r + 1's first scores with the heavy
    // tile's operand (nine wasted products: a step without next scores there, in a
    // branch of its own, made the compiler spill); a barrier (the producer takes it too)
    // frees item r's stage, which is refilled only in round r + 1; there the heavy
    // tile's rows are written and the light tile's operand is staged (its loads issued
    // before the barrier, so that their latency overlaps the row stores); item r + 1's
    // first scores are formed again as in the prologue, from reference 0 -- the same
    // arithmetic in every q mode, so the modes give the same outputs from the same
    // operand.
    auto round = [&](uint32_t r, auto special) {
        constexpr bool SPECIAL = decltype(special)::value;
        const uint32_t st = k_stage(r), st1 = k_stage(r + 1);
        if constexpr (SPECIAL) mask_if_needed(Sa, r, 0);
        step(Sa, Sb, 0, st, kptr(st, 1), kptr(st1, 0), std::true_type{}, std::true_type{});
        if constexpr (SPECIAL) mask_if_needed(Sb, r, 1);
        step(Sb, Sa, 1, st, kptr(st1, 0), kptr(st1, 1), std::true_type{}, std::true_type{});
        if constexpr (SPECIAL) {
            if (r + 1 == H) {  // the heavy tile is done: its rows, then the light tile's
                QRows in;
                q_load(in, pair);
                lds_sync();
                write_rows(heavy, area_of(st));
                q_form(qop, in, area_of(st));
                m_sh = 0.0f;
                mneg[0] = (f16)0.0f;
                first_scores(Sa, r + 1);
                zero_acc();
                thr = -INFINITY;
            }
        }
        lds_sync();
    };
    // The special rounds: the switch (round H - 1) and the items whose second half
    // crosses a q tile's first row (key tile kt of q tile qt with 64 kt + 63 > pos +
    // 32 qt, i.e. kt >= first_masked).
    auto first_masked = [&](uint32_t qtile) -> uint32_t { return (p.pos + qtile * kQRows + 1) / kKTile; };
    const uint32_t mh = min(first_masked(heavy), H), ml = H + first_masked(pair);
    auto next_special = [&](uint32_t r) -> uint32_t {  // the first special round >= r
        uint32_t ns = n_items;
        if (has_light) {
            ns = r <= H - 1 ? H - 1 : n_items;
            ns = min(ns, max(r, ml));
        }
        if (r < H && mh < H) ns = min(ns, max(r, mh));
        return ns;
    };
    for (uint32_t r = 0; r + 1 < n_items;) {
        const uint32_t stop = min(next_special(r), n_items - 1);
        for (; r < stop; r++) round(r, std::false_type{});
        if (r + 1 < n_items) round(r++, std::true_type{});
    }
    // the last item: its second half's scores, then nothing ahead; the rows go through
    // the stage of item n_items - 2 (every wavefront passed the barrier after it, and
    // nothing refills it; with one item, stage 3, never filled)
    {
        const uint32_t r = n_items - 1, st = k_stage(r);
        mask_if_needed(Sa, r, 0);
        step(Sa, Sb, 0, st, kptr(st, 1), nullptr, std::true_type{}, std::false_type{});
        mask_if_needed(Sb, r, 1);
        step(Sb, Sa, 1, st, nullptr, nullptr, std::false_type{}, std::false_type{});
    }
    write_rows(has_light ? pair : heavy, area_of(k_stage(n_items + kStages - 2)));
}
}  // namespace

bool prefill_prep_supported(uint32_t n_kv_heads, uint32_t head_dim) {
    return (uint64_t)n_kv_heads * head_dim <= kPrepMaxRow && (head_dim == 64 || head_dim == 128);
}

int launch_kv_prep(ds5_hip_ctx* ctx, const KvPrepLaunch& a) {
    if (a.n_tokens == 0) return DS5_OK;
    if (a.head_dim == 128)
        DS5_TIMED_LAUNCH(ctx, "prefill_prep_kernel", prefill_prep_kernel<128>, dim3(a.n_tokens), dim3(kPrepThreads), 0,
                         ctx->stream, a, *a.table);
    else
        DS5_TIMED_LAUNCH(ctx, "prefill_prep_kernel", prefill_prep_kernel<64>, dim3(a.n_tokens), dim3(kPrepThreads), 0,
                         ctx->stream, a, *a.table);
    return ds5_after_launch(ctx, "prefill_prep_kernel");
}

template <int D, int QM>
static void launch_prefill_k(ds5_hip_ctx* ctx, const PrefillParams& p) {
    DS5_TIMED_LAUNCH(ctx, "prefill_attention_kernel", (prefill_attention_kernel<D, QM>), dim3(p.n_items), dim3(kThreads),
                     0, ctx->stream, p);
}

int launch_prefill(ds5_hip_ctx* ctx, const PrefillLaunch& a) {
    if (a.n_tokens == 0) return DS5_OK;
    PrefillParams p{};
    p.q16 = a.q16;
    p.q = a.q;
    p.q_norm = a.q_norm;
    p.cs = a.cs;
    p.eps = a.eps;
    p.q_scale = a.q_scale;
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
    const int qm = a.q16 ? kQOperand : a.cs ? kQRaw : kQRotated;
    if (a.head_dim == 128) {
        if (qm == kQOperand) launch_prefill_k<128, kQOperand>(ctx, p);
        else if (qm == kQRaw) launch_prefill_k<128, kQRaw>(ctx, p);
        else launch_prefill_k<128, kQRotated>(ctx, p);
    } else {
        if (qm == kQOperand) launch_prefill_k<64, kQOperand>(ctx, p);
        else if (qm == kQRaw) launch_prefill_k<64, kQRaw>(ctx, p);
        else launch_prefill_k<64, kQRotated>(ctx, p);
    }
    return ds5_after_launch(ctx, "prefill_attention_kernel");
}
