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
// and the attention kernel's q operand: q normalised, rotated, times softmax
// scale * log2(e), rounded to f16 ([n_tokens, n_q_heads, head_dim]). The
// separate-op path packs an already normalised and rotated q the same way
// (q_pack_kernel). The attention block's projection GEMM can do the pre-pass
// in its epilogue instead (k_matmul.hip).
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
constexpr int kHeads = 4;      // q heads per workgroup, one compute wavefront each
constexpr int kThreads = (kHeads + 1) * 64;  // + the producer wavefront
constexpr int kQRows = 32;     // q rows per wavefront tile (MFMA N)
constexpr int kKTile = 64;     // keys per LDS stage
constexpr int kStages = 4;     // K/V ring: a stage is refilled three rounds ahead of its use
constexpr int kAhead = kStages - 1;
constexpr int kOpAhead = 3;    // LDS operand reads in flight ahead of their product
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
        for (int b = 0; b < NB; b++) {
            const int pos = 1024 * b + 16 * lane;
            const int r = pos / RS, c = (pos % RS) / 16;
            off[b] = (uint32_t)(r * 2 * D + (c < D / 8 ? 16 * c : 0));
        }
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
        const uint32_t last_row = kv_end - key0 - 1;  // rows of this tile below kv_end, minus one
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const uint32_t lds = __builtin_amdgcn_readfirstlane(stage_lds + 1024 * b);
            const uint32_t off = min(tp.off[b] / (2 * D), last_row) * (2 * D) + tp.off[b] % (2 * D);
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
template <int D>
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

    // the wavefront's q tile: lane (r32, h) holds query row t
    uint32_t t = heavy * kQRows + r32;
    bool keep = live && t < p.n_tokens;

    // q operand of lane (r32, h): row t, dims 16 ks + 8 h + [0, 8) for every k-step.
    // Rows past the last token and the heads of an unfilled group read clamped, valid
    // q rows: their scores stay in their own columns of S and O and are never written.
    f16x8 qop[KS], qnext[KS];
    auto load_q = [&](f16x8(&dst)[KS], uint32_t qtile) {
        const uint32_t tc = min(qtile * kQRows + r32, p.n_tokens - 1);
        const f16* qrow = p.q16 + ((uint64_t)tc * p.n_q_heads + hq) * D + 8 * h;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) dst[ks] = *(const f16x8*)(qrow + 16 * ks);
    };

    f32x16 O[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int i = 0; i < 16; i++) O[dt][i] = 0.0f;
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
#pragma unroll
    for (int i = 0; i < 16; i++) Lsum[i] = 0.0f;
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

    // The wavefront's rows of its q tile when every key of the tile went through it:
    // O over its row sum.
    auto write_rows = [&]() {
        const float l = Lsum[0];
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

    // Half kh of item i on a tile that crosses the diagonal: its causal mask, in place,
    // then its max again.
    auto mask_if_needed = [&](f32x16& s, uint32_t i, int kh) {
        if (__builtin_expect(masked_half(i, kh), 0)) {
            mask_half(s, i, kh);
            mx = half_max(s);
        }
    };

    // ---- prologue: both q tiles' operands (the producer streams items 0 .. kAhead - 1
    // meanwhile); the scores of item 0's first half and their row max before round 0.
    load_q(qop, heavy);
    f32x16 Sa, Sb;  // scores of the current item's first and second half
    wait_vm<0>();
    lds_sync();
    {
        const char* sk = s_kv + k_stage(0) + kb;
#pragma unroll
        for (int r = 0; r < 16; r++) Sa[r] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) Sa = mfma_32x32x16(*(const f16x8*)(sk + 32 * ks), qop[ks], Sa);
#pragma unroll
        for (int n = 0; n < AHEAD; n++) kop[n] = *(const f16x8*)(kptr(k_stage(0), 1) + 32 * n);
        mx = half_max(Sa);  // (a masked half's max is taken again after its mask)
    }

    // Round r (item r): step 0 (weights and PV of its first half; scores of its second
    // half), then step 1 (weights and PV of its second half; scores of item r + 1's
    // first half, from stage (r + 1) % kStages), then the round's barrier. A special
    // round also masks the halves that cross the diagonal, loads the light tile's q
    // operand or switches to the light tile; the others run the plain form, so the
    // loop over a run of plain rounds has no branch but the rare rescale.
    auto round = [&](uint32_t r, auto special) {
        constexpr bool SPECIAL = decltype(special)::value;
        const uint32_t st = k_stage(r), st1 = k_stage(r + 1);
        if constexpr (SPECIAL) {
            // The light tile's q operand loads one round in (not with the heavy tile's:
            // at the start every workgroup loads its q at once, and that burst is time
            // no product overlaps), or in round 0 when item 1 already starts the light
            // tile.
            if (has_light && r == min(1u, H - 1)) load_q(qnext, pair);
            mask_if_needed(Sa, r, 0);
        }
        step(Sa, Sb, 0, st, kptr(st, 1), kptr(st1, 0), std::true_type{}, std::true_type{});
        if constexpr (SPECIAL) {
            if (r + 1 == H) {  // item H's scores (the next step) start the light tile
                wait_vm<0>();
#pragma unroll
                for (int ks = 0; ks < KS; ks++) qop[ks] = qnext[ks];
            }
            mask_if_needed(Sb, r, 1);
        }
        step(Sb, Sa, 1, st, kptr(st1, 0), kptr(st1, 1), std::true_type{}, std::true_type{});
        if constexpr (SPECIAL) {
            if (r + 1 == H) {  // the heavy tile is done: its rows, then the light tile's state
                write_rows();
                t = pair * kQRows + r32;
                keep = live && t < p.n_tokens;
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
#pragma unroll
                    for (int i = 0; i < 16; i++) O[dt][i] = 0.0f;
                thr = -INFINITY;
#pragma unroll
                for (int i = 0; i < 16; i++) Lsum[i] = 0.0f;
            }
        }
        lds_sync();
    };
    // The special rounds: the light tile's q load (round min(1, H - 1)) and switch
    // (round H - 1), and the items whose second half crosses a q tile's first row
    // (key tile kt of q tile qt with 64 kt + 63 > pos + 32 qt, i.e. kt >= first_masked).
    auto first_masked = [&](uint32_t qtile) -> uint32_t { return (p.pos + qtile * kQRows + 1) / kKTile; };
    const uint32_t mh = min(first_masked(heavy), H), ml = H + first_masked(pair);
    auto next_special = [&](uint32_t r) -> uint32_t {  // the first special round >= r
        uint32_t ns = n_items;
        if (has_light) {
            ns = r <= min(1u, H - 1) ? min(1u, H - 1) : r <= H - 1 ? H - 1 : n_items;
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
    // the last item: its second half's scores, then nothing ahead
    {
        const uint32_t r = n_items - 1, st = k_stage(r);
        mask_if_needed(Sa, r, 0);
        step(Sa, Sb, 0, st, kptr(st, 1), nullptr, std::true_type{}, std::false_type{});
        mask_if_needed(Sb, r, 1);
        step(Sb, Sa, 1, st, nullptr, nullptr, std::false_type{}, std::false_type{});
    }
    write_rows();
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
