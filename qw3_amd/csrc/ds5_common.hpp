// ds5_common.hpp -- shared types and helpers of the gfx950 attention backend.
//
// Host side: the context object behind ds5_hip_ctx, error helpers, and the
// launch functions each kernel file exports to the C-ABI op layer.
// Device side: vector types, MFMA wrappers, wavefront reductions.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "ds5_hip.h"
#include "ds5_index.hpp"

// ---------------------------------------------------------------------------
// Vector types (clang ext_vector_type: what the MFMA builtins take)
// ---------------------------------------------------------------------------
typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Rope inverse-frequency table: inv[i] = theta^(-(2i)/head_dim) evaluated the
// way the reference's std.math.pow(f32) evaluates it (see ds5_rope_table in
// ds5_ops.hip). Passed by value as a kernel argument; head_dim <= 512.
// ---------------------------------------------------------------------------
constexpr int DS5_MAX_ROPE_HALF = 256;
struct RopeTable {
    float inv[DS5_MAX_ROPE_HALF];
};

// ---------------------------------------------------------------------------
// Context (the object behind the opaque ds5_hip_ctx handle)
// ---------------------------------------------------------------------------
struct ds5_hip_ctx {
    int device = 0;
    int cu_count = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev_begin = nullptr;
    hipEvent_t ev_end = nullptr;
    bool batch_open = false;
    uint64_t elapsed_ns = 0;
    std::vector<void*> owned;  // device allocations freed at deinit
    std::string last_error;
    // Split-K partial results: grown on demand, owned by the context.
    void* workspace = nullptr;
    size_t workspace_bytes = 0;
    // A second growable buffer for a row-normalised x that must live beside the
    // workspace (the fused calls' rmsNorm when it cannot run inside the kernels).
    void* aux = nullptr;
    size_t aux_bytes = 0;
    // The library's static device scratch array on this context's device (its
    // address from hipGetSymbolAddress, taken once per device at init). While
    // use_scratch is set -- the allocation-free entry point -- the workspace
    // comes from there and nothing is allocated.
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    bool use_scratch = false;
    // Decode tuning: positions per split-K workgroup (0 = heuristic); paged
    // plan: workgroups per launch the plan aims at (0 = two per CU).
    uint32_t decode_chunk = 0;
    uint32_t plan_items = 0;
    // DS5_HIP_MOE_TWO_LAUNCH: the experts' down GEMV and the combine as the two
    // launches that serve outputs beyond one grid, at any size (tests of that path)
    bool moe_two_launch = false;
    // Optional per-kernel timing: events recorded around every launch on the
    // context stream, resolved at submit / query time.
    bool kernel_timing = false;
    std::vector<hipEvent_t> event_pool;
    size_t event_next = 0;
    struct Pending {
        const char* name;
        hipEvent_t start, end;
    };
    std::vector<Pending> pending;
    std::map<std::string, std::pair<double, uint64_t>> kernel_ns;  // name -> (total ns, launches)
    // Device-time marks (ds5_hip_timing_*): events recorded on the stream, reused.
    std::vector<hipEvent_t> marks;
    size_t marks_used = 0;
};

// Per-kernel timing: a pooled event pair per launch, resolved at submit / query time.
hipEvent_t ds5_next_event(ds5_hip_ctx* ctx);
void ds5_timer_record(ds5_hip_ctx* ctx, const char* name, hipEvent_t start, hipEvent_t end);
int ds5_timers_resolve(ds5_hip_ctx* ctx);

int ds5_fail(ds5_hip_ctx* ctx, int code, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
int ds5_hip_status(ds5_hip_ctx* ctx, hipError_t err, const char* what);
int ds5_after_launch(ds5_hip_ctx* ctx, const char* what);
int ds5_workspace(ds5_hip_ctx* ctx, size_t bytes, void** out);
int ds5_aux_workspace(ds5_hip_ctx* ctx, size_t bytes, void** out);
// Looks up (once per device) the address of the static scratch array on the
// context's device, which must be current, and records it in the context.
int ds5_scratch_init(ds5_hip_ctx* ctx);
void ds5_rope_table(float theta, uint32_t head_dim, RopeTable* t);

// Launches a kernel on `stream`. With timing enabled the launch carries its own
// start/stop events (hipExtLaunchKernelGGL: the events belong to the dispatch
// itself, so they time the kernel's execution, as a profiler's kernel trace
// does, not the dispatch latency around it).
template <typename K, typename... Args>
inline void ds5_launch(ds5_hip_ctx* ctx, const char* name, K kernel, dim3 grid, dim3 block, uint32_t shmem,
                       hipStream_t stream, Args... args) {
    if (ctx->kernel_timing) {
        hipEvent_t start = ds5_next_event(ctx), stop = ds5_next_event(ctx);
        if (start && stop) {
            hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, start, stop, 0u, args...);
            ds5_timer_record(ctx, name, start, stop);
            return;
        }
    }
    hipLaunchKernelGGL(kernel, grid, block, shmem, stream, args...);
}
#define DS5_TIMED_LAUNCH(ctx, name, ...) ds5_launch((ctx), (name), __VA_ARGS__)

static inline void* ds5_ptr(ds5_buf b) { return (char*)b.handle + b.offset; }

// ---------------------------------------------------------------------------
// Launchers exported by the kernel files (preconditions already checked)
// ---------------------------------------------------------------------------
// Projection matmul (k_matmul.hip): out[m, n] = x[m, k] . W^T, W f32 or Q8_0 rows.
struct MatmulLaunch {
    const float* x;
    const uint8_t* w;
    bool q8;
    float* out;
    uint32_t m, n, k;
    const float* res = nullptr;  // out = res + x . W^T when set (res may be out itself)
};
// Which kernel runs: the row (GEMV) kernel, the Q8_0 matrix-core GEMM, or the
// serial one-thread-per-output kernel that takes any shape and alignment.
enum class MatmulPath { Generic, Rows, Gemm };
MatmulPath matmul_path(const MatmulLaunch& a, uint64_t w_len);
int launch_matmul(ds5_hip_ctx* ctx, const MatmulLaunch& a, MatmulPath path);
// Up to kMatmulGroupMax products sharing x (and m, k, the weight dtype).
constexpr int kMatmulGroupMax = DS5_MATMUL_GROUP_MAX;
struct MatmulGroupLaunch {
    const float* x;
    bool q8;
    uint32_t m, k;
    uint32_t count;
    const uint8_t* w[kMatmulGroupMax];
    float* out[kMatmulGroupMax];
    const float* res[kMatmulGroupMax];  // per entry, as MatmulLaunch::res
    uint32_t n[kMatmulGroupMax];
    // x normalised first (k > 256: the reference GPU kernel's tree order) by the row
    // kernel or the GEMM's x split as they read it; null: x as it is. Only the Rows
    // and Gemm paths take it.
    const float* norm_w;
    float norm_eps;
};
int launch_matmul_group(ds5_hip_ctx* ctx, const MatmulGroupLaunch& a, const MatmulPath* paths);
// The attention block's q/k/v projections with the prefill pre-pass in the GEMM's
// epilogue (Q8_0 weights, head_dim 128, m >= 16): k / v rows into the f16 caches
// at pos, the f16 q operand into q16. ws: qkv_prep_workspace_bytes (x split and
// the rope cos / sin of every token).
struct QkvPrepLaunch {
    const float* x;
    const uint8_t *wq, *wk, *wv;
    uint32_t m, k, n_q_heads, n_kv_heads, head_dim;
    const int32_t* positions;
    float freq_scale;
    const RopeTable* table;
    const float* q_norm;
    const float* k_norm;
    f16* q16;
    f16* k_cache;
    f16* v_cache;
    uint32_t pos, max_ctx;
    float eps, q_scale;
    void* ws;
    const float* norm_w;  // x normalised first, as MatmulGroupLaunch::norm_w (null: none)
    float norm_eps;
};
size_t qkv_prep_workspace_bytes(uint32_t m, uint32_t k, uint32_t head_dim);
int launch_qkv_prep(ds5_hip_ctx* ctx, const QkvPrepLaunch& a);
// Residual add out = x + y over n f32 elements (any views; out may be x or y).
int launch_add(ds5_hip_ctx* ctx, const void* x, const void* y, void* out, uint64_t n);

// MoE router (k_moe.hip): per token, ids / weights (device) and optionally the
// token-major dispatch pairs.
struct RouterLaunch {
    const float* x;
    const uint8_t* w;
    uint32_t w_dtype;
    uint64_t row_bytes;
    uint32_t n_tokens, dim, n_experts, top_k;
    bool norm;
    uint16_t* ids;
    float* weights;
    ds5_pair* pairs;  // may be null
    float* logits;    // scratch [n_tokens, n_experts]
    // x normalised first (f32 rows of dim % 4 == 0 and dim > 256, x and w 16-byte
    // aligned: the logits kernel's fast path; the tree order), the normalised rows
    // written to h_out for the experts; null: x as it is
    const float* x_norm_w;
    float x_norm_eps;
    float* h_out;
};
int launch_router(ds5_hip_ctx* ctx, const RouterLaunch& a);
// The router's logits run in token x expert tiles (router_logits_tile_kernel) from
// this many tokens, for f32 or f16 rows (dim % 4 == 0, x 16-byte and the rows 16- or
// 8-byte aligned) without an in-kernel norm.
constexpr uint32_t kRouterTileMinTokens = 32;
bool router_tiled(uint32_t w_dtype, uint32_t n_tokens, uint32_t dim, const void* x, const void* w);

// SwiGLU experts over device dispatch pairs; out accumulates. Token t's pairs
// are order[offsets[t] .. offsets[t + 1]) in list order, or t*top_k .. when
// offsets is null. h [n_pairs, ffn] and y [n_pairs, dim] are scratch.
struct ExpertLaunch {
    const float* x;
    const uint8_t *gate, *up, *down;
    bool q8;
    bool fast;  // the wavefront GEMVs (else the serial kernels)
    const ds5_pair* pairs;
    const uint32_t* order;
    const uint32_t* offsets;
    uint32_t top_k;
    float* out;
    const float* res;  // set: out = res + the experts' sum from zero; null: the sum accumulates into out
    float* h;
    float* y;
    uint32_t n_tokens, n_pairs, dim, ffn;
    uint64_t row_h, row_f, stride_gu, stride_d;
    // grouped: the products on the matrix cores over the pairs sorted by expert
    // (Q8_0 banks, many pairs per expert); the scratch below, h holding the gate
    // products and u the up products, y the down products in pair order
    bool grouped;
    uint32_t n_experts, max_tiles, tile_rows;
    uint16_t *xhi, *xlo, *hhi, *hlo;
    int *xexp, *hexp;
    float* u;
    uint32_t *perm, *xrow, *n_tiles;
    uint4* tiles;
};
// The grouped path's row tiles: at most P / rows + E of 64 or 128 rows (each expert's
// last one partial).
constexpr uint32_t kMoeMinTileRows = 64;
inline uint32_t moe_max_tiles(uint32_t n_pairs, uint32_t n_experts, uint32_t tile_rows = kMoeMinTileRows) {
    return n_pairs / tile_rows + n_experts + 1;
}
constexpr uint32_t kMoeGroupedMaxExperts = 2048;
int launch_experts(ds5_hip_ctx* ctx, const ExpertLaunch& a);
// The experts over rows sorted by expert on the matrix cores (k_matmul.hip): the
// tokens' x rows split into f16 planes; grouped Q8_0 products whose row tiles (of
// tile_rows rows) come from a device table (first row, end row, expert), x_rows (if
// not null) mapping each sorted row to its plane row; h = silu(g) * u split.
int launch_x_split_rows(ds5_hip_ctx* ctx, const float* x, uint32_t rows, uint32_t k, uint16_t* hi, uint16_t* lo,
                        int* row_exp);
int launch_moe_h_split(ds5_hip_ctx* ctx, const float* g, const float* u, uint32_t rows, uint32_t k, uint16_t* hi,
                       uint16_t* lo, int* row_exp);
int launch_q8_gemm_grouped(ds5_hip_ctx* ctx, const uint16_t* hi, const uint16_t* lo, const int* row_exp, uint32_t k,
                           const uint8_t* const* w, float* const* out, const uint32_t* n, uint32_t count,
                           const uint4* tiles, const uint32_t* n_tiles, uint32_t max_tiles, uint32_t tile_rows,
                           uint64_t w_stride, const uint32_t* x_rows, const uint32_t* out_rows);

struct RmsNormLaunch {
    const float* x;
    const float* w;
    float* out;
    uint32_t n_rows, dim;
    float eps;
};
int launch_rms_norm(ds5_hip_ctx* ctx, const RmsNormLaunch& a);

struct RopeLaunch {
    float* x;
    const int32_t* positions;
    uint32_t n_tokens, n_heads, head_dim;
    float freq_scale;
    const RopeTable* table;
};
int launch_rope(ds5_hip_ctx* ctx, const RopeLaunch& a);

struct KvAppendLaunch {
    const float* k_new;
    const float* v_new;
    void* k_cache;
    void* v_cache;
    uint32_t kv_dtype, pos, n_tokens, n_kv_heads, head_dim, max_ctx;
};
int launch_kv_append(ds5_hip_ctx* ctx, const KvAppendLaunch& a);

// Prefill pre-pass of the fused step: per token, the norm + rope + f16 append
// of every kv head's k row, f16 append of v, and the rope cos/sin of the token
// into cs [n_tokens, head_dim] (cos of pairs 0 .. head_dim/2 - 1, then sin),
// which the attention kernel rotates q with.
constexpr float kLog2e = 1.4426950408889634f;  // softmax runs in the log2 domain

struct KvPrepLaunch {
    const float* k;
    const float* v;
    const float* k_norm;
    const int32_t* positions;
    f16* k_cache;
    f16* v_cache;
    float* cs;
    uint32_t pos, n_tokens, n_kv_heads, head_dim, max_ctx;
    float eps, freq_scale;
    const RopeTable* table;
};
bool prefill_prep_supported(uint32_t n_kv_heads, uint32_t head_dim);
int launch_kv_prep(ds5_hip_ctx* ctx, const KvPrepLaunch& a);

// Generic causal GQA attention (any head_dim <= 512, f32 or f16 cache).
struct GenericAttnLaunch {
    const float* q;
    const void* k_cache;
    const void* v_cache;
    float* out;
    uint32_t kv_dtype, pos, n_tokens, n_q_heads, n_kv_heads, head_dim, max_ctx;
    float scale;
};
int launch_generic_attention(ds5_hip_ctx* ctx, const GenericAttnLaunch& a);

// Split-K MFMA decode (one query token per sequence), f16 cache, head_dim 64
// or 128. Covers the contiguous and paged caches, with or without the fused
// norm/rope/append prologue.
struct DecodeLaunch {
    // query / new token (fused: raw projections; unfused: q post-rope only)
    const float* q;          // [n_seqs, n_q_heads, head_dim]
    const float* k_new;      // fused only: [n_seqs, n_kv_heads, head_dim]
    const float* v_new;      // fused only
    const float* q_norm;     // fused only: [head_dim]
    const float* k_norm;     // fused only
    const int32_t* positions;  // fused contiguous: rope position of the token
    // cache (contiguous when page_table == nullptr)
    f16* k_cache;
    f16* v_cache;
    uint64_t cache_stride;   // positions per kv head: max_ctx or pool slots
    const int32_t* page_table;  // [n_seqs, max_pages] or nullptr
    const int32_t* seq_lens;    // [n_seqs] (paged) or nullptr
    uint32_t page_size, max_pages;
    uint32_t ctx_len;        // contiguous: attended positions (pos + 1)
    uint32_t max_len;        // upper bound of attended positions (sizes the grid)
    float* out;              // [n_seqs, n_q_heads * head_dim]
    uint32_t n_seqs, n_q_heads, n_kv_heads, head_dim;
    float scale, eps, freq_scale;
    bool fused;
    const RopeTable* table;
};
int launch_decode(ds5_hip_ctx* ctx, const DecodeLaunch& a);
// Split-K geometry of a decode launch and the workspace bytes it needs (0 when
// one split covers every sequence).
struct DecodeGeometry {
    uint32_t chunk, n_splits;
};
size_t decode_workspace_bytes(const ds5_hip_ctx* ctx, uint32_t n_seqs, uint32_t n_q_heads, uint32_t n_kv_heads,
                              uint32_t head_dim, uint32_t max_len);

// Causal flash-attention prefill on f16 MFMA (head_dim 128 or 64).
// The q operand is one of: q16 (a ready f16 operand, already scaled by softmax
// scale * log2(e)); q with cs (the raw f32 projection: RMSNorm with q_norm and
// eps, rotation with the pre-pass's cos/sin table, times q_scale); q alone (f32,
// already normalised and rotated: times q_scale).
struct PrefillLaunch {
    const f16* q16;          // [n_tokens, n_q_heads, head_dim] or null
    const float* q;          // [n_tokens, n_q_heads, head_dim] f32 (q16 null)
    const float* q_norm;     // [head_dim] (with cs)
    const float* cs;         // [n_tokens, head_dim] or null
    float eps, q_scale;      // q_scale = softmax scale * log2(e) (f32 q)
    const f16* k_cache;
    const f16* v_cache;
    float* out;
    uint32_t pos, n_tokens, n_q_heads, n_kv_heads, head_dim, max_ctx;
};
int launch_prefill(ds5_hip_ctx* ctx, const PrefillLaunch& a);

int launch_fill_normal_f16(ds5_hip_ctx* ctx, f16* out, uint64_t n, uint64_t seed);
int launch_stream_read(ds5_hip_ctx* ctx, const void* src, uint64_t len, uint32_t* sink);
int launch_empty(ds5_hip_ctx* ctx, uint32_t n_workgroups);
int launch_zero(ds5_hip_ctx* ctx, void* p, uint64_t len);

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
#if defined(__HIP_DEVICE_COMPILE__)
#define DS5_DEVICE_INLINE __device__ __forceinline__
#else
#define DS5_DEVICE_INLINE __device__ inline
#endif

DS5_DEVICE_INLINE f32x4 mfma_16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

DS5_DEVICE_INLINE f32x16 mfma_32x32x16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Lane exchange within the 64-wide wavefront (ds_bpermute based: an LDS round trip).
DS5_DEVICE_INLINE float lane_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

// VALU-only cross-lane operations (no LDS round trip).
// DPP move within rows of 16 lanes; CTRL is a DPP control word.
template <int CTRL>
DS5_DEVICE_INLINE float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// op(v[l], v[l ^ 16]) and op(v[l], v[l ^ 32]): v_permlane16_swap / v_permlane32_swap
// with both operands v return (own, partner) in some order, so a commutative op
// of the pair gives the combined value on every lane.
template <class F>
DS5_DEVICE_INLINE float swap16_op(float v, F op) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
template <class F>
DS5_DEVICE_INLINE float swap32_op(float v, F op) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// All-reduce over the 64 lanes in a fixed order: xor 1 and xor 2 (quad_perm),
// the quads of 8 lanes (row_half_mirror), the halves of 16 (row_mirror), then
// rows (permlane16 swap) and halves of the wave (permlane32 swap).
template <class F>
DS5_DEVICE_INLINE float wave_allreduce(float v, F op) {
    v = op(v, dpp_mov<0xB1>(v));   // quad_perm [1, 0, 3, 2]
    v = op(v, dpp_mov<0x4E>(v));   // quad_perm [2, 3, 0, 1]
    v = op(v, dpp_mov<0x141>(v));  // row_half_mirror
    v = op(v, dpp_mov<0x140>(v));  // row_mirror
    v = swap16_op(v, op);
    return swap32_op(v, op);
}
struct OpAdd {
    DS5_DEVICE_INLINE float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
    DS5_DEVICE_INLINE float operator()(float a, float b) const { return fmaxf(a, b); }
};

DS5_DEVICE_INLINE float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Q8_0 (GGUF): 34-byte blocks of an f16 scale and 32 int8; value = f32(scale) * q.
constexpr int kQ8Bytes = 34;

DS5_DEVICE_INLINE float f16_bits_to_f32(uint32_t bits) {
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

DS5_DEVICE_INLINE Q8Block q8_unpack(const uint32_t (&d)[9], uint32_t sh) {
    Q8Block r;
    r.scale = f16_bits_to_f32((d[0] >> (8 * sh)) & 0xffffu);
    const uint32_t sel = sh ? 0x07060504u : 0x05040302u;
#pragma unroll
    for (int i = 0; i < 8; i++) r.q[i] = __builtin_amdgcn_perm(d[i + 1], d[i], sel);
    return r;
}

// sum_i q_i * x_i over one block (four interleaved partial sums)
DS5_DEVICE_INLINE float q8_dot(const uint32_t (&q)[8], const float (&x)[32]) {
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


// Correctly rounded f32 square root. The compiler lowers __fsqrt_rn and
// sqrtf to v_sqrt_f32, which is only 1-ulp accurate, while the reference's
// @sqrt (and the C library's sqrtf) round correctly. The root is taken in f64
// and rounded to f32: rounding twice is innocuous for sqrt when the wide
// format has at least 2*24+2 significand bits (53 here), and a 24-bit input's
// square root lies at least 2^-51 (relative) away from every f32 midpoint, so
// an f64 root within 1 f64 ulp still rounds to the correct f32.
DS5_DEVICE_INLINE float sqrt_rn(float x) { return (float)__builtin_sqrt((double)x); }

// 1 / sqrt(sumsq / dim + eps) with each operation correctly rounded, the
// RMSNorm scale of kernels_a.zig:87.
DS5_DEVICE_INLINE float rms_inv(float sumsq, float dim, float eps) {
    return __fdiv_rn(1.0f, sqrt_rn(__fdiv_rn(sumsq, dim) + eps));
}

// rmsNorm of rows longer than 256 elements takes the reduction order of the
// reference's GPU kernel (kernels_a.metal:127-165): thread t < 256 of a block
// accumulates s = fma(v, v, s) over the row's elements t, t + 256, t + 512, ...
// in that order (kTreeParts partials), then the partials add in a halving tree,
// p[t] += p[t + s] for s = 128, 64, ..., 1. tree_rms_inv takes each thread's
// partial (threads >= 256 pass anything) and returns the row's rms_inv to every
// thread; part: kTreeParts floats of LDS, inv: one float of LDS; every thread of
// the block (at least 256) calls it, as it holds barriers.
constexpr uint32_t kTreeParts = 256;
// ds5_hip_rms_norm: rows of up to this many elements take the reference CPU
// path's serial sum, longer rows the tree order above.
constexpr uint32_t kRmsSerialMaxDim = 256;
DS5_DEVICE_INLINE float tree_rms_inv(float s, uint32_t dim, float eps, float* part, float* inv) {
    const uint32_t t = threadIdx.x;
    if (t < kTreeParts) part[t] = s;
    __syncthreads();
    if (t < kTreeParts / 2) part[t] = s + part[t + kTreeParts / 2];
    __syncthreads();
    if (t < 64) {
        float v = part[t] + part[t + 64];
#pragma unroll
        for (int k = 32; k > 0; k >>= 1) v += __shfl_down(v, k, 64);
        if (t == 0) *inv = rms_inv(v, (float)dim, eps);
    }
    __syncthreads();
    return *inv;
}

// The q/k arithmetic of a prefill step, shared by every kernel that produces the
// cache rows and the attention q operand (the pre-pass, the attention kernel and
// the projection GEMM's epilogue), each operation rounded on its own so they
// agree bit for bit:
//   k rows, the reference's operations (the cache is compared row for row):
//   qk_serial_sumsq: sum of squares in element order (kernels_a.zig:85-86)
//   qk_norm_mul:     (v * inv) * w                  (kernels_a.zig:89)
//   qk_rope_angle:   (pos * freq_scale) * inv_freq   (kernels_a.zig:120)
//   qk_rotate:       x0 c - x1 s, x0 s + x1 c        (kernels_a.zig:125-126)
//   the q operand, which only feeds attention as an f16 value (its f32 rounding
//   steps are far below the final f16 rounding), in fewer operations:
//   qk_quarter_sumsq: the squares of 4 rope pairs (i, i + D/2), accumulated
//                    x0[0]^2, x1[0]^2, x0[1]^2, ... with fma; a head's D/8
//                    quarters (pairs 4j .. 4j + 3) then add in a balanced tree
//                    in index order ((p0 + p1) + (p2 + p3)) + ...
//   qk_q_pair:       u0 = x0 w0, u1 = x1 w1 (the norm weights), y0 = u0 c - u1 s,
//                    y1 = u1 c + u0 s (each one fma over a rounded product),
//                    then f16 of y r, r = inv * q_scale: the norm, the rotation
//                    and the softmax scale * log2(e) in 8 operations per pair
//   qk_scaled_f16:   f16 of the f32 product y * s, rounded twice (to f32, then
//                    to f16). The backend turns a product that is converted
//                    to f16 into one mixed-precision fma (v_fma_mixlo_f16, a
//                    single rounding) in some kernels and not in others, even
//                    with contraction off; an empty asm that takes the product
//                    as a register value keeps the two roundings everywhere
DS5_DEVICE_INLINE float qk_serial_sumsq(const float* row, int dim) {
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

DS5_DEVICE_INLINE float qk_norm_mul(float v, float inv, float w) {
#pragma clang fp contract(off)
    return v * inv * w;
}

DS5_DEVICE_INLINE float qk_rope_angle(float pos, float freq_scale, float inv) {
#pragma clang fp contract(off)
    return pos * freq_scale * inv;
}

DS5_DEVICE_INLINE void qk_rotate(float x0, float x1, float c, float s, float& y0, float& y1) {
#pragma clang fp contract(off)
    y0 = x0 * c - x1 * s;
    y1 = x0 * s + x1 * c;
}

DS5_DEVICE_INLINE _Float16 qk_scaled_f16(float y, float s) {
#pragma clang fp contract(off)
    float p = y * s;
    asm volatile("" : "+v"(p));
    return (_Float16)p;
}

DS5_DEVICE_INLINE float qk_quarter_sumsq(float a0, float b0, float a1, float b1, float a2, float b2, float a3,
                                         float b3) {
#pragma clang fp contract(off)
    float p = a0 * a0;
    p = __builtin_fmaf(b0, b0, p);
    p = __builtin_fmaf(a1, a1, p);
    p = __builtin_fmaf(b1, b1, p);
    p = __builtin_fmaf(a2, a2, p);
    p = __builtin_fmaf(b2, b2, p);
    p = __builtin_fmaf(a3, a3, p);
    return __builtin_fmaf(b3, b3, p);
}

DS5_DEVICE_INLINE void qk_q_pair(float x0, float x1, float w0, float w1, float c, float s, float r, _Float16& o0,
                                 _Float16& o1) {
#pragma clang fp contract(off)
    const float u0 = x0 * w0, u1 = x1 * w1;
    const float y0 = __builtin_fmaf(u0, c, -(u1 * s));
    const float y1 = __builtin_fmaf(u1, c, u0 * s);
    o0 = qk_scaled_f16(y0, r);
    o1 = qk_scaled_f16(y1, r);
}
