/*
 * ds5_oracle.h -- CPU restatement of DS5's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP backend:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it. Nothing in the qw3_amd product links or calls it.
 *
 * Each function restates one function of the reference's CPU backend, in the
 * same loop order and with the same f32 operation order (compiled with
 * -ffp-contract=off, so a*b+c is never fused, like Zig's strict float mode):
 *
 *   ds5o_rms_norm       src/kernels/cpu/kernels_a.zig:68-91
 *   ds5o_rms_norm_tree  src/kernels/shaders/kernels_a.metal:127-165 (the
 *                       reference GPU kernel's reduction order, 256 fma
 *                       partials and a halving tree)
 *   ds5o_rope           src/kernels/cpu/kernels_a.zig:97-130
 *   ds5o_kv_append      src/kernels/cpu/kernels_a.zig:169-217
 *   ds5o_gqa_attention  src/kernels/cpu/kernels_b.zig:29-133
 *   ds5o_matmul         src/kernels/cpu/kernels_a.zig:136-163 (row dot :39-62)
 *   ds5o_add            src/kernels/cpu/kernels_a.zig:223-233
 *   ds5o_router_topk    src/kernels/cpu/kernels_c.zig:80-155
 *   ds5o_expert_mlp_swiglu  src/kernels/cpu/kernels_c.zig:157-214
 *
 * Argument structs mirror src/shared/contracts.zig:210-286 (Buf and the
 * RmsNorm/Rope/KvAppend/Attn args); buffer views honour offset and len as
 * src/kernels/cpu/ctx.zig:70-108 does, and the same ShapeMismatch /
 * UnsupportedDtype checks run before any arithmetic.
 *
 * The paged-KV functions have no reference code (the reference has no paged
 * cache); they are defined by reduction to the contiguous functions above.
 */
#ifndef DS5_ORACLE_H
#define DS5_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* contracts.zig:201-206 KernelError, as status codes. */
enum {
    DS5O_OK = 0,
    DS5O_SHAPE_MISMATCH = 1,
    DS5O_UNSUPPORTED_DTYPE = 2,
    DS5O_DEVICE_FAILURE = 3,
    DS5O_OUT_OF_MEMORY = 4,
};

/* contracts.zig:22-29 Dtype ids (GGML type ids). Q8_0 blocks: 32 elements in 34
 * bytes, an f16 scale then 32 int8 (contracts.zig:57,74); value = f32(scale) * q. */
enum { DS5O_F32 = 0, DS5O_F16 = 1, DS5O_Q8_0 = 8 };

/* contracts.zig:210-214 Buf: handle is a host pointer for this oracle. */
typedef struct ds5o_buf {
    void* handle;
    uint64_t offset;
    uint64_t len;
} ds5o_buf;

typedef struct ds5o_matmul_args { /* contracts.zig:242-250 MatmulArgs */
    ds5o_buf x;       /* f32 [m, k] */
    ds5o_buf w;       /* w_dtype: n rows of k elements (GGUF layout, ne = {k, n}) */
    uint32_t w_dtype; /* DS5O_F32 or DS5O_Q8_0 */
    ds5o_buf out;     /* f32 [m, n] */
    uint32_t m, n, k;
} ds5o_matmul_args;

typedef struct ds5o_rms_norm_args { /* contracts.zig:218-225 */
    ds5o_buf x, weight, out;
    uint32_t n_rows, dim;
    float eps;
} ds5o_rms_norm_args;

typedef struct ds5o_rope_args { /* contracts.zig:230-238 */
    ds5o_buf x, positions;
    uint32_t n_tokens, n_heads, head_dim;
    float theta, freq_scale;
} ds5o_rope_args;

typedef struct ds5o_kv_append_args { /* contracts.zig:256-267 */
    ds5o_buf k_new, v_new, k_cache, v_cache;
    uint32_t kv_dtype, pos, n_tokens, n_kv_heads, head_dim, max_ctx;
} ds5o_kv_append_args;

typedef struct ds5o_attn_args { /* contracts.zig:272-286 */
    ds5o_buf q, k_cache, v_cache;
    uint32_t kv_dtype;
    ds5o_buf out;
    uint32_t pos, n_tokens, n_q_heads, n_kv_heads, head_dim, max_ctx;
    float scale;
} ds5o_attn_args;

int ds5o_matmul(const ds5o_matmul_args* a);

typedef struct ds5o_add_args { /* contracts.zig:334-339 AddArgs */
    ds5o_buf x, y, out;        /* f32 [n_elems] each; out may alias x */
    uint64_t n_elems;
} ds5o_add_args;
int ds5o_add(const ds5o_add_args* a);

typedef struct ds5o_router_args { /* contracts.zig:293-304 RouterArgs */
    ds5o_buf x;                   /* f32 [n_tokens, dim] */
    ds5o_buf w;                   /* w_dtype (f32, f16, q8_0): n_experts rows of dim */
    uint32_t w_dtype;
    uint32_t n_tokens, dim, n_experts, top_k;
    uint32_t norm_topk_prob;      /* bool */
    uint16_t* out_ids;            /* host [n_tokens * top_k] */
    uint64_t out_ids_len;
    float* out_weights;           /* host [n_tokens * top_k] */
    uint64_t out_weights_len;
} ds5o_router_args;
int ds5o_router_topk(const ds5o_router_args* a);

typedef struct ds5o_pair { /* contracts.zig:308-312 PairDispatch (extern struct) */
    uint32_t token;
    uint32_t expert;
    float weight;
} ds5o_pair;

typedef struct ds5o_expert_mlp_args { /* contracts.zig:319-331 ExpertMlpArgs */
    ds5o_buf x;                       /* f32 [n_tokens, dim] */
    ds5o_buf gate, up, down;          /* expert banks: gate/up n_experts x ffn rows of dim, down x dim rows of ffn */
    uint32_t w_dtype;                 /* f32 or q8_0 */
    const ds5o_pair* pairs;           /* host */
    uint64_t n_pairs;
    ds5o_buf out;                     /* f32 [n_tokens, dim], accumulated into */
    uint32_t n_tokens, dim, ffn_dim, n_experts;
} ds5o_expert_mlp_args;
int ds5o_expert_mlp_swiglu(const ds5o_expert_mlp_args* a);
int ds5o_rms_norm(const ds5o_rms_norm_args* a);
int ds5o_rms_norm_tree(const ds5o_rms_norm_args* a);
int ds5o_rope(const ds5o_rope_args* a);
int ds5o_kv_append(const ds5o_kv_append_args* a);
int ds5o_gqa_attention(const ds5o_attn_args* a);

/* std.math.pow(f32, x, y) as Zig's standard library computes it (see the
 * definition for the algorithm); exported so tests can pin it. */
float ds5o_zig_powf(float x, float y);

/* f32 -> f16 bits, IEEE-754 round-to-nearest-even (Zig's @floatCast), and the
 * exact widening f16 -> f32. */
uint16_t ds5o_f32_to_f16(float x);
float ds5o_f16_to_f32(uint16_t h);
void ds5o_f32_to_f16_array(const float* x, uint16_t* out, uint64_t n);
void ds5o_f16_to_f32_array(const uint16_t* h, float* out, uint64_t n);

/* Paged KV (no reference counterpart). Pool layout is the frozen cache layout
 * [n_kv_heads, n_pages * page_size, head_dim] with slots grouped into pages of
 * page_size consecutive slots. Sequence position p lives in slot
 *     page_table[p / page_size] * page_size + p % page_size.             */
int64_t ds5o_paged_slot(const int32_t* page_table, uint32_t n_table, uint32_t page_size, uint32_t p);

/* Copy positions 0..len-1 of one sequence from a paged f16 pool into a
 * contiguous f16 cache [n_kv_heads, len, head_dim]. Returns a status code. */
int ds5o_paged_gather_f16(const uint16_t* pool, uint64_t pool_slots, const int32_t* page_table,
                          uint32_t n_table, uint32_t page_size, uint32_t len, uint32_t n_kv_heads,
                          uint32_t head_dim, uint16_t* out);

/* Post-norm, post-rope f32 per-head pipeline of one engine step on the
 * contiguous cache, in the engine's op order (src/engine/forward.zig:345-412):
 * q_norm, k_norm, rope q, rope k, kvAppend, gqaAttention. q, k, v are
 * modified in place like the engine's scratch buffers. */
typedef struct ds5o_step_args {
    ds5o_buf q, k, v, q_norm_w, k_norm_w, positions, k_cache, v_cache, out;
    uint32_t kv_dtype, pos, n_tokens, n_q_heads, n_kv_heads, head_dim, max_ctx;
    float eps, theta, freq_scale, scale;
} ds5o_step_args;
int ds5o_attention_step(const ds5o_step_args* a);

#ifdef __cplusplus
}
#endif
#endif
