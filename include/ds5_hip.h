/*
 * ds5_hip.h -- C ABI of the MI355X (gfx950) backend for DS5's attention path.
 *
 * libds5hip.so is a third kernel backend beside DS5's `cpu` and `metal`
 * providers. The Zig host binds it with @cImport of this header; every entry
 * point takes plain pointers, sizes and the structs below, never a torch
 * type.
 *
 * Two groups of entry points:
 *   1. the device context, one per engine, replacing the frozen GPU API
 *      contracts.assertGpuApi (src/shared/contracts.zig:374-384) that
 *      src/kernels/cpu/ctx.zig and src/metal/metal.zig implement;
 *   2. the kernel-provider ops of the attention path, replacing
 *      rmsNorm / rope / kvAppend / gqaAttention of contracts.assertKernelApi
 *      (src/shared/contracts.zig:358-367), plus the matmul of the projections
 *      on either side of it, and fused and paged extensions that the engine
 *      may pick up with @hasDecl.
 *
 * Status codes are contracts.KernelError (src/shared/contracts.zig:201-206):
 * every precondition the reference checks is checked here before any launch.
 * All ops enqueue on the context's single HIP stream and return without
 * waiting; ds5_hip_download and ds5_hip_submit synchronise.
 */
#ifndef DS5_HIP_H
#define DS5_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: contracts.zig:201-206 KernelError ------------------- */
#define DS5_OK 0
#define DS5_SHAPE_MISMATCH 1    /* KernelError.ShapeMismatch */
#define DS5_UNSUPPORTED_DTYPE 2 /* KernelError.UnsupportedDtype */
#define DS5_DEVICE_FAILURE 3    /* KernelError.DeviceFailure: any HIP error */
#define DS5_OUT_OF_MEMORY 4     /* KernelError.OutOfMemory */

/* ---- dtypes: contracts.zig:22-29 (GGML type ids) ------------------------ */
#define DS5_DTYPE_F32 0u
#define DS5_DTYPE_F16 1u
#define DS5_DTYPE_Q8_0 8u /* 32-element blocks of 34 bytes: f16 scale, 32 x int8 (contracts.zig:57,74) */

/* contracts.zig:210-214 `Buf = extern struct { handle, offset, len }`, 24 B.
 * handle = base of a device allocation owned by the context; offset and len
 * are bytes and every op honours them (ctx.zig:70-108 semantics). */
typedef struct ds5_buf {
    void* handle;
    uint64_t offset;
    uint64_t len;
} ds5_buf;

typedef struct ds5_hip_ctx ds5_hip_ctx;

/* ========================================================================
 * 1. Device context (contracts.zig:374-384 assertGpuApi)
 * ======================================================================== */

/* Ctx.init (metal.zig:131, ctx.zig:20): picks device `device_index`
 * (0 for the first visible GPU) and creates the context's stream and
 * timing events. */
int ds5_hip_init(int device_index, ds5_hip_ctx** out);

/* Ctx.deinit (ctx.zig:26-30): waits for the stream, frees every buffer the
 * context created, destroys the stream. */
void ds5_hip_deinit(ds5_hip_ctx* ctx);

/* Ctx.createBuffer (ctx.zig:32-38, metal.zig:239-250): zero-filled device
 * allocation of len bytes, owned by the context. */
int ds5_hip_create_buffer(ds5_hip_ctx* ctx, uint64_t len, ds5_buf* out);

/* Ctx.bufferFromBytes (metal.zig:280-306): HIP has no zero-copy wrap of
 * pageable host memory into device storage, so this allocates a context-owned
 * device buffer and copies the bytes; the caller keeps ownership of `bytes`. */
int ds5_hip_buffer_from_bytes(ds5_hip_ctx* ctx, const void* bytes, uint64_t len, ds5_buf* out);

/* Ctx.upload / Ctx.download (ctx.zig:47-55, metal.zig:309-336): byte copies
 * at `offset` within the view. Both return after the copy is complete;
 * download first drains everything already enqueued (the Metal glue's
 * auto-flush, metal.zig:326-329). */
int ds5_hip_upload(ds5_hip_ctx* ctx, ds5_buf buf, uint64_t offset, const void* bytes, uint64_t len);
int ds5_hip_download(ds5_hip_ctx* ctx, ds5_buf buf, uint64_t offset, void* out, uint64_t len);

/* Ctx.begin / Ctx.submit / Ctx.gpuElapsedNs (metal.zig:360-393): begin records
 * a start event on the stream; submit records an end event and blocks until
 * the stream is idle; gpu_elapsed_ns is the device time between the last
 * begin/submit pair (0 if no batch completed). */
void ds5_hip_begin(ds5_hip_ctx* ctx);
int ds5_hip_submit(ds5_hip_ctx* ctx);
uint64_t ds5_hip_gpu_elapsed_ns(ds5_hip_ctx* ctx);

/* Text of the most recent failure on this context (empty if none). */
const char* ds5_hip_last_error(ds5_hip_ctx* ctx);

/* The context's HIP stream (a hipStream_t), for hosts that interleave their
 * own device work with these ops. */
void* ds5_hip_stream(ds5_hip_ctx* ctx);

/* Per-kernel device timing (no reference counterpart; the reference times
 * whole command buffers, metal.zig:369-389). When enabled, every kernel
 * launch of this context is bracketed by events on its stream; submit and
 * ds5_hip_kernel_time resolve them. Enabling (or disabling) clears the
 * totals. kernel_time reports the launches and summed device nanoseconds of
 * the kernel named `kernel` (e.g. "decode_splitk_kernel"). */
int ds5_hip_set_kernel_timing(ds5_hip_ctx* ctx, int enable);
int ds5_hip_kernel_time(ds5_hip_ctx* ctx, const char* kernel, uint64_t* launches, double* total_ns);

/* Device-time marks for per-layer timing of a forward pass: the reference's
 * beginTiming / layerNs / endTiming (src/kernels/gpu/kernels.zig:442-472),
 * written to run metadata as gpu_ns_per_layer_boundary (src/main.zig:420-444).
 * timing_begin forgets earlier marks; timing_mark records an event on the
 * context stream (enqueued work before it is timed, nothing synchronises;
 * ShapeMismatch while the stream is capturing); timing_read synchronises and
 * writes the device nanoseconds between consecutive marks -- count = marks - 1
 * values, at most max of them. The engine marks before its first layer and
 * after every layer, so value i is layer i's device time (the reference's
 * boundary batch also spans the previous layer's post-router work, because its
 * router syncs the host mid-layer; here nothing does). */
int ds5_hip_timing_begin(ds5_hip_ctx* ctx);
int ds5_hip_timing_mark(ds5_hip_ctx* ctx);
int ds5_hip_timing_read(ds5_hip_ctx* ctx, uint64_t* ns, uint32_t max, uint32_t* count);

/* Stream capture into a replayable HIP graph (no reference counterpart; the
 * Metal glue batches a layer's dispatches into one command buffer,
 * kernels/gpu/kernels.zig:112-119). Ops called between capture_begin and
 * capture_end are recorded, not run; capture_end returns an executable graph
 * (a hipGraphExec_t) that graph_launch replays on the context stream with the
 * argument values of the capture. Ops that would allocate (a first split-K
 * decode at a new size grows the workspace) must run once before capture. */
int ds5_hip_capture_begin(ds5_hip_ctx* ctx);
int ds5_hip_capture_end(ds5_hip_ctx* ctx, void** graph_exec);
int ds5_hip_graph_launch(ds5_hip_ctx* ctx, void* graph_exec);
void ds5_hip_graph_destroy(void* graph_exec);

/* ========================================================================
 * 2. Kernel-provider ops (contracts.zig:358-367 assertKernelApi)
 * ======================================================================== */

/* contracts.zig:218-225 RmsNormArgs. y = x * (1/sqrt(mean(x^2) + eps)) * w
 * rowwise; `out` may alias `x`. Replaces kernels_a.zig:68-91 rmsNorm and the
 * Metal rmsnorm_f32 dispatch (kernels/gpu/kernels.zig:146-157). Rows of up to
 * 256 elements sum their squares in the CPU path's serial order; longer rows in
 * the Metal kernel's order (kernels/shaders/kernels_a.metal:127-165: 256
 * strided fma partials, then a halving tree). */
typedef struct ds5_rms_norm_args {
    ds5_buf x;      /* f32 [n_rows, dim] */
    ds5_buf weight; /* f32 [dim] */
    ds5_buf out;    /* f32 [n_rows, dim] */
    uint32_t n_rows;
    uint32_t dim;
    float eps;
} ds5_rms_norm_args;
int ds5_hip_rms_norm(ds5_hip_ctx* ctx, const ds5_rms_norm_args* args);

/* contracts.zig:230-238 RopeArgs. In-place NeoX rotation, element i pairs
 * with i + head_dim/2, angle = pos * freq_scale * theta^(-2i/head_dim).
 * Replaces kernels_a.zig:97-130 rope (Metal: kernels/gpu/kernels.zig:163-180).
 * head_dim must be even and at most 512. */
typedef struct ds5_rope_args {
    ds5_buf x;         /* f32 [n_tokens, n_heads, head_dim], rotated in place */
    ds5_buf positions; /* i32 [n_tokens] absolute positions */
    uint32_t n_tokens;
    uint32_t n_heads;
    uint32_t head_dim;
    float theta;
    float freq_scale; /* 1.0 in the reference engine */
} ds5_rope_args;
int ds5_hip_rope(ds5_hip_ctx* ctx, const ds5_rope_args* args);

/* contracts.zig:256-267 KvAppendArgs. Scatter [n_tokens, n_kv_heads,
 * head_dim] f32 into the frozen cache layout [n_kv_heads, max_ctx, head_dim]
 * at positions pos..pos+n_tokens-1; an f16 cache stores the IEEE
 * round-to-nearest-even cast. Replaces kernels_a.zig:169-217 kvAppend
 * (Metal: kernels/gpu/kernels.zig:210-235). */
typedef struct ds5_kv_append_args {
    ds5_buf k_new;   /* f32 [n_tokens, n_kv_heads, head_dim] */
    ds5_buf v_new;   /* f32 [n_tokens, n_kv_heads, head_dim] */
    ds5_buf k_cache; /* kv_dtype [n_kv_heads, max_ctx, head_dim] */
    ds5_buf v_cache; /* kv_dtype [n_kv_heads, max_ctx, head_dim] */
    uint32_t kv_dtype;
    uint32_t pos;
    uint32_t n_tokens;
    uint32_t n_kv_heads;
    uint32_t head_dim;
    uint32_t max_ctx;
} ds5_kv_append_args;
int ds5_hip_kv_append(ds5_hip_ctx* ctx, const ds5_kv_append_args* args);

/* contracts.zig:272-286 AttnArgs. Causal GQA attention: query token t sits at
 * pos + t and attends cache positions 0..pos+t; q head h reads kv head
 * h / (n_q_heads / n_kv_heads); softmax in f32. max_ctx is the cache STRIDE,
 * not the valid length. Replaces kernels_b.zig:29-133 gqaAttention (Metal:
 * kernels/gpu/kernels.zig:254-286). n_tokens == 1 runs the split-K
 * flash-decoding kernels, n_tokens > 1 the causal MFMA prefill kernel
 * (f16 cache, head_dim 64 or 128); other shapes and f32 caches run a generic
 * streaming kernel. All paths are device code. */
typedef struct ds5_attn_args {
    ds5_buf q;       /* f32 [n_tokens, n_q_heads, head_dim], post-norm post-rope */
    ds5_buf k_cache; /* kv_dtype [n_kv_heads, max_ctx, head_dim] */
    ds5_buf v_cache; /* kv_dtype [n_kv_heads, max_ctx, head_dim] */
    uint32_t kv_dtype;
    ds5_buf out;     /* f32 [n_tokens, n_q_heads * head_dim] */
    uint32_t pos;
    uint32_t n_tokens;
    uint32_t n_q_heads;
    uint32_t n_kv_heads;
    uint32_t head_dim;
    uint32_t max_ctx;
    float scale; /* 1/sqrt(head_dim) in the engine (forward.zig:308) */
} ds5_attn_args;
int ds5_hip_gqa_attention(ds5_hip_ctx* ctx, const ds5_attn_args* args);

/* contracts.zig:242-250 MatmulArgs. out[m, n] = x[m, k] . W^T with W a
 * GGUF-layout weight, n rows of k elements (ne = {k, n}): f32, or Q8_0 blocks
 * (value = f32(f16 scale) * int8 q, contracts.zig:194). Replaces
 * kernels_a.zig:136-163 matmul -- the q/k/v projections feeding the attention
 * step (forward.zig:337-339) and the output projection after it (:416-418).
 * Weight dtypes other than f32 / Q8_0 are UnsupportedDtype; k must be a
 * positive multiple of the dtype's block (32 for Q8_0). Each output is the
 * same dot product as the reference's serial one, summed as a fixed tree of
 * per-block partial sums, so it agrees to rounding (the serial kernel, used for
 * views the fast kernels cannot read, keeps the reference's order and is
 * bit-identical). From 16 tokens a Q8_0 product uses 4*m*k bytes of the
 * context workspace: run a shape once before capturing it in a graph. */
typedef struct ds5_matmul_args {
    ds5_buf x;        /* f32 [m, k] */
    ds5_buf w;        /* w_dtype: n rows of k elements */
    uint32_t w_dtype; /* DS5_DTYPE_F32 or DS5_DTYPE_Q8_0 */
    ds5_buf out;      /* f32 [m, n] */
    uint32_t m;
    uint32_t n;
    uint32_t k;
} ds5_matmul_args;
int ds5_hip_matmul(ds5_hip_ctx* ctx, const ds5_matmul_args* args);

/* contracts.zig:334-339 AddArgs. out = x + y over n_elems f32 (replaces
 * kernels_a.zig:223-233 add: the residual adds, forward.zig:418 after the
 * attention block). x, y, then out too small are ShapeMismatch, in that order;
 * out may be the same view as x or y. Bit-identical to the reference. */
typedef struct ds5_add_args {
    ds5_buf x;
    ds5_buf y;
    ds5_buf out;
    uint64_t n_elems;
} ds5_add_args;
int ds5_hip_add(ds5_hip_ctx* ctx, const ds5_add_args* args);

/* contracts.zig:293-304 RouterArgs; replaces kernels_c.zig:80-155 routerTopK.
 * logits = x . W^T, softmax over all n_experts, the top_k largest descending
 * (ties: the lower id), divided by their sum iff norm_topk_prob. The outputs
 * are HOST arrays, as in the reference: the call waits for the device and
 * copies them back. Checks in the reference's order: w_dtype (f32, f16, q8_0)
 * else UnsupportedDtype; top_k in 1..n_experts; dim a positive multiple of the
 * dtype's block; both output lengths == n_tokens * top_k; x; w -- each else
 * ShapeMismatch. Also ShapeMismatch here: a router row above 64 KiB, 4*dim plus a
 * row above 128 KiB, or n_experts above 16384 (LDS). Logits are the reference's serial
 * dot, bit for bit; exp is the device's, so weights agree within an ulp or so
 * and ids agree unless two probabilities do as well. */
typedef struct ds5_router_args {
    ds5_buf x;                 /* f32 [n_tokens, dim] */
    ds5_buf w;                 /* w_dtype: n_experts rows of dim */
    uint32_t w_dtype;
    uint32_t n_tokens;
    uint32_t dim;
    uint32_t n_experts;
    uint32_t top_k;
    uint32_t norm_topk_prob;   /* bool */
    uint16_t* out_ids;         /* host [n_tokens * top_k] */
    uint64_t out_ids_len;
    float* out_weights;        /* host [n_tokens * top_k] */
    uint64_t out_weights_len;
} ds5_router_args;
int ds5_hip_router_topk(ds5_hip_ctx* ctx, const ds5_router_args* args);

/* contracts.zig:308-312 PairDispatch (extern struct): one (token, expert) to run. */
typedef struct ds5_pair {
    uint32_t token;
    uint32_t expert;
    float weight;
} ds5_pair;

/* contracts.zig:319-331 ExpertMlpArgs; replaces kernels_c.zig:157-214
 * expertMlpSwiglu: per pair, out[token] += weight * down(silu(gate . x) *
 * (up . x)), in list order per token; out is accumulated into (the caller
 * zeroes it). Banks are GGUF 3-D tensors: expert e of gate/up at
 * e * ffn_dim * rowBytes(dim), of down at e * dim * rowBytes(ffn_dim). pairs is
 * a HOST array (uploaded by the call). Checks in the reference's order: w_dtype
 * (f32, q8_0); dim and ffn_dim positive multiples of the block; x, out, gate,
 * up, down sizes; then every pair's token and expert in range -- all before
 * anything runs (the reference adds the pairs before a bad one; here out is left
 * untouched). Dots agree with the reference's serial ones to rounding (the
 * serial kernels, for views the wavefront kernels cannot read, are exact). */
typedef struct ds5_expert_mlp_args {
    ds5_buf x;               /* f32 [n_tokens, dim] */
    ds5_buf gate;            /* w_dtype [n_experts, ffn_dim, dim] */
    ds5_buf up;              /* w_dtype [n_experts, ffn_dim, dim] */
    ds5_buf down;            /* w_dtype [n_experts, dim, ffn_dim] */
    uint32_t w_dtype;
    const ds5_pair* pairs;   /* host */
    uint64_t n_pairs;
    ds5_buf out;             /* f32 [n_tokens, dim] */
    uint32_t n_tokens;
    uint32_t dim;
    uint32_t ffn_dim;
    uint32_t n_experts;
} ds5_expert_mlp_args;
int ds5_hip_expert_mlp_swiglu(ds5_hip_ctx* ctx, const ds5_expert_mlp_args* args);

/* ========================================================================
 * 3. Fused extensions (optional decls; the engine uses them via @hasDecl)
 * ======================================================================== */

/* The MoE block of one layer without a host round trip (no reference
 * counterpart; the reference routes on the host and builds the pairs there):
 * routerTopK on the device, its token-major pairs (token t's experts in pick
 * order) kept in device memory, and expertMlpSwiglu over them, accumulating
 * into out. Equal to ds5_hip_router_topk then ds5_hip_expert_mlp_swiglu on
 * those pairs. Checked as the two calls are (router first); ids / weights,
 * when given (len >= 2 * and 4 * n_tokens * top_k), receive the router's
 * outputs on the device. residual, when given (len >= 4 * n_tokens * dim):
 * out = residual + the experts' sum, the sum started from zero -- the
 * engine's zeroed accumulator, the experts into it and add(x, proj -> x) of
 * forward.zig:445-468, bit for bit, without the accumulator, its clear and the
 * add launch; out may be residual. */
typedef struct ds5_moe_args {
    ds5_buf x;                 /* f32 [n_tokens, dim] */
    ds5_buf router_w;          /* router_dtype: n_experts rows of dim */
    uint32_t router_dtype;     /* f32, f16 or q8_0 */
    ds5_buf gate;
    ds5_buf up;
    ds5_buf down;
    uint32_t w_dtype;          /* f32 or q8_0 */
    ds5_buf out;               /* f32 [n_tokens, dim], accumulated into */
    ds5_buf ids;               /* optional u16 [n_tokens, top_k] */
    ds5_buf weights;           /* optional f32 [n_tokens, top_k] */
    uint32_t n_tokens;
    uint32_t dim;
    uint32_t ffn_dim;
    uint32_t n_experts;
    uint32_t top_k;
    uint32_t norm_topk_prob;
    ds5_buf residual;          /* optional f32 [n_tokens, dim] */
    ds5_buf x_norm;            /* optional f32 [dim]: ds5_hip_rms_norm(x, x_norm, x_norm_eps)
                                * first (forward.zig:420-428's ffn_norm), bit for bit, inside
                                * the router's logits kernel (f32 router, rows of more than
                                * 256 elements) or else into a context buffer; its checks
                                * come first; x itself is left as it is (it may be residual) */
    float x_norm_eps;
} ds5_moe_args;
int ds5_hip_moe(ds5_hip_ctx* ctx, const ds5_moe_args* args);

/* The output projection and residual of forward.zig:416-418 as one call:
 * out = residual + x . W^T, bit-identical to ds5_hip_matmul(x, w -> proj)
 * then ds5_hip_add(residual, proj -> out) for the same views, without the
 * proj buffer or the add launch. Checked as matmul (dtype, k, x, out, w),
 * then residual too small; residual and out must be 4-byte aligned views
 * (ShapeMismatch otherwise). out may be the same view as residual (the
 * engine's x = x + proj); it must not overlap x or w otherwise. */
typedef struct ds5_matmul_add_args {
    ds5_buf x;        /* f32 [m, k] */
    ds5_buf w;        /* w_dtype: n rows of k elements */
    uint32_t w_dtype; /* DS5_DTYPE_F32 or DS5_DTYPE_Q8_0 */
    ds5_buf residual; /* f32 [m, n] */
    ds5_buf out;      /* f32 [m, n] */
    uint32_t m;
    uint32_t n;
    uint32_t k;
} ds5_matmul_add_args;
int ds5_hip_matmul_add(ds5_hip_ctx* ctx, const ds5_matmul_add_args* args);

/* The engine's q, k and v projections (forward.zig:337-339: three matmul calls
 * on the same x) as one call: entry e is exactly ds5_hip_matmul(x, w[e],
 * w_dtype, out[e], m, n[e], k), same results bit for bit. All entries are
 * checked (in order, each as matmul checks) before anything is enqueued. When
 * every entry takes the same kernel the group is one launch per pass of tokens
 * (from 16 Q8_0 tokens: one split of x, then one launch). count is
 * 1..DS5_MATMUL_GROUP_MAX, else ShapeMismatch. */
#define DS5_MATMUL_GROUP_MAX 4u
typedef struct ds5_matmul_group_args {
    ds5_buf x;        /* f32 [m, k], shared */
    uint32_t w_dtype; /* DS5_DTYPE_F32 or DS5_DTYPE_Q8_0, shared */
    uint32_t m;
    uint32_t k;
    uint32_t count;
    ds5_buf w[DS5_MATMUL_GROUP_MAX];   /* entry e: n[e] rows of k elements */
    ds5_buf out[DS5_MATMUL_GROUP_MAX]; /* entry e: f32 [m, n[e]] */
    uint32_t n[DS5_MATMUL_GROUP_MAX];
} ds5_matmul_group_args;
int ds5_hip_matmul_group(ds5_hip_ctx* ctx, const ds5_matmul_group_args* args);

/* One layer's attention block in the engine's op order
 * (src/engine/forward.zig:345-412): per-head RMSNorm of q and k with
 * q_norm / k_norm, NeoX rope of q and k, append of k and v into the cache,
 * then causal GQA attention -- with the same cache rows and attention output
 * as the six separate ops. q and k are scratch: their contents after the call
 * are unspecified (the fused kernels leave them as they were; other shapes run
 * the separate ops in place). Decode (n_tokens == 1, f16 cache, head_dim
 * 64/128) is ONE kernel launch plus, for long contexts, a split-K merge
 * launch; prefill is a k/v append launch plus one attention launch that
 * normalises and rotates q itself. The engine's per-op trace points
 * (forward.zig:361-380) are not produced on this path. */
typedef struct ds5_attention_step_args {
    ds5_buf q;         /* f32 [n_tokens, n_q_heads, head_dim] q projection (in/out) */
    ds5_buf k;         /* f32 [n_tokens, n_kv_heads, head_dim] k projection (in/out) */
    ds5_buf v;         /* f32 [n_tokens, n_kv_heads, head_dim] v projection */
    ds5_buf q_norm;    /* f32 [head_dim] */
    ds5_buf k_norm;    /* f32 [head_dim] */
    ds5_buf positions; /* i32 [n_tokens]; the engine passes pos..pos+n_tokens-1 */
    ds5_buf k_cache;   /* kv_dtype [n_kv_heads, max_ctx, head_dim] */
    ds5_buf v_cache;
    ds5_buf out;       /* f32 [n_tokens, n_q_heads * head_dim] */
    uint32_t kv_dtype;
    uint32_t pos;
    uint32_t n_tokens;
    uint32_t n_q_heads;
    uint32_t n_kv_heads;
    uint32_t head_dim;
    uint32_t max_ctx;
    float eps;
    float theta;
    float freq_scale;
    float scale;
} ds5_attention_step_args;
int ds5_hip_attention_step(ds5_hip_ctx* ctx, const ds5_attention_step_args* args);

/* The attention block of a layer, forward.zig:337-412 as one call (no
 * reference counterpart: the reference makes nine provider calls): the q/k/v
 * projections of x (K.matmul by wq, wk, wv; kernels_a.zig:136-163), then the
 * attention step. The results -- cache rows and attention output -- are those
 * of ds5_hip_matmul_group(x; wq, wk, wv -> step.q, step.k, step.v) followed by
 * ds5_hip_attention_step(&step), bit for bit, and the preconditions are
 * theirs, in that order. For a prefill whose Q8_0 projections take the
 * matrix-core GEMM path (n_tokens >= 16, or hidden above 8192), with an f16
 * cache and head_dim 128, the step's pre-pass runs in
 * the projection GEMM's epilogue -- per-head RMSNorm, rope, f16 k/v append
 * and the f16 q operand -- so q, k and v are never written in f32 and no
 * pre-pass launches; every other case runs the two calls. step.q / step.k /
 * step.v are scratch. */
typedef struct ds5_attention_block_args {
    ds5_buf x;         /* f32 [n_tokens, hidden]: the attn_norm output (or its input, with x_norm) */
    ds5_buf wq;        /* [n_q_heads * head_dim rows of hidden] in w_dtype */
    ds5_buf wk;        /* [n_kv_heads * head_dim rows of hidden] */
    ds5_buf wv;        /* [n_kv_heads * head_dim rows of hidden] */
    uint32_t w_dtype;  /* DS5_DTYPE_F32 or DS5_DTYPE_Q8_0 */
    uint32_t hidden;
    ds5_attention_step_args step; /* q/k/v scratch, norms, positions, caches, out, shapes */
    ds5_buf x_norm;    /* optional f32 [hidden]: the block first applies
                        * ds5_hip_rms_norm(x, x_norm, x_norm_eps) (forward.zig:325-334's
                        * attn_norm), bit for bit, inside the projection kernels where
                        * they read x (rows of more than 256 elements), else into a
                        * context buffer; its checks come first */
    float x_norm_eps;
} ds5_attention_block_args;
int ds5_hip_attention_block(ds5_hip_ctx* ctx, const ds5_attention_block_args* args);

/* No reference counterpart. For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): ds5_hip_attention_step with the same kernels, arguments,
 * preconditions and results, but the split-K partials (decode) or the f16 q
 * operand (prefill) live in the library's static device scratch array of
 * DS5_NOALLOC_SCRATCH_BYTES per GPU instead of the context's workspace, and
 * the call allocates nothing. A call that would need more scratch than that
 * (e.g. a long prefill) fails with ShapeMismatch before any device work.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (other contexts or streams) race. Nothing in the array needs to start
 * at zero; each call writes what it reads. Per-kernel timing is off during
 * the call. */
#define DS5_NOALLOC_SCRATCH_BYTES (4u << 20)
int ds5_hip_attention_step_noalloc(ds5_hip_ctx* ctx, const ds5_attention_step_args* args);

/* ========================================================================
 * 4. Paged KV decode (no reference counterpart: the reference has no paged
 *    cache; its spec names a "KV page table", docs/specs/DS5_Project_Spec_v0.3.md:65)
 * ======================================================================== */

/* Pool layout: the frozen cache layout with the pool as the position axis,
 * f16 [n_kv_heads, n_pages * page_size, head_dim]; a page is page_size
 * consecutive slots. Sequence b's position p lives in slot
 *     page_table[b * max_pages + p / page_size] * page_size + p % page_size.
 * One decode token per sequence: its q/k/v are normalised and rotated at
 * position seq_lens[b] - 1, k/v are appended into that slot, and the token
 * attends positions 0..seq_lens[b]-1. max_seq_len is a host-side upper bound
 * of seq_lens (it sizes the launch). page_size must be a multiple of 16 (a
 * 16-position half-tile of the kernel never straddles pages). Entries the
 * device finds out of range -- a sequence length outside [1, max_seq_len] or a
 * page index outside [0, n_pages) -- are never dereferenced; that sequence's
 * output rows are set to NaN instead. */
typedef struct ds5_paged_decode_args {
    ds5_buf q;          /* f32 [n_seqs, n_q_heads, head_dim] (in/out: normalised + rotated) */
    ds5_buf k;          /* f32 [n_seqs, n_kv_heads, head_dim] (in/out) */
    ds5_buf v;          /* f32 [n_seqs, n_kv_heads, head_dim] */
    ds5_buf q_norm;     /* f32 [head_dim] */
    ds5_buf k_norm;     /* f32 [head_dim] */
    ds5_buf k_pool;     /* f16 [n_kv_heads, n_pages * page_size, head_dim] */
    ds5_buf v_pool;
    ds5_buf page_table; /* i32 [n_seqs, max_pages] */
    ds5_buf seq_lens;   /* i32 [n_seqs], each >= 1, includes the appended token */
    ds5_buf out;        /* f32 [n_seqs, n_q_heads * head_dim] */
    uint32_t n_seqs;
    uint32_t n_q_heads;
    uint32_t n_kv_heads;
    uint32_t head_dim;
    uint32_t page_size;
    uint32_t n_pages;
    uint32_t max_pages;
    uint32_t max_seq_len;
    float eps;
    float theta;
    float freq_scale;
    float scale;
} ds5_paged_decode_args;
int ds5_hip_paged_decode(ds5_hip_ctx* ctx, const ds5_paged_decode_args* args);

/* ========================================================================
 * 5. Bench/test utility (no reference counterpart)
 * ======================================================================== */

/* inv_freq[i] = theta^(-(2i)/head_dim), i < head_dim/2, exactly as the rope
 * kernels use it (std.math.pow(f32) evaluation order, kernels_a.zig:119-120).
 * Host-only; lets tests pin the table against the CPU reference. */
int ds5_hip_rope_table(float theta, uint32_t head_dim, float* out);

/* Fill `n` f16 values at buf with N(0,1) draws from a counter-based generator
 * (seed, element index) on the device. Lets benchmarks build multi-GB caches
 * without host generation; results are deterministic for a given seed. */
int ds5_hip_fill_normal_f16(ds5_hip_ctx* ctx, ds5_buf buf, uint64_t n, uint64_t seed);

/* Device-to-device byte copy on the context stream (the runtime's plain copy
 * kernel). The benchmark uses a copy of known size to calibrate the HBM
 * traffic counters (FETCH_SIZE / WRITE_SIZE) it reports. */
int ds5_hip_copy_device(ds5_hip_ctx* ctx, ds5_buf dst, ds5_buf src, uint64_t len);

/* Zero `len` bytes of a view on the context stream with a fill kernel: no host
 * copy and no synchronisation (the reference zeroes the MoE accumulator with a
 * host upload, forward.zig:452-454; a device-resident engine step does it here),
 * and no memset node when the call is captured into a graph. */
int ds5_hip_zero(ds5_hip_ctx* ctx, ds5_buf buf, uint64_t len);

/* Floor measurements for the benchmark: one launch that reads `len` bytes of
 * buf once (len % 16 == 0, 16-byte aligned view) with the decode kernel's
 * contiguous access -- 16-byte non-temporal loads, 64 KiB per 256-thread
 * workgroup -- and computes nothing (sink: 4 bytes, written only for one bit
 * pattern of the data); and one launch of an empty kernel over n_workgroups
 * workgroups. Captured per layer into a graph they give the cost of one
 * dependent launch and of one bare read of a layer's K/V. */
int ds5_hip_stream_read(ds5_hip_ctx* ctx, ds5_buf buf, uint64_t len, ds5_buf sink);
int ds5_hip_empty_launch(ds5_hip_ctx* ctx, uint32_t n_workgroups);

#ifdef __cplusplus
}
#endif
#endif /* DS5_HIP_H */
