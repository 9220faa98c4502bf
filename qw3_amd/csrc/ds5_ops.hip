// ds5_ops.hip -- the kernel-provider entry points of the C ABI.
//
// Each entry point checks the reference's preconditions, in the reference's
// order, before anything is enqueued (the GPU kernels have no error channel,
// as PORTING-kernels-a.md / -b.md require of the Metal glue), then dispatches:
//   rmsNorm       kernels_a.zig:68-91   -> rms_norm_rows_kernel (rows <= 256), rms_norm_tree_kernel
//   rope          kernels_a.zig:97-130  -> rope_kernel
//   kvAppend      kernels_a.zig:169-217 -> kv_append_kernel
//   gqaAttention  kernels_b.zig:29-133  -> decode_split_kernel (+ merge),
//                                          prefill_attention_kernel (f32 q),
//                                          or the generic kernel
#include <math.h>

#include <mutex>

#include "ds5_common.hpp"

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point (ds5_hip_attention_step_noalloc):
// a static device array, one copy per GPU, held until the process ends. Host
// code never passes the array's name to a kernel (on the host it is only a
// stand-in symbol): ds5_scratch_init looks up this device's address with
// hipGetSymbolAddress once per device, and the workspace calls hand out that
// address.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[DS5_NOALLOC_SCRATCH_BYTES];

int ds5_scratch_init(ds5_hip_ctx* ctx) {
    static std::mutex mu;
    static std::map<int, void*> per_device;  // device index -> address of `scratch` there
    std::lock_guard<std::mutex> lock(mu);
    auto it = per_device.find(ctx->device);
    if (it == per_device.end()) {
        void* ptr = nullptr;
        const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !ptr) {
            (void)hipGetLastError();  // do not leave the error for a later launch check
            return ds5_fail(ctx, DS5_DEVICE_FAILURE, "hipGetSymbolAddress(scratch) on device %d: %s", ctx->device,
                            hipGetErrorString(err));
        }
        it = per_device.emplace(ctx->device, ptr).first;
    }
    ctx->scratch = it->second;
    ctx->scratch_bytes = DS5_NOALLOC_SCRATCH_BYTES;
    return DS5_OK;
}

// ---------------------------------------------------------------------------
// Rope inverse frequencies, evaluated as the reference evaluates
// std.math.pow(f32, theta, -(2i/head_dim)) in kernels_a.zig:119-120: the Zig
// standard library splits |y| into integer and fraction parts, takes
// exp(frac * log x) (fractions above one half are shifted down by one into the
// integer part), multiplies in x^int by repeated squaring of frexp(x), and for
// a negative exponent takes the reciprocal before the final ldexp. The host C
// library supplies expf/logf. Built once per (theta, head_dim) on the host and
// passed to the kernels by value.
// ---------------------------------------------------------------------------
static float pow_f32_like_reference(float x, float y) {
    if (y == 0.0f || x == 1.0f) return 1.0f;
    if (isnan(x) || isnan(y)) return NAN;
    if (y == 1.0f) return x;
    if (!(x > 0.0f) || isinf(x) || isinf(y)) return powf(x, y);
    if (y == 0.5f) return sqrtf(x);
    if (y == -0.5f) return 1.0f / sqrtf(x);
    float int_part;
    float frac = modff(fabsf(y), &int_part);
    if (int_part >= 2147483648.0f) return powf(x, y);
    float mant_acc = 1.0f;
    int exp_acc = 0;
    if (frac != 0.0f) {
        if (frac > 0.5f) {
            frac -= 1.0f;
            int_part += 1.0f;
        }
        mant_acc = expf(frac * logf(x));
    }
    int xe;
    float xm = frexpf(x, &xe);
    for (int32_t n = (int32_t)int_part; n != 0; n >>= 1) {
        if (xe < -512 || xe > 512) {
            exp_acc += xe;
            break;
        }
        if (n & 1) {
            mant_acc *= xm;
            exp_acc += xe;
        }
        xm *= xm;
        xe <<= 1;
        if (xm < 0.5f) {
            xe -= 1;
            xm += xm;
        }
    }
    if (y < 0.0f) {
        mant_acc = 1.0f / mant_acc;
        exp_acc = -exp_acc;
    }
    return scalbnf(mant_acc, exp_acc);
}

void ds5_rope_table(float theta, uint32_t head_dim, RopeTable* t) {
    const uint32_t half = head_dim / 2;
    for (uint32_t i = 0; i < DS5_MAX_ROPE_HALF; i++) {
        if (i < half) {
            const float expnt = (float)(2 * i) / (float)head_dim;
            t->inv[i] = pow_f32_like_reference(theta, -expnt);
        } else {
            t->inv[i] = 0.0f;
        }
    }
}

namespace {

bool covers(ds5_buf b, uint64_t bytes) { return b.len >= bytes && (bytes == 0 || b.handle != nullptr); }

bool aligned16(ds5_buf b) { return ((uintptr_t)ds5_ptr(b) & 15u) == 0; }

uint64_t cache_elem_bytes(uint32_t kv_dtype) {
    return kv_dtype == DS5_DTYPE_F32 ? 4 : kv_dtype == DS5_DTYPE_F16 ? 2 : 0;
}

struct TableCache {
    float theta = NAN;
    uint32_t head_dim = 0;
    RopeTable table;
};

const RopeTable* rope_table_for(float theta, uint32_t head_dim) {
    static thread_local TableCache cache;
    if (!(cache.theta == theta) || cache.head_dim != head_dim) {
        ds5_rope_table(theta, head_dim, &cache.table);
        cache.theta = theta;
        cache.head_dim = head_dim;
    }
    return &cache.table;
}

// Runs after the preconditions, so shape errors are reported even without a
// device context (a null context then fails with DeviceFailure).
int set_device(ds5_hip_ctx* ctx) {
    if (!ctx) return DS5_DEVICE_FAILURE;
    return ds5_hip_status(ctx, hipSetDevice(ctx->device), "hipSetDevice");
}

}  // namespace

extern "C" {

int ds5_hip_rms_norm(ds5_hip_ctx* ctx, const ds5_rms_norm_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    const uint64_t n_rows = a->n_rows, dim = a->dim;
    if (dim == 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "rms_norm: dim == 0");
    if (!covers(a->x, n_rows * dim * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "rms_norm: x too small");
    if (!covers(a->out, n_rows * dim * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "rms_norm: out too small");
    if (!covers(a->weight, dim * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "rms_norm: weight too small");
    if (int rc = set_device(ctx)) return rc;
    RmsNormLaunch l{(const float*)ds5_ptr(a->x), (const float*)ds5_ptr(a->weight), (float*)ds5_ptr(a->out),
                    a->n_rows, a->dim, a->eps};
    return launch_rms_norm(ctx, l);
}

// kernels_a.zig:136-150: dtype first, then k, then the three buffer sizes.
static int check_matmul(ds5_hip_ctx* ctx, const char* op, ds5_buf x, ds5_buf w, uint32_t w_dtype, ds5_buf out,
                        uint64_t m, uint64_t n, uint64_t k) {
    const bool q8 = w_dtype == DS5_DTYPE_Q8_0;
    if (!q8 && w_dtype != DS5_DTYPE_F32)
        return ds5_fail(ctx, DS5_UNSUPPORTED_DTYPE, "%s: w_dtype %u (f32 and q8_0 are supported)", op, w_dtype);
    if (k == 0 || k % (q8 ? 32 : 1) != 0)
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: k = %llu is not a positive multiple of the weight block", op,
                        (unsigned long long)k);
    if (!covers(x, m * k * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: x too small", op);
    if (!covers(out, m * n * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: out too small", op);
    const uint64_t row_bytes = q8 ? k / 32 * 34 : k * 4;
    if (!covers(w, n * row_bytes)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: w too small", op);
    return DS5_OK;
}

int ds5_hip_matmul(ds5_hip_ctx* ctx, const ds5_matmul_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    if (int rc = check_matmul(ctx, "matmul", a->x, a->w, a->w_dtype, a->out, a->m, a->n, a->k)) return rc;
    if (a->m == 0 || a->n == 0) return DS5_OK;
    if (int rc = set_device(ctx)) return rc;
    const MatmulLaunch l{(const float*)ds5_ptr(a->x), (const uint8_t*)ds5_ptr(a->w), a->w_dtype == DS5_DTYPE_Q8_0,
                         (float*)ds5_ptr(a->out), a->m, a->n, a->k};
    return launch_matmul(ctx, l, matmul_path(l, a->w.len));
}

// kernels_a.zig:223-233: x, y, out sizes in order.
int ds5_hip_add(ds5_hip_ctx* ctx, const ds5_add_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    const uint64_t n = a->n_elems;
    if (!covers(a->x, n * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "add: x too small");
    if (!covers(a->y, n * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "add: y too small");
    if (!covers(a->out, n * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "add: out too small");
    if (n == 0) return DS5_OK;
    if (int rc = set_device(ctx)) return rc;
    return launch_add(ctx, ds5_ptr(a->x), ds5_ptr(a->y), ds5_ptr(a->out), n);
}

int ds5_hip_matmul_add(ds5_hip_ctx* ctx, const ds5_matmul_add_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    if (int rc = check_matmul(ctx, "matmul_add", a->x, a->w, a->w_dtype, a->out, a->m, a->n, a->k)) return rc;
    if (!covers(a->residual, (uint64_t)a->m * a->n * 4))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "matmul_add: residual too small");
    if ((((uintptr_t)ds5_ptr(a->residual) | (uintptr_t)ds5_ptr(a->out)) & 3u) != 0)
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "matmul_add: residual and out must be 4-byte aligned views");
    if (a->m == 0 || a->n == 0) return DS5_OK;
    if (int rc = set_device(ctx)) return rc;
    MatmulLaunch l{(const float*)ds5_ptr(a->x), (const uint8_t*)ds5_ptr(a->w), a->w_dtype == DS5_DTYPE_Q8_0,
                   (float*)ds5_ptr(a->out), a->m, a->n, a->k};
    l.res = (const float*)ds5_ptr(a->residual);
    return launch_matmul(ctx, l, matmul_path(l, a->w.len));
}

// ---------------------------------------------------------------------------
// MoE: router top-k and SwiGLU experts (kernels_c.zig)
// ---------------------------------------------------------------------------

static uint64_t row_bytes_of(uint32_t dtype, uint64_t k) {
    return dtype == DS5_DTYPE_Q8_0 ? k / 32 * 34 : k * (dtype == DS5_DTYPE_F16 ? 2 : 4);
}

// kernels_c.zig:81-95, without the output slices (checked by the caller).
static int check_router(ds5_hip_ctx* ctx, const char* op, ds5_buf x, ds5_buf w, uint32_t dt, uint64_t T,
                        uint64_t dim, uint64_t E, uint64_t K, bool outputs_ok) {
    if (dt != DS5_DTYPE_F32 && dt != DS5_DTYPE_F16 && dt != DS5_DTYPE_Q8_0)
        return ds5_fail(ctx, DS5_UNSUPPORTED_DTYPE, "%s: router w_dtype %u (f32, f16 and q8_0 are supported)", op, dt);
    if (K == 0 || K > E) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: top_k %llu of %llu experts", op,
                                         (unsigned long long)K, (unsigned long long)E);
    if (dim == 0 || dim % (dt == DS5_DTYPE_Q8_0 ? 32 : 1) != 0)
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: dim %llu is not a positive multiple of the block", op,
                        (unsigned long long)dim);
    if (!outputs_ok) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: output lengths are not n_tokens * top_k", op);
    if (!covers(x, T * dim * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: x too small", op);
    if (!covers(w, E * row_bytes_of(dt, dim))) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: router w too small", op);
    // LDS: a token's x and at least one router row (<= 128 KiB), the logits of a token (<= 64 KiB)
    if (row_bytes_of(dt, dim) > 65536 || dim * 4 + row_bytes_of(dt, dim) > 131072 || E > 16384)
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: dim %llu / n_experts %llu exceed the router's LDS", op,
                        (unsigned long long)dim, (unsigned long long)E);
    return DS5_OK;
}

// kernels_c.zig:157-183 (sizes; the pairs are checked by the caller).
static int check_experts(ds5_hip_ctx* ctx, const char* op, ds5_buf x, ds5_buf gate, ds5_buf up, ds5_buf down,
                         uint32_t dt, ds5_buf out, uint64_t T, uint64_t dim, uint64_t ffn, uint64_t E) {
    if (dt != DS5_DTYPE_F32 && dt != DS5_DTYPE_Q8_0)
        return ds5_fail(ctx, DS5_UNSUPPORTED_DTYPE, "%s: expert w_dtype %u (f32 and q8_0 are supported)", op, dt);
    const uint64_t block = dt == DS5_DTYPE_Q8_0 ? 32 : 1;
    if (dim == 0 || ffn == 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: dim or ffn_dim is 0", op);
    if (dim % block || ffn % block) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: dims not block multiples", op);
    if (!covers(x, T * dim * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: x too small", op);
    if (!covers(out, T * dim * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: out too small", op);
    const uint64_t gstride = row_bytes_of(dt, dim) * ffn, dstride = row_bytes_of(dt, ffn) * dim;
    if (!covers(gate, E * gstride)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: gate too small", op);
    if (!covers(up, E * gstride)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: up too small", op);
    if (!covers(down, E * dstride)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "%s: down too small", op);
    return DS5_OK;
}

// The wavefront GEMVs work in 32-element blocks (dim and ffn multiples of 32,
// as Q8_0 always is), read x / h as float4 and each Q8_0 block as the nine
// dwords from its dword floor (2 bytes past the last block unless the bank
// ends on a dword boundary or its view has 2 more bytes); f32 rows as floats.
static bool experts_fast(ds5_buf x, ds5_buf gate, ds5_buf up, ds5_buf down, uint32_t dt, uint64_t dim, uint64_t ffn,
                         uint64_t E) {
    if (dim % 32 || ffn % 32 || dim > 16384 || ((uintptr_t)ds5_ptr(x) & 15u)) return false;  // x staged in LDS
    const uint64_t ends[3] = {row_bytes_of(dt, dim) * ffn * E, row_bytes_of(dt, dim) * ffn * E,
                              row_bytes_of(dt, ffn) * dim * E};
    const ds5_buf banks[3] = {gate, up, down};
    for (int i = 0; i < 3; i++) {
        const uintptr_t a = (uintptr_t)ds5_ptr(banks[i]);
        if (a & 3u) return false;
        if (dt == DS5_DTYPE_Q8_0 && (a + ends[i]) % 4 != 0 && banks[i].len < ends[i] + 2) return false;
    }
    return true;
}

// The experts run grouped (sorted by expert, on the matrix cores) when their Q8_0
// banks take the wavefront kernels and the pairs share experts: from two pairs per
// expert on average, each expert's weights are read once instead of once per pair.
static bool experts_grouped(bool fast, uint32_t dt, uint64_t P, uint64_t E, uint64_t dim, uint64_t ffn) {
    return fast && dt == DS5_DTYPE_Q8_0 && E > 0 && E <= kMoeGroupedMaxExperts && P >= 2 * E &&
           P * std::max(dim, ffn) * 2 < (1ull << 32) && row_bytes_of(dt, std::max(dim, ffn)) * std::max(dim, ffn) <
                                                                (1ull << 31);
}

struct MoeScratch {
    float* logits;
    ds5_pair* pairs;
    uint32_t* order;
    uint32_t* offsets;
    float* h;
    float* y;
    uint16_t* ids;
    float* weights;
    float* h2;  // the normalised x, when the router applies the norm
    // grouped experts
    uint16_t *xhi, *xlo, *hhi, *hlo;
    int *xexp, *hexp;
    float* u;
    uint32_t *perm, *xrow, *n_tiles;
    uint4* tiles;
};

static size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

// Scratch for the router (E experts' logits; 0: none) and the experts; nE: the
// bank's expert count when the experts run grouped (0: not grouped).
static int moe_scratch(ds5_hip_ctx* ctx, uint64_t T, uint64_t E, uint64_t P, uint64_t dim, uint64_t ffn,
                       MoeScratch* s, uint64_t nE = 0) {
    const uint64_t G = nE ? P : 0, GT = nE ? T : 0;  // rows of the grouped h and x planes
    const size_t sz[19] = {up256(T * E * 4), up256(P * sizeof(ds5_pair)), up256(P * 4), up256((T + 1) * 4),
                           up256(P * ffn * 4), up256(P * dim * 4), up256(P * 2), up256(P * 4), up256(T * dim * 4),
                           up256(GT * dim * 2), up256(GT * dim * 2), up256(G * ffn * 2), up256(G * ffn * 2),
                           up256(GT * 4), up256(G * 4), up256(G * ffn * 4), up256(G * 4), up256(G * 4),
                           up256(nE ? 16 : 0)};
    const size_t tiles_sz = nE ? up256((size_t)moe_max_tiles((uint32_t)P, (uint32_t)nE) * 16) : 0;
    size_t total = tiles_sz;
    for (size_t v : sz) total += v;
    void* ws = nullptr;
    if (int rc = ds5_workspace(ctx, total, &ws)) return rc;
    char* p = (char*)ws;
    void** dst[19] = {(void**)&s->logits, (void**)&s->pairs, (void**)&s->order, (void**)&s->offsets,
                      (void**)&s->h, (void**)&s->y, (void**)&s->ids, (void**)&s->weights, (void**)&s->h2,
                      (void**)&s->xhi, (void**)&s->xlo, (void**)&s->hhi, (void**)&s->hlo, (void**)&s->xexp,
                      (void**)&s->hexp, (void**)&s->u, (void**)&s->perm, (void**)&s->xrow, (void**)&s->n_tiles};
    for (int i = 0; i < 19; i++) {
        *dst[i] = p;
        p += sz[i];
    }
    s->tiles = nE ? (uint4*)p : nullptr;
    if (!nE) s->n_tiles = nullptr;
    return DS5_OK;
}

static ExpertLaunch expert_launch(const ds5_buf& x, const ds5_buf& gate, const ds5_buf& up, const ds5_buf& down,
                                  uint32_t dt, const ds5_buf& out, uint32_t T, uint32_t P, uint32_t dim, uint32_t ffn,
                                  uint32_t E, const MoeScratch& s) {
    ExpertLaunch l{};
    l.x = (const float*)ds5_ptr(x);
    l.gate = (const uint8_t*)ds5_ptr(gate);
    l.up = (const uint8_t*)ds5_ptr(up);
    l.down = (const uint8_t*)ds5_ptr(down);
    l.q8 = dt == DS5_DTYPE_Q8_0;
    l.fast = experts_fast(x, gate, up, down, dt, dim, ffn, E);
    l.pairs = s.pairs;
    l.out = (float*)ds5_ptr(out);
    l.h = s.h;
    l.y = s.y;
    l.n_tokens = T;
    l.n_pairs = P;
    l.dim = dim;
    l.ffn = ffn;
    l.row_h = row_bytes_of(dt, dim);
    l.row_f = row_bytes_of(dt, ffn);
    l.stride_gu = l.row_h * ffn;
    l.stride_d = l.row_f * dim;
    l.grouped = s.tiles != nullptr && s.n_tiles != nullptr && experts_grouped(l.fast, dt, P, E, dim, ffn);
    if (l.grouped) {
        l.n_experts = E;
        // 128-row tiles (8 wavefronts) from ~96 pairs per expert; below, 64-row tiles (4
        // wavefronts) leave fewer rows of each expert's last tile empty (2048 tokens x 8
        // over 128 experts: 1.01 ms with 128 rows, 1.12 with 64; 512 tokens: 0.53, 0.41)
        l.tile_rows = P >= 96ull * E ? 128 : kMoeMinTileRows;
        l.max_tiles = moe_max_tiles(P, E, l.tile_rows);
        l.xhi = s.xhi;
        l.xlo = s.xlo;
        l.hhi = s.hhi;
        l.hlo = s.hlo;
        l.xexp = s.xexp;
        l.hexp = s.hexp;
        l.u = s.u;
        l.perm = s.perm;
        l.xrow = s.xrow;
        l.n_tiles = s.n_tiles;
        l.tiles = s.tiles;
    }
    return l;
}

int ds5_hip_router_topk(ds5_hip_ctx* ctx, const ds5_router_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    const uint64_t TK = (uint64_t)a->n_tokens * a->top_k;
    if (int rc = check_router(ctx, "router_topk", a->x, a->w, a->w_dtype, a->n_tokens, a->dim, a->n_experts, a->top_k,
                              a->out_ids_len == TK && a->out_weights_len == TK))
        return rc;
    if ((TK && (!a->out_ids || !a->out_weights))) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "router_topk: null output");
    if (a->n_tokens == 0) return DS5_OK;
    if (int rc = set_device(ctx)) return rc;
    MoeScratch s{};
    if (int rc = moe_scratch(ctx, a->n_tokens, a->n_experts, TK, 0, 0, &s)) return rc;
    RouterLaunch r{(const float*)ds5_ptr(a->x), (const uint8_t*)ds5_ptr(a->w), a->w_dtype,
                   row_bytes_of(a->w_dtype, a->dim), a->n_tokens, a->dim, a->n_experts, a->top_k,
                   a->norm_topk_prob != 0, s.ids, s.weights, nullptr, s.logits};
    if (int rc = launch_router(ctx, r)) return rc;
    // host outputs (the reference's contract): wait, then copy back
    int rc = ds5_hip_status(ctx, hipMemcpyAsync(a->out_ids, s.ids, TK * 2, hipMemcpyDeviceToHost, ctx->stream), "ids");
    if (!rc) rc = ds5_hip_status(ctx, hipMemcpyAsync(a->out_weights, s.weights, TK * 4, hipMemcpyDeviceToHost,
                                                     ctx->stream), "weights");
    if (!rc) rc = ds5_hip_status(ctx, hipStreamSynchronize(ctx->stream), "router sync");
    return rc;
}

int ds5_hip_expert_mlp_swiglu(ds5_hip_ctx* ctx, const ds5_expert_mlp_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    if (int rc = check_experts(ctx, "expert_mlp", a->x, a->gate, a->up, a->down, a->w_dtype, a->out, a->n_tokens,
                               a->dim, a->ffn_dim, a->n_experts))
        return rc;
    const uint64_t P = a->n_pairs;
    if (P && !a->pairs) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "expert_mlp: null pairs");
    for (uint64_t p = 0; p < P; p++)
        if (a->pairs[p].token >= a->n_tokens || a->pairs[p].expert >= a->n_experts)
            return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "expert_mlp: pair %llu (token %u, expert %u) out of range",
                            (unsigned long long)p, a->pairs[p].token, a->pairs[p].expert);
    if (P == 0 || a->n_tokens == 0) return DS5_OK;
    if (P > 0xffffffffull) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "expert_mlp: too many pairs");
    if (int rc = set_device(ctx)) return rc;
    // token-ordered view of the list, each token's pairs in list order
    std::vector<uint32_t> offsets(a->n_tokens + 1, 0), order(P);
    for (uint64_t p = 0; p < P; p++) offsets[a->pairs[p].token + 1]++;
    for (uint32_t t = 0; t < a->n_tokens; t++) offsets[t + 1] += offsets[t];
    {
        std::vector<uint32_t> fill(offsets.begin(), offsets.end() - 1);
        for (uint64_t p = 0; p < P; p++) order[fill[a->pairs[p].token]++] = (uint32_t)p;
    }
    MoeScratch s{};
    const bool grouped = experts_grouped(experts_fast(a->x, a->gate, a->up, a->down, a->w_dtype, a->dim, a->ffn_dim,
                                                      a->n_experts),
                                         a->w_dtype, P, a->n_experts, a->dim, a->ffn_dim);
    if (int rc = moe_scratch(ctx, a->n_tokens, 0, P, a->dim, a->ffn_dim, &s, grouped ? a->n_experts : 0)) return rc;
    int rc = ds5_hip_status(ctx, hipMemcpyAsync(s.pairs, a->pairs, P * sizeof(ds5_pair), hipMemcpyHostToDevice,
                                                ctx->stream), "pairs");
    if (!rc) rc = ds5_hip_status(ctx, hipMemcpyAsync(s.order, order.data(), P * 4, hipMemcpyHostToDevice, ctx->stream),
                                 "pair order");
    if (!rc) rc = ds5_hip_status(ctx, hipMemcpyAsync(s.offsets, offsets.data(), offsets.size() * 4,
                                                     hipMemcpyHostToDevice, ctx->stream), "pair offsets");
    // the host arrays must outlive the copies
    if (!rc) rc = ds5_hip_status(ctx, hipStreamSynchronize(ctx->stream), "pairs sync");
    if (rc) return rc;
    ExpertLaunch l = expert_launch(a->x, a->gate, a->up, a->down, a->w_dtype, a->out, a->n_tokens, (uint32_t)P, a->dim,
                                   a->ffn_dim, a->n_experts, s);
    l.order = s.order;
    l.offsets = s.offsets;
    return launch_experts(ctx, l);
}

int ds5_hip_moe(ds5_hip_ctx* ctx, const ds5_moe_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    const uint64_t TK = (uint64_t)a->n_tokens * a->top_k;
    // x_norm: rmsNorm(x -> h) first (its checks first), then the block on h
    const bool norm = a->x_norm.len != 0;
    if (norm) {
        const uint64_t T = a->n_tokens, D = a->dim;
        if (D == 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "moe: dim == 0");
        if (!covers(a->x, T * D * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "moe: x too small");
        if (!covers(a->x_norm, D * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "moe: x_norm too small");
    }
    if (int rc = check_router(ctx, "moe", a->x, a->router_w, a->router_dtype, a->n_tokens, a->dim, a->n_experts,
                              a->top_k, true))
        return rc;
    if (int rc = check_experts(ctx, "moe", a->x, a->gate, a->up, a->down, a->w_dtype, a->out, a->n_tokens, a->dim,
                               a->ffn_dim, a->n_experts))
        return rc;
    if ((a->ids.len && !covers(a->ids, TK * 2)) || (a->weights.len && !covers(a->weights, TK * 4)))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "moe: ids / weights outputs too small");
    if (a->residual.len && !covers(a->residual, (uint64_t)a->n_tokens * a->dim * 4))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "moe: residual too small");
    if (a->n_tokens == 0) return DS5_OK;
    if (TK > 0xffffffffull) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "moe: too many pairs");
    if (int rc = set_device(ctx)) return rc;
    // The norm runs inside the router's per-token logits kernel (its f32 fast path, rows
    // of more than 256 elements: the tree order), which also writes h for the experts;
    // otherwise (also where the logits run in tiles) rmsNorm writes h to the context's
    // second buffer first and the block runs on h.
    const bool norm_inside = norm && a->dim > kRmsSerialMaxDim && a->dim % 4 == 0 &&
                             a->router_dtype == DS5_DTYPE_F32 && aligned16(a->x) && aligned16(a->router_w) &&
                             aligned16(a->x_norm) &&
                             !router_tiled(a->router_dtype, a->n_tokens, a->dim, ds5_ptr(a->x), ds5_ptr(a->router_w));
    if (norm && !norm_inside) {
        void* h = nullptr;
        const uint64_t bytes = (uint64_t)a->n_tokens * a->dim * 4;
        if (int rc = ds5_aux_workspace(ctx, bytes, &h)) return rc;
        if (int rc = launch_rms_norm(ctx, RmsNormLaunch{(const float*)ds5_ptr(a->x), (const float*)ds5_ptr(a->x_norm),
                                                        (float*)h, a->n_tokens, a->dim, a->x_norm_eps}))
            return rc;
        ds5_moe_args b = *a;
        b.x = ds5_buf{h, 0, bytes};
        b.x_norm = ds5_buf{};
        return ds5_hip_moe(ctx, &b);
    }
    MoeScratch s{};
    // the experts read x, or h2 (aligned scratch) when the router normalises
    const bool fast = experts_fast(norm_inside ? ds5_buf{} : a->x, a->gate, a->up, a->down, a->w_dtype, a->dim,
                                   a->ffn_dim, a->n_experts);
    const bool grouped = experts_grouped(fast, a->w_dtype, TK, a->n_experts, a->dim, a->ffn_dim);
    if (int rc = moe_scratch(ctx, a->n_tokens, a->n_experts, TK, a->dim, a->ffn_dim, &s, grouped ? a->n_experts : 0))
        return rc;
    RouterLaunch r{(const float*)ds5_ptr(a->x), (const uint8_t*)ds5_ptr(a->router_w), a->router_dtype,
                   row_bytes_of(a->router_dtype, a->dim), a->n_tokens, a->dim, a->n_experts, a->top_k,
                   a->norm_topk_prob != 0,
                   a->ids.len ? (uint16_t*)ds5_ptr(a->ids) : s.ids,
                   a->weights.len ? (float*)ds5_ptr(a->weights) : s.weights, s.pairs, s.logits};
    if (norm_inside) {
        r.x_norm_w = (const float*)ds5_ptr(a->x_norm);
        r.x_norm_eps = a->x_norm_eps;
        r.h_out = s.h2;
    }
    if (int rc = launch_router(ctx, r)) return rc;
    const ds5_buf ex = norm_inside ? ds5_buf{s.h2, 0, (uint64_t)a->n_tokens * a->dim * 4} : a->x;
    ExpertLaunch l = expert_launch(ex, a->gate, a->up, a->down, a->w_dtype, a->out, a->n_tokens, (uint32_t)TK,
                                   a->dim, a->ffn_dim, a->n_experts, s);
    l.top_k = a->top_k;  // token t's pairs are t * top_k .. (t + 1) * top_k - 1
    l.res = a->residual.len ? (const float*)ds5_ptr(a->residual) : nullptr;  // every token has top_k >= 1 pairs
    return launch_experts(ctx, l);
}

// The group's launch and each entry's kernel path (the checks done).
static void group_launch_of(const ds5_matmul_group_args* a, MatmulGroupLaunch& g, MatmulPath* paths) {
    g.x = (const float*)ds5_ptr(a->x);
    g.q8 = a->w_dtype == DS5_DTYPE_Q8_0;
    g.m = a->m;
    g.k = a->k;
    g.count = a->count;
    for (uint32_t e = 0; e < a->count; e++) {
        g.w[e] = (const uint8_t*)ds5_ptr(a->w[e]);
        g.out[e] = (float*)ds5_ptr(a->out[e]);
        g.n[e] = a->n[e];
        paths[e] = matmul_path(MatmulLaunch{g.x, g.w[e], g.q8, g.out[e], g.m, g.n[e], g.k}, a->w[e].len);
    }
}

int ds5_hip_matmul_group(ds5_hip_ctx* ctx, const ds5_matmul_group_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    if (a->count == 0 || a->count > DS5_MATMUL_GROUP_MAX)
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "matmul_group: count = %u (1..%u)", a->count, DS5_MATMUL_GROUP_MAX);
    for (uint32_t e = 0; e < a->count; e++)
        if (int rc = check_matmul(ctx, "matmul_group", a->x, a->w[e], a->w_dtype, a->out[e], a->m, a->n[e], a->k))
            return rc;
    if (a->m == 0) return DS5_OK;
    if (int rc = set_device(ctx)) return rc;
    MatmulGroupLaunch g{};
    MatmulPath paths[kMatmulGroupMax];
    group_launch_of(a, g, paths);
    return launch_matmul_group(ctx, g, paths);
}

int ds5_hip_rope(ds5_hip_ctx* ctx, const ds5_rope_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    const uint64_t T = a->n_tokens, H = a->n_heads, hd = a->head_dim;
    if (hd == 0 || hd % 2 != 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "rope: head_dim must be even and > 0");
    if (!covers(a->x, T * H * hd * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "rope: x too small");
    if (!covers(a->positions, T * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "rope: positions too small");
    if (hd > 2 * DS5_MAX_ROPE_HALF) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "rope: head_dim > 512");
    if (int rc = set_device(ctx)) return rc;
    RopeLaunch l{(float*)ds5_ptr(a->x), (const int32_t*)ds5_ptr(a->positions), a->n_tokens, a->n_heads,
                 a->head_dim, a->freq_scale, rope_table_for(a->theta, a->head_dim)};
    return launch_rope(ctx, l);
}

int ds5_hip_kv_append(ds5_hip_ctx* ctx, const ds5_kv_append_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    const uint64_t T = a->n_tokens, H = a->n_kv_heads, hd = a->head_dim, cap = a->max_ctx;
    if (hd == 0 || H == 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "kv_append: head_dim/n_kv_heads == 0");
    if ((uint64_t)a->pos + T > cap) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "kv_append: pos + n_tokens > max_ctx");
    const uint64_t new_bytes = T * H * hd * 4;
    if (!covers(a->k_new, new_bytes) || !covers(a->v_new, new_bytes))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "kv_append: k_new/v_new too small");
    const uint64_t eb = cache_elem_bytes(a->kv_dtype);
    if (!eb) return ds5_fail(ctx, DS5_UNSUPPORTED_DTYPE, "kv_append: kv_dtype %u", a->kv_dtype);
    if (!covers(a->k_cache, H * cap * hd * eb) || !covers(a->v_cache, H * cap * hd * eb))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "kv_append: cache too small");
    if (int rc = set_device(ctx)) return rc;
    KvAppendLaunch l{(const float*)ds5_ptr(a->k_new), (const float*)ds5_ptr(a->v_new), ds5_ptr(a->k_cache),
                     ds5_ptr(a->v_cache), a->kv_dtype, a->pos, a->n_tokens, a->n_kv_heads, a->head_dim,
                     a->max_ctx};
    return launch_kv_append(ctx, l);
}

static int check_attention(ds5_hip_ctx* ctx, const ds5_attn_args* a) {
    const uint64_t hq = a->n_q_heads, hkv = a->n_kv_heads, hd = a->head_dim;
    const uint64_t T = a->n_tokens, pos = a->pos, cap = a->max_ctx;
    if (hq == 0 || hkv == 0 || hd == 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "attention: zero heads or head_dim");
    if (hq % hkv != 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "attention: n_q_heads %% n_kv_heads != 0");
    if (pos + T > cap) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "attention: pos + n_tokens > max_ctx");
    const uint64_t q_bytes = T * hq * hd * 4;
    if (!covers(a->q, q_bytes) || !covers(a->out, q_bytes))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "attention: q/out too small");
    const uint64_t eb = cache_elem_bytes(a->kv_dtype);
    if (!eb) return ds5_fail(ctx, DS5_UNSUPPORTED_DTYPE, "attention: kv_dtype %u", a->kv_dtype);
    if (!covers(a->k_cache, hkv * cap * hd * eb) || !covers(a->v_cache, hkv * cap * hd * eb))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "attention: cache too small");
    if (hd > 512) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "attention: head_dim > 512");
    return DS5_OK;
}

// MFMA kernels: f16 cache, head_dim 64 or 128, 16-byte aligned views.
static bool mfma_shape(uint32_t kv_dtype, uint32_t head_dim, std::initializer_list<ds5_buf> bufs) {
    if (kv_dtype != DS5_DTYPE_F16 || (head_dim != 64 && head_dim != 128)) return false;
    for (const ds5_buf& b : bufs)
        if (!aligned16(b)) return false;
    return true;
}

int ds5_hip_gqa_attention(ds5_hip_ctx* ctx, const ds5_attn_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    if (int rc = check_attention(ctx, a)) return rc;
    if (a->n_tokens == 0) return DS5_OK;
    if (int rc = set_device(ctx)) return rc;
    if (mfma_shape(a->kv_dtype, a->head_dim, {a->q, a->k_cache, a->v_cache, a->out})) {
        if (a->n_tokens == 1) {
            DecodeLaunch l{};
            l.q = (const float*)ds5_ptr(a->q);
            l.k_cache = (f16*)ds5_ptr(a->k_cache);
            l.v_cache = (f16*)ds5_ptr(a->v_cache);
            l.cache_stride = a->max_ctx;
            l.ctx_len = a->pos + 1;
            l.max_len = a->pos + 1;
            l.out = (float*)ds5_ptr(a->out);
            l.n_seqs = 1;
            l.n_q_heads = a->n_q_heads;
            l.n_kv_heads = a->n_kv_heads;
            l.head_dim = a->head_dim;
            l.scale = a->scale;
            return launch_decode(ctx, l);
        }
        // the kernel scales q (already normalised and rotated) into its f16 operand
        PrefillLaunch l{};
        l.q = (const float*)ds5_ptr(a->q);
        l.q_scale = a->scale * kLog2e;
        l.k_cache = (const f16*)ds5_ptr(a->k_cache);
        l.v_cache = (const f16*)ds5_ptr(a->v_cache);
        l.out = (float*)ds5_ptr(a->out);
        l.pos = a->pos;
        l.n_tokens = a->n_tokens;
        l.n_q_heads = a->n_q_heads;
        l.n_kv_heads = a->n_kv_heads;
        l.head_dim = a->head_dim;
        l.max_ctx = a->max_ctx;
        return launch_prefill(ctx, l);
    }
    GenericAttnLaunch g{(const float*)ds5_ptr(a->q), ds5_ptr(a->k_cache), ds5_ptr(a->v_cache), (float*)ds5_ptr(a->out),
                        a->kv_dtype, a->pos, a->n_tokens, a->n_q_heads, a->n_kv_heads, a->head_dim, a->max_ctx,
                        a->scale};
    return launch_generic_attention(ctx, g);
}

// Workspace of the fused prefill step: the pre-pass's rope cos/sin table [T, head_dim] f32.
static size_t prefill_step_workspace_bytes(uint64_t T, uint64_t head_dim) { return (size_t)(T * head_dim * sizeof(float)); }
// A multi-token step on the MFMA shapes runs fused (pre-pass + attention kernel) when
// the pre-pass takes the kv width and q_norm is 16-byte aligned (the attention
// kernel reads it in float4s); otherwise it runs the separate ops.
static bool prefill_step_fused(const ds5_attention_step_args* a) {
    return prefill_prep_supported(a->n_kv_heads, a->head_dim) && aligned16(a->q_norm);
}

// The attention step's preconditions: rmsNorm(q), rmsNorm(k), rope(q), rope(k),
// kvAppend and gqaAttention checks, in that order.
static int check_step(ds5_hip_ctx* ctx, const ds5_attention_step_args* a) {
    const uint64_t T = a->n_tokens, hq = a->n_q_heads, hkv = a->n_kv_heads, hd = a->head_dim;
    if (hd == 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "step: head_dim == 0");
    if (!covers(a->q, T * hq * hd * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "step: q too small");
    if (!covers(a->q_norm, hd * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "step: q_norm too small");
    if (!covers(a->k, T * hkv * hd * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "step: k too small");
    if (!covers(a->k_norm, hd * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "step: k_norm too small");
    if (hd % 2 != 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "step: head_dim must be even");
    if (!covers(a->positions, T * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "step: positions too small");
    if (hkv == 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "step: n_kv_heads == 0");
    if ((uint64_t)a->pos + T > a->max_ctx) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "step: pos + n_tokens > max_ctx");
    if (!covers(a->v, T * hkv * hd * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "step: v too small");
    const ds5_attn_args at{a->q, a->k_cache, a->v_cache, a->kv_dtype, a->out, a->pos, a->n_tokens,
                           a->n_q_heads, a->n_kv_heads, a->head_dim, a->max_ctx, a->scale};
    if (int rc = check_attention(ctx, &at)) return rc;
    if (T == 0) return DS5_OK;
    if (hd > 2 * DS5_MAX_ROPE_HALF) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "step: head_dim > 512");
    return DS5_OK;
}

int ds5_hip_attention_step(ds5_hip_ctx* ctx, const ds5_attention_step_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    if (int rc = check_step(ctx, a)) return rc;
    const uint64_t T = a->n_tokens, hq = a->n_q_heads, hkv = a->n_kv_heads, hd = a->head_dim;
    const ds5_attn_args at{a->q, a->k_cache, a->v_cache, a->kv_dtype, a->out, a->pos, a->n_tokens,
                           a->n_q_heads, a->n_kv_heads, a->head_dim, a->max_ctx, a->scale};
    if (T == 0) return DS5_OK;
    if (int rc = set_device(ctx)) return rc;
    const RopeTable* table = rope_table_for(a->theta, a->head_dim);

    if (mfma_shape(a->kv_dtype, a->head_dim, {a->q, a->k, a->v, a->k_cache, a->v_cache, a->out})) {
        if (T == 1) {
            DecodeLaunch l{};
            l.q = (const float*)ds5_ptr(a->q);
            l.k_new = (const float*)ds5_ptr(a->k);
            l.v_new = (const float*)ds5_ptr(a->v);
            l.q_norm = (const float*)ds5_ptr(a->q_norm);
            l.k_norm = (const float*)ds5_ptr(a->k_norm);
            l.positions = (const int32_t*)ds5_ptr(a->positions);
            l.k_cache = (f16*)ds5_ptr(a->k_cache);
            l.v_cache = (f16*)ds5_ptr(a->v_cache);
            l.cache_stride = a->max_ctx;
            l.ctx_len = a->pos + 1;
            l.max_len = a->pos + 1;
            l.out = (float*)ds5_ptr(a->out);
            l.n_seqs = 1;
            l.n_q_heads = a->n_q_heads;
            l.n_kv_heads = a->n_kv_heads;
            l.head_dim = a->head_dim;
            l.scale = a->scale;
            l.eps = a->eps;
            l.freq_scale = a->freq_scale;
            l.fused = true;
            l.table = table;
            return launch_decode(ctx, l);
        }
        if (prefill_step_fused(a)) {
            // the pre-pass's rope cos/sin table [n_tokens, head_dim] in the workspace;
            // the attention kernel normalises, rotates and scales q itself
            void* ws = nullptr;
            if (int rc = ds5_workspace(ctx, prefill_step_workspace_bytes(T, hd), &ws)) return rc;
            KvPrepLaunch kp{};
            kp.k = (const float*)ds5_ptr(a->k);
            kp.v = (const float*)ds5_ptr(a->v);
            kp.k_norm = (const float*)ds5_ptr(a->k_norm);
            kp.positions = (const int32_t*)ds5_ptr(a->positions);
            kp.k_cache = (f16*)ds5_ptr(a->k_cache);
            kp.v_cache = (f16*)ds5_ptr(a->v_cache);
            kp.cs = (float*)ws;
            kp.pos = a->pos;
            kp.n_tokens = a->n_tokens;
            kp.n_kv_heads = a->n_kv_heads;
            kp.head_dim = a->head_dim;
            kp.max_ctx = a->max_ctx;
            kp.eps = a->eps;
            kp.freq_scale = a->freq_scale;
            kp.table = table;
            if (int rc = launch_kv_prep(ctx, kp)) return rc;
            PrefillLaunch l{};
            l.q = (const float*)ds5_ptr(a->q);
            l.q_norm = (const float*)ds5_ptr(a->q_norm);
            l.cs = kp.cs;
            l.eps = a->eps;
            l.q_scale = a->scale * kLog2e;
            l.k_cache = (const f16*)ds5_ptr(a->k_cache);
            l.v_cache = (const f16*)ds5_ptr(a->v_cache);
            l.out = (float*)ds5_ptr(a->out);
            l.pos = a->pos;
            l.n_tokens = a->n_tokens;
            l.n_q_heads = a->n_q_heads;
            l.n_kv_heads = a->n_kv_heads;
            l.head_dim = a->head_dim;
            l.max_ctx = a->max_ctx;
            return launch_prefill(ctx, l);
        }
    }

    // Other shapes: the six separate device ops, in place on q and k.
    float* q = (float*)ds5_ptr(a->q);
    float* k = (float*)ds5_ptr(a->k);
    int rc = launch_rms_norm(ctx, RmsNormLaunch{q, (const float*)ds5_ptr(a->q_norm), q, (uint32_t)(T * hq),
                                                a->head_dim, a->eps});
    if (!rc) rc = launch_rms_norm(ctx, RmsNormLaunch{k, (const float*)ds5_ptr(a->k_norm), k, (uint32_t)(T * hkv),
                                                     a->head_dim, a->eps});
    const int32_t* positions = (const int32_t*)ds5_ptr(a->positions);
    if (!rc) rc = launch_rope(ctx, RopeLaunch{q, positions, a->n_tokens, a->n_q_heads, a->head_dim, a->freq_scale, table});
    if (!rc) rc = launch_rope(ctx, RopeLaunch{k, positions, a->n_tokens, a->n_kv_heads, a->head_dim, a->freq_scale, table});
    if (!rc) rc = launch_kv_append(ctx, KvAppendLaunch{k, (const float*)ds5_ptr(a->v), ds5_ptr(a->k_cache),
                                                       ds5_ptr(a->v_cache), a->kv_dtype, a->pos, a->n_tokens,
                                                       a->n_kv_heads, a->head_dim, a->max_ctx});
    if (!rc) rc = ds5_hip_gqa_attention(ctx, &at);
    return rc;
}

int ds5_hip_attention_block(ds5_hip_ctx* ctx, const ds5_attention_block_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    const ds5_attention_step_args& s = a->step;
    const uint32_t hd = s.head_dim;
    // x_norm: rmsNorm(x -> h) first (its checks first), then the block on h
    const bool norm = a->x_norm.len != 0;
    if (norm) {
        const uint64_t T = s.n_tokens, H = a->hidden;
        if (H == 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "attention_block: hidden == 0");
        if (!covers(a->x, T * H * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "attention_block: x too small");
        if (!covers(a->x_norm, H * 4)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "attention_block: x_norm too small");
    }
    ds5_matmul_group_args g{};
    g.x = a->x;
    g.w_dtype = a->w_dtype;
    g.m = s.n_tokens;
    g.k = a->hidden;
    g.count = 3;
    g.w[0] = a->wq;
    g.w[1] = a->wk;
    g.w[2] = a->wv;
    g.out[0] = s.q;
    g.out[1] = s.k;
    g.out[2] = s.v;
    g.n[0] = s.n_q_heads * hd;
    g.n[1] = g.n[2] = s.n_kv_heads * hd;
    // the calls' preconditions, in their order: the three projections, then the step
    for (uint32_t e = 0; e < 3; e++)
        if (int rc = check_matmul(ctx, "attention_block", g.x, g.w[e], g.w_dtype, g.out[e], g.m, g.n[e], g.k)) return rc;
    if (int rc = check_step(ctx, &s)) return rc;
    if (s.n_tokens == 0) return DS5_OK;
    if (int rc = set_device(ctx)) return rc;
    MatmulGroupLaunch gl{};
    MatmulPath paths[kMatmulGroupMax];
    group_launch_of(&g, gl, paths);
    // The norm runs inside the projection's kernels (the row kernel or the GEMM's x
    // split, as they read x) for rows of more than 256 elements (the tree order) when
    // every projection takes one of them; otherwise rmsNorm writes h to the context's
    // second buffer first and the block runs on h.
    const bool all_rows = paths[0] == MatmulPath::Rows && paths[1] == MatmulPath::Rows && paths[2] == MatmulPath::Rows;
    const bool all_gemm = paths[0] == MatmulPath::Gemm && paths[1] == MatmulPath::Gemm && paths[2] == MatmulPath::Gemm;
    const bool norm_inside = norm && a->hidden > kRmsSerialMaxDim && aligned16(a->x_norm) && (all_rows || all_gemm);
    if (norm && !norm_inside) {
        void* h = nullptr;
        const uint64_t bytes = (uint64_t)s.n_tokens * a->hidden * 4;
        if (int rc = ds5_aux_workspace(ctx, bytes, &h)) return rc;
        if (int rc = launch_rms_norm(ctx, RmsNormLaunch{(const float*)ds5_ptr(a->x), (const float*)ds5_ptr(a->x_norm),
                                                        (float*)h, s.n_tokens, a->hidden, a->x_norm_eps}))
            return rc;
        ds5_attention_block_args b = *a;
        b.x = ds5_buf{h, 0, bytes};
        b.x_norm = ds5_buf{};
        return ds5_hip_attention_block(ctx, &b);
    }
    if (norm_inside) {
        gl.norm_w = (const float*)ds5_ptr(a->x_norm);
        gl.norm_eps = a->x_norm_eps;
    }
    // Fused: the prefill pre-pass in the projection GEMM's epilogue (the paths the two
    // calls would take: the GEMM for every weight, the fused MFMA prefill step).
    const bool fused = a->w_dtype == DS5_DTYPE_Q8_0 && hd == 128 && s.n_tokens >= 2 &&
                       mfma_shape(s.kv_dtype, hd, {s.q, s.k, s.v, s.k_cache, s.v_cache, s.out}) &&
                       prefill_prep_supported(s.n_kv_heads, hd) && aligned16(a->x) && aligned16(s.q_norm) &&
                       aligned16(s.k_norm) && all_gemm;
    if (!fused) {
        if (int rc = launch_matmul_group(ctx, gl, paths)) return rc;
        return ds5_hip_attention_step(ctx, &s);
    }
    const uint64_t T = s.n_tokens;
    const size_t q16_bytes = (size_t)T * s.n_q_heads * hd * sizeof(uint16_t);
    const size_t prep_bytes = qkv_prep_workspace_bytes(s.n_tokens, a->hidden, hd);
    void* ws = nullptr;
    if (int rc = ds5_workspace(ctx, q16_bytes + prep_bytes, &ws)) return rc;
    QkvPrepLaunch qp{};
    qp.x = (const float*)ds5_ptr(a->x);
    qp.wq = (const uint8_t*)ds5_ptr(a->wq);
    qp.wk = (const uint8_t*)ds5_ptr(a->wk);
    qp.wv = (const uint8_t*)ds5_ptr(a->wv);
    qp.m = s.n_tokens;
    qp.k = a->hidden;
    qp.n_q_heads = s.n_q_heads;
    qp.n_kv_heads = s.n_kv_heads;
    qp.head_dim = hd;
    qp.positions = (const int32_t*)ds5_ptr(s.positions);
    qp.freq_scale = s.freq_scale;
    qp.table = rope_table_for(s.theta, hd);
    qp.q_norm = (const float*)ds5_ptr(s.q_norm);
    qp.k_norm = (const float*)ds5_ptr(s.k_norm);
    qp.q16 = (f16*)ws;
    qp.k_cache = (f16*)ds5_ptr(s.k_cache);
    qp.v_cache = (f16*)ds5_ptr(s.v_cache);
    qp.pos = s.pos;
    qp.max_ctx = s.max_ctx;
    qp.eps = s.eps;
    qp.q_scale = s.scale * kLog2e;
    qp.ws = (char*)ws + q16_bytes;
    qp.norm_w = gl.norm_w;
    qp.norm_eps = gl.norm_eps;
    if (int rc = launch_qkv_prep(ctx, qp)) return rc;
    PrefillLaunch l{};
    l.q16 = (const f16*)ws;
    l.k_cache = qp.k_cache;
    l.v_cache = qp.v_cache;
    l.out = (float*)ds5_ptr(s.out);
    l.pos = s.pos;
    l.n_tokens = s.n_tokens;
    l.n_q_heads = s.n_q_heads;
    l.n_kv_heads = s.n_kv_heads;
    l.head_dim = hd;
    l.max_ctx = s.max_ctx;
    return launch_prefill(ctx, l);
}

// Workspace bytes ds5_hip_attention_step takes for these arguments: the same
// kernel choices as its dispatch (the fused MFMA decode or prefill, else the
// separate ops followed by ds5_hip_gqa_attention's own choice).
static size_t step_workspace_bytes(const ds5_hip_ctx* ctx, const ds5_attention_step_args* a) {
    const uint64_t T = a->n_tokens, hq = a->n_q_heads, hkv = a->n_kv_heads, hd = a->head_dim;
    if (T == 0 || hkv == 0 || hd == 0) return 0;
    const bool fused = mfma_shape(a->kv_dtype, a->head_dim, {a->q, a->k, a->v, a->k_cache, a->v_cache, a->out});
    if (fused && (T == 1 || prefill_step_fused(a)))
        return T == 1 ? decode_workspace_bytes(ctx, 1, a->n_q_heads, a->n_kv_heads, a->head_dim, a->pos + 1)
                      : prefill_step_workspace_bytes(T, hd);
    if (mfma_shape(a->kv_dtype, a->head_dim, {a->q, a->k_cache, a->v_cache, a->out}))
        return T == 1 ? decode_workspace_bytes(ctx, 1, a->n_q_heads, a->n_kv_heads, a->head_dim, a->pos + 1) : 0;
    return 0;
}

int ds5_hip_attention_step_noalloc(ds5_hip_ctx* ctx, const ds5_attention_step_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    if (!ctx) return ds5_hip_attention_step(ctx, a);  // preconditions, then DeviceFailure
    if (!ctx->scratch) return ds5_fail(ctx, DS5_DEVICE_FAILURE, "attention_step_noalloc: no scratch on this device");
    const size_t need = step_workspace_bytes(ctx, a);
    if (need > ctx->scratch_bytes)
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH,
                        "attention_step_noalloc: this call needs %zu bytes of scratch; the allocation-free entry "
                        "point holds at most %zu (use ds5_hip_attention_step)", need, ctx->scratch_bytes);
    // For the duration of the call: workspace from the static scratch array, and
    // no per-kernel timing (its event pool grows by allocation).
    struct Scope {
        ds5_hip_ctx* c;
        bool timing;
        explicit Scope(ds5_hip_ctx* c_) : c(c_), timing(c_->kernel_timing) {
            c->use_scratch = true;
            c->kernel_timing = false;
        }
        ~Scope() {
            c->use_scratch = false;
            c->kernel_timing = timing;
        }
    } scope(ctx);
    return ds5_hip_attention_step(ctx, a);
}

int ds5_hip_paged_decode(ds5_hip_ctx* ctx, const ds5_paged_decode_args* a) {
    if (!a) return DS5_SHAPE_MISMATCH;
    const uint64_t B = a->n_seqs, hq = a->n_q_heads, hkv = a->n_kv_heads, hd = a->head_dim;
    if (hq == 0 || hkv == 0 || hd == 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: zero heads or head_dim");
    if (hq % hkv != 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: n_q_heads %% n_kv_heads != 0");
    if (hd != 64 && hd != 128) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: head_dim must be 64 or 128");
    if (a->page_size == 0 || a->n_pages == 0 || a->max_pages == 0)
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: empty page geometry");
    if (a->page_size % 16 != 0)
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: page_size must be a multiple of 16");
    if ((uint64_t)a->max_seq_len > (uint64_t)a->max_pages * a->page_size)
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: max_seq_len exceeds max_pages * page_size");
    const uint64_t slots = (uint64_t)a->n_pages * a->page_size;
    if (!covers(a->q, B * hq * hd * 4) || !covers(a->out, B * hq * hd * 4))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: q/out too small");
    if (!covers(a->k, B * hkv * hd * 4) || !covers(a->v, B * hkv * hd * 4))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: k/v too small");
    if (!covers(a->q_norm, hd * 4) || !covers(a->k_norm, hd * 4))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: norm weights too small");
    if (!covers(a->k_pool, hkv * slots * hd * 2) || !covers(a->v_pool, hkv * slots * hd * 2))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: pool too small");
    if (!covers(a->page_table, B * a->max_pages * 4) || !covers(a->seq_lens, B * 4))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: page_table/seq_lens too small");
    for (const ds5_buf& b : {a->q, a->k, a->v, a->k_pool, a->v_pool, a->out})
        if (!aligned16(b)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: views must be 16-byte aligned");
    if (B == 0 || a->max_seq_len == 0) return DS5_OK;
    if (hd > 2 * DS5_MAX_ROPE_HALF) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "paged: head_dim > 512");
    if (int rc = set_device(ctx)) return rc;
    DecodeLaunch l{};
    l.q = (const float*)ds5_ptr(a->q);
    l.k_new = (const float*)ds5_ptr(a->k);
    l.v_new = (const float*)ds5_ptr(a->v);
    l.q_norm = (const float*)ds5_ptr(a->q_norm);
    l.k_norm = (const float*)ds5_ptr(a->k_norm);
    l.k_cache = (f16*)ds5_ptr(a->k_pool);
    l.v_cache = (f16*)ds5_ptr(a->v_pool);
    l.cache_stride = slots;
    l.page_table = (const int32_t*)ds5_ptr(a->page_table);
    l.seq_lens = (const int32_t*)ds5_ptr(a->seq_lens);
    l.page_size = a->page_size;
    l.max_pages = a->max_pages;
    l.max_len = a->max_seq_len;
    l.out = (float*)ds5_ptr(a->out);
    l.n_seqs = a->n_seqs;
    l.n_q_heads = a->n_q_heads;
    l.n_kv_heads = a->n_kv_heads;
    l.head_dim = a->head_dim;
    l.scale = a->scale;
    l.eps = a->eps;
    l.freq_scale = a->freq_scale;
    l.fused = true;
    l.table = rope_table_for(a->theta, a->head_dim);
    return launch_decode(ctx, l);
}

int ds5_hip_rope_table(float theta, uint32_t head_dim, float* out) {
    if (!out || head_dim == 0 || head_dim % 2 != 0 || head_dim > 2 * DS5_MAX_ROPE_HALF) return DS5_SHAPE_MISMATCH;
    RopeTable t;
    ds5_rope_table(theta, head_dim, &t);
    for (uint32_t i = 0; i < head_dim / 2; i++) out[i] = t.inv[i];
    return DS5_OK;
}

int ds5_hip_copy_device(ds5_hip_ctx* ctx, ds5_buf dst, ds5_buf src, uint64_t len) {
    if (!covers(dst, len) || !covers(src, len)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "copy_device: view too small");
    if (int rc = set_device(ctx)) return rc;
    if (len == 0) return DS5_OK;
    return ds5_hip_status(ctx, hipMemcpyAsync(ds5_ptr(dst), ds5_ptr(src), len, hipMemcpyDeviceToDevice, ctx->stream),
                          "copy_device");
}

int ds5_hip_stream_read(ds5_hip_ctx* ctx, ds5_buf buf, uint64_t len, ds5_buf sink) {
    if (len % 16 != 0 || !covers(buf, len) || !aligned16(buf))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "stream_read: len must be a multiple of 16 in a 16-byte aligned view");
    if (!covers(sink, 4) || ((uintptr_t)ds5_ptr(sink) & 3u))
        return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "stream_read: sink must be a 4-byte aligned view of 4 bytes");
    if (int rc = set_device(ctx)) return rc;
    return launch_stream_read(ctx, ds5_ptr(buf), len, (uint32_t*)ds5_ptr(sink));
}

int ds5_hip_zero(ds5_hip_ctx* ctx, ds5_buf buf, uint64_t len) {
    if (!covers(buf, len)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "zero: view too small");
    if (int rc = set_device(ctx)) return rc;
    return launch_zero(ctx, ds5_ptr(buf), len);
}

int ds5_hip_empty_launch(ds5_hip_ctx* ctx, uint32_t n_workgroups) {
    if (n_workgroups == 0) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "empty_launch: no workgroups");
    if (int rc = set_device(ctx)) return rc;
    return launch_empty(ctx, n_workgroups);
}

int ds5_hip_fill_normal_f16(ds5_hip_ctx* ctx, ds5_buf buf, uint64_t n, uint64_t seed) {
    if (!covers(buf, n * 2)) return ds5_fail(ctx, DS5_SHAPE_MISMATCH, "fill_normal_f16: buffer too small");
    if (int rc = set_device(ctx)) return rc;
    return launch_fill_normal_f16(ctx, (f16*)ds5_ptr(buf), n, seed);
}

}  // extern "C"
