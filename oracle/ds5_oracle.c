/*
 * ds5_oracle.c -- CPU restatement of DS5's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP backend, never part of the
 * shipped path. Build with -O2 -ffp-contract=off (oracle/build.py) so that no
 * a*b+c is contracted into an fma, matching Zig's default strict float mode.
 *
 * Transcendentals: the reference calls Zig's std.math.pow(f32), @cos, @sin and
 * @exp (kernels_a.zig:120-122, kernels_b.zig:115). @cos/@sin/@exp lower to the
 * C-library cosf/sinf/expf; here they are glibc's, which agree with Zig's
 * compiler-rt versions to within 1 ulp (bitwise agreement is not pinned).
 * std.math.pow(f32) is not a C-library call: ds5o_zig_powf restates its
 * algorithm (modf split, exp(yf*log x), frexp/squaring loop, reciprocal for a
 * negative exponent, final scalbn), because it can differ from a correctly
 * rounded powf by a few ulp and the rope angle multiplies that error by the
 * position.
 */
#include "ds5_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Buffer views (src/kernels/cpu/ctx.zig:70-108): a Buf is handle+offset and  */
/* len bytes; typed views cover exactly [offset, offset+len).               */
/* ------------------------------------------------------------------------ */

static void* view(ds5o_buf b) { return (char*)b.handle + b.offset; }

/* ------------------------------------------------------------------------ */
/* f16 <-> f32                                                               */
/* ------------------------------------------------------------------------ */

uint16_t ds5o_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax >= 0x38800000u) {                                  /* f16 normal range */
        uint32_t h = (ax - 0x38000000u) >> 13;                  /* rebias 127 -> 15 */
        const uint32_t rb = ax & 0x1fffu;
        if (rb > 0x1000u || (rb == 0x1000u && (h & 1u))) h += 1u; /* carry may bump exponent */
        return (uint16_t)(sign | h);
    }
    /* f16 subnormal: value = k * 2^-24 with k = m * 2^(e - 126). */
    const uint32_t e = ax >> 23;
    const int shift = 126 - (int)e;
    if (shift > 24) return (uint16_t)sign;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t k = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (k & 1u))) k += 1u;
    return (uint16_t)(sign | k);
}

float ds5o_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0x1fu) {
        x = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        x = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        x = sign;
    } else { /* subnormal: normalise */
        int ee = 113;
        while (!(m & 0x400u)) {
            m <<= 1;
            ee -= 1;
        }
        m &= 0x3ffu;
        x = sign | ((uint32_t)ee << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void ds5o_f32_to_f16_array(const float* x, uint16_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = ds5o_f32_to_f16(x[i]);
}

void ds5o_f16_to_f32_array(const uint16_t* h, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = ds5o_f16_to_f32(h[i]);
}

/* ------------------------------------------------------------------------ */
/* std.math.pow(f32) (Zig 0.16 standard library, lib/std/math/pow.zig).     */
/* The library's algorithm, restated for the inputs the path can produce   */
/* (finite x > 0; the sign/zero/inf special cases reduce to the C99 pow    */
/* special cases and are delegated to powf):                               */
/*   y == 0 or x == 1 -> 1;  y == 1 -> x;  y == +-0.5 -> sqrt / 1/sqrt;     */
/*   (yi, yf) = modf(|y|); if yf > 0.5 { yf -= 1; yi += 1 }                 */
/*   a1 = exp(yf * log(x)); (x1, xe) = frexp(x);                            */
/*   for i = yi; i != 0; i >>= 1 { if i&1 { a1 *= x1; ae += xe }            */
/*                                 x1 *= x1; xe <<= 1;                      */
/*                                 if x1 < 0.5 { xe -= 1; x1 += x1 } }      */
/*   if y < 0 { a1 = 1/a1; ae = -ae };  return scalbn(a1, ae)               */
/* ------------------------------------------------------------------------ */

float ds5o_zig_powf(float x, float y) {
    if (y == 0.0f || x == 1.0f) return 1.0f;
    if (isnan(x) || isnan(y)) return NAN;
    if (y == 1.0f) return x;
    if (!(x > 0.0f) || isinf(x) || isinf(y)) return powf(x, y);
    if (y == 0.5f) return sqrtf(x);
    if (y == -0.5f) return 1.0f / sqrtf(x);

    float yi;
    float yf = modff(fabsf(y), &yi);
    if (yi >= 2147483648.0f) return powf(x, y); /* over/underflow for every x != 1 */

    float a1 = 1.0f;
    int ae = 0;
    if (yf != 0.0f) {
        if (yf > 0.5f) {
            yf -= 1.0f;
            yi += 1.0f;
        }
        a1 = expf(yf * logf(x));
    }
    int xe;
    float x1 = frexpf(x, &xe);
    for (int32_t i = (int32_t)yi; i != 0; i >>= 1) {
        if (xe < -(1 << 9) || (1 << 9) < xe) {
            ae += xe;
            break;
        }
        if (i & 1) {
            a1 *= x1;
            ae += xe;
        }
        x1 *= x1;
        xe <<= 1;
        if (x1 < 0.5f) {
            xe -= 1;
            x1 += x1;
        }
    }
    if (y < 0.0f) {
        a1 = 1.0f / a1;
        ae = -ae;
    }
    return scalbnf(a1, ae);
}

/* ------------------------------------------------------------------------ */
/* matmul -- kernels_a.zig:136-163: out[m, n] = x[m, k] . W^T, one serial    */
/* f32 dot per (row, output) (dotRow, kernels_a.zig:39-62): f32 weights add */
/* w*x in k order; Q8_0 adds (f32(scale) * f32(q)) * x block by block, in   */
/* k order.                                                                 */
/* ------------------------------------------------------------------------ */

static float dot_row(const float* x, const uint8_t* row, uint32_t w_dtype, uint64_t k) {
    float acc = 0.0f;
    if (w_dtype == DS5O_F32) {
        const float* w = (const float*)row;
        for (uint64_t i = 0; i < k; i++) acc += w[i] * x[i];
    } else if (w_dtype == DS5O_F16) { /* kernels_c.zig:47-52 (router weights only) */
        for (uint64_t i = 0; i < k; i++)
            acc += ds5o_f16_to_f32((uint16_t)(row[2 * i] | (row[2 * i + 1] << 8))) * x[i];
    } else { /* DS5O_Q8_0 */
        for (uint64_t b = 0; b < k / 32; b++) {
            const uint8_t* blk = row + b * 34;
            const float scale = ds5o_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8))); /* little endian */
            const int8_t* qs = (const int8_t*)(blk + 2);
            for (int i = 0; i < 32; i++) acc += (scale * (float)qs[i]) * x[b * 32 + i];
        }
    }
    return acc;
}

int ds5o_matmul(const ds5o_matmul_args* a) {
    if (a->w_dtype != DS5O_F32 && a->w_dtype != DS5O_Q8_0) return DS5O_UNSUPPORTED_DTYPE;
    const uint64_t m = a->m, n = a->n, k = a->k;
    const uint64_t block = a->w_dtype == DS5O_Q8_0 ? 32 : 1;
    if (k == 0 || k % block != 0) return DS5O_SHAPE_MISMATCH;
    if (a->x.len < m * k * 4) return DS5O_SHAPE_MISMATCH;
    if (a->out.len < m * n * 4) return DS5O_SHAPE_MISMATCH;
    const uint64_t row_bytes = a->w_dtype == DS5O_Q8_0 ? k / 32 * 34 : k * 4;
    if (a->w.len < n * row_bytes) return DS5O_SHAPE_MISMATCH;

    const float* x = (const float*)view(a->x);
    const uint8_t* w = (const uint8_t*)view(a->w);
    float* out = (float*)view(a->out);
    for (uint64_t mi = 0; mi < m; mi++)
        for (uint64_t ni = 0; ni < n; ni++) out[mi * n + ni] = dot_row(x + mi * k, w + ni * row_bytes, a->w_dtype, k);
    return DS5O_OK;
}

/* ------------------------------------------------------------------------ */
/* routerTopK -- kernels_c.zig:80-155                                         */
/* logits = x . W^T (f32, serial), softmax over all experts, the top_k largest */
/* probabilities descending with ties to the lower id (ascending scan, strict  */
/* >), then optionally divided by their sum.                                   */
/* ------------------------------------------------------------------------ */

int ds5o_router_topk(const ds5o_router_args* a) {
    if (a->w_dtype != DS5O_F32 && a->w_dtype != DS5O_F16 && a->w_dtype != DS5O_Q8_0) return DS5O_UNSUPPORTED_DTYPE;
    const uint64_t T = a->n_tokens, dim = a->dim, E = a->n_experts, K = a->top_k;
    const uint64_t block = a->w_dtype == DS5O_Q8_0 ? 32 : 1;
    if (K == 0 || K > E) return DS5O_SHAPE_MISMATCH;
    if (dim == 0 || dim % block != 0) return DS5O_SHAPE_MISMATCH;
    if (a->out_ids_len != T * K) return DS5O_SHAPE_MISMATCH;
    if (a->out_weights_len != T * K) return DS5O_SHAPE_MISMATCH;
    if (a->x.len < T * dim * 4) return DS5O_SHAPE_MISMATCH;
    const uint64_t row_bytes = a->w_dtype == DS5O_Q8_0 ? dim / 32 * 34 : dim * (a->w_dtype == DS5O_F16 ? 2 : 4);
    if (a->w.len < E * row_bytes) return DS5O_SHAPE_MISMATCH;

    float* probs = (float*)malloc(E * sizeof(float));
    unsigned char* taken = (unsigned char*)malloc(E);
    if (!probs || !taken) {
        free(probs);
        free(taken);
        return DS5O_OUT_OF_MEMORY;
    }
    const float* x = (const float*)view(a->x);
    const uint8_t* w = (const uint8_t*)view(a->w);
    for (uint64_t t = 0; t < T; t++) {
        const float* xr = x + t * dim;
        float mx = -INFINITY;
        for (uint64_t e = 0; e < E; e++) {
            probs[e] = dot_row(xr, w + e * row_bytes, a->w_dtype, dim);
            mx = fmaxf(mx, probs[e]);
        }
        float sum = 0.0f;
        for (uint64_t e = 0; e < E; e++) {
            probs[e] = expf(probs[e] - mx);
            sum += probs[e];
        }
        const float inv_sum = 1.0f / sum;
        for (uint64_t e = 0; e < E; e++) probs[e] *= inv_sum;
        memset(taken, 0, E);
        float picked = 0.0f;
        for (uint64_t j = 0; j < K; j++) {
            uint64_t best = 0;
            float best_p = -1.0f;
            for (uint64_t e = 0; e < E; e++)
                if (!taken[e] && probs[e] > best_p) {
                    best = e;
                    best_p = probs[e];
                }
            taken[best] = 1;
            a->out_ids[t * K + j] = (uint16_t)best;
            a->out_weights[t * K + j] = best_p;
            picked += best_p;
        }
        if (a->norm_topk_prob) {
            const float inv = 1.0f / picked;
            for (uint64_t j = 0; j < K; j++) a->out_weights[t * K + j] *= inv;
        }
    }
    free(probs);
    free(taken);
    return DS5O_OK;
}

/* ------------------------------------------------------------------------ */
/* expertMlpSwiglu -- kernels_c.zig:157-214                                   */
/* per pair, in list order: h = silu(gate . x) * (up . x) over ffn_dim, then   */
/* out[token] += weight * (down . h); silu(v) = v / (1 + exp(-v)). A pair out  */
/* of range is ShapeMismatch when it is reached (earlier pairs already added). */
/* ------------------------------------------------------------------------ */

int ds5o_expert_mlp_swiglu(const ds5o_expert_mlp_args* a) {
    if (a->w_dtype != DS5O_F32 && a->w_dtype != DS5O_Q8_0) return DS5O_UNSUPPORTED_DTYPE;
    const uint64_t dim = a->dim, ffn = a->ffn_dim, T = a->n_tokens;
    const uint64_t block = a->w_dtype == DS5O_Q8_0 ? 32 : 1;
    if (dim == 0 || ffn == 0) return DS5O_SHAPE_MISMATCH;
    if (dim % block != 0 || ffn % block != 0) return DS5O_SHAPE_MISMATCH;
    if (a->x.len < T * dim * 4) return DS5O_SHAPE_MISMATCH;
    if (a->out.len < T * dim * 4) return DS5O_SHAPE_MISMATCH;
    const uint64_t row_h = a->w_dtype == DS5O_Q8_0 ? dim / 32 * 34 : dim * 4;  /* gate / up rows */
    const uint64_t row_f = a->w_dtype == DS5O_Q8_0 ? ffn / 32 * 34 : ffn * 4;  /* down rows */
    const uint64_t gate_stride = row_h * ffn, down_stride = row_f * dim;
    if (a->gate.len < a->n_experts * gate_stride) return DS5O_SHAPE_MISMATCH;
    if (a->up.len < a->n_experts * gate_stride) return DS5O_SHAPE_MISMATCH;
    if (a->down.len < a->n_experts * down_stride) return DS5O_SHAPE_MISMATCH;

    float* h = (float*)malloc((ffn ? ffn : 1) * sizeof(float));
    if (!h) return DS5O_OUT_OF_MEMORY;
    const float* x = (const float*)view(a->x);
    float* out = (float*)view(a->out);
    const uint8_t* gate = (const uint8_t*)view(a->gate);
    const uint8_t* up = (const uint8_t*)view(a->up);
    const uint8_t* down = (const uint8_t*)view(a->down);
    for (uint64_t p = 0; p < a->n_pairs; p++) {
        const ds5o_pair pr = a->pairs[p];
        if (pr.token >= T || pr.expert >= a->n_experts) {
            free(h);
            return DS5O_SHAPE_MISMATCH;
        }
        const float* xr = x + (uint64_t)pr.token * dim;
        const uint8_t* g = gate + (uint64_t)pr.expert * gate_stride;
        const uint8_t* u = up + (uint64_t)pr.expert * gate_stride;
        const uint8_t* d = down + (uint64_t)pr.expert * down_stride;
        for (uint64_t j = 0; j < ffn; j++) {
            const float gv = dot_row(xr, g + j * row_h, a->w_dtype, dim);
            const float uv = dot_row(xr, u + j * row_h, a->w_dtype, dim);
            h[j] = gv / (1.0f + expf(-gv)) * uv;
        }
        float* orow = out + (uint64_t)pr.token * dim;
        for (uint64_t i = 0; i < dim; i++) orow[i] += pr.weight * dot_row(h, d + i * row_f, a->w_dtype, ffn);
    }
    free(h);
    return DS5O_OK;
}

/* ------------------------------------------------------------------------ */
/* add -- kernels_a.zig:223-233: the three sizes in order, then out = x + y   */
/* ------------------------------------------------------------------------ */

int ds5o_add(const ds5o_add_args* a) {
    const uint64_t n = a->n_elems;
    if (a->x.len < n * 4) return DS5O_SHAPE_MISMATCH;
    if (a->y.len < n * 4) return DS5O_SHAPE_MISMATCH;
    if (a->out.len < n * 4) return DS5O_SHAPE_MISMATCH;
    const float* x = (const float*)view(a->x);
    const float* y = (const float*)view(a->y);
    float* out = (float*)view(a->out);
    for (uint64_t i = 0; i < n; i++) out[i] = x[i] + y[i]; /* element i read before written */
    return DS5O_OK;
}

/* ------------------------------------------------------------------------ */
/* rmsNorm -- kernels_a.zig:68-91                                            */
/* ------------------------------------------------------------------------ */

int ds5o_rms_norm(const ds5o_rms_norm_args* a) {
    const uint64_t n_rows = a->n_rows, dim = a->dim;
    if (dim == 0) return DS5O_SHAPE_MISMATCH;
    if (a->x.len < n_rows * dim * 4) return DS5O_SHAPE_MISMATCH;
    if (a->out.len < n_rows * dim * 4) return DS5O_SHAPE_MISMATCH;
    if (a->weight.len < dim * 4) return DS5O_SHAPE_MISMATCH;

    const float* x = (const float*)view(a->x);
    const float* w = (const float*)view(a->weight);
    float* out = (float*)view(a->out);
    for (uint64_t r = 0; r < n_rows; r++) {
        const float* xr = x + r * dim;
        float* orow = out + r * dim;
        float sumsq = 0.0f;
        for (uint64_t i = 0; i < dim; i++) sumsq += xr[i] * xr[i];
        const float inv = 1.0f / sqrtf(sumsq / (float)dim + a->eps);
        /* alias-safe when out == x: element i is read before it is written */
        for (uint64_t i = 0; i < dim; i++) orow[i] = xr[i] * inv * w[i];
    }
    return DS5O_OK;
}

/* ------------------------------------------------------------------------ */
/* rmsNorm, the reference GPU kernel's order -- kernels_a.metal:127-165       */
/* (rmsnorm_f32, RMSNORM_TG = 256 threads per row): thread t accumulates      */
/* s = fma(x[i], x[i], s) over i = t, t + 256, ...; partial[t] += partial[t + */
/* stride] for stride = 128 .. 1; inv = 1 / sqrt(partial[0] / dim + eps);    */
/* out[i] = x[i] * inv * w[i]. The same preconditions as ds5o_rms_norm.       */
/* ------------------------------------------------------------------------ */

int ds5o_rms_norm_tree(const ds5o_rms_norm_args* a) {
    enum { TG = 256 };
    const uint64_t n_rows = a->n_rows, dim = a->dim;
    if (dim == 0) return DS5O_SHAPE_MISMATCH;
    if (a->x.len < n_rows * dim * 4) return DS5O_SHAPE_MISMATCH;
    if (a->out.len < n_rows * dim * 4) return DS5O_SHAPE_MISMATCH;
    if (a->weight.len < dim * 4) return DS5O_SHAPE_MISMATCH;

    const float* x = (const float*)view(a->x);
    const float* w = (const float*)view(a->weight);
    float* out = (float*)view(a->out);
    float partial[TG];
    for (uint64_t r = 0; r < n_rows; r++) {
        const float* xr = x + r * dim;
        float* orow = out + r * dim;
        for (uint64_t t = 0; t < TG; t++) {
            float s = 0.0f;
            for (uint64_t i = t; i < dim; i += TG) s = fmaf(xr[i], xr[i], s);
            partial[t] = s;
        }
        for (uint64_t stride = TG / 2; stride > 0; stride >>= 1)
            for (uint64_t t = 0; t < stride; t++) partial[t] += partial[t + stride];
        const float inv = 1.0f / sqrtf(partial[0] / (float)dim + a->eps);
        for (uint64_t i = 0; i < dim; i++) orow[i] = xr[i] * inv * w[i];
    }
    return DS5O_OK;
}

/* ------------------------------------------------------------------------ */
/* rope -- kernels_a.zig:97-130 (NeoX pairing i <-> i + head_dim/2)          */
/* ------------------------------------------------------------------------ */

int ds5o_rope(const ds5o_rope_args* a) {
    const uint64_t n_tokens = a->n_tokens, n_heads = a->n_heads, head_dim = a->head_dim;
    if (head_dim == 0 || head_dim % 2 != 0) return DS5O_SHAPE_MISMATCH;
    if (a->x.len < n_tokens * n_heads * head_dim * 4) return DS5O_SHAPE_MISMATCH;
    if (a->positions.len < n_tokens * 4) return DS5O_SHAPE_MISMATCH;

    const uint64_t half = head_dim / 2;
    float* x = (float*)view(a->x);
    const int32_t* positions = (const int32_t*)view(a->positions);
    for (uint64_t t = 0; t < n_tokens; t++) {
        const float pos = (float)positions[t];
        for (uint64_t h = 0; h < n_heads; h++) {
            float* head = x + (t * n_heads + h) * head_dim;
            for (uint64_t i = 0; i < half; i++) {
                const float expnt = (float)(2 * i) / (float)head_dim;
                const float angle = pos * a->freq_scale * ds5o_zig_powf(a->theta, -expnt);
                const float c = cosf(angle);
                const float s = sinf(angle);
                const float x0 = head[i];
                const float x1 = head[i + half];
                head[i] = x0 * c - x1 * s;
                head[i + half] = x0 * s + x1 * c;
            }
        }
    }
    return DS5O_OK;
}

/* ------------------------------------------------------------------------ */
/* kvAppend -- kernels_a.zig:169-217                                         */
/* ------------------------------------------------------------------------ */

int ds5o_kv_append(const ds5o_kv_append_args* a) {
    const uint64_t n_tokens = a->n_tokens, n_kv_heads = a->n_kv_heads;
    const uint64_t head_dim = a->head_dim, max_ctx = a->max_ctx;
    if (head_dim == 0 || n_kv_heads == 0) return DS5O_SHAPE_MISMATCH;
    if ((uint64_t)a->pos + a->n_tokens > a->max_ctx) return DS5O_SHAPE_MISMATCH;

    const uint64_t new_bytes = n_tokens * n_kv_heads * head_dim * 4;
    if (a->k_new.len < new_bytes || a->v_new.len < new_bytes) return DS5O_SHAPE_MISMATCH;

    uint64_t cache_bytes;
    if (a->kv_dtype == DS5O_F32)
        cache_bytes = n_kv_heads * max_ctx * head_dim * 4;
    else if (a->kv_dtype == DS5O_F16)
        cache_bytes = n_kv_heads * max_ctx * head_dim * 2;
    else
        return DS5O_UNSUPPORTED_DTYPE;
    if (a->k_cache.len < cache_bytes || a->v_cache.len < cache_bytes) return DS5O_SHAPE_MISMATCH;

    const float* k_new = (const float*)view(a->k_new);
    const float* v_new = (const float*)view(a->v_new);
    for (uint64_t t = 0; t < n_tokens; t++) {
        for (uint64_t h = 0; h < n_kv_heads; h++) {
            const uint64_t src = (t * n_kv_heads + h) * head_dim;
            const uint64_t dst = (h * max_ctx + (a->pos + t)) * head_dim;
            if (a->kv_dtype == DS5O_F32) {
                memcpy((float*)view(a->k_cache) + dst, k_new + src, head_dim * 4);
                memcpy((float*)view(a->v_cache) + dst, v_new + src, head_dim * 4);
            } else {
                uint16_t* kc = (uint16_t*)view(a->k_cache);
                uint16_t* vc = (uint16_t*)view(a->v_cache);
                for (uint64_t d = 0; d < head_dim; d++) {
                    kc[dst + d] = ds5o_f32_to_f16(k_new[src + d]);
                    vc[dst + d] = ds5o_f32_to_f16(v_new[src + d]);
                }
            }
        }
    }
    return DS5O_OK;
}

/* ------------------------------------------------------------------------ */
/* gqaAttention -- kernels_b.zig:29-133 (f32 branch :68-95, f16 :96-127)     */
/* ------------------------------------------------------------------------ */

int ds5o_gqa_attention(const ds5o_attn_args* a) {
    const uint64_t hq = a->n_q_heads, hkv = a->n_kv_heads, hd = a->head_dim;
    const uint64_t n_tokens = a->n_tokens, pos = a->pos, max_ctx = a->max_ctx;

    if (hq == 0 || hkv == 0 || hd == 0) return DS5O_SHAPE_MISMATCH;
    if (hq % hkv != 0) return DS5O_SHAPE_MISMATCH;
    if (pos + n_tokens > max_ctx) return DS5O_SHAPE_MISMATCH;

    const uint64_t q_bytes = n_tokens * hq * hd * 4;
    if (a->q.len < q_bytes || a->out.len < q_bytes) return DS5O_SHAPE_MISMATCH;

    uint64_t cache_bytes;
    if (a->kv_dtype == DS5O_F32)
        cache_bytes = hkv * max_ctx * hd * 4;
    else if (a->kv_dtype == DS5O_F16)
        cache_bytes = hkv * max_ctx * hd * 2;
    else
        return DS5O_UNSUPPORTED_DTYPE;
    if (a->k_cache.len < cache_bytes || a->v_cache.len < cache_bytes) return DS5O_SHAPE_MISMATCH;

    const uint64_t group = hq / hkv;
    const float* q = (const float*)view(a->q);
    float* out = (float*)view(a->out);

    float* scores = (float*)malloc(sizeof(float) * (pos + n_tokens));
    if (!scores) return DS5O_OUT_OF_MEMORY;

    for (uint64_t t = 0; t < n_tokens; t++) {
        const uint64_t ctx_len = pos + t + 1;
        for (uint64_t h = 0; h < hq; h++) {
            const uint64_t kh = h / group;
            const float* qr = q + (t * hq + h) * hd;
            float* out_row = out + t * hq * hd + h * hd;
            float row_max = -INFINITY;
            if (a->kv_dtype == DS5O_F32) {
                const float* k_head = (const float*)view(a->k_cache) + kh * max_ctx * hd;
                const float* v_head = (const float*)view(a->v_cache) + kh * max_ctx * hd;
                for (uint64_t p = 0; p < ctx_len; p++) {
                    float acc = 0.0f;
                    for (uint64_t d = 0; d < hd; d++) acc += qr[d] * k_head[p * hd + d];
                    const float s = acc * a->scale;
                    scores[p] = s;
                    row_max = fmaxf(row_max, s);
                }
                float sum = 0.0f;
                for (uint64_t p = 0; p < ctx_len; p++) {
                    scores[p] = expf(scores[p] - row_max);
                    sum += scores[p];
                }
                const float inv_sum = 1.0f / sum;
                memset(out_row, 0, hd * 4);
                for (uint64_t p = 0; p < ctx_len; p++) {
                    const float w = scores[p] * inv_sum;
                    for (uint64_t d = 0; d < hd; d++) out_row[d] += w * v_head[p * hd + d];
                }
            } else {
                const uint16_t* k_head = (const uint16_t*)view(a->k_cache) + kh * max_ctx * hd;
                const uint16_t* v_head = (const uint16_t*)view(a->v_cache) + kh * max_ctx * hd;
                for (uint64_t p = 0; p < ctx_len; p++) {
                    float acc = 0.0f;
                    for (uint64_t d = 0; d < hd; d++) acc += qr[d] * ds5o_f16_to_f32(k_head[p * hd + d]);
                    const float s = acc * a->scale;
                    scores[p] = s;
                    row_max = fmaxf(row_max, s);
                }
                float sum = 0.0f;
                for (uint64_t p = 0; p < ctx_len; p++) {
                    scores[p] = expf(scores[p] - row_max);
                    sum += scores[p];
                }
                const float inv_sum = 1.0f / sum;
                memset(out_row, 0, hd * 4);
                for (uint64_t p = 0; p < ctx_len; p++) {
                    const float w = scores[p] * inv_sum;
                    for (uint64_t d = 0; d < hd; d++) out_row[d] += w * ds5o_f16_to_f32(v_head[p * hd + d]);
                }
            }
        }
    }
    free(scores);
    return DS5O_OK;
}

/* ------------------------------------------------------------------------ */
/* Paged KV: defined by reduction to the contiguous layout.                  */
/* ------------------------------------------------------------------------ */

int64_t ds5o_paged_slot(const int32_t* page_table, uint32_t n_table, uint32_t page_size, uint32_t p) {
    const uint32_t page = p / page_size;
    if (page_size == 0 || page >= n_table || page_table[page] < 0) return -1;
    return (int64_t)page_table[page] * page_size + p % page_size;
}

int ds5o_paged_gather_f16(const uint16_t* pool, uint64_t pool_slots, const int32_t* page_table,
                          uint32_t n_table, uint32_t page_size, uint32_t len, uint32_t n_kv_heads,
                          uint32_t head_dim, uint16_t* out) {
    for (uint32_t p = 0; p < len; p++) {
        const int64_t slot = ds5o_paged_slot(page_table, n_table, page_size, p);
        if (slot < 0 || (uint64_t)slot >= pool_slots) return DS5O_SHAPE_MISMATCH;
        for (uint32_t h = 0; h < n_kv_heads; h++) {
            memcpy(out + ((uint64_t)h * len + p) * head_dim,
                   pool + ((uint64_t)h * pool_slots + (uint64_t)slot) * head_dim, (size_t)head_dim * 2);
        }
    }
    return DS5O_OK;
}

/* ------------------------------------------------------------------------ */
/* One engine step of the path, in forward.zig:345-412 order.                */
/* ------------------------------------------------------------------------ */

int ds5o_attention_step(const ds5o_step_args* a) {
    int rc;
    const ds5o_rms_norm_args qn = {a->q, a->q_norm_w, a->q, a->n_tokens * a->n_q_heads, a->head_dim, a->eps};
    if ((rc = ds5o_rms_norm(&qn))) return rc;
    const ds5o_rms_norm_args kn = {a->k, a->k_norm_w, a->k, a->n_tokens * a->n_kv_heads, a->head_dim, a->eps};
    if ((rc = ds5o_rms_norm(&kn))) return rc;
    const ds5o_rope_args rq = {a->q, a->positions, a->n_tokens, a->n_q_heads, a->head_dim, a->theta, a->freq_scale};
    if ((rc = ds5o_rope(&rq))) return rc;
    const ds5o_rope_args rk = {a->k, a->positions, a->n_tokens, a->n_kv_heads, a->head_dim, a->theta, a->freq_scale};
    if ((rc = ds5o_rope(&rk))) return rc;
    const ds5o_kv_append_args ap = {a->k, a->v, a->k_cache, a->v_cache, a->kv_dtype,
                                    a->pos, a->n_tokens, a->n_kv_heads, a->head_dim, a->max_ctx};
    if ((rc = ds5o_kv_append(&ap))) return rc;
    const ds5o_attn_args at = {a->q, a->k_cache, a->v_cache, a->kv_dtype, a->out, a->pos, a->n_tokens,
                               a->n_q_heads, a->n_kv_heads, a->head_dim, a->max_ctx, a->scale};
    return ds5o_gqa_attention(&at);
}
