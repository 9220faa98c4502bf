// k_generic.hip -- causal GQA attention for every shape the MFMA kernels do
// not take: f32 caches, head_dim other than 64/128, misaligned views.
//
// Semantics are those of kernels_b.zig:29-133: query token t (absolute
// position pos + t) of q head h attends cache positions 0..pos+t of kv head
// h / (n_q_heads / n_kv_heads); scores = scale * (q . k), softmax in f32 with
// max subtraction, out = sum_p softmax_p * v_p. One workgroup per (t, h)
// streams the positions in 256-wide blocks with an online softmax (the exact
// softmax, reassociated).
#include "ds5_common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxDim = 512;

__device__ float block_reduce_max(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < kThreads / 64; w++) m = fmaxf(m, red[w]);
    return m;
}

__device__ float block_reduce_sum(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int w = 0; w < kThreads / 64; w++) s += red[w];
    return s;
}

template <typename T>
__device__ inline float ld(const T* p, uint64_t i) {
    return (float)p[i];
}

template <typename T>
__global__ __launch_bounds__(kThreads) void generic_attention_kernel(GenericAttnLaunch a) {
    __shared__ float s_q[kMaxDim];
    __shared__ float s_p[kThreads];
    __shared__ float red[kThreads / 64];
    const uint32_t t = blockIdx.x, h = blockIdx.y;
    const uint32_t hd = a.head_dim, hq = a.n_q_heads;
    const uint32_t kh = h / (hq / a.n_kv_heads);
    const uint64_t ctx_len = (uint64_t)a.pos + t + 1;
    const T* kc = (const T*)a.k_cache + (uint64_t)kh * a.max_ctx * hd;
    const T* vc = (const T*)a.v_cache + (uint64_t)kh * a.max_ctx * hd;
    const float* q = a.q + ((uint64_t)t * hq + h) * hd;
    for (uint32_t d = threadIdx.x; d < hd; d += kThreads) s_q[d] = q[d];
    __syncthreads();

    float o[kMaxDim / kThreads] = {};
    float m = -INFINITY, l = 0.0f;
    for (uint64_t base = 0; base < ctx_len; base += kThreads) {
        const uint64_t p = base + threadIdx.x;
        float s = -INFINITY;
        if (p < ctx_len) {
            float acc = 0.0f;
            for (uint32_t d = 0; d < hd; d++) acc += s_q[d] * ld(kc, p * hd + d);
            s = acc * a.scale;
        }
        const float m_new = fmaxf(m, block_reduce_max(s, red));
        const float alpha = expf(m - m_new);
        const float pr = (p < ctx_len) ? expf(s - m_new) : 0.0f;
        s_p[threadIdx.x] = pr;
        l = l * alpha + block_reduce_sum(pr, red);
        m = m_new;
        const uint32_t n = (uint32_t)min<uint64_t>(kThreads, ctx_len - base);
        for (uint32_t k = 0; k < (hd + kThreads - 1) / kThreads; k++) {
            const uint32_t d = threadIdx.x + k * kThreads;
            if (d >= hd) break;
            float acc = o[k] * alpha;
            for (uint32_t j = 0; j < n; j++) acc += s_p[j] * ld(vc, (base + j) * hd + d);
            o[k] = acc;
        }
        __syncthreads();
    }
    float* out = a.out + (uint64_t)t * hq * hd + (uint64_t)h * hd;
    for (uint32_t k = 0; k < (hd + kThreads - 1) / kThreads; k++) {
        const uint32_t d = threadIdx.x + k * kThreads;
        if (d < hd) out[d] = o[k] / l;
    }
}

}  // namespace

int launch_generic_attention(ds5_hip_ctx* ctx, const GenericAttnLaunch& a) {
    if (a.n_tokens == 0) return DS5_OK;
    const dim3 grid(a.n_tokens, a.n_q_heads);
    if (a.kv_dtype == DS5_DTYPE_F16)
        DS5_TIMED_LAUNCH(ctx, "generic_attention_kernel", generic_attention_kernel<f16>, grid, dim3(kThreads), 0, ctx->stream, a);
    else
        DS5_TIMED_LAUNCH(ctx, "generic_attention_kernel", generic_attention_kernel<float>, grid, dim3(kThreads), 0, ctx->stream, a);
    return ds5_after_launch(ctx, "generic_attention_kernel");
}
