/* ds5_index.h -- host exports of the gfx950 kernels' address arithmetic.
 *
 * No reference counterpart: these are test hooks. The kernels compute their
 * load and store addresses with the __host__ __device__ helpers of
 * qw3_amd/csrc/ds5_index.hpp; these functions run the same helpers on the host,
 * so the CPU tests (tests/test_address_ranges.py) enumerate every access of a
 * launch with the kernels' own arithmetic. Nothing here touches the device. */
#ifndef DS5_INDEX_H
#define DS5_INDEX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* decode_split_kernel: out = [tile, waves, heads, max_splits];
 * prefill_attention_kernel: out = [heads, q_rows, key_tile]. */
void ds5_index_decode_shape(uint32_t* out);
void ds5_index_prefill_shape(uint32_t* out);

/* Split-K geometry of a contiguous decode launch (chunk positions per split). */
void ds5_index_decode_geometry(uint32_t cu_count, uint32_t decode_chunk, uint32_t n_seqs, uint32_t n_kv_heads,
                               uint32_t n_sub, uint32_t max_len, uint32_t* chunk, uint32_t* n_splits);

/* The K and V loads of one decode tile in issue order: K [2][head_dim/32][64]
 * and V [head_dim/16][64] rows (positions, or pool slots when paged) and f16
 * columns (8 elements per load). */
void ds5_index_decode_tile(uint32_t p0, uint32_t end, uint32_t head_dim, int paged, uint64_t row_a, uint64_t row_b,
                           uint64_t* k_rows, uint32_t* k_cols, uint64_t* v_rows, uint32_t* v_cols);
uint32_t ds5_index_half_pos(uint32_t p0, uint32_t end, int st);
uint64_t ds5_index_page_index(uint32_t b, uint32_t max_pages, uint32_t pos, uint32_t page_size);
uint64_t ds5_index_page_first(int32_t entry, uint32_t n_pages, uint32_t page_size, int* bad);

/* Paged plan arithmetic. */
void ds5_index_plan_bounds(uint32_t max_len, uint32_t* cmin, uint32_t* cmax);
uint32_t ds5_index_plan_len(int32_t len, uint32_t max_len);
uint32_t ds5_index_plan_items(uint32_t len, uint32_t chunk);
uint32_t ds5_index_plan_whole(uint32_t len, uint32_t chunk);
uint32_t ds5_index_plan_partial(uint32_t len, uint32_t chunk);

/* matmul_q8_mfma_kernel: a wavefront's x-plane offsets [nx][64] and raw-q dword
 * index, tile row and even/odd-block offsets [nq][64]. */
void ds5_index_gemm_x(uint32_t wave, uint32_t W, uint32_t nx, uint32_t BM, uint32_t m0, uint32_t m, uint32_t k,
                      uint32_t* x_off);
/* The grouped MoE form: tile row r reads plane row x_rows[min(m0 + r, m - 1)]. */
void ds5_index_gemm_x_rows(uint32_t wave, uint32_t W, uint32_t nx, uint32_t BM, uint32_t m0, uint32_t m, uint32_t k,
                           const uint32_t* x_rows, uint32_t* x_off);
void ds5_index_gemm_q(uint32_t wave, uint32_t threads, uint32_t nq, uint32_t w_rows, uint32_t row_dw, uint32_t n0,
                      uint32_t n, uint32_t row_bytes, uint32_t* q_dw, uint32_t* q_row, uint32_t* q_even,
                      uint32_t* q_odd);

/* prefill_attention_kernel: byte offsets [loads][64] of a K (v = 0) or V tile's
 * direct-to-LDS loads from key0 (clamped past kv_end); returns the load count.
 * A q tile row's token. */
uint32_t ds5_index_prefill_tile(uint32_t head_dim, int v, uint32_t key0, uint32_t kv_end, uint32_t* off);
uint32_t ds5_index_pf_q_token(uint32_t q0, uint32_t row, uint32_t n_tokens);

#ifdef __cplusplus
}
#endif

#endif /* DS5_INDEX_H */
