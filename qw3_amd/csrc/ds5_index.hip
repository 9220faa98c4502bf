// ds5_index.hip -- host exports of the kernels' address arithmetic
// (ds5_index.hpp), for the CPU tests that enumerate every access of a launch.
// No reference counterpart; nothing here touches the device.
#include <stdint.h>

#include "ds5_index.hpp"
#include "ds5_index.h"

extern "C" {

// [tile, waves, heads, max_splits] of the decode kernel; [heads, q_rows, key_tile]
// of the prefill kernel.
void ds5_index_decode_shape(uint32_t* out) {
    out[0] = ds5idx::kDecTile;
    out[1] = ds5idx::kDecWaves;
    out[2] = ds5idx::kDecHeads;
    out[3] = ds5idx::kDecMaxSplits;
}
void ds5_index_prefill_shape(uint32_t* out) {
    out[0] = ds5idx::kPfHeads;
    out[1] = ds5idx::kPfQRows;
    out[2] = ds5idx::kPfKTile;
}

void ds5_index_decode_geometry(uint32_t cu_count, uint32_t decode_chunk, uint32_t n_seqs, uint32_t n_kv_heads,
                               uint32_t n_sub, uint32_t max_len, uint32_t* chunk, uint32_t* n_splits) {
    ds5idx::dec_geometry(cu_count, decode_chunk, n_seqs, n_kv_heads, n_sub, max_len, *chunk, *n_splits);
}

// The K and V loads of one decode tile, in the kernel's issue order: K half st,
// k-step kk, lane l -> k_rows/k_cols[(st * KK + kk) * 64 + l] (KK = head_dim / 32);
// V chunk r, lane l -> v_rows/v_cols[r * 64 + l] (VC = 32 * head_dim / 8 / 64). Rows
// are cache positions (contiguous) or pool slots (paged: row_a / row_b are the
// halves' first slots); columns are f16 elements, each load 8 of them.
void ds5_index_decode_tile(uint32_t p0, uint32_t end, uint32_t head_dim, int paged, uint64_t row_a, uint64_t row_b,
                           uint64_t* k_rows, uint32_t* k_cols, uint64_t* v_rows, uint32_t* v_cols) {
    const int KK = (int)head_dim / 32, RC = (int)head_dim / 8, VC = ds5idx::kDecTile * RC / 64;
    for (int st = 0; st < 2; st++)
        for (int kk = 0; kk < KK; kk++)
            for (int lane = 0; lane < 64; lane++) {
                const int g = lane >> 4, c16 = lane & 15, i = (st * KK + kk) * 64 + lane;
                k_rows[i] = paged ? ds5idx::dec_k_row_paged(row_a, row_b, st, c16) : ds5idx::dec_k_row(p0, end, st, c16);
                k_cols[i] = ds5idx::dec_k_col(kk, g);
            }
    for (int r = 0; r < VC; r++)
        for (int lane = 0; lane < 64; lane++) {
            const int c = lane + 64 * r, tr = c / RC, i = r * 64 + lane;
            v_rows[i] = paged ? ds5idx::dec_v_row_paged(row_a, row_b, r, VC, tr) : ds5idx::dec_v_row(p0, end, tr);
            v_cols[i] = ds5idx::dec_v_col(c, RC);
        }
}

// The position whose page holds half st of tile p0; the page-table index of a
// position; the first slot of the page an entry names (bad: entry out of range).
uint32_t ds5_index_half_pos(uint32_t p0, uint32_t end, int st) { return ds5idx::dec_half_pos(p0, end, st); }
uint64_t ds5_index_page_index(uint32_t b, uint32_t max_pages, uint32_t pos, uint32_t page_size) {
    return ds5idx::dec_page_index(b, max_pages, pos, page_size);
}
uint64_t ds5_index_page_first(int32_t entry, uint32_t n_pages, uint32_t page_size, int* bad) {
    bool b = false;
    const uint64_t r = ds5idx::dec_page_first(entry, n_pages, page_size, b);
    *bad = b;
    return r;
}

// The paged plan's arithmetic: [cmin, cmax] for max_len, a sequence's staged
// length, and per chunk its item count and whole / partial chunk counts.
void ds5_index_plan_bounds(uint32_t max_len, uint32_t* cmin, uint32_t* cmax) {
    const uint32_t step = ds5idx::kDecWaves * ds5idx::kDecTile;
    *cmin = ds5idx::plan_cmin(max_len, step, ds5idx::kDecMaxSplits);
    *cmax = ds5idx::plan_cmax(max_len, step);
}
uint32_t ds5_index_plan_len(int32_t len, uint32_t max_len) { return ds5idx::plan_len(len, max_len); }
uint32_t ds5_index_plan_items(uint32_t len, uint32_t chunk) { return ds5idx::plan_items(len, chunk); }
uint32_t ds5_index_plan_whole(uint32_t len, uint32_t chunk) { return ds5idx::plan_whole(len, chunk); }
uint32_t ds5_index_plan_partial(uint32_t len, uint32_t chunk) { return ds5idx::plan_partial(len, chunk); }

// GEMM: the x-plane byte offsets (block 0) of wavefront `wave`'s nx loads
// (x_off[i * 64 + lane]), and its nq raw-q loads' dword index, tile row and
// even/odd-block offsets (q_*[i * 64 + lane]).
void ds5_index_gemm_x(uint32_t wave, uint32_t W, uint32_t nx, uint32_t BM, uint32_t m0, uint32_t m, uint32_t k,
                      uint32_t* x_off) {
    for (uint32_t i = 0; i < nx; i++)
        for (uint32_t lane = 0; lane < 64; lane++)
            x_off[i * 64 + lane] = ds5idx::gemm_x_off(1024u * (wave + W * i) + 16u * lane, lane, BM, m0, m, k);
}
// The grouped MoE form: tile row r reads plane row x_rows[min(m0 + r, m - 1)].
void ds5_index_gemm_x_rows(uint32_t wave, uint32_t W, uint32_t nx, uint32_t BM, uint32_t m0, uint32_t m, uint32_t k,
                           const uint32_t* x_rows, uint32_t* x_off) {
    for (uint32_t i = 0; i < nx; i++)
        for (uint32_t lane = 0; lane < 64; lane++) {
            const uint32_t r = ds5idx::gemm_x_tile_row(1024u * (wave + W * i) + 16u * lane, BM);
            x_off[i * 64 + lane] = ds5idx::gemm_x_off_row(r, lane, x_rows[ds5idx::umin(m0 + r, m - 1)], k);
        }
}
void ds5_index_gemm_q(uint32_t wave, uint32_t threads, uint32_t nq, uint32_t w_rows, uint32_t row_dw, uint32_t n0,
                      uint32_t n, uint32_t row_bytes, uint32_t* q_dw, uint32_t* q_row, uint32_t* q_even,
                      uint32_t* q_odd) {
    for (uint32_t i = 0; i < nq; i++)
        for (uint32_t lane = 0; lane < 64; lane++) {
            const uint32_t j = i * 64 + lane;
            q_dw[j] = ds5idx::gemm_q_dword(i, lane, w_rows, row_dw);
            q_row[j] = ds5idx::gemm_q_row(q_dw[j], wave, threads, row_dw);
            ds5idx::gemm_q_off(q_dw[j], q_row[j], n0, n, row_bytes, row_dw, q_even[j], q_odd[j]);
        }
}

// Prefill: the byte offsets (from the tile's first key row) of every lane of
// every 1 KiB load of a K (rs = pf_rsk) or V (rs = pf_rsv) tile starting at key0,
// clamped when the tile reaches past kv_end: off[b * 64 + lane]; returns the load
// count. Also the strides, and a q tile row's token.
uint32_t ds5_index_prefill_tile(uint32_t head_dim, int v, uint32_t key0, uint32_t kv_end, uint32_t* off) {
    const int D = (int)head_dim, RS = v ? ds5idx::pf_rsv(D) : ds5idx::pf_rsk(D);
    const int NB = ds5idx::kPfKTile * RS / 1024;
    const bool whole = key0 + ds5idx::kPfKTile <= kv_end;
    for (int b = 0; b < NB; b++)
        for (int lane = 0; lane < 64; lane++) {
            const uint32_t o = ds5idx::pf_tile_off(b, lane, D, RS);
            off[b * 64 + lane] = whole ? o : ds5idx::pf_clamped_off(o, key0, kv_end, D);
        }
    return (uint32_t)NB;
}
uint32_t ds5_index_pf_q_token(uint32_t q0, uint32_t row, uint32_t n_tokens) {
    return ds5idx::pf_q_token(q0, row, n_tokens);
}

}  // extern "C"
