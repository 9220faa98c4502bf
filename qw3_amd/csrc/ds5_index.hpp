// ds5_index.hpp -- the per-lane address arithmetic of the hot kernels, as
// __host__ __device__ functions: the kernels call them, and the library
// exports host wrappers (ds5_index_*, ds5_index.hip) through which the CPU
// tests enumerate every access of a launch. A change here changes both.
//
//   decode_split_kernel (k_decode.hip): the rows and columns of a tile's K and V
//     loads (issue_tile), the page-table slot of a paged position (page_base), and
//     the arithmetic of the paged plan (paged_plan);
//   matmul_q8_mfma_kernel (k_matmul.hip): the lane offsets of the direct-to-LDS
//     x-plane and raw Q8_0 row loads;
//   prefill_attention_kernel (k_prefill.hip): the lane offsets of a K/V tile's
//     direct-to-LDS loads and their clamp, and the staged q and output rows.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#endif

#if defined(__HIPCC__)
#define DS5_HD __host__ __device__ __forceinline__
#define DS5_HDC __host__ __device__ constexpr
#else
#define DS5_HD inline
#define DS5_HDC constexpr
#endif

namespace ds5idx {

DS5_HD uint32_t umin(uint32_t a, uint32_t b) { return a < b ? a : b; }
DS5_HD uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

// decode_split_kernel's shape: 32-position tiles, four wavefronts (one per SIMD),
// up to 16 q heads of one kv head per workgroup, at most 64 splits per sequence.
constexpr int kDecTile = 32, kDecWaves = 4, kDecHeads = 16;
constexpr uint32_t kDecMaxSplits = 64;
// prefill_attention_kernel's shape: 4 q heads per workgroup, 32-row q tiles,
// 64-key K/V tiles; LDS row strides of K and V (bytes), padded for conflict-free reads.
constexpr int kPfHeads = 4, kPfQRows = 32, kPfKTile = 64;
DS5_HDC int pf_rsk(int D) { return 2 * D + 16; }
DS5_HDC int pf_rsv(int D) { return 2 * D + 64; }

// Split-K geometry of a contiguous decode launch: positions per split (a multiple
// of 128, at least max_len / 64; about four workgroups per CU unless decode_chunk
// fixes it) and the split count.
DS5_HD void dec_geometry(uint32_t cu_count, uint32_t decode_chunk, uint32_t n_seqs, uint32_t n_kv_heads,
                         uint32_t n_sub, uint32_t max_len, uint32_t& chunk, uint32_t& n_splits) {
    const uint32_t step = kDecWaves * kDecTile;
    chunk = decode_chunk;
    if (chunk == 0) {
        const uint64_t units = (uint64_t)n_seqs * n_kv_heads * n_sub;
        const uint64_t target = 4ull * (cu_count > 0 ? cu_count : 256);
        const uint64_t c = (max_len * units + target - 1) / target;
        chunk = (uint32_t)(c < max_len ? c : max_len);
    }
    chunk = umax((chunk + step - 1) / step * step, step);
    chunk = umax(chunk, (max_len + kDecMaxSplits - 1) / kDecMaxSplits);
    chunk = (chunk + step - 1) / step * step;
    n_splits = (max_len + chunk - 1) / chunk;
}

// ---------------------------------------------------------------------------
// decode_split_kernel: a 32-position tile [p0, p0 + 32) of a split ending at `end`.
// K: lane (g = lane / 16, c16 = lane % 16), half st, k-step kk reads 8 halves
//    (16 bytes) of row dec_k_row at column dec_k_col.
// V: 16-byte chunk c = lane + 64 r (r < VC) reads row dec_v_row (tile row
//    tr = c / RC, RC = head_dim / 8 chunks per row) at column dec_v_col.
// Contiguous cache: rows past `end` are clamped to end - 1. Paged: each
// 16-position half sits inside one page (page_size % 16 == 0, p0 % 32 == 0);
// rowA / rowB are the pool slots of the halves' first positions.
// ---------------------------------------------------------------------------
DS5_HD uint32_t dec_half_pos(uint32_t p0, uint32_t end, int st) { return st ? umin(p0 + 16, end - 1) : p0; }
DS5_HD uint64_t dec_k_row(uint32_t p0, uint32_t end, int st, int c16) {
    return umin(p0 + 16 * (uint32_t)st + (uint32_t)c16, end - 1);
}
DS5_HD uint64_t dec_v_row(uint32_t p0, uint32_t end, int tr) { return umin(p0 + (uint32_t)tr, end - 1); }
DS5_HD uint64_t dec_k_row_paged(uint64_t rowA, uint64_t rowB, int st, int c16) { return (st ? rowB : rowA) + c16; }
DS5_HD uint64_t dec_v_row_paged(uint64_t rowA, uint64_t rowB, int r, int VC, int tr) {
    return (r < VC / 2 ? rowA : rowB) + (tr & 15);
}
DS5_HD uint32_t dec_k_col(int kk, int g) { return (uint32_t)(kk * 32 + 8 * g); }
DS5_HD uint32_t dec_v_col(int c, int RC) { return (uint32_t)((c % RC) * 8); }
// Page-table entry of sequence b for position pos, and the first pool slot of
// the page it names (a position's slot adds pos % page_size). An entry outside
// [0, n_pages) reads page 0 and raises `bad`.
DS5_HD uint64_t dec_page_index(uint32_t b, uint32_t max_pages, uint32_t pos, uint32_t page_size) {
    return (uint64_t)b * max_pages + pos / page_size;
}
DS5_HD uint64_t dec_page_first(int32_t entry, uint32_t n_pages, uint32_t page_size, bool& bad) {
    const bool ok = (uint32_t)entry < n_pages;
    bad |= !ok;
    return (uint64_t)(ok ? entry : 0) * page_size;
}

// Paged plan: a length outside [1, max_len] is poisoned (0, one item); the chunk
// is the smallest multiple of `step` in [plan_cmin, plan_cmax] whose item count
// sum_b plan_items(L_b, c) fits the cap. Items: every sequence's whole chunks
// first, then the partial last chunks (and the poisoned sequences).
DS5_HD uint32_t plan_len(int32_t len, uint32_t max_len) {
    return (len < 1 || (uint32_t)len > max_len) ? 0u : (uint32_t)len;
}
DS5_HD uint32_t plan_items(uint32_t len, uint32_t c) { return len == 0 ? 1u : (len + c - 1) / c; }
DS5_HD uint32_t plan_cmax(uint32_t max_len, uint32_t step) { return (max_len + step - 1) / step * step; }
DS5_HD uint32_t plan_cmin(uint32_t max_len, uint32_t step, uint32_t max_splits) {
    return umax(step, (max_len + max_splits - 1) / max_splits + step - 1) / step * step;
}
DS5_HD uint32_t plan_whole(uint32_t len, uint32_t chunk) { return len / chunk; }
DS5_HD uint32_t plan_partial(uint32_t len, uint32_t chunk) { return (len == 0 || len % chunk != 0) ? 1u : 0u; }

// ---------------------------------------------------------------------------
// matmul_q8_mfma_kernel: block b's direct-to-LDS loads.
// x: load i of wavefront `wave` fills stage bytes o = 1024 (wave + W i) + 16 lane;
//    its plane byte offset (block 0) is row min(m0 + r, m - 1), swizzled chunk c.
// raw q: dword d = min(64 i + lane, 9 * rows - 1) of the wavefront's area is dword
//    d % 9 of local row d / 9 = tile row 16 wave + (threads / 4) (lr / 16) + lr % 16;
//    the offsets from the block's scalar base (w + 34 b, or w + 34 b - 2 for odd b).
// ---------------------------------------------------------------------------
DS5_HD uint32_t gemm_x_tile_row(uint32_t o, uint32_t BM) { return (o % (BM * 64)) / 64; }
// the offset of tile row r's swizzled chunk in plane row `row`
DS5_HD uint32_t gemm_x_off_row(uint32_t r, uint32_t lane, uint32_t row, uint32_t k) {
    return row * k * 2 + 16 * ((lane & 3) ^ ((r >> 2) & 3));
}
DS5_HD uint32_t gemm_x_off(uint32_t o, uint32_t lane, uint32_t BM, uint32_t m0, uint32_t m, uint32_t k) {
    const uint32_t r = gemm_x_tile_row(o, BM);
    return gemm_x_off_row(r, lane, umin(m0 + r, m - 1), k);
}
DS5_HD uint32_t gemm_q_row(uint32_t d, uint32_t wave, uint32_t threads, uint32_t row_dw) {
    const uint32_t lr = d / row_dw;
    return 16 * wave + (threads / 4) * (lr / 16) + lr % 16;
}
DS5_HD uint32_t gemm_q_dword(uint32_t i, uint32_t lane, uint32_t w_rows, uint32_t row_dw) {
    return umin(64u * i + lane, w_rows * row_dw - 1);
}
DS5_HD void gemm_q_off(uint32_t d, uint32_t row, uint32_t n0, uint32_t n, uint32_t row_bytes, uint32_t row_dw,
                       uint32_t& even, uint32_t& odd) {
    const uint32_t rb = umin(n0 + row, n - 1) * row_bytes;
    even = (rb & ~3u) + 4 * (d % row_dw);
    odd = ((rb + 2) & ~3u) + 4 * (d % row_dw);
}

// ---------------------------------------------------------------------------
// prefill_attention_kernel: a K (or V) tile's direct-to-LDS loads fill one stage
// of 64 rows at row stride RS bytes; load b's lane covers stage bytes
// 1024 b + 16 lane: row r, chunk slot c (a padding slot re-reads the row's first
// chunk). pf_tile_off is that lane's byte offset from the tile's first key row
// (row bytes 2 D); on a tile that reaches past kv_end, rows at or past it are
// clamped to kv_end - 1 (pf_clamped_off).
// ---------------------------------------------------------------------------
DS5_HD uint32_t pf_tile_off(int b, int lane, int D, int RS) {
    const int pos = 1024 * b + 16 * lane;
    const int r = pos / RS, c = (pos % RS) / 16;
    return (uint32_t)(r * 2 * D + (c < D / 8 ? 16 * c : 0));
}
DS5_HD uint32_t pf_clamped_off(uint32_t off, uint32_t key0, uint32_t kv_end, int D) {
    const uint32_t last_row = kv_end - key0 - 1;
    return umin(off / (2 * D), last_row) * (2 * D) + off % (2 * D);
}
// A q tile's row `row` (< 32) reads token min(q0 + row, n_tokens - 1).
DS5_HD uint32_t pf_q_token(uint32_t q0, uint32_t row, uint32_t n_tokens) { return umin(q0 + row, n_tokens - 1); }

}  // namespace ds5idx
