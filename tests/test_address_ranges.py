"""Every load and store address of the hot kernels, enumerated on the CPU with the
kernels' own index arithmetic (no GPU).

The kernels compute their per-lane offsets and clamps with the __host__ __device__
helpers of qw3_amd/csrc/ds5_index.hpp; libds5hip.so exports host wrappers of the same
helpers (include/ds5_index.h), and these tests call them for every tile, load and lane
of a launch at the BASELINE shapes (C0-C4) and at the Q8_0 shapes whose blocks start 2
bytes off a dword, then assert that every access stays inside its view (and that the
paged plan covers every position exactly once). A change to a helper changes the kernel
and what these tests see alike. A GPU memory fault once came from exactly such
arithmetic (an offset that went negative and wrapped as an unsigned 32-bit value).

What remains written here is the launch structure around the helpers: which tiles a
workgroup's wavefronts issue (k_decode.hip), the grid of the GEMM (k_matmul.hip) and the
items of a prefill workgroup (k_prefill.hip), and the paged plan's cap and item order.
"""
import ctypes as C
import os
import re

import numpy as np
import pytest

from qw3_amd import synth

U32 = 1 << 32
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def ix(hip):
    """The ds5_index_* exports of the built library, typed."""
    lib = hip.LIB
    u32, u64, i32, P = C.c_uint32, C.c_uint64, C.c_int32, C.c_void_p
    sig = {
        "ds5_index_decode_shape": ([P], None), "ds5_index_prefill_shape": ([P], None),
        "ds5_index_decode_geometry": ([u32] * 6 + [P, P], None),
        "ds5_index_decode_tile": ([u32, u32, u32, C.c_int, u64, u64, P, P, P, P], None),
        "ds5_index_half_pos": ([u32, u32, C.c_int], u32), "ds5_index_page_index": ([u32] * 4, u64),
        "ds5_index_page_first": ([i32, u32, u32, P], u64), "ds5_index_plan_bounds": ([u32, P, P], None),
        "ds5_index_plan_len": ([i32, u32], u32), "ds5_index_plan_items": ([u32, u32], u32),
        "ds5_index_plan_whole": ([u32, u32], u32), "ds5_index_plan_partial": ([u32, u32], u32),
        "ds5_index_gemm_x": ([u32] * 7 + [P], None), "ds5_index_gemm_q": ([u32] * 8 + [P] * 4, None),
        "ds5_index_gemm_x_rows": ([u32] * 7 + [P, P], None),
        "ds5_index_prefill_tile": ([u32, C.c_int, u32, u32, P], u32), "ds5_index_pf_q_token": ([u32] * 3, u32),
    }
    for name, (a, r) in sig.items():
        f = getattr(lib, name)
        f.argtypes, f.restype = a, r
    return lib


def _u32s(n):
    return np.zeros(n, np.uint32)


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def test_index_header_symbols_exported(hip):
    """Every function include/ds5_index.h declares is exported by the library."""
    text = open(os.path.join(ROOT, "include", "ds5_index.h")).read()
    names = set(re.findall(r"^\s*(?:void|uint32_t|uint64_t)\s+(ds5_index_\w+)\(", text, re.M))
    assert len(names) == 17
    for n in names:
        assert getattr(hip.LIB, n) is not None


# ---------------------------------------------------------------------------
# decode_split_kernel (k_decode.hip)
# ---------------------------------------------------------------------------

def decode_shape(ix):
    out = _u32s(4)
    ix.ds5_index_decode_shape(_ptr(out))
    return tuple(int(v) for v in out)  # tile, waves, heads, max_splits


def decode_geometry(ix, n_seqs, n_kv_heads, n_sub, max_len, cu_count=256):
    """decode_geometry_of: (chunk, n_splits)."""
    ch, ns = C.c_uint32(), C.c_uint32()
    ix.ds5_index_decode_geometry(cu_count, 0, n_seqs, n_kv_heads, n_sub, max_len, C.byref(ch), C.byref(ns))
    return ch.value, ns.value


def paged_plan(ix, lens, max_len, n_kv_units, cu_count=256):
    """The paged plan: the smallest admissible chunk (the kernel's binary search finds
    the same one: the item count does not grow with the chunk) whose item count fits
    the cap launch_decode gives the grid (about two workgroups per CU, at least one
    per sequence); items are every sequence's whole chunks, then the partial last
    chunks and the poisoned sequences. Returns (chunk, cap, items)."""
    tile, waves, _, _ = decode_shape(ix)
    step = tile * waves
    cap = max((2 * cu_count + n_kv_units - 1) // n_kv_units, len(lens))
    staged = [ix.ds5_index_plan_len(int(L), max_len) for L in lens]
    cmin, cmax = C.c_uint32(), C.c_uint32()
    ix.ds5_index_plan_bounds(max_len, C.byref(cmin), C.byref(cmax))
    count = lambda c: sum(ix.ds5_index_plan_items(L, c) for L in staged)
    chunk = next(c for c in range(cmin.value, cmax.value + 1, step) if count(c) <= cap)
    items = [(b, sp) for b, L in enumerate(staged) for sp in range(ix.ds5_index_plan_whole(L, chunk))]
    items += [(b, ix.ds5_index_plan_whole(L, chunk)) for b, L in enumerate(staged)
              if ix.ds5_index_plan_partial(L, chunk)]
    assert len(items) <= cap
    return chunk, cap, items


def tile_rows(ix, p0, end, D, row_a=0, row_b=0, paged=False):
    """issue_tile's K and V loads of the tile at p0: rows (positions, or pool slots
    when paged) and element columns, from the kernel's helpers."""
    KK, VC = D // 32, 32 * (D // 8) // 64
    kr, kc = np.zeros(2 * KK * 64, np.uint64), _u32s(2 * KK * 64)
    vr, vc = np.zeros(VC * 64, np.uint64), _u32s(VC * 64)
    ix.ds5_index_decode_tile(p0, end, D, int(paged), row_a, row_b, _ptr(kr), _ptr(kc), _ptr(vr), _ptr(vc))
    return kr.astype(np.int64), kc.astype(np.int64), vr.astype(np.int64), vc.astype(np.int64)


def check_decode(ix, n_seqs, hq, hkv, D, lens, cache_stride, page_size=0, page_table=None, n_pages=0,
                 max_len=None, fused=True):
    """Every access of one decode launch. lens: attended positions per sequence (the
    contiguous cache passes one length). Returns the number of checked 16-byte loads."""
    K_TILE, K_WAVES, K_HEADS, MAX_SPLITS = decode_shape(ix)
    group = hq // hkv
    n_sub = (group + K_HEADS - 1) // K_HEADS
    max_len = max_len if max_len is not None else int(max(lens))
    paged = page_table is not None
    if paged:  # planned launch: chunk from the lengths, kMaxSplits partial slots per row
        chunk, _, items = paged_plan(ix, lens, max_len, hkv * n_sub)
        n_splits = MAX_SPLITS
        assert all(sp < n_splits for _, sp in items)
    else:
        chunk, n_splits = decode_geometry(ix, n_seqs, hkv, n_sub, max_len)
    cache_elems = hkv * cache_stride * D            # per K (and V) cache, f16 elements
    q_elems = n_seqs * hq * D
    part_elems = n_seqs * hq * n_splits * D if n_splits > 1 else 0
    TPH = D // 8
    checked = 0
    item_set = set(items) if paged else set()
    table = page_table.reshape(-1) if paged else None
    max_pages = page_table.shape[1] if paged else 0

    def page_first(b, pos):
        idx = ix.ds5_index_page_index(b, max_pages, pos, page_size)
        assert 0 <= idx < table.size  # the page-table read itself
        bad = C.c_int()
        return ix.ds5_index_page_first(int(table[idx]), n_pages, page_size, C.byref(bad))

    for b in range(n_seqs):
        L = int(lens[b]) if len(lens) > 1 else int(lens[0])
        if paged and not (1 <= L <= max_len):
            continue  # poisoned sequence: only its output is written
        for kv in range(hkv):
            for sub in range(n_sub):
                n0 = sub * K_HEADS
                NS = min(K_HEADS, group - n0)
                qrow0 = b * hq + kv * group + n0
                # q-operand loads: thread t reads 4 floats at (qrow0 + min(t / TPH, NS - 1)) * D + 4 (t % TPH) (+ D/2)
                t = np.arange(256)
                qoff = (qrow0 + np.minimum(t // TPH, NS - 1)) * D + 4 * (t % TPH)
                assert qoff.min() >= 0 and (qoff + D // 2 + 4).max() <= q_elems
                for split in range(n_splits):
                    start = split * chunk
                    if start >= L:
                        continue
                    assert not paged or (b, split) in item_set  # every split the kernel reads has a workgroup
                    end = min(L, start + chunk)
                    n_tiles = (end - start + K_TILE - 1) // K_TILE
                    newpos = L - 1
                    for wave in range(K_WAVES):
                        # the first tile is issued unconditionally (clamped), then one ahead
                        tiles = [start + min(wave, n_tiles - 1) * K_TILE]
                        it = wave
                        while it < n_tiles and it + K_WAVES < n_tiles:
                            it += K_WAVES
                            tiles.append(start + it * K_TILE)
                        for p0 in tiles:
                            ra = rb = 0
                            if paged:
                                ra = page_first(b, ix.ds5_index_half_pos(p0, end, 0)) + p0 % page_size
                                rb = page_first(b, ix.ds5_index_half_pos(p0, end, 1)) + (p0 + 16) % page_size
                            kr, kc, vr, vc = tile_rows(ix, p0, end, D, ra, rb, paged)
                            for rows, cols in ((kr, kc), (vr, vc)):
                                off = (kv * cache_stride + rows) * D + cols
                                assert off.min() >= 0 and (off + 8).max() <= cache_elems, (b, kv, split, p0)
                                checked += off.size
                    if fused and start <= newpos < end:
                        slot = page_first(b, newpos) + newpos % page_size if paged else newpos
                        off = (kv * cache_stride + slot) * D + np.arange(D)
                        assert off.min() >= 0 and off.max() < cache_elems
                    if n_splits > 1:
                        qi = qrow0 + np.arange(NS)
                        off = ((qi * n_splits + split) * D)[:, None] + np.arange(0, D, 4)[None, :]
                        assert off.min() >= 0 and (off + 4).max() <= part_elems
    return checked


@pytest.mark.parametrize("config", [0, 1, 3])
def test_decode_contiguous_addresses(ix, config):
    cfg = synth.CONFIGS[config]
    s = cfg["shape"]
    n = check_decode(ix, 1, s.n_q_heads, s.n_kv_heads, s.head_dim, [cfg["pos"] + 1], cfg["cap"])
    assert n > 0


@pytest.mark.parametrize("L,cap,hq,hkv,D", [
    (1, 1, 32, 4, 128), (33, 40, 32, 4, 128), (129, 129, 8, 2, 64), (1000, 1024, 64, 4, 128),
    (8191, 8192, 32, 4, 128), (4097, 5000, 6, 3, 128), (300, 300, 40, 2, 128),
])
def test_decode_contiguous_addresses_edges(ix, L, cap, hq, hkv, D):
    """Lengths that leave partial tiles, single tiles, and a group of 20 heads (two head sub-groups)."""
    assert check_decode(ix, 1, hq, hkv, D, [L], cap) > 0


def test_decode_paged_addresses_config4(ix):
    cfg = synth.CONFIGS[4]
    s = cfg["shape"]
    lay = synth.paged_layout(cfg["n_seqs"], cfg["lo"], cfg["hi"], cfg["page_size"], seed=0)
    n = check_decode(ix, cfg["n_seqs"], s.n_q_heads, s.n_kv_heads, s.head_dim, lay.seq_lens, lay.n_pages * 16, 16,
                     lay.page_table, lay.n_pages, int(lay.seq_lens.max()))
    assert n > 0


@pytest.mark.parametrize("page_size", [32, 64])
def test_decode_paged_addresses_larger_pages(ix, page_size):
    """The GPU suite's 32- and 64-position page cases (7 sequences, lengths 1..700)."""
    s = synth.Shape()
    lay = synth.paged_layout(7, 1, 700, page_size, seed=11)
    n = check_decode(ix, 7, s.n_q_heads, s.n_kv_heads, s.head_dim, lay.seq_lens, lay.n_pages * page_size, page_size,
                     lay.page_table, lay.n_pages, int(lay.seq_lens.max()))
    assert n > 0


def test_paged_plan_fits_and_is_smallest(ix):
    """The plan's chunk is the smallest admissible one: the next smaller multiple of
    128 (when admissible) overflows the cap. C4's lengths give ~2 workgroups per CU."""
    cfg = synth.CONFIGS[4]
    lay = synth.paged_layout(cfg["n_seqs"], cfg["lo"], cfg["hi"], cfg["page_size"], seed=0)
    max_len = int(lay.seq_lens.max())
    chunk, cap, items = paged_plan(ix, lay.seq_lens, max_len, 4)
    assert cap == 128 and len(items) <= cap and chunk % 128 == 0
    smaller = chunk - 128
    if smaller >= max(128, -(-max_len // 64)):
        assert sum(-(-int(L) // smaller) for L in lay.seq_lens) > cap
    # every position of every sequence is in exactly one item
    for b, L in enumerate(lay.seq_lens):
        spans = sorted(sp for bb, sp in items if bb == b)
        assert spans == list(range(-(-int(L) // chunk)))


def test_decode_paged_addresses_invalid_entries(ix):
    """Page ids outside the pool and lengths outside [1, max_len] (the device-side
    entries the host cannot check) are never used as addresses."""
    lay = synth.paged_layout(5, 40, 300, 16, seed=11)
    table, lens = lay.page_table.copy(), lay.seq_lens.copy()
    max_len = int(lens.max())
    table[1, 0] = lay.n_pages + 3
    table[4, :] = -7
    lens[2] = 0
    lens[3] = max_len + 1
    assert check_decode(ix, 5, 32, 4, 128, lens, lay.n_pages * 16, 16, table, lay.n_pages, max_len) > 0


def test_decode_rows_clamp_at_the_split_end(ix):
    """The tile helpers clamp every row past the split's end to its last position (the
    tile at 64 of a split ending at 80 reads rows 64..79 and none past them)."""
    kr, kc, vr, vc = tile_rows(ix, 64, 80, 128)
    assert kr.max() == 79 and vr.max() == 79 and kr.min() == 64 and vr.min() == 64
    assert kc.max() + 8 <= 128 and vc.max() + 8 <= 128


# ---------------------------------------------------------------------------
# matmul_q8_mfma_kernel direct-to-LDS loads (k_matmul.hip)
# ---------------------------------------------------------------------------

Q8 = 34


def gemm_path_ok(w_addr, n, k, w_len, m=1):
    """matmul_path's Q8_0 requirements of the weight view for the GEMM: the row
    kernel's end condition, and plane and weight offsets that fit 32 bits
    (gemm_offsets_fit)."""
    end = n * (k // 32) * Q8
    fits = m * k * 2 < U32 and end + 2 < U32
    return w_addr % 4 == 0 and ((w_addr + end) % 4 == 0 or w_len >= end + 2) and fits


def check_gemm(ix, m, n, k, w_addr, w_len, BM, BN, WM, WN):
    """Every x-plane and weight byte the GEMM's direct-to-LDS loads read, for each
    block b of every tile (offsets from the kernel's helpers); returns one past the
    highest weight byte read."""
    W = WM * WN
    nb = k // 32
    row_bytes = nb * Q8
    b = np.arange(nb)[:, None]
    lane = np.arange(64)
    # x: load i of wavefront w fills stage bytes 1024 (w + W i) + 16 lane of one plane; its
    # 32-bit lane offset (block 0) from gemm_x_off, plus 64 b per block
    nx = 2 * BM * 64 // 1024 // W
    assert nx >= 1 and nx * 1024 * W == 2 * BM * 64
    for m0 in range(0, m, BM):
        for w in range(W):
            off = _u32s(nx * 64)
            ix.ds5_index_gemm_x(w, W, nx, BM, m0, m, k, _ptr(off))
            for i in range(nx):
                o = 1024 * (w + W * i) + 16 * lane
                plane = o // (BM * 64)
                assert (plane == plane[0]).all()  # one plane per load
                byte = off[i * 64:(i + 1) * 64].astype(np.int64)[None, :] + 64 * b
                assert byte.min() >= 0 and (byte + 16).max() <= m * k * 2
    # raw q: the dwords of each row's block from the dword boundary at or below it, a
    # scalar base (34 b, or 34 b - 2 for odd b) plus the lane's even/odd offset
    threads = W * 64
    b_per = BN * 4 // threads
    w_rows = 16 * b_per
    nq = (w_rows * 9 + 63) // 64
    hi = None
    for n0 in range(0, n, BN):
        for w in range(W):
            dw, row, even, odd = (_u32s(nq * 64) for _ in range(4))
            ix.ds5_index_gemm_q(w, threads, nq, w_rows, 9, n0, n, row_bytes, _ptr(dw), _ptr(row), _ptr(even),
                                _ptr(odd))
            dw, row, even, odd = (a.astype(np.int64) for a in (dw, row, even, odd))
            base = Q8 * b - (b % 2) * 2                    # the scalar base (non-negative: b >= 1 when odd)
            assert base.min() >= 0
            byte = base + np.where(b % 2 == 0, even[None, :], odd[None, :])
            rb = np.minimum(n0 + row, n - 1) * row_bytes
            # the bytes are those of the dword boundary at or below the block
            want = (rb[None, :] + Q8 * b) // 4 * 4 + 4 * (dw % 9)[None, :]
            assert (byte == want).all()
            assert ((w_addr + byte) % 4 == 0).all()  # dword loads stay aligned
            top = int((byte + 4).max())
            hi = top if hi is None else max(hi, top)
            # the wavefront loaded exactly the rows its threads convert (thread c: row c / 4)
            conv = {(c + threads * u) // 4 for c in range(64 * w, 64 * w + 64) for u in range(b_per)}
            assert set(row.tolist()) == conv
    return hi


@pytest.mark.parametrize("m,n,k", [
    (16, 512, 2048), (2048, 4096, 2048), (2048, 512, 2048), (200, 300, 96), (130, 70, 32 * 65),
    (17, 256, 256), (16, 5, 32 * 3), (33, 129, 32 * 7),
    (128, 256, 32), (130, 128, 64), (256, 384, 96), (136, 200, 160),
])
@pytest.mark.parametrize("tile", [(128, 128, 4, 2), (32, 64, 2, 2), (64, 128, 2, 2), (128, 128, 2, 2)])
def test_gemm_load_block_addresses(ix, m, n, k, tile):
    """Both GEMM tiles; odd block counts put every other row's blocks at 2 mod 4."""
    end = n * (k // 32) * Q8
    for w_len in (end, end + 2):
        if not gemm_path_ok(0, n, k, w_len, m):
            continue  # matmul_path sends this view to the serial kernel
        hi = check_gemm(ix, m, n, k, 0, w_len, *tile)
        assert hi <= w_len, (hi, w_len)


def _moe_tiles(pairs_expert, E, rows):
    """The grouped MoE's sorted rows and row tiles as moe_sort_kernel builds them: each
    expert's rows consecutive in expert order, tiles of `rows` rows (first, end, expert)."""
    cnt = np.bincount(pairs_expert, minlength=E)
    off = np.concatenate([[0], np.cumsum(cnt)])
    tiles = [(off[e] + rows * t, off[e] + cnt[e], e) for e in range(E) for t in range(-(-cnt[e] // rows))]
    return np.argsort(pairs_expert, kind="stable"), tiles


@pytest.mark.parametrize("T,K,E,dim,ffn", [(64, 8, 16, 2048, 768), (40, 8, 12, 512, 256), (24, 3, 8, 256, 96),
                                           (2048, 8, 128, 2048, 768)])
@pytest.mark.parametrize("tile", [(64, 128, 2, 2), (128, 128, 4, 2)])
def test_grouped_moe_gemm_x_rows(ix, hip, T, K, E, dim, ffn, tile):
    """The grouped MoE products' x loads: gate / up read sorted row r's token's row of the
    T-row x planes (x_rows = the pairs' tokens in sorted order), down the P-row h planes
    (no map); every load stays inside its planes, reads a row of the tile's own expert,
    and the tile count stays within moe_max_tiles (P / rows + E + 1)."""
    BM, BN, WM, WN = tile
    W = WM * WN
    g = np.random.default_rng(T + E)
    P = T * K
    tokens = np.repeat(np.arange(T), K)
    expert = g.integers(0, E, P)
    expert[g.random(P) < 0.3] = 1  # one heavy expert: several tiles
    perm, tiles = _moe_tiles(expert, E, BM)
    assert len(tiles) <= P // BM + E + 1
    x_rows = tokens[perm].astype(np.uint32)
    nx = 2 * BM * 64 // 1024 // W
    lane = np.arange(64)
    for m0, m, e in tiles:
        for w in range(W):
            o = 1024 * (w + W * np.arange(nx)[:, None]) + 16 * lane[None, :]
            r = (o % (BM * 64)) // 64
            srow = np.minimum(m0 + r, m - 1)
            assert (expert[perm[srow]] == e).all()  # the tile's own expert, rows past the end included
            for k, rows_map, plane_rows in ((dim, x_rows, T), (ffn, None, P)):
                off = _u32s(nx * 64)
                if rows_map is None:
                    ix.ds5_index_gemm_x(w, W, nx, BM, int(m0), int(m), k, _ptr(off))
                    want_row = srow
                else:
                    ix.ds5_index_gemm_x_rows(w, W, nx, BM, int(m0), int(m), k, _ptr(rows_map), _ptr(off))
                    want_row = tokens[perm[srow]]
                off = off.astype(np.int64).reshape(nx, 64)
                assert (off // (2 * k) == want_row).all()
                last = off + 64 * (k // 32 - 1) + 16  # the last block's 16 bytes
                assert off.min() >= 0 and last.max() <= plane_rows * k * 2


def test_gemm_slack_rule_is_needed(ix):
    """Without matmul_path's rule the last run of an odd-block view ending at 2 mod 4
    reads 2 bytes past the view: the rule is what keeps the GEMM inside it."""
    n, k = 129, 32 * 7
    end = n * (k // 32) * Q8
    assert end % 4 == 2 and not gemm_path_ok(0, n, k, end)
    assert check_gemm(ix, 64, n, k, 0, end, 32, 64, 2, 2) == end + 2


# ---------------------------------------------------------------------------
# prefill_attention_kernel DMA (k_prefill.hip)
# ---------------------------------------------------------------------------

def check_prefill(ix, pos, T, hq, hkv, D, max_ctx):
    """Every direct-to-LDS load, staged q-row load and output row store of one prefill
    launch (tile offsets and the q rows' tokens from the kernel's helpers)."""
    shape = _u32s(3)
    ix.ds5_index_prefill_shape(_ptr(shape))
    P_HEADS, P_QROWS, P_KTILE = (int(v) for v in shape)
    group = hq // hkv
    n_qtiles = (T + P_QROWS - 1) // P_QROWS
    n_pairs = (n_qtiles + 1) // 2
    n_hgroups = (group + P_HEADS - 1) // P_HEADS
    head_bytes = max_ctx * 2 * D
    calls = set()
    kv_end_of = lambda qt: pos + min(T, qt * P_QROWS + P_QROWS)
    lane = np.arange(64)
    tok = np.vectorize(lambda q0, r: ix.ds5_index_pf_q_token(int(q0), int(r), T))
    for pair in range(n_pairs):
        heavy = n_qtiles - 1 - pair
        has_light = pair < heavy
        H = (kv_end_of(heavy) + P_KTILE - 1) // P_KTILE
        L = (kv_end_of(pair) + P_KTILE - 1) // P_KTILE if has_light else 0
        # items: the heavy tile's key tiles 0 .. H - 1, then the light tile's 0 .. L - 1
        for qt, n in ((heavy, H), (pair, L)):
            for j in range(n):
                calls.add((j * P_KTILE, kv_end_of(qt)))
        for sel in range(2):
            if sel == 1 and not has_light:
                break
            q0 = (heavy if sel == 0 else pair) * P_QROWS
            # q rows, staged along rows: D/8 lanes per row; f16 operand lane (g, m) reads
            # elements 8 m + [0, 8), f32 q lane (g, m) elements 4 m + [0, 4) and D/2 + 4 m +
            # [0, 4), and the same of its cos/sin row (D floats per token)
            LPR = D // 8
            RPI = 64 // LPR
            rows = tok(q0, RPI * np.arange(P_QROWS // RPI)[:, None] + lane[None, :] // LPR)
            for els in (8 * (lane % LPR)[:, None] + np.arange(8),
                        np.concatenate([4 * (lane % LPR)[:, None] + np.arange(4),
                                        D // 2 + 4 * (lane % LPR)[:, None] + np.arange(4)], 1)):
                assert els.min() >= 0 and els.max() < D
            assert rows.min() >= 0 and (rows * D + D).max() <= T * D  # cos/sin rows
            for hg in range(n_hgroups):
                for hw in range(P_HEADS):
                    hin = hg * P_HEADS + hw
                    for kvh in range(hkv):
                        hqi = kvh * group + (hin if hin < group else 0)
                        off = (rows * hq + hqi) * D
                        assert off.min() >= 0 and (off + D).max() <= T * hq * D
            # output rows: lane l stores row q0 + 8 it + l / 8 (rows past T are skipped),
            # elements 32 dt + 4 (l % 8) + [0, 4)
            orow = q0 + 8 * np.arange(P_QROWS // 8)[:, None] + lane[None, :] // 8
            ocol = 32 * np.arange(D // 32)[:, None] + 4 * (lane % 8)[None, :]
            assert (ocol + 4).max() <= D and ((orow[orow < T] + 1) * hq * D).max() <= T * hq * D
    off = _u32s(64 * 64)
    for key0, end in calls:
        assert 0 < end <= max_ctx
        for v in (0, 1):
            nb = ix.ds5_index_prefill_tile(D, v, key0, end, _ptr(off))
            a = key0 * 2 * D + off[:nb * 64].astype(np.int64)
            assert a.min() >= 0 and (a + 16).max() <= head_bytes, (key0, end, v)
            if key0 + P_KTILE > end:  # a clamped tile reads no row at or past kv_end
                assert (a // (2 * D)).max() <= end - 1
    return len(calls)


@pytest.mark.parametrize("pos,T,hq,hkv,D,cap", [
    (0, 2048, 32, 4, 128, 2048),     # C2
    (0, 300, 32, 4, 128, 307), (100, 130, 32, 4, 128, 237), (5, 77, 32, 4, 64, 89), (0, 2, 32, 4, 128, 9),
    (0, 97, 32, 4, 128, 104), (48, 160, 32, 4, 128, 215), (31, 200, 64, 4, 128, 238), (3, 96, 6, 3, 128, 106), (0, 65, 8, 8, 64, 72),
])
def test_prefill_dma_addresses(ix, pos, T, hq, hkv, D, cap):
    """C2 and the GPU parity suite's prefill shapes (chunked continuations, odd q-tile counts)."""
    assert check_prefill(ix, pos, T, hq, hkv, D, cap) > 0
