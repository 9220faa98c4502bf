"""Host replicas of the device kernels' load/store address arithmetic (no GPU).

Each replica restates, per lane, the byte offsets a kernel reads or writes --
with the same clamps, wrap-free unsigned arithmetic and launch geometry as the
kernel source it cites -- and the tests assert that every access of every
workgroup stays inside its view at the BASELINE shapes (C0-C4) and at the
Q8_0 shapes whose blocks start 2 bytes off a dword. A GPU memory fault once came
from exactly such arithmetic (an offset that went negative and wrapped as an
unsigned 32-bit value); a replica catches that class of mistake on the CPU.

Replicated:
  qw3_amd/csrc/k_decode.hip  decode_geometry_of, paged_plan, issue_tile, the q-operand and
                             new-row accesses and the partial stores of
                             decode_split_kernel (contiguous and paged caches)
  qw3_amd/csrc/k_matmul.hip  the direct-to-LDS loads of matmul_q8_mfma_kernel (x
                             planes, raw Q8_0 rows) and matmul_path's slack rule
  qw3_amd/csrc/k_prefill.hip TilePlan / dma_tile of prefill_attention_kernel (every
                             direct-to-LDS load of every item), its staged q-row and
                             cos/sin-row loads and its output row stores
"""
import numpy as np
import pytest

from qw3_amd import synth

U32 = 1 << 32


# ---------------------------------------------------------------------------
# decode_split_kernel (k_decode.hip)
# ---------------------------------------------------------------------------

K_TILE, K_WAVES, K_HEADS = 32, 4, 16


def decode_geometry(n_seqs, n_kv_heads, n_sub, max_len, cu_count=256, decode_chunk=0):
    """decode_geometry_of: (chunk, n_splits)."""
    step = K_WAVES * K_TILE
    chunk = decode_chunk
    if chunk == 0:
        units = n_seqs * n_kv_heads * n_sub
        target = 4 * cu_count
        chunk = min((max_len * units + target - 1) // target, max_len)
    chunk = max((chunk + step - 1) // step * step, step)
    chunk = max(chunk, (max_len + 63) // 64)
    chunk = (chunk + step - 1) // step * step
    return chunk, (max_len + chunk - 1) // chunk


def paged_plan(lens, max_len, n_kv_units, cu_count=256, max_splits=64):
    """paged_plan (k_decode.hip): the smallest chunk (a multiple of 128, at least
    max_len / max_splits) whose item count sum_b ceil(L_b / chunk) fits the cap; a
    length outside [1, max_len] counts one item. Returns (chunk, cap, items)."""
    step = K_WAVES * K_TILE
    cap = max((2 * cu_count + n_kv_units - 1) // n_kv_units, len(lens))
    lens = [int(L) if 1 <= int(L) <= max_len else 0 for L in lens]
    cmin = max(step, -(-max_len // max_splits) + step - 1) // step * step
    cmax = -(-max_len // step) * step
    count = lambda c: sum(1 if L == 0 else -(-L // c) for L in lens)
    chunk = next(c for c in range(cmin, cmax + 1, step) if count(c) <= cap)
    # whole chunks of every sequence first, then the partial last chunks (and poisoned sequences)
    items = [(b, sp) for b, L in enumerate(lens) for sp in range(L // chunk)]
    items += [(b, L // chunk) for b, L in enumerate(lens) if L == 0 or L % chunk]
    assert len(items) <= cap
    return chunk, cap, items


def tile_rows(p0, end, D, paged, page_row=None):
    """issue_tile: the cache rows (positions, or pool slots when paged) of the K and V
    loads of the tile starting at p0, and each load's element offset inside its row:
    K: lane (g, c16), half st, step kk -> row (p0 + 16 st + c16 clamped), dims kk*32 + 8g;
    V: chunk c = lane + 64 r -> row p0 + c / RC (clamped), dims (c % RC) * 8."""
    KK, RC = D // 32, D // 8
    VC = K_TILE * RC // 64
    lane = np.arange(64)
    g, c16 = lane >> 4, lane & 15
    krow, kcol, vrow, vcol = [], [], [], []
    for st in range(2):
        for kk in range(KK):
            if paged:
                krow.append(page_row(p0, st) + c16)
            else:
                krow.append(np.minimum(p0 + 16 * st + c16, end - 1))
            kcol.append(kk * 32 + 8 * g)
    for r in range(VC):
        c = lane + 64 * r
        tr = c // RC
        if paged:
            vrow.append(page_row(p0, 0 if r < VC // 2 else 1) + (tr & 15))
        else:
            vrow.append(np.minimum(p0 + tr, end - 1))
        vcol.append((c % RC) * 8)
    return (np.concatenate(krow), np.concatenate(kcol), np.concatenate(vrow), np.concatenate(vcol))


def check_decode(n_seqs, hq, hkv, D, lens, cache_stride, page_size=0, page_table=None, n_pages=0, max_len=None,
                 fused=True):
    """Every access of one decode launch. lens: attended positions per sequence (the
    contiguous cache passes one length). Returns the number of checked 16-byte loads."""
    group = hq // hkv
    n_sub = (group + K_HEADS - 1) // K_HEADS
    max_len = max_len if max_len is not None else int(max(lens))
    paged = page_table is not None
    if paged:  # planned launch: chunk from the lengths, kMaxSplits partial slots per row
        chunk, _, items = paged_plan(lens, max_len, hkv * n_sub)
        n_splits = 64
        assert all(sp < n_splits for _, sp in items)
    else:
        chunk, n_splits = decode_geometry(n_seqs, hkv, n_sub, max_len)
    cache_elems = hkv * cache_stride * D            # per K (and V) cache, f16 elements
    q_elems = n_seqs * hq * D
    part_elems = n_seqs * hq * n_splits * D if n_splits > 1 else 0
    TPH = D // 8
    checked = 0
    item_set = set(items) if paged else set()
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

                    def page_row(p0, st):
                        pos = p0 if st == 0 else min(p0 + 16, end - 1)
                        idx = b * page_table.shape[1] + pos // page_size
                        assert 0 <= idx < page_table.size  # the page-table read itself
                        pg = int(page_table.reshape(-1)[idx])
                        base = (pg if 0 <= pg < n_pages else 0) * page_size
                        return base + (p0 + 16 * st) % page_size

                    for wave in range(K_WAVES):
                        # the first tile is issued unconditionally (clamped), then one ahead
                        tiles = [start + min(wave, n_tiles - 1) * K_TILE]
                        it = wave
                        while it < n_tiles and it + K_WAVES < n_tiles:
                            it += K_WAVES
                            tiles.append(start + it * K_TILE)
                        for p0 in tiles:
                            kr, kc, vr, vc = tile_rows(p0, end, D, paged, page_row if paged else None)
                            for rows, cols in ((kr, kc), (vr, vc)):
                                off = ((kv * cache_stride + rows) * D + cols).astype(np.int64)
                                assert off.min() >= 0 and (off + 8).max() <= cache_elems, (b, kv, split, p0)
                                checked += off.size
                    if fused and start <= newpos < end:
                        slot = newpos
                        if paged:
                            idx = b * page_table.shape[1] + newpos // page_size
                            pg = int(page_table.reshape(-1)[idx])
                            slot = (pg if 0 <= pg < n_pages else 0) * page_size + newpos % page_size
                        off = (kv * cache_stride + slot) * D + np.arange(D)
                        assert off.min() >= 0 and off.max() < cache_elems
                    if n_splits > 1:
                        qi = qrow0 + np.arange(NS)
                        off = ((qi * n_splits + split) * D)[:, None] + np.arange(0, D, 4)[None, :]
                        assert off.min() >= 0 and (off + 4).max() <= part_elems
    return checked


@pytest.mark.parametrize("config", [0, 1, 3])
def test_decode_contiguous_addresses(config):
    cfg = synth.CONFIGS[config]
    s = cfg["shape"]
    n = check_decode(1, s.n_q_heads, s.n_kv_heads, s.head_dim, [cfg["pos"] + 1], cfg["cap"])
    assert n > 0


@pytest.mark.parametrize("L,cap,hq,hkv,D", [
    (1, 1, 32, 4, 128), (33, 40, 32, 4, 128), (129, 129, 8, 2, 64), (1000, 1024, 64, 4, 128),
    (8191, 8192, 32, 4, 128), (4097, 5000, 6, 3, 128), (300, 300, 40, 2, 128),
])
def test_decode_contiguous_addresses_edges(L, cap, hq, hkv, D):
    """Lengths that leave partial tiles, single tiles, and a group of 20 heads (two head sub-groups)."""
    assert check_decode(1, hq, hkv, D, [L], cap) > 0


def test_decode_paged_addresses_config4():
    cfg = synth.CONFIGS[4]
    s = cfg["shape"]
    lay = synth.paged_layout(cfg["n_seqs"], cfg["lo"], cfg["hi"], cfg["page_size"], seed=0)
    n = check_decode(cfg["n_seqs"], s.n_q_heads, s.n_kv_heads, s.head_dim, lay.seq_lens, lay.n_pages * 16, 16,
                     lay.page_table, lay.n_pages, int(lay.seq_lens.max()))
    assert n > 0


@pytest.mark.parametrize("page_size", [32, 64])
def test_decode_paged_addresses_larger_pages(page_size):
    """The GPU suite's 32- and 64-position page cases (7 sequences, lengths 1..700)."""
    s = synth.Shape()
    lay = synth.paged_layout(7, 1, 700, page_size, seed=11)
    n = check_decode(7, s.n_q_heads, s.n_kv_heads, s.head_dim, lay.seq_lens, lay.n_pages * page_size, page_size,
                     lay.page_table, lay.n_pages, int(lay.seq_lens.max()))
    assert n > 0


def test_paged_plan_fits_and_is_smallest():
    """The plan's chunk is the smallest admissible one: the next smaller multiple of
    128 (when admissible) overflows the cap. C4's lengths give ~2 workgroups per CU."""
    cfg = synth.CONFIGS[4]
    lay = synth.paged_layout(cfg["n_seqs"], cfg["lo"], cfg["hi"], cfg["page_size"], seed=0)
    max_len = int(lay.seq_lens.max())
    chunk, cap, items = paged_plan(lay.seq_lens, max_len, 4)
    assert cap == 128 and len(items) <= cap and chunk % 128 == 0
    smaller = chunk - 128
    if smaller >= max(128, -(-max_len // 64)):
        assert sum(-(-int(L) // smaller) for L in lay.seq_lens) > cap
    # every position of every sequence is in exactly one item
    for b, L in enumerate(lay.seq_lens):
        spans = sorted(sp for bb, sp in items if bb == b)
        assert spans == list(range(-(-int(L) // chunk)))


def test_decode_paged_addresses_invalid_entries():
    """Page ids outside the pool and lengths outside [1, max_len] (the device-side
    entries the host cannot check) are never used as addresses."""
    lay = synth.paged_layout(5, 40, 300, 16, seed=11)
    table, lens = lay.page_table.copy(), lay.seq_lens.copy()
    max_len = int(lens.max())
    table[1, 0] = lay.n_pages + 3
    table[4, :] = -7
    lens[2] = 0
    lens[3] = max_len + 1
    assert check_decode(5, 32, 4, 128, lens, lay.n_pages * 16, 16, table, lay.n_pages, max_len) > 0


def test_decode_replica_catches_a_wrapped_offset():
    """A plausible mistake -- the half-tile row taken as p0 - 16 + c16 instead of
    p0 + 16 + c16, wrapping below zero for the first tile -- is caught."""
    kr, kc, _, _ = tile_rows(0, 100, 128, paged=False)
    bad = np.minimum(0 - 16 + (np.arange(64) & 15), 99) % U32  # unsigned 32-bit wrap
    assert kr.min() >= 0 and bad.max() >= U32 - 16


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


def check_gemm(m, n, k, w_addr, w_len, BM, BN, WM, WN):
    """Every x-plane and weight byte the GEMM's direct-to-LDS loads read, for each
    block b of every tile; returns one past the highest weight byte read."""
    W = WM * WN
    nb = k // 32
    row_bytes = nb * Q8
    b = np.arange(nb)[:, None]
    lane = np.arange(64)
    # x: load i of wavefront w: stage byte o = 1024 (w + W i) + 16 lane -> plane o / (64 BM),
    # row r = (o % (64 BM)) / 64, chunk (lane % 4) ^ ((r / 4) % 4); plane byte
    # min(m0 + r, m - 1) * 2k + 16 chunk + 64 b, 16 bytes; the offset is a 32-bit lane value
    nx = 2 * BM * 64 // 1024 // W
    assert nx >= 1 and nx * 1024 * W == 2 * BM * 64
    for m0 in range(0, m, BM):
        for w in range(W):
            for i in range(nx):
                o = 1024 * (w + W * i) + 16 * lane
                plane = o // (BM * 64)
                assert (plane == plane[0]).all()  # one plane per load
                r = (o % (BM * 64)) // 64
                c = (lane & 3) ^ ((r >> 2) & 3)
                off = np.minimum(m0 + r, m - 1) * k * 2 + 16 * c
                assert off.max() < 2 ** 32
                byte = off[None, :] + 64 * b
                assert byte.min() >= 0 and (byte + 16).max() <= m * k * 2
    # raw q: 9 dwords per tile row from the dword boundary at or below the row's block,
    # each wavefront loading the rows of its own threads' runs: local row lr < 16 b_per
    # is tile row 16 w + (threads / 4) (lr / 16) + lr % 16; dword d = 64 i + lane
    # (clamped to the last) is dword d % 9 of local row d / 9; rb = min(n0 + row, n - 1)
    # * row_bytes: weight byte (34 b) + (rb & ~3) + 4 (d % 9) for even b, (34 b - 2) +
    # ((rb + 2) & ~3) + 4 (d % 9) for odd b -- a scalar base plus a 32-bit lane offset
    threads = W * 64
    b_per = BN * 4 // threads
    w_rows = 16 * b_per
    nq = (w_rows * 9 + 63) // 64
    hi = None
    for n0 in range(0, n, BN):
        for w in range(W):
            covered = set()
            for i in range(nq):
                d = np.minimum(64 * i + lane, w_rows * 9 - 1)
                lr = d // 9
                row = 16 * w + (threads // 4) * (lr // 16) + lr % 16
                covered.update(row.tolist())
                rb = np.minimum(n0 + row, n - 1) * row_bytes
                even = (rb & ~3) + 4 * (d % 9)        # lane offsets: sums of non-negative terms
                odd = ((rb + 2) & ~3) + 4 * (d % 9)
                assert min(even.min(), odd.min()) >= 0 and max(even.max(), odd.max()) < 2 ** 32
                base = Q8 * b - (b % 2) * 2               # the scalar base (non-negative: b >= 1 when odd)
                assert base.min() >= 0
                byte = base + np.where(b % 2 == 0, even[None, :], odd[None, :])
                # the bytes are those of the dword boundary at or below the block
                want = (rb[None, :] + Q8 * b) // 4 * 4 + 4 * (d % 9)[None, :]
                assert (byte == want).all()
                assert ((w_addr + byte) % 4 == 0).all()  # dword loads stay aligned
                assert byte.min() >= 0
                top = int((byte + 4).max())
                hi = top if hi is None else max(hi, top)
            # the wavefront loaded exactly the rows its threads convert (thread c: row c / 4)
            conv = {(c + threads * u) // 4 for c in range(64 * w, 64 * w + 64) for u in range(b_per)}
            assert covered == conv
    return hi


@pytest.mark.parametrize("m,n,k", [
    (16, 512, 2048), (2048, 4096, 2048), (2048, 512, 2048), (200, 300, 96), (130, 70, 32 * 65),
    (17, 256, 256), (16, 5, 32 * 3), (33, 129, 32 * 7),
    (128, 256, 32), (130, 128, 64), (256, 384, 96), (136, 200, 160),
])
@pytest.mark.parametrize("tile", [(128, 128, 4, 2), (32, 64, 2, 2), (64, 128, 2, 2), (128, 128, 2, 2)])
def test_gemm_load_block_addresses(m, n, k, tile):
    """Both GEMM tiles; odd block counts put every other row's blocks at 2 mod 4."""
    end = n * (k // 32) * Q8
    for w_len in (end, end + 2):
        if not gemm_path_ok(0, n, k, w_len, m):
            continue  # matmul_path sends this view to the serial kernel
        hi = check_gemm(m, n, k, 0, w_len, *tile)
        assert hi <= w_len, (hi, w_len)


def test_gemm_slack_rule_is_needed():
    """Without matmul_path's rule the last run of an odd-block view ending at 2 mod 4
    reads 2 bytes past the view: the rule is what keeps the GEMM inside it."""
    n, k = 129, 32 * 7
    end = n * (k // 32) * Q8
    assert end % 4 == 2 and not gemm_path_ok(0, n, k, end)
    assert check_gemm(64, n, k, 0, end, 32, 64, 2, 2) == end + 2


# ---------------------------------------------------------------------------
# prefill_attention_kernel DMA (k_prefill.hip)
# ---------------------------------------------------------------------------

P_HEADS, P_QROWS, P_KTILE = 4, 32, 64


def tile_plan(D, RS):
    """TilePlan: each lane's byte offset inside a 64-row tile, for every 1 KiB load of
    the stage (load b fills stage bytes [1024 b, +1024); a padding lane re-reads its
    row's first chunk)."""
    NB = P_KTILE * RS // 1024
    offs = []
    for b in range(NB):
        pos = 1024 * b + 16 * np.arange(64)
        r, c = pos // RS, (pos % RS) // 16
        offs.append(r * 2 * D + np.where(c < D // 8, 16 * c, 0))
    return np.concatenate(offs)


def dma_extent(D, offs, key0, kv_end):
    """dma_tile: byte range [lo, hi) read from the kv head's rows for one call."""
    if key0 + P_KTILE <= kv_end:  # whole tile: scalar tile base + offset
        a = key0 * 2 * D + offs
    else:
        last_row = kv_end - key0 - 1
        a = key0 * 2 * D + np.minimum(offs // (2 * D), last_row) * (2 * D) + offs % (2 * D)
    return int(a.min()), int(a.max()) + 16


def check_prefill(pos, T, hq, hkv, D, max_ctx):
    """Every direct-to-LDS load and q-operand load of one prefill launch."""
    RB = 2 * D
    RSK, RSV = RB + 16, RB + 64
    pk, pv = tile_plan(D, RSK), tile_plan(D, RSV)
    group = hq // hkv
    n_qtiles = (T + P_QROWS - 1) // P_QROWS
    n_pairs = (n_qtiles + 1) // 2
    n_hgroups = (group + P_HEADS - 1) // P_HEADS
    head_bytes = max_ctx * 2 * D
    calls = set()
    kv_end_of = lambda qt: pos + min(T, qt * P_QROWS + P_QROWS)
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
            qt = heavy if sel == 0 else pair
            q0 = qt * P_QROWS
            # q rows, staged along rows: kQOperand lane (g, m) reads f16 elements
            # 8 m + [0, 8) of row min(q0 + RPI it + g, T - 1); f32 q lane (g, m) reads
            # elements 4 m + [0, 4) and D/2 + 4 m + [0, 4) of that row, and the same of
            # its cos/sin row (D floats per token)
            lane = np.arange(64)
            for LPR, els in ((D // 8, 8 * (lane % (D // 8))[:, None] + np.arange(8)),
                             (D // 8, np.concatenate([4 * (lane % (D // 8))[:, None] + np.arange(4),
                                                      D // 2 + 4 * (lane % (D // 8))[:, None] + np.arange(4)], 1))):
                RPI = 64 // LPR
                rows = np.minimum(q0 + (RPI * np.arange(P_QROWS // RPI)[:, None] + lane[None, :] // LPR), T - 1)
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
    for key0, end in calls:
        assert 0 < end <= max_ctx
        for plan in (pk, pv):
            lo, hi = dma_extent(D, plan, key0, end)
            assert lo >= 0 and hi <= head_bytes, (key0, end, lo, hi)
    return len(calls)


@pytest.mark.parametrize("pos,T,hq,hkv,D,cap", [
    (0, 2048, 32, 4, 128, 2048),     # C2
    (0, 300, 32, 4, 128, 307), (100, 130, 32, 4, 128, 237), (5, 77, 32, 4, 64, 89), (0, 2, 32, 4, 128, 9),
    (0, 97, 32, 4, 128, 104), (48, 160, 32, 4, 128, 215), (31, 200, 64, 4, 128, 238), (3, 96, 6, 3, 128, 106), (0, 65, 8, 8, 64, 72),
])
def test_prefill_dma_addresses(pos, T, hq, hkv, D, cap):
    """C2 and the GPU parity suite's prefill shapes (chunked continuations, odd q-tile counts)."""
    assert check_prefill(pos, T, hq, hkv, D, cap) > 0
