"""Host-side replay of the kernels' index mapping for every entry of the explicit tile lists (the
analogue of the reference's gemm/verifier.py mapping_check, :135-176): at ragged shapes, each output
is written exactly once, each weight chunk / k step is read and reduced exactly once, and every load
either lands inside its buffer at the element it stands for or is a deliberate out-of-range offset
(answered with zeros by the buffer resource) that cannot wrap the 32-bit offset. The entries come
from the library (q4_gemv_config_info, q4_gemv_mx_config_info, gemm_f16_config_info,
q4_linear_ws_config_info); the index formulas restate the kernels (file:function cited per test).
No GPU is needed."""

import numpy as np
import pytest

from q4llm._lib import config_table

OOB = 0x80000000


def cdiv(a, b):
    return -(-a // b)


# ------------------------------------------------------------------------------------------------
# VALU decode GEMV (csrc/q4_gemv.hip: q4_gemv_kernel, load_item / compute_item / stage_store)
# ------------------------------------------------------------------------------------------------

def gemv_fits(cfg, N, K):
    lpr, cpl, r, waves, xw, multi = cfg
    cpr = K // 32
    if K // 8 > xw * 64 * waves:
        return False
    if not multi and lpr * cpl < cpr:
        return False
    return True


def replay_gemv(cfg, N, K, gshift, paired):
    lpr, cpl, R, waves, xw, multi = cfg
    cpr, spr, nwords = K // 32, (K // 32) >> gshift, K // 8
    rows_per_wave = R * (64 // lpr)
    rows_wg = rows_per_wave * waves
    n_blocks = cdiv(N, rows_wg)
    grid = min(n_blocks, 1024) if multi else n_blocks
    n_kpass = cdiv(cpr, lpr * cpl) if multi else 1
    wbytes, sbytes = N * (K // 2), N * spr * 2
    reads = np.zeros((N, cpr), np.int32)
    sreads = np.zeros((N, spr), np.int32)
    stores = np.zeros(N if not paired else N // 2, np.int32)

    def phys(v):
        if not paired:
            return v
        pr, b = v >> 1, v & 1
        return N if pr >= N // 2 else pr + b * (N // 2)  # SwiGLU pairing

    lane = np.arange(64)
    lr, rg = lane % lpr, lane // lpr
    for blk in range(grid):
        my = cdiv(n_blocks - blk, grid) if blk < n_blocks else 0
        n_items = my * n_kpass if multi else 1
        # grid-stride loops run items in pairs (it, it + 1); the odd tail item is past the end
        items = range(n_items + (n_items % 2) if multi else 1)
        for wave in range(waves):
            for it in items:
                kp = it % n_kpass
                row0 = (blk + (it // n_kpass) * grid) * rows_wg + wave * rows_per_wave + rg * R
                for rr in range(R):
                    v = row0 + rr
                    row = np.array([phys(int(x)) for x in v])
                    for i in range(cpl):
                        c = kp * (lpr * cpl) + i * lpr + lr
                        woff = np.where(c < cpr, row.astype(np.int64) * (K // 2) + c * 16, OOB)
                        soff = np.where(c < cpr, (row.astype(np.int64) * spr + (c >> gshift)) * 2, OOB)
                        assert (woff < 2 ** 32).all() and (soff < 2 ** 32).all(), "offset wraps"
                        live = (woff < wbytes) & (c < cpr)
                        assert ((woff >= wbytes) | live).all()
                        np.add.at(reads, (row[live], c[live]), 1)
                        sl = soff < sbytes
                        np.add.at(sreads, (row[sl], (c[sl] >> gshift)), 1)
                if kp == n_kpass - 1:
                    last = lr == lpr - 1
                    if paired:
                        pr = (row0[last] >> 1)
                        np.add.at(stores, pr[pr < N // 2], 1)
                    else:
                        for rr in range(R):
                            rows = (row0 + rr)[last]
                            np.add.at(stores, rows[rows < N], 1)
    assert (reads == 1).all(), "weight chunks read other than once"
    assert (sreads == 1 << gshift).all(), "each scale feeds its group's chunks"
    assert (stores == 1).all(), "outputs stored other than once"
    # x staging: word wd = thread + i * threads, i < xw, each word of K staged once
    thr = np.arange(64 * waves)
    wd = (thr[None, :] + np.arange(xw)[:, None] * 64 * waves).ravel()
    staged = np.bincount(wd[wd < nwords], minlength=nwords)
    assert (staged == 1).all()


@pytest.mark.parametrize("idx", range(len(config_table("gemv"))))
def test_gemv_entries_cover_once(idx):
    cfg = config_table("gemv")[idx]
    lpr, cpl, r, waves, xw, multi = cfg
    ran = 0
    for K in (256, 704, 1024, 3072, 4096, 8192):
        for N in (40, 1000, 3 * 64 * waves + 7):
            if not gemv_fits(cfg, N, K) or (multi and N > 2000):
                continue
            for gshift in (0, 2):
                if (K // 32) % (1 << gshift):
                    continue
                replay_gemv(cfg, N, K, gshift, False)
                if r == 2 and not multi:
                    replay_gemv(cfg, N - N % 2, K, gshift, True)
                ran += 1
            break
    assert ran > 0


# ------------------------------------------------------------------------------------------------
# Matrix-core decode GEMV (csrc/q4_gemv_mx.hip: q4_gemv_mx_kernel issue / compute, both layouts)
# ------------------------------------------------------------------------------------------------

def mx_fits(cfg, n_tiles, nblk):
    rbw, wpb, tpw, rpb, multi = cfg
    return n_tiles == wpb * tpw and 64 * rbw * wpb >= nblk


def replay_mx(cfg, N, K, G, pair, tiled):
    rbw, wpb, tpw, rpb, multi = cfg
    seg_per_tile = 4 * G // 128
    n_tiles = cdiv(K, 4 * G)
    nseg = n_tiles * seg_per_tile
    kg = K // G
    n_rb = cdiv(N // 2, 8) if pair else cdiv(N, rpb)
    n_t16 = cdiv(N // 2, 8) if pair else cdiv(N, 16)
    wbytes = n_t16 * nseg * 1024 if tiled else N * (K // 2)
    n_wg = cdiv(n_rb, rbw)
    grid = min(n_wg, 1024) if multi else n_wg
    reads = np.zeros((N, cdiv(K, 32)), np.int32)
    stores = np.zeros(N // 2 if pair else N, np.int32)

    def phys(rb, v):  # q4_gemv_mx.hip phys_row (SwiGLU pairing for pair=True)
        if not pair:
            r = rb * rpb + v
            return r if (v < rpb and r < N) else -1
        p = rb * 8 + (v & 7)
        if p >= N // 2:
            return -1
        return p + (N // 2 if v >= 8 else 0)

    lane = np.arange(64)
    c, b = lane & 15, lane >> 4
    for wg0 in range(grid):
        my = cdiv(n_wg - wg0, grid) if wg0 < n_wg else 0
        wgs = [wg0 + it * grid for it in range(my)] if multi else [wg0]
        for wg in wgs:
            for wave in range(rbw * wpb):
                rbl, wp = wave // wpb, wave % wpb
                rb = wg * rbw + rbl
                for i in range(tpw):
                    T = wp * tpw + i
                    for sg in range(seg_per_tile):
                        seg = T * seg_per_tile + sg
                        for ln in range(64):
                            if rb >= n_rb:
                                continue
                            k0 = seg * 128 + 32 * b[ln]
                            row = phys(rb, c[ln])
                            if tiled:
                                vr = rb * rpb + c[ln] if not pair else rb * 16 + c[ln]
                                ok = rb < n_rb and c[ln] < rpb and (pair or vr < N) and k0 < K
                                off = ((vr >> 4) * nseg + seg) * 1024 + (vr & 15) * 64 + 16 * b[ln] if ok else OOB
                            else:
                                ok = row >= 0 and k0 < K
                                off = row * (K // 2) + 64 * seg + 16 * b[ln] if ok else OOB
                            assert off < 2 ** 32
                            if off < wbytes and row >= 0 and k0 < K:
                                if not tiled:
                                    assert off == row * (K // 2) + k0 // 2
                                reads[row, k0 // 32] += 1
            # epilogue: thread tid < 16 RBW finishes virtual row tid % 16 of block tid / 16
            for tid in range(16 * rbw):
                rb, v = wg * rbw + tid // 16, tid % 16
                if rb >= n_rb:
                    continue
                if pair:
                    p = rb * 8 + v
                    if v < 8 and p < N // 2:
                        stores[p] += 1
                else:
                    row = rb * rpb + v
                    if v < rpb and row < N:
                        stores[row] += 1
    assert (reads == 1).all(), "weight chunks read other than once"
    assert (stores == 1).all(), "outputs stored other than once"
    if tiled and not pair:
        # T16 scales: lane group b of row block rb loads 4 consecutive rows vs..vs+3 (one 8-byte load):
        # aligned, inside one 16-row tile, and covering every used row of the block once
        seen = np.zeros(N, np.int32)
        for rb in range(n_rb):
            for bb in range(4):
                if 4 * bb >= rpb:
                    continue
                vs = rb * rpb + 4 * bb
                assert vs % 4 == 0 and (vs >> 4) == ((vs + 3) >> 4)
                for t in range(4):
                    if 4 * bb + t < rpb and vs + t < N:
                        seen[vs + t] += 1
        assert (seen == 1).all(), "scale rows loaded other than once"
    # x prologue: thread tid owns 16-k block tid (< nblk)
    assert 64 * rbw * wpb >= n_tiles * (4 * G // 16)


@pytest.mark.parametrize("idx", range(len(config_table("gemv_mx"))))
def test_mx_entries_cover_once(idx):
    cfg = config_table("gemv_mx")[idx]
    rbw, wpb, tpw, rpb, multi = cfg
    ran = 0
    for G, K in ((128, 3072), (128, 8192), (32, 256), (32, 704)):
        n_tiles = cdiv(K, 4 * G)
        if not mx_fits(cfg, n_tiles, n_tiles * 4 * G // 16):
            continue
        if G == 32 and idx not in (0, 1, 2, 3, 17):
            continue
        for N in (48, 250):
            for tiled in (False, True):
                replay_mx(cfg, N, K, G, False, tiled)
                if rpb == 16:
                    replay_mx(cfg, N, K, G, True, tiled)
                ran += 1
        break
    assert ran > 0


# ------------------------------------------------------------------------------------------------
# fp16 GEMM (csrc/gemm_f16.hip: gemm_f16_nt_kernel)
# ------------------------------------------------------------------------------------------------

def swz(bk, r):
    return (r >> 1) & 7 if bk == 64 else (r >> 2) & 3


def tile_of(bid, tiles_m, tiles_n, remap):
    ntiles = tiles_m * tiles_n
    if remap:
        bid = (bid % 8) * (ntiles // 8) + bid // 8
    group = bid // (4 * tiles_n)
    first_m = group * 4
    gsize = min(tiles_m - first_m, 4)
    in_group = bid - group * 4 * tiles_n
    return first_m + in_group % gsize, in_group // gsize


def gemm_split(cfg, M, N, K, force=None):
    """K split of a tile entry (csrc/gemm_f16.hip: gemm_split_plan): (n_split, nk_split)."""
    bm, bn, wm, wn, nst, bk, sp = cfg
    if N % 4 or M <= 1:
        return 1, 0
    nk = cdiv(K, bk)
    tiles = cdiv(M, bm) * cdiv(N, bn)
    want = min(256 // tiles, nk // 4) if M < 512 else 1
    if 2.0 * M * N * K < 4e9:  # small problems: ~256 workgroups, K ranges of >= 8 steps
        want = min((512 // tiles + 1) // 2, nk // 8)
    if force is not None:
        want = force
    if want <= 1 or nk < 2:
        return 1, 0
    nk_s = cdiv(nk, min(want, nk))
    S = cdiv(nk, nk_s)
    return (S, nk_s) if S >= 2 else (1, 0)


def replay_gemm(cfg, M, N, K, force_split=None):
    """gemm_f16_nt_kernel: workgroup -> (K range, tile) mapping, the direct loads of one stage (lane
    offsets, row blocks, LDS slots), operand reads and epilogue stores."""
    bm, bn, wm, wn, nst, bk, sp = cfg
    waves = wm * wn
    row_b = bk * 2
    rows_per_inst = 1024 // row_b
    kcpr = bk // 8
    kai = cdiv(bm // rows_per_inst, waves)
    kbi = cdiv(bn // rows_per_inst, waves)
    rows_per_j = waves * rows_per_inst
    tiles_m, tiles_n = cdiv(M, bm), cdiv(N, bn)
    ntiles = tiles_m * tiles_n
    nk = cdiv(K, bk)
    S, nk_s = gemm_split(cfg, M, N, K, force_split)
    grid = ntiles * S
    remap = 1 if grid % 8 == 0 else 0
    seen = np.zeros((S, tiles_m, tiles_n), np.int32)
    for g in range(grid):
        gg = (g % 8) * (grid // 8) + g // 8 if remap else g
        ksp = gg // ntiles
        tm, tn = tile_of(gg - ksp * ntiles, tiles_m, tiles_n, 0)
        seen[ksp, tm, tn] += 1
    assert (seen == 1).all(), "workgroup order is not a permutation of (K range, tile)"
    ksteps = np.zeros(nk, np.int32)
    for ksp in range(S):
        kt0 = ksp * nk_s if S > 1 else 0
        n = min(nk_s, nk - kt0) if S > 1 else nk
        assert n >= 1, "empty K range"
        ksteps[kt0:kt0 + n] += 1
    assert (ksteps == 1).all(), "K steps reduced other than once"
    lane = np.arange(64)
    lda = ldb = K
    abytes, bbytes = (M - 1) * lda * 2 + K * 2, (N - 1) * ldb * 2 + K * 2
    # one stage of the first and of the last (ragged) tile, at the first and the last K step
    for (m0, n0) in ((0, 0), ((tiles_m - 1) * bm, (tiles_n - 1) * bn)):
        full = m0 + bm <= M and n0 + bn <= N
        for nrows, base, nbytes, ld, ni, limit in ((bm, m0, abytes, lda, kai, M), (bn, n0, bbytes, ldb, kbi, N)):
            for k0 in (0, (nk - 1) * bk):
                filled = np.zeros((nrows, kcpr), np.int32)
                fast = full and k0 + bk <= K
                for wave in range(waves):
                    r0 = wave * rows_per_inst + lane // kcpr
                    chunk = (lane % kcpr) ^ swz(bk, r0)
                    lane_off = (base + r0) * ld * 2 + chunk * 16
                    left = limit - base - r0
                    for j in range(ni):
                        blk = wave + j * waves
                        r = r0 + j * rows_per_j
                        real = blk < nrows // rows_per_inst
                        if not real:
                            continue  # spare instructions land in the junk area
                        # the chunk formula of row r gives the lane's chunk for every j
                        assert (chunk == ((lane % kcpr) ^ swz(bk, r))).all()
                        for ln in range(64):
                            g_row, g_k = base + r[ln], k0 + 8 * chunk[ln]
                            in_range = g_row < limit and g_k < K
                            if fast:
                                off = lane_off[ln] + k0 * 2 + j * rows_per_j * ld * 2
                                assert in_range
                            else:
                                ok = g_k < K and j * rows_per_j < left[ln]
                                assert ok == in_range
                                off = lane_off[ln] + j * rows_per_j * ld * 2 + k0 * 2 if ok else OOB
                            assert off < 2 ** 31 or off == OOB
                            if in_range:
                                assert off == g_row * ld * 2 + g_k * 2 and off < nbytes
                            filled[r[ln], ln % kcpr] += 1
                            # the reader of (row, chunk c) looks at slot c ^ swz(row): it holds chunk c
                            assert ((ln % kcpr) ^ swz(bk, r[ln])) == chunk[ln]
                assert (filled == 1).all(), "LDS stage slots filled other than once"
    # operand reads: lane supplies row lane % 32 and chunk 2 kk + lane / 32 of each 16-k step
    ks = np.zeros(bk // 8, np.int32)
    for kk in range(bk // 16):
        for ln in range(64):
            ks[2 * kk + ln // 32] += 1
    assert (ks == 32).all()
    # epilogue: (i, j, e, lane) -> (row, col) covers the tile once
    wtm, wtn = bm // wm, bn // wn
    out = np.zeros((bm, bn), np.int32)
    for wave in range(waves):
        wmi, wni = wave // wn, wave % wn
        for i in range(wtm // 32):
            for j in range(wtn // 32):
                for e in range(16):
                    row = wmi * wtm + i * 32 + 8 * (e // 4) + 4 * (lane >> 5) + (e % 4)
                    col = wni * wtn + j * 32 + (lane & 31)
                    np.add.at(out, (row, col), 1)
    assert (out == 1).all(), "tile outputs stored other than once"


@pytest.mark.parametrize("idx", range(len(config_table("gemm"))))
def test_gemm_entries_cover_once(idx):
    cfg = config_table("gemm")[idx]
    for (M, N, K) in ((300, 520, 200), (cfg[0] * 2, cfg[1] * 4, 512), (256, 3072, 8192)):
        replay_gemm(cfg, M, N, K)
    for force in (2, 3, 5):  # K splits: forced counts, ragged K, and the automatic rule
        replay_gemm(cfg, 300, 520, 200 + 64 * 9, force)
    replay_gemm(cfg, 256, 5120, 3072)


def test_gemm_split_rule_fills_the_cus():
    """The automatic K split of the 256-row config-3 shapes on the pipelined 128x128 entry."""
    cfg = next(c for c in config_table("gemm") if c[:6] == (128, 128, 2, 2, 4, 64) and c[6])
    assert gemm_split(cfg, 256, 5120, 3072) == (3, 16)   # 80 tiles x 3
    assert gemm_split(cfg, 256, 3072, 8192) == (5, 26)   # 48 tiles x 5 (last range 24 steps)
    assert gemm_split(cfg, 256, 16384, 3072) == (1, 0)   # 256 tiles fill the CUs
    assert gemm_split(cfg, 1024, 5120, 3072) == (1, 0)   # no split from 512 rows on
    # problems under 4 GFLOP (the reference's S1-S8) take the 64x64 entry and about 256 workgroups
    c64 = next(c for c in config_table("gemm") if c[:2] == (64, 64))
    assert gemm_split(c64, 1024, 1024, 1024) == (1, 0)   # S1: 256 tiles
    assert gemm_split(c64, 128, 3072, 3072) == (3, 16)   # S2: 96 tiles x 3
    assert gemm_split(c64, 4096, 64, 1024) == (2, 8)     # S3: 64 tiles x 2 (8-step ranges)
    assert gemm_split(c64, 16, 4096, 4096) == (4, 16)    # S4: 64 tiles x 4
    assert gemm_split(c64, 256, 256, 8192) == (16, 8)    # S5: 16 tiles x 16
    assert gemm_split(c64, 768, 768, 768) == (1, 0)      # S8: 144 tiles, 12 steps


# ------------------------------------------------------------------------------------------------
# W4A16 prefill GEMM (csrc/q4_linear.hip: q4_linear_ws_kernel)
# ------------------------------------------------------------------------------------------------

def replay_linear_ws(cfg, M, N, K, group):
    bm, bn, wm, wn, nst, ks_n, pipe = cfg
    waves = wm * wn * ks_n
    kai = cdiv(bm // 8, waves)
    kbi = cdiv(bn // 32, waves)
    gshift = group.bit_length() - 1
    spr = K >> gshift
    tiles_n = cdiv(N, bn)
    tiles = cdiv(M, bm) * tiles_n
    seen = np.zeros(tiles, np.int32)
    lane = np.arange(64)
    for blk in range(tiles):
        seen[(blk // tiles_n) * tiles_n + blk % tiles_n] += 1
    assert (seen == 1).all()
    # x planes: rows 8b..8b+7 per instruction, slot lane % 8 of row 8b + lane / 8 holds chunk slot ^ ((r >> 1) & 7)
    xfill = np.zeros((bm, 8), np.int32)
    for wave in range(waves):
        for j in range(kai):
            b = wave + j * waves
            if b >= bm // 8:
                continue
            r = 8 * b + (lane >> 3)
            chunk = (lane & 7) ^ ((r >> 1) & 7)
            np.add.at(xfill, (r, lane & 7), 1)
            # the reader of chunk c of row r (c ^ ((r >> 1) & 7) slot) finds chunk c
            assert (((lane & 7) ^ ((r >> 1) & 7)) == chunk).all()
    assert (xfill == 1).all()
    # weights: rows 32b + lane / 2, 16-byte half lane % 2 of the 32-byte (64-nibble) step row
    wfill = np.zeros((bn, 2), np.int32)
    for wave in range(waves):
        for j in range(kbi):
            b = wave + j * waves
            if b >= bn // 32:
                continue
            np.add.at(wfill, (32 * b + (lane >> 1), lane & 1), 1)
    assert (wfill == 1).all()
    # k split: 16-k step kk of each 64-k stage belongs to wave group kk // (4 / KS); every step once
    kk_owner = np.zeros(4, np.int32)
    for ksi in range(ks_n):
        for q in range(4 // ks_n):
            kk_owner[ksi * (4 // ks_n) + q] += 1
    assert (kk_owner == 1).all()
    # group scales: applied once per group at its last 16-k step (or, k-split, per wave part)
    applied = np.zeros((K >> gshift), np.int32)
    for k0 in range(0, K, 64):
        for ksi in range(ks_n):
            for q in range(4 // ks_n):
                kk = ksi * (4 // ks_n) + q
                k = k0 + 16 * kk
                ends_here = ((k + 16) & (group - 1)) == 0
                ends_in_stage = ks_n > 1 and q == 4 // ks_n - 1 and ((((k >> gshift) + 1) << gshift) <= k0 + 64)
                if ends_here or ends_in_stage:
                    applied[k >> gshift] += 1
                    # the scale slot used must be one of the stage's two groups
                    assert (k >> gshift) - (k0 >> gshift) in (0, 1)
    per_group = ks_n if group < 64 else 1
    assert (applied >= 1).all()
    if ks_n == 1:
        assert (applied == 1).all()
    # epilogue: each tile output once
    wtm, wtn = bm // wm, bn // wn
    out = np.zeros((bm, bn), np.int32)
    for wt in range(wm * wn):
        wmi, wni = wt // wn, wt % wn
        for i in range(wtm // 32):
            for j in range(wtn // 32):
                for e in range(16):
                    row = wmi * wtm + i * 32 + 8 * (e // 4) + 4 * (lane >> 5) + (e % 4)
                    col = wni * wtn + j * 32 + (lane & 31)
                    np.add.at(out, (row, col), 1)
    assert (out == 1).all()
    del per_group


@pytest.mark.parametrize("idx", range(len(config_table("linear_ws"))))
def test_linear_ws_entries_cover_once(idx):
    cfg = config_table("linear_ws")[idx]
    for group in (32, 128):
        replay_linear_ws(cfg, 100, 3 * cfg[1] + 32, 512, group)


@pytest.mark.parametrize("bk", [64, 32])
def test_gemm_swizzle_is_bank_conflict_free(bk):
    """An MFMA operand read takes 16 consecutive tile rows at one 16-byte chunk; gfx950's LDS serves
    16 lanes x 16 bytes per clock from 16 groups of 16 bytes, so the 16 addresses must fall in 16
    distinct groups (csrc/gemm_f16.hip swz)."""
    row_b = bk * 2
    for c in range(bk // 8):
        for r0 in range(0, 256, 16):
            groups = {((r * row_b + ((c ^ swz(bk, r)) << 4)) // 16) % 16 for r in range(r0, r0 + 16)}
            assert len(groups) == 16, (c, r0)
    # and the identity mapping (no swizzle) would not be: the check discriminates
    groups = {((r * row_b) // 16) % 16 for r in range(16)}
    assert len(groups) < 16


# ------------------------------------------------------------------------------------------------
# W4A16 prefill GEMM reading the decode T16 copy (csrc/q4_linear.hip: q4_linear_ws_kernel, T16 = true;
# layout: csrc/q4_t16.hip t16_pack_weights / t16_pack_scales / t16_row)
# ------------------------------------------------------------------------------------------------

def t16_row(vr, N, pairing, hd):
    """Weight row of T16 virtual row vr (-1: padding); pairing 0 none, 1 SwiGLU, 2 RoPE."""
    if pairing == 0:
        return vr if vr < N else -1
    v = vr & 15
    p = (vr >> 4) * 8 + (v & 7)
    if p >= N // 2:
        return -1
    if pairing == 1:
        return p + (N // 2 if v >= 8 else 0)
    hh = hd // 2
    head, d = divmod(p, hh)
    return head * hd + d + (hh if v >= 8 else 0)


def t16_pack(qbytes, sc, N, K, group, pairing, hd):
    """Byte image of the T16 tiles and the fp16 scale array, restated from q4_t16.hip."""
    tile_k = 4 * group
    n_tiles = cdiv(K, tile_k)
    nseg = n_tiles * tile_k // 128
    n_t16 = cdiv(N, 16) if pairing == 0 else cdiv(N // 2, 8)
    tiles = np.zeros((n_t16, nseg, 16, 64), np.uint8)
    scales = np.zeros((n_t16, n_tiles, 4, 16), np.uint16)
    kg = K // group
    for t in range(n_t16):
        for v in range(16):
            row = t16_row(16 * t + v, N, pairing, hd)
            if row < 0:
                continue
            for seg in range(nseg):
                k0 = seg * 128
                if k0 < K:
                    tiles[t, seg, v] = qbytes[row, k0 // 2:k0 // 2 + 64]
            for T in range(n_tiles):
                for q in range(4):
                    if 4 * T + q < kg:
                        scales[t, T, q, v] = sc[row, 4 * T + q]
    return tiles.reshape(-1), scales.reshape(-1), n_t16, n_tiles, nseg


@pytest.mark.parametrize("pairing,N,K,group", [(0, 200, 1024, 128), (2, 256 + 64, 768, 128), (1, 512 + 32, 512, 32),
                                               (0, 96, 1536, 32)])
def test_linear_ws_t16_loads_and_outputs(pairing, N, K, group):
    """Every 1 KB weight load of a 64-k stage of 32 virtual columns brings, for LDS row r (lane / 2), the
    64 nibbles of weight row t16_row(column) at that stage; every scale slot holds the fp16 scale of that
    row and the stage's group; and the epilogue writes each virtual column to t16_row (EPI 0, every
    pairing) and, for the SwiGLU epilogue, each pair once from the lane holding gate with up 8 columns
    away."""
    hd = 64
    cfg = config_table("linear_ws")[-1]
    bm, bn, wm, wn, nst, ks_n, pipe = cfg
    assert bn % 128 == 0 and ks_n == 1 and pipe == 1
    waves = wm * wn
    rng = np.random.default_rng(N + K)
    qbytes = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    sc = rng.integers(0, 0x7BFF, size=(N, K // group), dtype=np.uint16)
    tiles, scales, n_t16, n_tiles, nseg = t16_pack(qbytes, sc, N, K, group, pairing, hd)
    lane = np.arange(64)
    gshift = group.bit_length() - 1
    for n0 in range(0, cdiv(N, bn) * bn, bn):
        for kt in range(K // 64):
            k0 = 64 * kt
            # weights: instruction j of wave w fills virtual rows 32 b .. 32 b + 31, b = w + j waves
            for b in range(bn // 32):
                t = (n0 + 32 * b) // 16 + (lane >> 5)
                off = t * nseg * 1024 + ((lane & 31) >> 1) * 64 + (lane & 1) * 16 + (kt >> 1) * 1024 + (kt & 1) * 32
                for ln in range(64):
                    vc = n0 + 32 * b + ln // 2
                    got = tiles[off[ln]:off[ln] + 16] if t[ln] < n_t16 else np.zeros(16, np.uint8)
                    row = t16_row(vc, N, pairing, hd) if vc < 16 * n_t16 else -1
                    want = qbytes[row, k0 // 2 + 16 * (ln & 1): k0 // 2 + 16 * (ln & 1) + 16] if row >= 0 else 0
                    assert (got == want).all(), (n0, kt, b, ln)
            # scales: instruction i (< 2 bn / 128) fills slot i // (bn / 128), part i % (bn / 128)
            parts = bn // 128
            for i in range(2 * parts):
                slot, part = divmod(i, parts)
                g = (k0 >> gshift) if slot == 0 else ((k0 + 63) >> gshift)
                t = n0 // 16 + part * 8 + (lane >> 3)
                e = ((t * n_tiles + (g >> 2)) * 4 + (g & 3)) * 16 + 2 * (lane & 7)
                for ln in range(64):
                    for h in range(2):
                        col = part * 128 + 2 * ln + h  # virtual column of the fp16 in LDS
                        vc = n0 + col
                        row = t16_row(vc, N, pairing, hd) if vc < 16 * n_t16 else -1
                        got = scales[e[ln] + h] if t[ln] < n_t16 else 0
                        assert got == (sc[row, g] if row >= 0 else 0), (n0, kt, i, ln, h)
        assert waves * 1 >= 2 * (bn // 128)  # one scale instruction per wave covers both slots
    # epilogue column mapping (q4_linear_ws_kernel: the T16 branches of the EPI 0 / EPI 1 stores)
    cols = np.arange(16 * n_t16)
    if pairing == 1:
        # tiles j, j + 1 (32 columns each) paired: lane l with l % 16 < 8 takes gate column c of tile j
        # and its up at c + 8 (from lane l ^ 8); lane l with l % 16 >= 8 takes up column c of tile j + 1
        # and its gate at c - 8; both write pair 8 (c / 16) + c % 8
        seen = np.zeros(N // 2, np.int32)
        for base in range(0, 16 * n_t16, 64):
            for ln in range(32):
                hi8 = (ln & 8) != 0
                vc = base + (32 if hi8 else 0) + ln
                gate_c, up_c = (vc - 8, vc) if hi8 else (vc, vc + 8)
                pr = 8 * (vc >> 4) + (vc & 7)
                if vc < 16 * n_t16 and pr < N // 2:
                    assert t16_row(gate_c, N, 1, hd) == pr and t16_row(up_c, N, 1, hd) == pr + N // 2
                    seen[pr] += 1
        assert (seen == 1).all()
        # EPI 0 (K-split partials, or gate/up before a separate SwiGLU): each virtual column to its row
        seen = np.zeros(N, np.int32)
        for vc in cols:
            pr = 8 * (vc >> 4) + (vc & 7)
            col = pr + (N // 2 if vc & 8 else 0) if pr < N // 2 else N
            if col < N:
                assert col == t16_row(vc, N, 1, hd)
                seen[col] += 1
        assert (seen == 1).all()
    else:
        seen = np.zeros(N, np.int32)
        for vc in cols:
            col = vc
            if pairing == 2:
                pr, hh = 8 * (vc >> 4) + (vc & 7), hd >> 1
                sh = hh.bit_length() - 1
                head = pr >> sh
                col = head * hd + (pr - (head << sh)) + (hh if vc & 8 else 0) if pr < N // 2 else N
            if col < N:
                assert col == t16_row(vc, N, pairing, hd)
                seen[col] += 1
        assert (seen == 1).all()

