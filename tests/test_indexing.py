"""The indexing contract of every kernel route, checked on the CPU.

For each projection shape the library's own host routing decides the
launch (w8a8_diag_linear_route / w8a8_diag_argmax_route: the kernel family,
its compile-time shape and grid -- gemm_route / gemv_route in the library),
and this file replays that kernel's address arithmetic over the whole grid,
with numpy over every workgroup, wave and lane.  Every global read must lie
inside its operand, every LDS access inside the kernel's LDS array, every
store inside its output, and every output element (every slab element for a
split-K launch) must be written exactly once.  K loops are checked at their
extreme iterations: each address is affine in the loop counter.

The replay restates the index expressions of the kernels, each function
citing the source lines it follows; the table in the design notes states the
same bounds in words.  Shapes: the benchmark configurations (C1-C5: the
decode shapes at M = 1, the lm_head, M = 129 and 512, the ragged M = 4 / 16 /
64), the M = 129 tails (M = 129-135 and 136-159, sampled), N not a multiple
of 96, K not a multiple of 128, and the folded producers' and SwiGLU
kernels' fixed launch shapes.  This is the reference's checked build
(tools/cuda.sh:15-19) in host form.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import seeded_linear_shapes
from inferrous_amd import _lib

F32, BF16, I32 = 0, 1, 2  # W8A8_OUT_* (include/inferrous_w8a8.h)
AUTO, DOT4, MFMA = 0, 1, 2  # W8A8_PATH_*
ROUTE_LEN = 20
DECODE = [(6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288)]


def route(m, n, k, dtype=BF16, residual=False, path=AUTO, workspace=0):
    r = np.zeros(ROUTE_LEN, np.int32)
    st = _lib.lib().w8a8_diag_linear_route(m, n, k, dtype, int(residual), path, workspace, r.ctypes.data,
                                           ROUTE_LEN)
    assert st == 0, st
    keys = ("family grid_x grid_y block bm bn wm wn sa sb ma mt s u splits nt epi_cols rows kc waves").split()
    return dict(zip(keys, (int(v) for v in r)))


def argmax_route(n, k):
    r = np.zeros(ROUTE_LEN, np.int32)
    assert _lib.lib().w8a8_diag_argmax_route(n, k, r.ctypes.data, ROUTE_LEN) == 0
    keys = ("family grid_x grid_y block bm bn wm wn sa sb ma mt s u splits nt epi_cols rows kc waves").split()
    return dict(zip(keys, (int(v) for v in r)))


def workspace_bytes(m, n, k):
    return int(_lib.lib().w8a8_linear_workspace_bytes(m, n, k))


# ------------------------------------------------------------------ helpers
def within(name, lo, hi, size):
    """Every access [lo, hi) (arrays of byte or element offsets) inside [0, size)."""
    lo = np.asarray(lo)
    hi = np.asarray(hi)
    if lo.size == 0:
        return
    assert lo.min() >= 0, f"{name}: access below the buffer ({lo.min()})"
    assert hi.max() <= size, f"{name}: access past the buffer ({hi.max()} > {size})"


def written_once(name, idx, total):
    """Stores at element offsets idx: inside [0, total) and each element once."""
    idx = np.asarray(idx, np.int64).ravel()
    assert idx.size == total, f"{name}: {idx.size} stores for {total} elements"
    within(name, idx, idx + 1, total)
    counts = np.bincount(idx, minlength=total)
    assert counts.max() == 1 and counts.min() == 1, f"{name}: an element is written {counts.max()} times " \
                                                    f"or not at all"


def xcd_slot(b, G):
    """Workgroup b's slot among G (gemm.hip / gemv.hip xcd_slot): XCD-major when G % 8 == 0."""
    b = np.asarray(b)
    return (b % 8) * (G // 8) + b // 8 if G % 8 == 0 else b


def mfma32_rows_cols(lane, v):
    """Row / column of value v of lane l in a 32 x 32 i32 MFMA block (gemm.hip:382-384)."""
    return (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3), lane & 31


def frag_offsets():
    """gemm_dma / gemm_tall fragment reads: lane l, sub-step i -> byte offset
    inside a 32-row block of 128-byte LDS rows (gemm.hip:559-562, :829-832)."""
    lane = np.arange(64)
    fr, fh = lane & 31, lane >> 5
    return np.stack([fr * 128 + (((2 * i + fh) ^ ((fr >> 1) & 7)) * 16) for i in range(4)])  # [4, 64]


# ------------------------------------------------------------------ GEMM routes
def store_blocks(m, n, row0, col0, FM, FN):
    """(rows, cols) that store_blocks writes for wave tiles with top-left
    corners (row0, col0) (broadcast arrays), guarded by r < m, c < n
    (gemm.hip:389-460).  Its epilogue loads are clamped (min(r, m - 1),
    min(c, n - 1)), hence always in bounds."""
    lane = np.arange(64)[:, None]
    v = np.arange(16)[None, :]
    rr, cc = mfma32_rows_cols(lane, v)                      # [64, 16]
    # [..., FM, FN, lane, v]
    rows = np.asarray(row0)[..., None, None, None, None] + 32 * np.arange(FM)[:, None, None, None] + rr
    cols = (np.asarray(col0)[..., None, None, None, None] + 32 * np.arange(FN)[:, None, None]
            + np.zeros_like(v) + (lane & 31))
    rows, cols = np.broadcast_arrays(rows, cols)
    keep = (rows < m) & (cols < n)
    return rows[keep].astype(np.int64), cols[keep].astype(np.int64)


def check_dma(m, n, k, r, residual):
    """gemm_dma (gemm.hip:483-629) over its grid: DMA sources, LDS ring slots,
    fragment reads, the stores of store_blocks."""
    BM, BN, WM, WN, SA, SB, splits = r["bm"], r["bn"], r["wm"], r["wn"], r["sa"], r["sb"], r["splits"]
    tm, tn = -(-m // BM), -(-n // BN)
    T, G = tm * tn, tm * tn * splits
    assert r["grid_x"] == G and r["block"] == 512
    assert k % 128 == 0 and (k // 128) % splits == 0
    KT = k // 128 // splits
    LA, LB = BM // 64, BN // 64
    ASL, BSL = BM * 128, BN * 128
    assert SA * ASL + SB * BSL <= 160 * 1024
    Lt = xcd_slot(np.arange(G), G)
    split, Lt = Lt // T, Lt % T
    m0, n0 = (Lt % tm) * BM, (Lt // tm) * BN
    wave, lane = np.arange(8)[:, None], np.arange(64)[None, :]
    kbase = split * KT * 128
    chunk = lambda row: ((lane & 7) ^ ((row >> 1) & 7)) * 16  # noqa: E731
    for j in range(LA):
        row = 8 * (wave * LA + j) + (lane >> 3)                              # [8, 64]
        g = m0[:, None, None] + row
        src = np.where(g < m, g, 0) * k + kbase[:, None, None] + chunk(row)
        within("gemm_dma A", src, src + (KT - 1) * 128 + 16, m * k)
        dst = (wave * LA + j) * 1024 + lane * 16
        within("gemm_dma A ring slot", dst, dst + 16, ASL)
    for j in range(LB):
        row = 8 * (wave * LB + j) + (lane >> 3)
        g = n0[:, None, None] + row
        src = np.where(g < n, g, 0) * k + kbase[:, None, None] + chunk(row)
        within("gemm_dma B", src, src + (KT - 1) * 128 + 16, n * k)
        dst = (wave * LB + j) * 1024 + lane * 16
        within("gemm_dma B ring slot", dst, dst + 16, BSL)
    off = frag_offsets()
    wm0, wn0 = (np.arange(8) // (BN // WN)) * WM, (np.arange(8) % (BN // WN)) * WN
    for f in range(WM // 32):
        a = (wm0 + 32 * f)[:, None, None] * 128 + off[None]
        within("gemm_dma A fragments", a, a + 16, ASL)
    for f in range(WN // 32):
        b = (wn0 + 32 * f)[:, None, None] * 128 + off[None]
        within("gemm_dma B fragments", b, b + 16, BSL)
    rows, cols = store_blocks(m, n, (m0[:, None] + wm0[None, :]), (n0[:, None] + wn0[None, :]), WM // 32, WN // 32)
    if splits == 1:
        written_once("gemm_dma out", rows * n + cols, m * n)
    else:
        # slab index of each store: repeat the per-workgroup split over its stores
        per_wg = [store_blocks(m, n, m0[w] + wm0, n0[w] + wn0, WM // 32, WN // 32) for w in range(G)]
        idx = np.concatenate([split[w] * m * n + rr * n + cc for w, (rr, cc) in enumerate(per_wg)])
        written_once("gemm_dma slabs", idx, splits * m * n)
        check_epilogue(m, n, r, residual)


def check_tall(m, n, k, r, residual):
    """gemm_tall (gemm.hip:746-945): per-wave DMA instruction dealing, the
    rings, the two compute mappings, the stores."""
    BN, SA, SB, MA, splits = r["bn"], r["sa"], r["sb"], r["ma"], r["splits"]
    FN, ASL, BSL, NB = BN // 32, MA * 128, BN * 128, BN // 8
    kMaxA, kMaxB = (MA // 8 + 7) // 8, (NB + 7) // 8
    assert SA * ASL + SB * BSL <= 160 * 1024 and m <= MA
    tn = -(-n // BN)
    G = tn * splits
    assert r["grid_x"] == G
    KT = k // 128 // splits
    assert k % 128 == 0 and KT * splits * 128 == k
    Lt = xcd_slot(np.arange(G), G)
    split, n0 = Lt // tn, (Lt % tn) * BN
    kbase = split * KT * 128
    NA = -(-m // 8)
    for wave in range(8):
        na, nb = (NA + 7 - wave) // 8, (NB + 7 - wave) // 8
        assert na <= kMaxA and nb <= kMaxB
        lane = np.arange(64)
        for j in range(na):
            row = 8 * (wave + 8 * j) + (lane >> 3)
            assert row.max() < MA  # the ring slot row: 1024 (wave + 8 j) + 16 lane < MA * 128
            src = np.minimum(row, m - 1) * k + kbase[:, None] + ((lane & 7) ^ ((row >> 1) & 7)) * 16
            within("gemm_tall A", src, src + (KT - 1) * 128 + 16, m * k)
            dst = 1024 * (wave + 8 * j) + lane * 16
            within("gemm_tall A ring slot", dst, dst + 16, ASL)
        for j in range(nb):
            br = 8 * (wave + 8 * j) + (lane >> 3)
            src = np.minimum(n0[:, None] + br, n - 1) * k + kbase[:, None] + ((lane & 7) ^ ((br >> 1) & 7)) * 16
            within("gemm_tall B", src, src + (KT - 1) * 128 + 16, n * k)
            dst = 1024 * (wave + 8 * j) + lane * 16
            within("gemm_tall B ring slot", dst, dst + 16, BSL)
    off = frag_offsets()
    stores = []
    if MA == 64:
        T = -(-m // 32) * FN
        for wave in range(min(T, 8)):
            mb, nbk = wave // FN, wave % FN
            a = mb * 32 * 128 + off
            b = nbk * 32 * 128 + off
            within("gemm_tall A fragments", a, a + 16, ASL)
            within("gemm_tall B fragments", b, b + 16, BSL)
            stores.append((32 * mb + 0 * n0, n0 + 32 * nbk, 1, 1))
        assert T <= 8, "one 32 x 32 block per wave"
    else:
        for wave in range(8):
            if 32 * wave >= m:
                continue
            a = 32 * wave * 128 + off
            within("gemm_tall A fragments", a, a + 16, ASL)
            for jj in range(FN):
                b = 32 * jj * 128 + off
                within("gemm_tall B fragments", b, b + 16, BSL)
            stores.append((32 * wave + 0 * n0, n0, 1, FN))
    idx = []
    for w in range(G):
        for (row0, col0, fm, fn) in stores:
            rr, cc = store_blocks(m, n, row0[w], col0[w], fm, fn)
            idx.append(split[w] * m * n + rr * n + cc)
    written_once("gemm_tall slabs" if splits > 1 else "gemm_tall out", np.concatenate(idx), splits * m * n)
    if splits > 1:
        check_epilogue(m, n, r, residual)


def check_epilogue(m, n, r, residual):
    """splitk_epilogue / splitk_epilogue8 (gemm.hip:960-1093): grid
    (ceil(n / cols / 256), min(m, 65535)), thread columns c .. c + cols - 1,
    rows blockIdx.y, + gridDim.y, ...; slab index clamped to splits - 1."""
    cols, splits = r["epi_cols"], r["splits"]
    assert n % cols == 0, "the epilogue works on whole column groups"
    gx, gy = -(-(n // cols) // 256), min(m, 65535)
    c = (np.arange(gx)[:, None] * 256 + np.arange(256)[None, :]).ravel() * cols
    c = c[c < n]
    rows = np.arange(m)  # row r is visited by blockIdx.y = r mod gy
    i = rows[:, None] * n + c[None, :]
    for s in range(4):  # kMaxSplits slab loads, clamped
        base = min(s, splits - 1) * m * n + i
        within("split-K epilogue slabs", base, base + cols, splits * m * n)
    within("split-K epilogue ws", c, c + cols, n)
    if residual:
        within("split-K epilogue residual", i, i + cols, m * n)
    written_once("split-K epilogue out", (i[..., None] + np.arange(cols)).ravel(), m * n)


def check_skinny(m, n, k, r):
    """gemm_skinny (gemm.hip:92-144): grid (ceil(n / 16), 1), S waves split K in
    64-byte steps; loads guarded by kk + koff < K (16-byte reads, K % 16 == 0)."""
    MT, S, U = r["mt"], r["s"], r["u"]
    assert r["grid_x"] == -(-n // 16) and r["grid_y"] == 1 and 16 * MT >= m and k % 16 == 0
    n0 = np.arange(r["grid_x"]) * 16
    steps = -(-k // 64)
    per = -(-steps // S)
    lane = np.arange(64)
    koff = (lane >> 4) * 16
    for wave in range(S):
        s0, s1 = min(wave * per, steps), min(wave * per + per, steps)
        for s in ({s0, s1 - 1} if s1 > s0 else set()):
            kk = s * 64
            ok = kk + koff < k
            wrow = np.minimum(n0[:, None] + (lane & 15), n - 1)
            src = (wrow * k + koff + kk)[:, ok]
            within("gemm_skinny W", src, src + 16, n * k)
            for t in range(MT):
                arow = t * 16 + (lane & 15)
                src = (arow * k + koff + kk)[ok & (arow < m)]
                within("gemm_skinny A", src, src + 16, m * k)
    # epilogue: thread i -> (t, v, l); r = m0 + 16 t + 4 (l >> 4) + v, c = n0 + (l & 15)
    i = np.arange(MT * 4 * 64)
    l, v, t = i & 63, (i >> 6) & 3, i >> 8
    rr = t * 16 + 4 * (l >> 4) + v
    cc = n0[:, None] + (l & 15)
    rr = np.broadcast_to(rr, cc.shape)
    keep = (rr < m) & (cc < n)
    written_once("gemm_skinny out", rr[keep] * n + cc[keep], m * n)


def check_narrow(m, n, k, r):
    """gemm_narrow (gemm.hip:268-380, plan :1125): grid ceil(n / 16) x 64 S
    threads; wave w sums ST = K / (128 S) of the 128-byte K chunks through
    its own R-stage ring: at S = 4 stage s reads chunk w ST + s, at S = 8
    chunk ((s + b) mod ST) S + w for workgroup b; the chunks of all waves
    and stages of a workgroup must be every chunk of K exactly once.  DMA
    instruction j < 2 + LAL fills rows 8j .. 8j + 7 of a stage (lane l: row
    8j + l / 8, 16-byte piece (l % 8) ^ (row % 8)); rows 0-15 are weight
    rows n0 + row clamped to n - 1, rows 16.. activation rows row - 16,
    loaded only below M."""
    MB, S, LAL, R = r["mt"], r["s"], r["u"], r["sa"]
    assert r["grid_x"] == -(-n // 16) and r["grid_y"] == 1 and r["block"] == 64 * S and r["splits"] == 1
    assert k % (128 * S) == 0 and 16 * MB >= m
    # every row below M has its DMA instruction, and every issued instruction has a live lane
    assert 8 * LAL >= m and 8 * (LAL - 1) < m, (m, LAL)
    ROWS, L = 16 * (1 + MB), 2 + LAL
    STAGE, RING = ROWS * 128, R * ROWS * 128
    assert L <= ROWS // 8 and S * RING <= 160 * 1024
    ST = k // (128 * S)
    n0 = np.arange(r["grid_x"])[:, None] * 16
    lane = np.arange(64)
    b = np.arange(r["grid_x"])

    def kchunk(wave, st):
        """K chunk of stage st of wave `wave`, per workgroup."""
        if S >= 8:
            return ((st + b) % ST) * S + wave
        return np.full(b.shape, wave * ST + st)

    seen = np.zeros((r["grid_x"], k // 128), np.int64)
    for wave in range(S):
        for st in range(ST):
            np.add.at(seen, (b, kchunk(wave, st)), 1)
    assert (seen == 1).all(), "every K chunk exactly once per workgroup"
    for wave in range(S):
        for st in ({0, ST - 1} if ST > 0 else set()):
            for j in range(L):
                row = 8 * j + (lane >> 3)
                chunk = ((lane & 7) ^ (row & 7)) * 16
                koff = kchunk(wave, st)[:, None] * 128 + chunk
                if j < 2:
                    src = np.minimum(n0 + row, n - 1) * k + koff
                    within("gemm_narrow W", src, src + 16, n * k)
                else:
                    g = row - 16
                    live = g < m
                    src = (g * k + koff)[:, live]
                    within("gemm_narrow A", src, src + 16, m * k)
                dst = wave * RING + (st % R) * STAGE + j * 1024 + lane * 16
                within("gemm_narrow LDS DMA", dst, dst + 16, S * RING)
    fr, fq = lane & 15, lane >> 4
    for h in range(2):
        c = 4 * h + fq
        b = fr * 128 + ((c ^ (fr & 7)) * 16)
        within("gemm_narrow B fragments", b, b + 16, STAGE)
        for t in range(MB):
            row = 16 + 16 * t + fr
            a = row * 128 + ((c ^ (row & 7)) * 16)
            within("gemm_narrow A fragments", a, a + 16, STAGE)
    red = ((np.arange(S)[:, None, None, None] * MB + np.arange(MB)[:, None, None]) * 4
           + np.arange(4)[:, None]) * 64 + lane
    within("gemm_narrow reduction", red * 4, red * 4 + 4, S * RING)
    # epilogue: index i = tid, tid + 64 S, ... < MB * 256 -> (t, v, l)
    i = np.arange(MB * 4 * 64)
    l, v, t = i & 63, (i >> 6) & 3, i >> 8
    rr = 16 * t + 4 * (l >> 4) + v
    cc = n0 + (l & 15)
    rr = np.broadcast_to(rr, cc.shape)
    keep = (rr < m) & (cc < n)
    written_once("gemm_narrow out", rr[keep] * n + cc[keep], m * n)


def check_tiled(m, n, k, r):
    """gemm_tiled (gemm.hip:147-241): guarded 16-byte loads (gm < M, kk < K),
    LDS rows of PITCH = 144 bytes, XCD-aware tile numbering."""
    BM, BN, WM, WN = r["bm"], r["bn"], r["wm"], r["wn"]
    PITCH = 144
    tm, tn = -(-m // BM), -(-n // BN)
    T = tm * tn
    assert r["grid_x"] == T and k % 16 == 0
    L = xcd_slot(np.arange(T), T)
    m0, n0 = (L % tm) * BM, (L // tm) * BN
    tid = np.arange(256)
    KT = -(-k // 128)
    for i in range(BM * 8 // 256):
        idd = tid + i * 256
        row, kc = idd >> 3, idd & 7
        within("gemm_tiled A slot", row * PITCH + kc * 16, row * PITCH + kc * 16 + 16, BM * PITCH)
        for kt in {0, KT - 1}:
            gm, kk = m0[:, None] + row, kt * 128 + kc * 16
            ok = (gm < m) & (kk < k)
            src = (gm * k + kk)[ok]
            within("gemm_tiled A", src, src + 16, m * k)
    for i in range(BN * 8 // 256):
        idd = tid + i * 256
        row, kc = idd >> 3, idd & 7
        for kt in {0, KT - 1}:
            gn, kk = n0[:, None] + row, kt * 128 + kc * 16
            ok = (gn < n) & (kk < k)
            src = (gn * k + kk)[ok]
            within("gemm_tiled B", src, src + 16, n * k)
    lane = np.arange(64)
    frow, fk = lane & 15, (lane >> 4) * 16
    wave = np.arange(4)
    wm0, wn0 = (wave // (BN // WN)) * WM, (wave % (BN // WN)) * WN
    for ks in range(2):
        for ii in range(WM // 16):
            a = (wm0[:, None] + ii * 16 + frow) * PITCH + ks * 64 + fk
            within("gemm_tiled A fragments", a, a + 16, BM * PITCH)
    rows, cols = [], []
    for ii in range(WM // 16):
        for jj in range(WN // 16):
            for v in range(4):
                rr = m0[:, None, None] + wm0[None, :, None] + ii * 16 + 4 * (lane >> 4) + v
                cc = n0[:, None, None] + wn0[None, :, None] + jj * 16 + (lane & 15)
                rr, cc = np.broadcast_arrays(rr, cc)
                keep = (rr < m) & (cc < n)
                rows.append(rr[keep])
                cols.append(cc[keep])
    written_once("gemm_tiled out", np.concatenate(rows) * n + np.concatenate(cols), m * n)


# ------------------------------------------------------------------ GEMV routes
def check_gemv_m1(m, n, k, r, residual, argmax=False):
    """gemv_m1_one / gemv_m1 (gemv.hip:205-325): wave g owns rows R g ..
    R g + R - 1; loads clamped to n - 1; lanes < R store rows < n."""
    R, KC, W = r["rows"], r["kc"], r["waves"]
    assert m == 1 and k == KC * 1024
    groups = -(-n // R)
    assert r["grid_x"] == -(-groups // W)
    g = np.arange(r["grid_x"] * W)
    live = g < groups
    row0 = np.where(live, g * R, 0)
    lane = np.arange(64)
    within("gemv q", lane * 16, lane * 16 + 16 + (KC - 1) * 1024, k)
    erow = np.minimum(row0[:, None] + np.minimum(lane, R - 1), n - 1)
    within("gemv ws / residual", erow, erow + 1, n)
    for rr in range(R):
        src = np.minimum(row0 + rr, n - 1)[:, None] * k + lane * 16
        within("gemv W", src, src + (KC - 1) * 1024 + 16, n * k)
    row = row0[:, None] + lane
    keep = live[:, None] & (lane < R) & (row < n)
    written_once("gemv out", row[keep], n)
    if argmax:
        # one key per workgroup into a workspace of argmax_keys_for(n) keys
        assert r["grid_x"] <= -(-n // 4), "selection keys exceed the workspace bound"


def check_gemv_mt(m, n, k, r, residual):
    """gemv_mt (gemv.hip:348-423): 4-row groups, MT activation rows per pass
    (blockIdx.y), 1 KiB chunks with rotation, loads guarded by kk < K."""
    MT, R = r["mt"], 4
    groups = -(-n // R)
    assert r["grid_x"] == -(-groups // 4) and r["grid_y"] == -(-m // MT)
    g = np.arange(r["grid_x"] * 4)
    live = g < groups
    row0 = np.where(live, g * R, 0)
    lane = np.arange(64)
    nch = -(-k // 1024)
    for ci in {0, nch - 1}:
        kk = ci * 1024 + lane * 16
        ok = kk < k
        for rr in range(R):
            src = (np.minimum(row0 + rr, n - 1)[:, None] * k + kk)[:, ok]
            within("gemv_mt W", src, src + 16, n * k)
        m0 = np.arange(r["grid_y"]) * MT
        for t in range(MT):
            xr = m0 + t
            src = (np.where(xr < m, xr, 0)[:, None] * k + kk)[xr < m][:, ok]
            within("gemv_mt q", src, src + 16, m * k)
    V = R * MT
    m0 = np.arange(r["grid_y"]) * MT
    t = m0[:, None, None] + (lane // R)[None, None, :]
    row = row0[None, :, None] + (lane % R)[None, None, :]
    t, row = np.broadcast_arrays(t, row)
    keep = live[None, :, None] & (lane < V)[None, None, :] & (row < n) & (t < m)
    written_once("gemv_mt out", (t * n + row)[keep], m * n)


def check_linear(m, n, k, dtype=BF16, residual=False, path=AUTO, workspace=0):
    r = route(m, n, k, dtype, residual, path, workspace)
    fam = r["family"]
    if fam in (1, 2):
        check_gemv_m1(m, n, k, r, residual)
    elif fam == 3:
        check_gemv_mt(m, n, k, r, residual)
    elif fam == 11:
        check_skinny(m, n, k, r)
    elif fam == 12:
        check_tall(m, n, k, r, residual)
    elif fam == 13:
        check_dma(m, n, k, r, residual)
    elif fam == 14:
        check_tiled(m, n, k, r)
    elif fam == 15:
        check_narrow(m, n, k, r)
    else:
        raise AssertionError(f"no route for {(m, n, k)}: {r}")
    return r


# ------------------------------------------------------------------ tests
@pytest.mark.parametrize("n,k", DECODE)
def test_decode_shapes_m1(n, k):
    """C1 / C2: the decode projections at M = 1, and with a residual."""
    for residual in (False, True):
        r = check_linear(1, n, k, residual=residual)
        assert r["family"] == 1


def test_lm_head_argmax():
    """C3: the 151,936-row head's fused-selection GEMV."""
    n, k = 151936, 4096
    r = argmax_route(n, k)
    assert r["family"] == 2 and r["waves"] == 16
    check_gemv_m1(1, n, k, r, False, argmax=True)
    for nn in (1, 3, 4097, 50000):
        check_gemv_m1(1, nn, k, argmax_route(nn, k), False, argmax=True)


@pytest.mark.parametrize("m", [129, 512])
@pytest.mark.parametrize("n,k", DECODE)
def test_prefill_shapes(m, n, k):
    """C4: M = 129 and 512 on the four layer shapes, with and without the
    split-K workspace, plain and with a residual."""
    for ws in (0, workspace_bytes(m, n, k)):
        for residual in (False, True):
            check_linear(m, n, k, residual=residual, workspace=ws)


@pytest.mark.parametrize("m", [130, 131, 135, 136, 140, 159])
@pytest.mark.parametrize("n,k", DECODE)
def test_m129_tails(m, n, k):
    """The rows past a 32-row block and past the 128-row tile: M = 129-135
    and 136-159 (sampled)."""
    check_linear(m, n, k, workspace=workspace_bytes(m, n, k))
    check_linear(m, n, k, residual=True)


@pytest.mark.parametrize("m", [4, 16, 64])
@pytest.mark.parametrize("n,k", [(24576, 4096), (4096, 12288)])
def test_ragged_small_m(m, n, k):
    """C5: the ragged batches on gate_up and down, on both families."""
    for path in (DOT4, MFMA):
        for ws in (0, workspace_bytes(m, n, k)):
            check_linear(m, n, k, path=path, workspace=ws)


@pytest.mark.parametrize("m", [2, 3, 7, 8, 17, 33, 65, 100, 200, 255, 256, 257, 300])
def test_other_m_and_n_not_multiple_of_96(m):
    """Every family at M between the configurations, with N % 96 != 0 (and
    not a multiple of 64 or 16 where the routes allow it)."""
    for n, k in [(4000, 4096), (6100, 4096), (24500, 4096), (1000, 12288), (4100, 4096)]:
        for ws in (0, workspace_bytes(m, n, k)):
            check_linear(m, n, k, workspace=ws)
        check_linear(m, n, k, residual=True)


@pytest.mark.parametrize("m,n,k", [(100, 4096, 4112), (300, 1000, 1040), (65, 777, 2064), (1, 5000, 1040),
                                   (3, 333, 48)])
def test_k_not_multiple_of_128(m, n, k):
    """gemm_tiled (K % 128 != 0 at M > 64), gemm_skinny and gemv_mt at odd K."""
    check_linear(m, n, k)
    check_linear(m, n, k, path=DOT4)


@pytest.mark.parametrize("n,k", [(4096, 4096), (6144, 4096), (4096, 12288), (1000, 512), (4100, 8192), (333, 2048),
                                 (17, 12288)])
def test_narrow_every_m(n, k):
    """gemm_narrow at every M it takes (1-16, and 17-32 at K <= 4096 on
    N <= 4096): both wave counts (K below and from 8192), one to four live
    activation loads per stage, N not a multiple of 16, a one-stage slice
    (K = 512)."""
    took = 0
    for m in range(1, 33):
        for path in (AUTO, MFMA):
            r = check_linear(m, n, k, path=path, workspace=workspace_bytes(m, n, k))
            if path == MFMA and m <= 16:
                assert r["family"] == 15, (m, n, k, r)
            took += r["family"] == 15
    assert took >= 16


@pytest.mark.parametrize("m,n,k", seeded_linear_shapes())
def test_seeded_shape_sweep(m, n, k):
    """The shapes of the GPU sweep (test_gpu_parity.test_linear_seeded_shape_sweep),
    replayed first here on every path it runs: AUTO with and without the
    split-K workspace, BF16 and f32 with the residual; the dot4 GEMV and
    the MFMA family forced."""
    wsb = workspace_bytes(m, n, k)
    for path in (AUTO, DOT4, MFMA):
        for workspace in ((0, wsb) if path != DOT4 else (0,)):
            check_linear(m, n, k, path=path, workspace=workspace)
            check_linear(m, n, k, F32, residual=True, path=path, workspace=workspace)
    check_linear(m, n, k, I32, path=MFMA, workspace=wsb)


def test_every_family_is_replayed():
    """The shapes above reach every GEMM and GEMV family."""
    seen = set()
    for (m, n, k, ws) in [(1, 4096, 4096, 0), (1, 4096, 1040, 0), (3, 4096, 4096, 0), (3, 4096, 1040, 0),
                          (129, 4096, 4096, 1 << 30), (512, 24576, 4096, 0), (100, 4096, 4112, 0)]:
        seen.add(route(m, n, k, workspace=ws)["family"])
    seen.add(argmax_route(4096, 4096)["family"])
    assert seen == {1, 2, 3, 11, 12, 13, 14, 15}, seen


# ------------------------------------------------------------------ folded producers
def check_rows_split(n, NS, RS, K):
    """gemv_m1_split / gemv_rowtail_split streaming waves (gemv.hip:690-757,
    :856-965): row r of wave wv of workgroup b is (r NS + wv) G + slot(b),
    loads clamped to n - 1, stores guarded by row < n."""
    G = -(-n // (NS * RS))
    b, wv, rr = np.meshgrid(np.arange(G), np.arange(NS), np.arange(RS), indexing="ij")
    row = (rr * NS + wv) * G + xcd_slot(b, G)
    er = np.minimum(row, n - 1)
    lane = np.arange(64)
    src = er[..., None] * K + lane * 16
    within("split W", src, src + K - 1024 + 16, n * K)
    written_once("split out", row[row < n], n)


def check_swiglu_split(n, NS=12, CS=4):
    """gemv_swiglu_split (gemv.hip:763-842): coordinate k of wave wv of
    workgroup b is (k NS + wv) G + slot(b)."""
    G = -(-n // (NS * CS))
    b, wv, kk = np.meshgrid(np.arange(G), np.arange(NS), np.arange(CS), indexing="ij")
    c = (kk * NS + wv) * G + xcd_slot(b, G)
    src = np.minimum(c, n - 1)[..., None] * 4096 + np.arange(64) * 16
    within("swiglu split W", src, src + 3 * 1024 + 16, n * 4096)
    written_once("swiglu split out", c[c < n], n)


@pytest.mark.parametrize("n", [1, 15, 16, 17, 1000, 4095, 4096, 4097, 5000, 6143, 6144, 6145, 24576, 40000])
def test_folded_producer_rows(n):
    """Every row of the folded-producer GEMVs written once, every weight load
    inside the matrix: 8 streaming waves x 2 rows up to N = 4096 and 12 x 2
    beyond (K = 4096), 8 x 2 for the down fold (K = 12,288)."""
    check_rows_split(n, 8 if n <= 4096 else 12, 2, 4096)
    check_rows_split(n, 8, 2, 12288)


@pytest.mark.parametrize("n", [1, 47, 48, 49, 4096, 12287, 12288, 12289, 30000])
def test_swiglu_split_coordinates(n):
    check_swiglu_split(n)


def test_producer_row_layout():
    """The producer waves' row loads: thread pt of the four reads x[pt + 256 i]
    (i < 16) of a 4096-wide row, and for the down fold elements
    4 (pt + 256 j) .. + 3 (j < 12) of the 12,288-wide act row; codes go to
    LDS byte pt + 256 i, or word pt + 256 j."""
    pt = np.arange(256)[:, None]
    x = pt + 256 * np.arange(16)
    written_once("producer row", x, 4096)
    e = 4 * (pt + 256 * np.arange(12))
    written_once("rowtail act", (e[..., None] + np.arange(4)).ravel(), 12288)


# ------------------------------------------------------------------ planted mistakes
def test_checker_catches_planted_mistakes():
    """The checks above must fail on the mistakes they exist for: a tail row
    read without its clamp, a store written twice or not at all, a slot
    mapping off by one."""
    m, n, k = 129, 4096, 4096
    r = route(m, n, k, workspace=workspace_bytes(m, n, k))
    assert r["family"] == 12  # gemm_tall, 160-row tile, split K
    lane = np.arange(64)
    row = 8 * (0 + 8 * 2) + (lane >> 3)  # wave 0's third activation row group: rows 128-135
    KT = k // 128 // r["splits"]
    unclamped = row * k + ((lane & 7) ^ ((row >> 1) & 7)) * 16 + (r["splits"] - 1) * KT * 128
    with pytest.raises(AssertionError, match="past the buffer"):
        within("unclamped A", unclamped, unclamped + (KT - 1) * 128 + 16, m * k)
    clamped = np.minimum(row, m - 1) * k + ((lane & 7) ^ ((row >> 1) & 7)) * 16 + (r["splits"] - 1) * KT * 128
    within("clamped A", clamped, clamped + (KT - 1) * 128 + 16, m * k)
    with pytest.raises(AssertionError):
        written_once("duplicate", np.array([0, 1, 1, 3]), 4)
    with pytest.raises(AssertionError):
        written_once("missing", np.array([0, 1, 3]), 4)
    # folded-producer rows with the slot shifted by one workgroup
    n, NS, RS = 6144, 12, 2
    G = -(-n // (NS * RS))
    b, wv, rr = np.meshgrid(np.arange(G), np.arange(NS), np.arange(RS), indexing="ij")
    bad = (rr * NS + wv) * G + (xcd_slot(b, G) + 1)
    with pytest.raises(AssertionError):
        written_once("shifted rows", bad[bad < n], n)
    # a 32 x 32 MFMA block's value layout with the half-wave term dropped
    lane2 = np.arange(64)[:, None]
    v = np.arange(16)[None, :]
    wrong = (v >> 2) * 8 + (v & 3) + 0 * lane2
    with pytest.raises(AssertionError):
        written_once("block rows", (wrong * 32 + (lane2 & 31)).ravel(), 32 * 32)
    rows, cols = mfma32_rows_cols(lane2, v)
    written_once("block rows", (rows * 32 + np.broadcast_to(cols, rows.shape)).ravel(), 32 * 32)
    # gemm_narrow: activation rows loaded without the live mask (M = 3: rows 3-7 of the first
    # activation instruction), and a live-load count one short of the rows (M = 9, LAL = 1)
    m, n, k = 3, 4096, 4096
    r = route(m, n, k, path=MFMA)
    assert r["family"] == 15
    g = (8 * 2 + (lane >> 3)) - 16
    src = g * k + ((lane & 7) ^ ((g + 16) & 7)) * 16 + (r["s"] - 1) * (k // r["s"])
    with pytest.raises(AssertionError, match="past the buffer"):
        within("unmasked A", src, src + (k // r["s"] - 128) + 16, m * k)
    bad = dict(route(9, n, k, path=MFMA), u=1)
    with pytest.raises(AssertionError):
        check_narrow(9, n, k, bad)
