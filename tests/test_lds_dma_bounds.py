"""CPU replay of the direct global-to-LDS loads (ld16_to_lds, csrc/lrq_common.h).

Four kernels move 16 bytes per lane from global memory straight into LDS with
__builtin_amdgcn_global_load_lds: k_encode_rows and k_encode_tiles (csrc/lrq_encode.hip),
k_softmax_rows (csrc/lrq_rowops.hip) and k_wht_rows (csrc/lrq_wht.hip).  This file restates, in numpy, the
host launch arithmetic (grid, row blocks per workgroup) and each kernel's source and
destination address arithmetic, and checks for every instance and launch shape that the
library's callers use (bench.py's configurations and the GPU tests' shapes) that

  * every global byte read lies inside the caller's tensor (rows clamped to the last row),
  * every LDS byte written lies inside the workgroup's allocation and inside the wave's own
    region (encode) or the block's tile (softmax, rotation),
  * no two lanes of one workgroup write the same LDS bytes for one row block.

For k_encode_tiles, whose tiles are swizzled (chunk c of tile row r at position c ^ r), the
replay also checks that the read-back (projection / quantisation layout and the rotation's
layout) finds every column where the loads put it.

No GPU is needed; a change to any of these kernels' addressing must be mirrored here.
"""

from __future__ import annotations

import numpy as np
import pytest

LDS_BYTES = 160 * 1024
CU_COUNTS = (256, 304, 80)  # MI355X, and two other counts the launch arithmetic must also survive


def _rows_per_wg(nrb: int, wgs: int) -> tuple[int, int]:
    rbw = (nrb + wgs - 1) // wgs
    return rbw, (nrb + rbw - 1) // rbw


def _blocks(grid: int, rbw: int, nrb: int):
    """Row blocks each workgroup loads: rb0 .. rb0 + nblk - 1 (the kernels return early when
    rb0 >= nrb, and their next-block loads stay below rb0 + nblk)."""
    for wg in range(grid):
        rb0 = wg * rbw
        if rb0 >= nrb:
            continue
        yield np.arange(rb0, rb0 + min(rbw, nrb - rb0))


def _check(gsrc, ldst, *, gbytes, lds_alloc, lo, hi, what):
    """gsrc / ldst: int64 arrays of the first byte each lane moves (16 bytes each)."""
    assert gsrc.min() >= 0 and (gsrc + 16).max() <= gbytes, f"{what}: global read out of the tensor"
    assert ldst.min() >= 0 and (ldst + 16).max() <= lds_alloc, f"{what}: LDS write out of the allocation"
    assert (ldst >= lo).all() and (ldst + 16 <= hi).all(), f"{what}: LDS write out of its region"


# ----------------------------------------------------------------------------- k_encode_rows
def encode_rows_replay(M, N, ldx, cus, bits=4, group=64, rank=16, upw=4, nw=8):
    """k_encode_rows<bits, group, rank, nw, upw> as launch_rows() launches it."""
    NP, RT = 8 // bits, rank // 16
    PIECE = upw * group * 2
    PITCH = NP * PIECE + 16
    REGION = 16 * PITCH
    PPL = 1024 // PIECE
    LPL = 64 // PPL
    NLD = 16 * NP // PPL
    PART = nw * RT * 64 * 16
    LDS = nw * REGION + 2 * PART
    assert LDS <= LDS_BYTES
    if PPL != NP:
        return 0  # this instance stages through registers (no direct loads)
    RPL = PPL // NP
    nrb = (M + 15) // 16
    rbw = (nrb + cus - 1) // cus
    grid = (nrb + rbw - 1) // rbw
    lane = np.arange(64)
    lpc, loff = lane // LPL, (lane % LPL) * 16
    lrow = lpc // NP
    checked = 0
    for w in range(nw):
        ub = w * upw
        xlane = ((lpc % NP) * (N // NP) + ub * group) * 2 + loff        # unit_base(p, ub) * 2 + loff
        for rbs in _blocks(grid, rbw, nrb):
            rb = rbs[:, None, None]
            i = np.arange(NLD)[None, :, None]
            r0 = rb * 16 + RPL * i
            full = r0 + RPL <= M
            row = np.where(full, r0 + lrow, np.minimum(r0 + lrow, M - 1))
            gsrc = row * ldx * 2 + xlane                                 # gaddr()
            ldst = np.broadcast_to(w * REGION + i * PITCH + lane * 16, gsrc.shape)  # region + i*PITCH, lane*16
            _check(gsrc, ldst, gbytes=((M - 1) * ldx + N) * 2, lds_alloc=LDS, lo=w * REGION,
                   hi=(w + 1) * REGION, what=f"k_encode_rows M={M} N={N} ldx={ldx} cus={cus} w={w}")
            # within one block the waves' lanes write disjoint bytes
            if w == 0 and rbs[0] == 0:
                allw = (np.arange(nw)[:, None, None] * REGION + np.arange(NLD)[None, :, None] * PITCH
                        + lane[None, None, :] * 16).ravel()
                assert np.unique(allw).size == allw.size
            checked += gsrc.size
    return checked


ENCODE_SHAPES = [  # (rows, ldx extra columns): bench north_star / c1 / lora, GPU-test shapes
    (16384, 0), (2048, 0), (1, 0), (5, 0), (16, 0), (17, 0), (37, 0), (64, 0), (96, 0), (100, 0),
    (4100, 0), (9000, 0), (100, 64), (33, 8),
]


@pytest.mark.parametrize("cus", CU_COUNTS)
def test_encode_rows_direct_loads_stay_in_bounds(cus):
    n = 0
    for rows, extra in ENCODE_SHAPES:
        n += encode_rows_replay(rows, 4096, 4096 + extra, cus)
    assert n > 0
    # the 2-unit-per-wave instance (hidden 2048) stages through registers: nothing to check
    assert encode_rows_replay(64, 2048, 2048, 256, upw=2) == 0


# ----------------------------------------------------------------------------- k_encode_tiles
def encode_tiles_replay(M, N, ldx, cus, upw=5, nw=8):
    """k_encode_tiles<upw, rot> as encode_tiles_dispatch() launches it (int4/g64: units of 128
    columns, tiles of 16 rows x 128 columns, 4 KB)."""
    NT, TILE = nw * upw, 16 * 256
    LDS = NT * TILE
    assert N == NT * 128 and LDS <= LDS_BYTES
    nrb = (M + 15) // 16
    rbw = (nrb + cus - 1) // cus
    grid = (nrb + rbw - 1) // rbw
    lane = np.arange(64)
    lr, lq = lane >> 4, lane & 15
    checked = 0
    for rbs in _blocks(grid, rbw, nrb):
        for rb in (rbs[0], rbs[-1]):
            dst_all, col_at = [], np.full(LDS // 16, -1, dtype=np.int64)  # LDS chunk -> (row, global chunk)
            for w in range(nw):
                for i in range(upw):
                    t = w + nw * i
                    for k in range(4):
                        r = 4 * k + lr
                        row = np.minimum(rb * 16 + r, M - 1)
                        gsrc = row * ldx * 2 + 256 * t + 16 * (lq ^ r)        # issue_one()
                        ldst = t * TILE + 1024 * k + 16 * lane
                        _check(gsrc, ldst, gbytes=((M - 1) * ldx + N) * 2, lds_alloc=LDS, lo=t * TILE,
                               hi=(t + 1) * TILE, what=f"k_encode_tiles M={M} N={N} ldx={ldx} cus={cus} w={w}")
                        assert ((gsrc % (ldx * 2)) // 256 == t).all(), "a tile holds columns of another tile"
                        dst_all.append(ldst)
                        col_at[ldst // 16] = r * 1000 + (gsrc % (ldx * 2)) // 16
                        checked += gsrc.size
            d = np.concatenate(dst_all)
            assert np.unique(d).size == d.size == LDS // 16, "every LDS chunk written exactly once per block"
            # read-back: lane (j, g) of wave w reads unit u = w*upw + uu, plane p, chunk
            # 8(u%2) + 2g + k of tile p*NT/2 + u/2, row j, at position chunk ^ j
            j, g = lane & 15, lane >> 4
            for w in range(nw):
                for uu in range(upw):
                    u = w * upw + uu
                    for p in range(2):
                        tp = p * (NT // 2) + u // 2
                        for k in range(2):
                            c = 8 * (u % 2) + 2 * g + k
                            pos = (tp * TILE + 256 * j + 16 * (c ^ j)) // 16
                            want_col = (p * (N // 2) + 64 * u + 16 * g + 8 * k)   # unit_base(p, u) + 16g + 8k
                            assert (col_at[pos] == j * 1000 + want_col // 8).all(), "read-back finds other columns"
                # the rotation's layout: lane (j, g) chunks 4g + c of its tiles' row j
                for i in range(upw):
                    t = w + nw * i
                    for c in range(4):
                        pos = (t * TILE + 256 * j + 16 * ((4 * g + c) ^ j)) // 16
                        assert (col_at[pos] == j * 1000 + (128 * t) // 8 + 4 * g + c).all()
    return checked


@pytest.mark.parametrize("cus", CU_COUNTS)
def test_encode_tiles_direct_loads_stay_in_bounds(cus):
    n = 0
    for rows, extra in [(16384, 0), (1, 0), (5, 0), (16, 0), (37, 0), (48, 0), (64, 0), (100, 0), (4100, 0),
                        (5000, 0), (64, 64), (33, 8)]:
        n += encode_tiles_replay(rows, 5120, 5120 + extra, cus)
    assert n > 0


# ----------------------------------------------------------------------------- k_softmax_rows
def softmax_rows_replay(M, N, lddp, cus, bits, group):
    """k_softmax_rows<bits, group, rank, NW> as softmax_units() / softmax_rows_launch() launch it."""
    NP = 8 // bits
    units = N // (group * NP)
    UB = group * NP * 2
    if units not in (8, 16) or (units * UB) % 1024:
        return 0
    NW = units
    ROWB = NW * group * NP * 2
    PITCH = ROWB + 16
    TILE = 16 * PITCH
    CPR = ROWB // 1024
    DPW = 16 * CPR // NW
    LDS = 2 * TILE + NW * 16 * 4
    if LDS > LDS_BYTES:
        return 0  # softmax_units() has no instance for this width (its compile-time LDS check)
    assert (16 * CPR) % NW == 0
    nrb = (M + 15) // 16
    per_cu = max(1, min(4, LDS_BYTES // LDS))
    wgs = max(1, min(nrb, cus * per_cu))
    rbw, grid = _rows_per_wg(nrb, wgs)
    lane = np.arange(64)
    checked = 0
    for rbs in _blocks(grid, rbw, nrb):
        for tb in (0, 1):
            dsts = []
            for w in range(NW):
                q = w * DPW + np.arange(DPW)[:, None]
                r, c = q // CPR, q % CPR
                row = np.minimum(rbs[:, None, None] * 16 + r[None], M - 1)
                gsrc = row * lddp * 2 + c[None] * 1024 + lane * 16
                ldst = np.broadcast_to(tb * TILE + r * PITCH + c * 1024 + lane * 16, (DPW, 64))
                _check(gsrc, ldst, gbytes=((M - 1) * lddp + N) * 2, lds_alloc=LDS, lo=tb * TILE,
                       hi=tb * TILE + TILE, what=f"k_softmax_rows M={M} N={N} bits={bits} w={w}")
                # a row's chunks stay inside the row's ROWB bytes of the tile
                assert ((ldst - tb * TILE) % PITCH + 16 <= ROWB).all()
                dsts.append(ldst.ravel())
                checked += gsrc.size
            d = np.concatenate(dsts)
            assert np.unique(d).size == d.size
    return checked


@pytest.mark.parametrize("cus", CU_COUNTS)
@pytest.mark.parametrize("bits,group,N", [(4, 64, 2048), (4, 64, 1024), (8, 128, 2048), (8, 128, 1024),
                                          (8, 64, 1024), (4, 128, 4096)])
def test_softmax_rows_direct_loads_stay_in_bounds(cus, bits, group, N):
    n = 0
    for rows in (1, 16, 40, 64, 100, 9000):
        n += softmax_rows_replay(rows, N, N, cus, bits, group)
    if (bits, group, N) == (4, 64, 2048):
        n += softmax_rows_replay(2 * 32 * 2048, N, N, cus, bits, group)  # config 5
    assert (n > 0) == ((bits, group, N) != (4, 128, 4096))  # 16 units of 512 B rows: no tile fits


# ----------------------------------------------------------------------------- k_wht_rows
def wht_rows_replay(M, N, ldx, cus):
    """k_wht_rows as lrq_wht128 launches it (hidden % 512 == 0)."""
    PITCH = 1024 + 16
    TILE = 16 * PITCH
    LDS = 2 * TILE
    nrb = (M + 15) // 16
    slabs = N // 512
    ranges = max(1, min(nrb, cus * 4 // slabs))
    rbw = (nrb + ranges - 1) // ranges
    grid = (nrb + rbw - 1) // rbw
    lane = np.arange(64)
    checked = 0
    for by in range(slabs):
        c0 = by * 512
        for rbs in _blocks(grid, rbw, nrb):
            for tb in (0, 1):
                dsts = []
                for w in range(4):
                    r = 4 * w + np.arange(4)[:, None]
                    row = np.minimum(rbs[:, None, None] * 16 + r[None], M - 1)
                    gsrc = c0 * 2 + row * ldx * 2 + lane * 16
                    ldst = np.broadcast_to(tb * TILE + r * PITCH + lane * 16, (4, 64))
                    _check(gsrc, ldst, gbytes=((M - 1) * ldx + N) * 2, lds_alloc=LDS, lo=tb * TILE,
                           hi=tb * TILE + TILE, what=f"k_wht_rows M={M} N={N} slab={by} w={w}")
                    dsts.append(ldst.ravel())
                    checked += gsrc.size
                d = np.concatenate(dsts)
                assert np.unique(d).size == d.size
    return checked


@pytest.mark.parametrize("cus", CU_COUNTS)
def test_wht_rows_direct_loads_stay_in_bounds(cus):
    n = 0
    for rows, N, extra in [(16384, 5120, 0), (20000, 512, 0), (64, 1024, 0), (33, 2048, 0), (100, 4096, 8),
                           (1, 512, 0), (5000, 5120, 0)]:
        n += wht_rows_replay(rows, N, N + extra, cus)
    assert n > 0


def test_replay_catches_a_planted_overrun():
    """The check is live: a replay whose row clamp is dropped (rows past the end read) fails."""
    M, N = 37, 4096
    nrb = (M + 15) // 16
    row = np.arange(nrb * 16)  # no clamp
    gsrc = row * N * 2
    with pytest.raises(AssertionError):
        _check(gsrc, np.zeros_like(gsrc), gbytes=((M - 1) * N + N) * 2, lds_alloc=LDS_BYTES, lo=0, hi=LDS_BYTES,
               what="planted")
