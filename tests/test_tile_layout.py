"""The LDS tile layout of fna2_amd/csrc/fna2_tile.h, modelled on the CPU.

The formulas below restate swz4 / tile_off / Dma::slot_offset / RowLane /
TrLane.  Checked: the layout is a bijection of 16-byte slots, the DMA plan
fills every slot with the chunk that belongs there, and both MFMA operand
reads are free of bank conflicts for 32 and for 64 four-byte banks (one LDS
cycle serves 128 or 256 bytes: 8 or 16 lanes of a 16-byte read, 16 or 32
lanes of an 8-byte read).  The same checks cover RowStage, the epilogue
staging layout: its 8-byte accumulator writes and 16-byte row reads.
"""
from collections import Counter

import pytest


def swz4(r):
    return ((((r >> 1) ^ (r >> 3)) & 1) << 1) | ((r >> 2) & 1)


def tile_off(rows, row, chunk):
    return (chunk >> 2) * rows * 64 + row * 64 + (((chunk & 3) ^ swz4(row)) << 4)


def max_bank_use(accesses, nbanks):
    c = Counter()
    for addr, nbytes in accesses:
        for w in range(addr // 4, (addr + nbytes) // 4):
            c[w % nbanks] += 1
    return max(c.values())


SHAPES = [(rows, c) for rows in (32, 64, 128) for c in (4, 8, 16)]


@pytest.mark.parametrize("rows,C", SHAPES)
def test_bijection_and_dma_plan(rows, C):
    offs = sorted(tile_off(rows, r, c) for r in range(rows) for c in range(C))
    assert offs == list(range(0, rows * C * 16, 16))
    # Dma::slot_offset: slot p holds logical (row, col); its address must be 16 p
    for p in range(rows * C):
        grp, rem = divmod(p, rows * 4)
        row, slot = rem >> 2, rem & 3
        col = 4 * grp + (slot ^ swz4(row))
        assert tile_off(rows, row, col) == 16 * p


@pytest.mark.parametrize("nbanks", [32, 64])
@pytest.mark.parametrize("rows,C", SHAPES)
def test_row_reads_conflict_free(nbanks, rows, C):
    per_cycle = nbanks * 4 // 16
    for r0 in range(0, rows, 32):
        for s in range(C // 2):
            acc = []
            for lane in range(64):
                l, hl = lane & 31, lane >> 5
                # RowLane: offset l*64 + ((2(s&1)+hl) ^ swz4(l))*16, plus immediates
                a = (s >> 1) * rows * 64 + r0 * 64 + l * 64 + (((2 * (s & 1) + hl) ^ swz4(l)) << 4)
                assert a == tile_off(rows, r0 + l, 2 * s + hl)
                acc.append((a, 16))
            for ph in range(0, 64, per_cycle):
                assert max_bank_use(acc[ph:ph + per_cycle], nbanks) == 1


@pytest.mark.parametrize("nbanks", [32, 64])
@pytest.mark.parametrize("rows,C", SHAPES)
def test_transpose_reads_conflict_free(nbanks, rows, C):
    per_cycle = nbanks * 4 // 8
    for k0 in range(0, rows, 16):
        for m0 in range(0, C * 8, 32):
            for second in (0, 1):
                acc = []
                for lane in range(64):
                    row = 4 * (lane >> 5) + ((lane & 15) >> 2) + 8 * second
                    chunk = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1)
                    byte = 8 * (lane & 1)
                    # TrLane offset + immediates (m0 / 32 column groups, k0 rows)
                    a = (m0 >> 5) * rows * 64 + k0 * 64 + row * 64 + ((chunk ^ swz4(row)) << 4) + byte
                    assert a == tile_off(rows, k0 + row, (m0 >> 3) + chunk) + byte
                    acc.append((a, 8))
                for ph in range(0, 64, per_cycle):
                    assert max_bank_use(acc[ph:ph + per_cycle], nbanks) == 1


# RowStage<W> (epilogue staging of a wave's 32 rows of W bf16 values).
def stage_pos(W, r, c):
    if W == 128:
        return c ^ (r & 15)
    if W == 64:
        return c ^ (((r >> 1) & 3) | (((r ^ (r >> 3)) & 1) << 2))
    return c ^ ((r >> 2) & 3)


def stage_hswap(W, r):
    return ((r >> 1) ^ (r >> 4)) & 1 if W == 32 else ((r >> 3) ^ (r >> 4)) & 1


def stage_off(W, row, col):
    """Byte offset of values col .. col + 3 of `row` (col a multiple of 4)."""
    return row * W * 2 + (stage_pos(W, row, col >> 3) << 4) + \
        ((((col >> 2) & 1) ^ stage_hswap(W, row)) << 3)


@pytest.mark.parametrize("W", [32, 64, 128])
def test_row_stage_bijection(W):
    offs = sorted(stage_off(W, r, col) for r in range(32) for col in range(0, W, 4))
    assert offs == list(range(0, 32 * W * 2, 8))


@pytest.mark.parametrize("nbanks", [32, 64])
@pytest.mark.parametrize("W", [32, 64, 128])
def test_row_stage_conflict_free(nbanks, W):
    # put4: one 8-byte write per lane, lane = (row l32, half hl) at column
    # 32 d + 8 q + 4 hl; one cycle serves nbanks * 4 / 8 lanes.
    per_cycle = nbanks * 4 // 8
    for chunk in range(W // 8):
        acc = [(stage_off(W, lane & 31, 8 * chunk + 4 * (lane >> 5)), 8) for lane in range(64)]
        for ph in range(0, 64, per_cycle):
            assert max_bank_use(acc[ph:ph + per_cycle], nbanks) == 1, (W, chunk, ph)
    # store: 16-byte reads of whole chunks, RPI rows per instruction, and the
    # read chunk holds the row's values col .. col + 7 (halves exchanged back)
    cpr, per_cycle = W // 8, nbanks * 4 // 16
    rpi = 64 // cpr
    for i in range(32 // rpi):
        acc = []
        for lane in range(64):
            r, ch = i * rpi + lane // cpr, lane % cpr
            a = r * W * 2 + (stage_pos(W, r, ch) << 4)
            lo, hi = stage_off(W, r, 8 * ch), stage_off(W, r, 8 * ch + 4)
            assert {lo, hi} == {a, a + 8} and (lo == a + 8) == bool(stage_hswap(W, r))
            if W != 32:  # the exchange is the same for every lane of a store
                assert stage_hswap(W, r) == stage_hswap(W, i * rpi)
            acc.append((a, 16))
        for ph in range(0, 64, per_cycle):
            assert max_bank_use(acc[ph:ph + per_cycle], nbanks) == 1, (W, i, ph)


def test_row_stage_checker_catches_a_plain_rotation():
    # the chunk rotation alone (no half exchange) leaves rows r, r + 16 on the
    # same banks of an 8-byte write at 64 banks
    acc = [((lane & 31) * 256 + ((3 ^ ((lane & 31) & 15)) << 4) + 8 * (lane >> 5), 8)
           for lane in range(64)]
    assert max_bank_use(acc[:32], 64) == 2
