"""The LDS tile layout of fna2_amd/csrc/fna2_tile.h, modelled on the CPU.

The formulas below restate swz4 / tile_off / Dma::slot_offset / RowLane /
TrLane.  Checked: the layout is a bijection of 16-byte slots, the DMA plan
fills every slot with the chunk that belongs there, and both MFMA operand
reads are free of bank conflicts for 32 and for 64 four-byte banks (one LDS
cycle serves 128 or 256 bytes: 8 or 16 lanes of a 16-byte read, 16 or 32
lanes of an 8-byte read).
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
