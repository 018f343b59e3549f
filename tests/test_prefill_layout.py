"""Index arithmetic of the load-to-LDS prefill kernel (redline_amd/csrc/prefill.hip,
PfDma and prefill_dma_kernel), checked on the host against the properties the
kernel relies on:

- the DMA pieces of a tile cover every (key row, 16-byte chunk) exactly once;
- a K fragment read returns the chunk the MFMA operand needs, and the 16 lanes
  of one 16-byte LDS read hit 16 distinct 16-byte slots of a 256-byte span
  (conflict-free with 64 banks of 4 bytes);
- the transposing V reads (8 bytes a lane) address the rows and dims the
  V^T operand needs, with 32 lanes at distinct 8-byte slots of 256 bytes;
- the dim-tile shortcut for D = 128 (offset of dt + 4 = offset of dt ^ 128).

The formulas are those of the kernel; what is checked is their consequence,
not their text."""
import itertools

import pytest


def kswz(D, r):
    return r & 15 if D == 128 else (r >> 1) & 7


def vswz(D, r):
    return (r & 7) << 1 if D == 128 else ((r >> 1) & 3) << 1


def waves(D):
    return 8 if D == 128 else 4


@pytest.mark.parametrize("D,int8", [(128, False), (64, False), (128, True), (64, True)])
def test_dma_pieces_cover_the_tile_once(D, int8):
    raw_row = D if int8 else 2 * D
    tile = 64 * raw_row
    W = waves(D)
    pieces = tile // 1024 // W
    rnd = W * 1024 // raw_row
    seen = {}
    for wave, u, lane in itertools.product(range(W), range(pieces), range(64)):
        byte0 = wave * 1024 + lane * 16
        r0, c = byte0 // raw_row, (byte0 % raw_row) // 16
        r = r0 + rnd * u
        # LDS destination of this lane: piece (wave + W u), 16 bytes per lane
        lds = (wave + W * u) * 1024 + lane * 16
        assert lds == r * raw_row + c * 16  # row-major image
        src_chunk = c if int8 else c ^ kswz(D, r)
        key = (r, src_chunk)
        assert key not in seen
        seen[key] = lds
        if pieces > 1:
            assert kswz(D, r) == kswz(D, r0) and vswz(D, r) == vswz(D, r0)
    assert len(seen) == 64 * (raw_row // 16)


@pytest.mark.parametrize("D", [128, 64])
def test_k_fragment_reads(D):
    row_bytes = 2 * D
    # LDS chunk c of row r holds K chunk c ^ kswz(r)
    for t, ks in itertools.product(range(4), range(D // 32)):
        slots = {}
        for qd, c16 in itertools.product(range(4), range(16)):
            row = 16 * t + c16
            phys = (4 * ks + qd) ^ kswz(D, c16)
            assert phys ^ kswz(D, row) == 4 * ks + qd  # the operand's chunk
            addr = row * row_bytes + phys * 16
            slots.setdefault(qd, []).append((addr % 256) // 16)
        for qd, s in slots.items():  # one 16-lane pass per qd group
            assert len(set(s)) == 16, (t, ks, qd)


@pytest.mark.parametrize("D", [128, 64])
def test_v_transposing_reads(D):
    row_bytes = 2 * D
    kvrd = 4 if D == 128 else D // 16
    for j, dt in itertools.product(range(2), range(D // 16)):
        for half in range(2):  # rows +0 and +16
            slots = {}
            for qd, c16 in itertools.product(range(4), range(16)):
                tk, tm = c16 >> 2, c16 & 3
                row0 = 4 * qd + tk
                vrd = [row0 * row_bytes + ((((2 * d + (tm >> 1)) ^ vswz(D, row0)) << 4) | ((tm & 1) << 3))
                       for d in range(kvrd)]
                off = vrd[dt] if dt < kvrd else vrd[dt - kvrd] ^ 128
                addr = off + 32 * j * row_bytes + 16 * half * row_bytes
                row = addr // row_bytes
                assert row == 32 * j + 16 * half + 4 * qd + tk
                phys = (addr % row_bytes) // 16
                logical = phys ^ vswz(D, row)
                dims = logical * 8 + ((addr % 16) // 8) * 4
                assert dims == 16 * dt + 4 * tm  # lane reads dims 16 dt + 4 tm .. + 3 of its row
                slots.setdefault(qd // 2, []).append((addr % 256) // 8)
            for g, s in slots.items():  # one 32-lane pass per pair of qd groups
                assert len(set(s)) == 32, (j, dt, half, g)
