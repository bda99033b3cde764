"""Host-side check of qmm_lds_kernel's LDS layout (infer.net_amd/csrc/qmm.hip), CPU only.

The kernel's direct global->LDS copies (global_load_lds: lane L of a copy writes its 16 or 4
bytes at the wave-uniform LDS address + L * size) and its MFMA operand reads are restated
here from the kernel's index expressions, for every tile shape the template can take
(8/5-bit, 1/2/4 route tiles of 32, four or eight waves, one or two 32-row slabs). The test
then checks what the kernel relies on:
* the copies of one step land inside their stage and never overlap;
* every operand byte a lane reads was written by that step's copies;
* and it is the byte the MFMA needs: weight row `wr`, codes 32h + 8j .. +7 of the K step
  for MFMA j in lane half h, and route slot n's activations 32h + 8j .. +7 likewise;
* the epilogue's accumulator layout covers each (row, route slot) of the tile exactly once.
NT = 1 (32-route tiles, built for the 8-bit grouped down projection of sparse routing) is
checked as well.
"""
import itertools

import pytest


def stage_layout(bits, nt, mode, rs):
    """mode: 'down' (one matrix, four waves), 'gated' (gate and up, four waves, each wave
    both), 'split' (gate and up, eight waves, waves 4-7 the up matrix)."""
    split = mode == "split"
    nw = 8 if split else 4
    tr = 128 * rs
    ab = 64 * bits // 8
    a_st = tr * ab
    nmat = 1 if mode == "down" else 2
    wmat = 2 if mode == "gated" else 1
    bn = 32 * nt
    st = nmat * a_st + bn * 128
    aq = (2 if bits == 8 else 5) * rs
    nbw = 4 * nt // nw
    return dict(nw=nw, tr=tr, ab=ab, a_st=a_st, nmat=nmat, wmat=wmat, bn=bn, st=st, aq=aq, nbw=nbw, split=split)


def copies(bits, nt, mode, rs):
    """LDS byte -> what it holds after one step's copies: ('w', matrix, row, byte) or
    ('x', route slot, element)."""
    L = stage_layout(bits, nt, mode, rs)
    split = L["split"]
    lds = {}

    def put(addr, val):
        assert 0 <= addr < L["st"], (addr, L["st"])
        assert addr not in lds, ("two copies write one LDS byte", addr)
        lds[addr] = val

    for wave in range(L["nw"]):
        slab = wave & 3
        mw = wave >> 2 if split else 0
        for mm in range(L["wmat"]):
            m = mm + mw
            for q in range(L["aq"]):
                for lane in range(64):
                    if bits == 8:
                        rl, sl = 16 * q + (lane >> 2), lane & 3
                        crow = slab * 32 * rs + rl
                        coff = 16 * (sl ^ ((rl >> 2) & 3))
                        dst = m * L["a_st"] + (slab * 32 * rs + 16 * q) * 64 + 16 * lane
                        for b in range(16):
                            put(dst + b, ("w", m, crow, coff + b))
                    else:
                        i = 64 * q + lane
                        rl = i // 10
                        crow = slab * 32 * rs + rl
                        coff = 4 * (i - rl * 10)
                        dst = m * L["a_st"] + slab * 32 * rs * 40 + q * 256 + 4 * lane
                        for b in range(4):
                            put(dst + b, ("w", m, crow, coff + b))
        for i in range(L["nbw"]):
            for lane in range(64):
                n = (L["nw"] * i + wave) * 8 + (lane >> 3)
                sl = lane & 7
                src_el = 8 * (sl ^ ((n >> 1) & 7))
                dst = L["nmat"] * L["a_st"] + (L["nw"] * i + wave) * 8 * 128 + 16 * lane
                for b in range(16):
                    put(dst + b, ("x", n, src_el + b // 2, b % 2))
    return L, lds


SHAPES = [(bits, nt, mode, rs) for bits, nt, mode, rs in itertools.product((8, 5), (1, 2, 4), ("down", "gated", "split"), (1, 2))
          if (mode == "down" or rs == 1) and (4 * nt) % (8 if mode == "split" else 4) == 0]


@pytest.mark.parametrize("bits,nt,mode,rs", SHAPES)
def test_operand_reads_see_their_copies(bits, nt, mode, rs):
    L, lds = copies(bits, nt, mode, rs)
    nw, split = L["nw"], L["split"]
    for wave in range(nw):
        slab = wave & 3
        mw = wave >> 2 if split else 0
        for lane in range(64):
            r, h = lane & 31, lane >> 5
            # weights: the lane's chunk (codes 32h..32h+31 of row wr in this K step)
            for rsi, mm in itertools.product(range(rs), range(L["wmat"])):
                wr = slab * 32 * rs + 32 * rsi + r
                m = mm + mw
                if bits == 8:
                    sw = (r >> 2) & 3
                    ra = m * L["a_st"] + wr * 64
                    got = [lds[ra + 16 * ((2 * h) ^ sw) + b] for b in range(16)] + \
                          [lds[ra + 16 * ((2 * h + 1) ^ sw) + b] for b in range(16)]
                    want = [("w", m, wr, 32 * h + b) for b in range(32)]
                else:
                    ra = m * L["a_st"] + (wr * 10 + 5 * h) * 4
                    got = [lds[ra + b] for b in range(20)]
                    want = [("w", m, wr, 20 * h + b) for b in range(20)]
                assert got == want, (wave, lane, rsi, m)
            # activations: MFMA j reads route slot n's elements 32h + 8j .. +7
            bb = L["nmat"] * L["a_st"]
            for j in range(4):
                for i in range(nt):
                    n = 32 * i + r
                    pc = 4 * h + j
                    addr = bb + n * 128 + 16 * (pc ^ ((n >> 1) & 7))
                    got = [lds[addr + b] for b in range(16)]
                    want = [("x", n, 32 * h + 8 * j + b // 2, b % 2) for b in range(16)]
                    assert got == want, (wave, lane, j, i)


@pytest.mark.parametrize("bits,nt,mode,rs", SHAPES)
def test_copies_fill_the_stage(bits, nt, mode, rs):
    """Each step's copies write every byte of the weight rows and route slots once."""
    L, lds = copies(bits, nt, mode, rs)
    weights = sorted(v for v in lds.values() if v[0] == "w")
    want_w = sorted(("w", m, row, b) for m in range(L["nmat"]) for row in range(L["tr"]) for b in range(L["ab"]))
    assert weights == want_w
    acts = sorted(v for v in lds.values() if v[0] == "x")
    want_x = sorted(("x", n, e, half) for n in range(L["bn"]) for e in range(64) for half in range(2))
    assert acts == want_x


@pytest.mark.parametrize("nt", [1, 2, 4])
def test_epilogue_covers_each_output_once(nt):
    """Accumulator element k of lane (r, h) in route tile i of slab `slab` is output row
    slab*32 + 8*(k/4) + 4h + k%4 of the tile and route slot 32i + r (the 32x32x16 MFMA's
    C layout), as the epilogue stores it."""
    seen = {}
    for slab in range(4):
        for lane in range(64):
            r, h = lane & 31, lane >> 5
            for i in range(nt):
                for q in range(4):
                    for k in range(4):
                        row = slab * 32 + 8 * q + 4 * h + k
                        key = (row, 32 * i + r)
                        assert key not in seen
                        seen[key] = True
    assert len(seen) == 128 * 32 * nt


def _tile_major_offsets(rows, rs, experts, G):
    """Byte offsets (into the tile-major copy) of every 4-byte piece the streaming kernel's
    copies read, padding rows included, and the (expert, row, piece offset, K step) each
    one belongs to. The copy pads an expert's rows to whole 256-row tiles (Matrix::tiled_rows);
    a copy lane's offset is tile * TR * row_bytes + (crow >> 7) * 128 * row_bytes +
    (crow & 127) * 40 + its piece offset, plus 128 * 40 per K step (qmm_lds_kernel)."""
    import numpy as np
    ab, row_bytes = 40, 40 * G
    rows_pad = (rows + 255) // 256 * 256
    tr = 128 * rs
    e, rt, slab, q, lane, kg = np.meshgrid(np.arange(experts), np.arange((rows + tr - 1) // tr), np.arange(4),
                                           np.arange(5 * rs), np.arange(64), np.arange(G), indexing="ij")
    i = 64 * q + lane
    rl = i // 10
    crow, coff = slab * 32 * rs + rl, 4 * (i - rl * 10)
    row = rt * tr + crow
    tpart = (crow >> 7) * 128 * row_bytes + (crow & 127) * ab + coff
    t_off = e * rows_pad * row_bytes + rt * tr * row_bytes + tpart + kg * 128 * ab
    return t_off, e, row, coff, kg, rows_pad


@pytest.mark.parametrize("rows,rs", [(256, 1), (200, 1), (384, 2), (300, 2), (129, 2)])
def test_tile_major_reads_match_row_major(rows, rs):
    """5-bit streaming launches read the codes from the tile-major copy that
    retile5_kernel writes ([expert][row tile][K step][row in tile][40 bytes], rows padded to
    whole 256-row tiles). Restates both index maps (the kernel's and the retile kernel's) on
    two experts and checks every byte a copy reads is the byte the row-major layout holds
    at row * row_bytes + K step * 40 + piece offset, for rows of the matrix, and zero
    padding inside the copy for the rows past it (their outputs are not stored)."""
    import numpy as np
    experts, G = 2, 8
    row_bytes = 40 * G
    t_off, e, row, coff, kg, rows_pad = _tile_major_offsets(rows, rs, experts, G)
    packed = np.arange(experts * rows * row_bytes, dtype=np.int64)   # byte b holds b
    words = packed.reshape(experts * rows, G, 10, 4)
    tiled = np.full(experts * rows_pad * row_bytes, -1, dtype=np.int64)
    for f in range(experts * rows):                                   # retile5_kernel
        ee, rr = divmod(f, rows)
        tile = ee * (rows_pad // 128) + rr // 128
        for k in range(G):
            for d in range(10):
                dst = ((tile * G + k) * 128 + rr % 128) * 10 + d
                tiled[4 * dst:4 * dst + 4] = words[f, k, d]
    assert t_off.min() >= 0 and t_off.max() + 4 <= tiled.size
    valid = row < rows
    r_off = (e * rows + row) * row_bytes + coff + kg * 40
    for b in range(4):
        assert np.array_equal(tiled[t_off[valid] + b], packed[r_off[valid] + b])
        assert (tiled[t_off[~valid] + b] == -1).all()


@pytest.mark.parametrize("rows", [16400, 16384 + 128, 16384 + 129, 4100, 300])
def test_tile_major_two_slab_copies_stay_in_bounds(rows):
    """Dense two-slab launches (256-row tiles) of single-expert 5-bit matrices: every byte
    a copy reads lies inside the tile-major copy, for rows % 256 in 1..128 (where 128-row
    padding would leave the last tile's upper slabs outside it) and above."""
    G = 8
    t_off, _, _, _, _, rows_pad = _tile_major_offsets(rows, 2, 1, G)
    tiled_bytes = rows_pad * 40 * G
    assert t_off.min() >= 0 and t_off.max() + 4 <= tiled_bytes
