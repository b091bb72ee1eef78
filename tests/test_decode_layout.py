"""Host checks of the decode kernel's index arithmetic (fa_decode.hip), run on
the CPU before any GPU run: a restatement of the kernel's lane -> address
formulas, checked against what the MFMA operand layout and the buffers
require.

  * K read as rows: lane l of load instruction i reads row
    l / CH + RPI i, dims 8 (l % CH) .. + 7 (CH = D / 8 lanes per row); every
    (row, 16-byte chunk) of a tile is read exactly once.
  * The wavefront's LDS K tile (kt_at): the rows written land on distinct
    16-byte slots inside the wavefront's TP x D f16 tile, and the MFMA
    B-operand read (position 16 grp + l % 16, dims 32 ks + 8 (l / 16))
    returns exactly that K block; the 16 lanes of one read column fall on 16
    distinct 16-byte bank groups.
  * The combine's record offsets stay inside the pair's records.
"""
import itertools

import pytest


def kt_at(D, r, c):
    nch = D // 8
    f = (r >> 1) if D == 64 else r
    return r * D + 8 * (c ^ (f & (nch - 1)))


def dec_record_floats(D, G):
    return G * D + ((2 * G + 3) & ~3)


@pytest.mark.parametrize("D,kv32", [(128, False), (64, False), (128, True), (64, True)])
def test_k_tile_transpose(D, kv32):
    TP = 16 if kv32 else 32
    CH = D // 8
    RPI = 64 // CH
    NV = TP // RPI
    NG = TP // 16
    KS = D // 32
    KT_FLOATS = TP * D // 2
    # load layout: every (row, chunk) once
    seen = set()
    for i in range(NV):
        for l in range(64):
            rc = (l // CH + RPI * i, l % CH)
            assert rc not in seen
            seen.add(rc)
    assert seen == {(r, c) for r in range(TP) for c in range(CH)}
    # LDS writes: distinct 8-half slots inside the region
    lds = {}
    for (r, c) in seen:
        off = kt_at(D, r, c)
        assert off % 8 == 0 and 0 <= off and off + 8 <= 2 * KT_FLOATS
        assert off not in lds
        lds[off] = (r, c)          # the slot holds K[row r][dims 8c .. 8c + 7]
    # MFMA B operand reads: position 16 grp + l % 16, dims 32 ks + 8 (l / 16)
    for grp, ks, l in itertools.product(range(NG), range(KS), range(64)):
        p = 16 * grp + (l & 15)
        c = 4 * ks + (l >> 4)
        assert lds[kt_at(D, p, c)] == (p, c)
    # bank groups of one read column (16 lanes sharing l / 16): distinct
    # 16-byte slots modulo 256 bytes at hd 128 and hd 64
    for grp, ks, hi in itertools.product(range(NG), range(KS), range(4)):
        slots = {(2 * kt_at(D, 16 * grp + lo, 4 * ks + hi) % 256) // 16 for lo in range(16)}
        assert len(slots) == 16


@pytest.mark.parametrize("D,G", [(64, 1), (64, 4), (128, 1), (128, 2), (128, 4)])
def test_merge_offsets(D, G):
    RS = dec_record_floats(D, G)
    assert (RS * 4) % 16 == 0 and RS >= G * D + 2 * G
    for ns in (2, 5, 8, 9, 16, 17, 32, 33, 64):
        maxs = 8 if ns > 32 else 4 if ns > 16 else 2 if ns > 8 else 1
        assert maxs * 8 >= ns
        for h, sl, lane, i in itertools.product(range(G), range(D // 32), range(64), range(maxs)):
            f, grp = lane % 8, lane // 8
            rec = min(grp + 8 * i, ns - 1) * RS * 4
            for off in (rec + 4 * (h * D + 32 * sl + 4 * f), rec + 4 * (G * D + h), rec + 4 * (G * D + G + h)):
                assert 0 <= off and off + 4 <= ns * RS * 4
            assert rec + 4 * (h * D + 32 * sl + 4 * f) + 16 <= ns * RS * 4
