"""CPU model of the wgrad kernel's tile mapping
(system-lab_amd/csrc/smoe_gemm_wgrad.hip: one-dimensional grid of
ceil(E/8)*8 * KT * NT workgroups dealt to the 8 XCDs round robin; XCD x takes
experts x, x+8, ... and all NT x KT tiles of one expert before the next).  It
checks, without a GPU, that every (expert, n-tile, k-tile) is produced by
exactly one workgroup, that padding workgroups map to experts >= E (which
leave), and that each expert's tiles all land on one XCD."""
import numpy as np
import pytest

WN = WK = 256


def wgrad_tiles(E, N, Kd):
    """(block, xcd, e, n0, k0) for every workgroup that does not leave."""
    KT, NT = -(-Kd // WK), -(-N // WN)
    nblk = -(-E // 8) * 8 * KT * NT
    out = []
    for b in range(nblk):
        xcd, tslot = b & 7, b >> 3
        e = (tslot // (NT * KT)) * 8 + xcd
        if e >= E:
            continue
        rem = tslot % (NT * KT)
        out.append((b, xcd, e, (rem // KT) * WN, (rem % KT) * WK))
    return out, nblk


@pytest.mark.parametrize("E,N,Kd", [(1, 128, 128), (4, 384, 640), (8, 2048, 768), (11, 384, 640),
                                    (128, 1536, 2048), (128, 2048, 768), (1024, 256, 128),
                                    (13, 7168, 2048)])
def test_every_wgrad_tile_once(E, N, Kd):
    tiles, nblk = wgrad_tiles(E, N, Kd)
    KT, NT = -(-Kd // WK), -(-N // WN)
    assert nblk < 2 ** 31
    seen = {(e, n0, k0) for _, _, e, n0, k0 in tiles}
    assert len(seen) == len(tiles), "a tile is produced twice"
    want = {(e, n * WN, k * WK) for e in range(E) for n in range(NT) for k in range(KT)}
    assert seen == want
    for _, _, e, n0, k0 in tiles:
        assert 0 <= n0 < N and 0 <= k0 < Kd


@pytest.mark.parametrize("E,N,Kd", [(11, 384, 640), (128, 1536, 2048)])
def test_wgrad_expert_stays_on_one_xcd(E, N, Kd):
    tiles, _ = wgrad_tiles(E, N, Kd)
    xcd_of = {}
    for _, xcd, e, _, _ in tiles:
        assert xcd_of.setdefault(e, xcd) == xcd, f"expert {e} split over XCDs"
        assert xcd == e % 8
    # within an XCD, one expert's tiles are consecutive in dispatch order
    per_xcd = {}
    for b, xcd, e, _, _ in sorted(tiles):
        per_xcd.setdefault(xcd, []).append(e)
    for seq in per_xcd.values():
        assert seq == sorted(seq)
        assert np.all(np.diff(np.unique(seq, return_index=True)[1]) > 0)
