"""CPU model of the wgrad kernel's tile mapping
(system-lab_amd/csrc/smoe_gemm_wgrad.hip).  Tiles are numbered expert-major
(expert e owns tiles e*NT*KT .., n-tile major); a tile of expert e costs
steps(e) + 4 row-group steps; the sequence is cut into 8 contiguous ranges
of about equal cost; workgroup b (XCD b%8, index j = b//8) runs tiles
T_x + j, T_x + j + per_xcd, ... of its XCD's range, per_xcd =
min(ceil(tiles / 8), CUs per XCD) (the launch: one workgroup per CU).
Checked without a GPU: every (expert, n-tile, k-tile) is
produced exactly once for valid and malformed pad[], each XCD's tiles are a
contiguous run (so an expert's tiles stay together), and under Zipf loads
the most loaded XCD carries close to 1/8 of the work where the earlier
expert-per-XCD order put a hot expert's whole work on one XCD."""
import numpy as np
import pytest

WN = WK = 256
FIXED = 4


def _costs(pad, E, ld, TE):
    g0 = np.maximum(pad[:-1], 0)
    g1 = np.minimum(pad[1:], ld)
    steps = np.where(g1 > g0, (g1 - g0) // 128, 0)
    return TE * (steps + FIXED), steps


def wgrad_tiles(pad, N, Kd, ld, cus_per_xcd=32):
    """-> list of (block, xcd, e, n0, k0) and per-XCD cost, following the
    kernel's integer arithmetic and the launch's grid."""
    E = len(pad) - 1
    KT, NT = -(-Kd // WK), -(-N // WN)
    TE = KT * NT
    cost, steps = _costs(np.asarray(pad, np.int64), E, ld, TE)
    cpre = np.concatenate([[0], np.cumsum(cost)])
    W = int(cpre[-1])
    total = E * TE
    per_xcd = min(-(-total // 8), cus_per_xcd)

    def first_tile(c):
        lo = int(np.searchsorted(cpre, c, side="right") - 1)
        lo = min(lo, E - 1)
        per_tile = (cpre[lo + 1] - cpre[lo]) // TE
        r = (c - cpre[lo] + per_tile - 1) // per_tile
        return lo * TE + min(r, TE)

    bounds = [0] + [first_tile(W * x // 8) for x in range(1, 8)] + [total]
    out, work = [], np.zeros(8)
    for b in range(per_xcd * 8):
        x, j = b & 7, b >> 3
        for t in range(bounds[x] + j, bounds[x + 1], per_xcd):
            e, rem = t // TE, t % TE
            out.append((b, x, e, (rem // KT) * WN, (rem % KT) * WK))
            work[x] += steps[e] + FIXED
    return out, work, bounds


def _pad_from_counts(counts):
    groups = [-(-c // 128) for c in counts]
    return np.concatenate([[0], np.cumsum(groups)]) * 128


CASES = [([130, 0, 5, 256, 1], 128, 128), ([1000] * 11, 384, 640), ([1024] * 128, 1536, 2048),
         ([1024] * 128, 2048, 768), ([1] * 1024, 256, 128), ([3] * 13, 7168, 2048),
         ([0] * 4, 256, 256), ([50000, 10, 0, 7000, 0, 0, 3], 512, 768)]


@pytest.mark.parametrize("cus", [32, 1, 5, 1 << 20])
@pytest.mark.parametrize("counts,N,Kd", CASES)
def test_every_wgrad_tile_once(counts, N, Kd, cus):
    pad = _pad_from_counts(counts)
    E = len(counts)
    tiles, _, bounds = wgrad_tiles(pad, N, Kd, int(pad[-1]) or 128, cus)
    KT, NT = -(-Kd // WK), -(-N // WN)
    assert bounds[-1] == E * NT * KT and all(b1 >= b0 for b0, b1 in zip(bounds, bounds[1:]))
    seen = [(e, n0, k0) for _, _, e, n0, k0 in tiles]
    assert len(set(seen)) == len(seen), "a tile is produced twice"
    assert set(seen) == {(e, n * WN, k * WK) for e in range(E) for n in range(NT) for k in range(KT)}


@pytest.mark.parametrize("seed", range(30))
def test_malformed_pad_still_covers_every_tile(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(1, 40))
    pad = np.sort(rng.integers(-500, 5000, E + 1)) if seed % 2 else rng.integers(-500, 5000, E + 1)
    ld = 4096
    tiles, _, _ = wgrad_tiles(pad, 512, 384, ld, 1 + seed % 4)
    seen = [(e, n0, k0) for _, _, e, n0, k0 in tiles]
    assert len(set(seen)) == len(seen) == E * 2 * 2


def test_xcd_ranges_are_contiguous_expert_runs():
    pad = _pad_from_counts([1024] * 128)
    tiles, work, _ = wgrad_tiles(pad, 1536, 2048, int(pad[-1]))
    per = {}
    for b, x, e, _, _ in tiles:
        per.setdefault(x, []).append(e)
    for seq in per.values():
        # the XCD's experts form one contiguous run
        es = sorted(set(seq))
        assert es == list(range(es[0], es[-1] + 1))
    # uniform loads: 16 whole experts per XCD, equal work
    assert all(len(set(seq)) == 16 for seq in per.values())
    assert work.max() == work.min()


def test_zipf_loads_are_balanced():
    """Config-5 fc1 wgrad shape with Zipf(1.2) loads over 128 experts (one
    expert holds a large share): the most loaded XCD carries at most 1/8 of
    the work plus one expert's tile group, against the whole hot expert on
    one XCD under an expert-per-XCD order."""
    rng = np.random.default_rng(0)
    w = 1.0 / np.arange(1, 129) ** 1.2
    counts = np.floor(w / w.sum() * 131072).astype(int)
    counts[0] += 131072 - counts.sum()
    rng.shuffle(counts)
    pad = _pad_from_counts(counts)
    tiles, work, _ = wgrad_tiles(pad, 1536, 2048, int(pad[-1]))
    total = work.sum()
    TE = 6 * 8
    steps = np.diff(pad) // 128
    assert work.max() <= total / 8 + (steps.max() + FIXED) * 2
    old = np.zeros(8)
    for e in range(128):
        old[e % 8] += TE * (steps[e] + FIXED)
    assert work.max() < 0.6 * old.max()
