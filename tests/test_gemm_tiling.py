"""CPU model of the grouped GEMM's tile mapping and address arithmetic
(system-lab_amd/csrc/smoe_gemm.hip, Cfg<2,4,8,2>: 256x256 tiles, chip-wide
groups of 32 m-tiles, 8 waves loading 1 KiB segments).  It checks, without a
GPU, that every real (m-tile, n-tile) is produced by exactly one workgroup,
and that every activation, scale, weight and output access of every lane
stays inside its buffer, for valid offsets and for malformed ones
(decreasing, negative or past R), which the kernel clamps to rows [0, R)."""
import numpy as np

BM = BN = 256
CHIP_M, XM, BK = 32, 4, 128
LANES = np.arange(64)


def tile_row(p):
    return (p & ~15) | ((p & 1) << 3) | ((p & 15) >> 1)


def cdiv_trunc(a, b):  # C integer division (truncates toward zero)
    return int(a / b) if a * b >= 0 else -((-a) // b)


def model(R, N, Kd, offsets):
    E = len(offsets) - 1
    mt_bound = (R + BM - 1) // BM + E
    NT = (N + BN - 1) // BN
    nblk = ((mt_bound + CHIP_M - 1) // CHIP_M * CHIP_M * NT + 7) // 8 * 8
    mstart = [0]
    for e in range(E):
        mstart.append(mstart[-1] + cdiv_trunc(int(offsets[e + 1]) - int(offsets[e]) + BM - 1, BM))
    m_all = min(mstart[E], mt_bound)
    full, m_last = m_all // CHIP_M, m_all - (m_all // CHIP_M) * CHIP_M
    chunk = (m_last * NT + 7) // 8
    ksb = Kd // BK
    sizes = {"A": R * Kd, "AS": R * ksb * 4, "B": E * N * Kd, "C": R * N * 2}
    tiles, bad = [], []
    for bid in range(nblk):
        xcd, kx = bid & 7, bid >> 3
        if kx < full * XM * NT:
            g, rem = kx // (XM * NT), kx % (XM * NT)
            mt, nt = g * CHIP_M + XM * xcd + rem % XM, rem // XM
        else:
            j = kx - full * XM * NT
            tl = xcd * chunk + j
            if j >= chunk or tl >= m_last * NT:
                continue
            mt, nt = full * CHIP_M + tl % m_last, tl // m_last
        lo, hi = 0, E
        while hi - lo > 1:
            mid = (lo + hi) >> 1
            lo, hi = (mid, hi) if mstart[mid] <= mt else (lo, mid)
        e = lo
        row0 = int(offsets[e]) + (mt - mstart[e]) * BM
        rows = min(BM, min(int(offsets[e + 1]), R) - row0)
        if row0 < 0 or rows <= 0:
            continue
        tiles.append((mt, nt))
        n0 = nt * BN
        ncols = min(BN, N - n0)
        slot = LANES & 7
        for wid in range(8):
            for seg in range(4):
                row = tile_row((wid * 4 + seg) * 8 + (LANES >> 3))
                oa = np.minimum(row, rows - 1) * Kd + ((slot ^ (row & 7)) << 4)
                ob = np.minimum(row, ncols - 1) * Kd + ((slot ^ (row & 7)) << 4)
                for kb in (0, ksb - 1):
                    if (row0 * Kd + kb * BK + oa).max() + 16 > sizes["A"]:
                        bad.append(("A", bid))
                    if ((e * N + n0) * Kd + kb * BK + ob).max() + 16 > sizes["B"]:
                        bad.append(("B", bid))
            if wid < 4:
                os_ = np.minimum(wid * 64 + LANES, rows - 1) * ksb * 4
                if (row0 * ksb * 4 + (ksb - 1) * 4 + os_).max() + 4 > sizes["AS"]:
                    bad.append(("AS", bid))
        if (row0 + rows - 1) * N * 2 + (n0 + ncols) * 2 > sizes["C"]:
            bad.append(("C", bid))
    return tiles, bad, mstart, NT


def test_every_tile_once_and_in_bounds_for_valid_offsets():
    rng = np.random.default_rng(1)
    for _ in range(60):
        E = int(rng.integers(1, 40))
        counts = rng.integers(0, 700, E)
        counts[rng.random(E) < 0.3] = 0
        R = int(counts.sum()) + int(rng.integers(0, 300))  # rows past offsets[E] are allowed
        R = max(R, 1)
        N = 128 * int(rng.integers(1, 6))
        offsets = np.concatenate([[0], np.cumsum(counts)])
        tiles, bad, mstart, NT = model(R, N, 256, offsets)
        assert not bad, bad[:4]
        want = {(mt, nt) for mt in range(mstart[E]) for nt in range(NT)}
        assert len(tiles) == len(set(tiles)) and set(tiles) == want


def test_in_bounds_for_malformed_offsets():
    rng = np.random.default_rng(2)
    for _ in range(150):
        E = int(rng.integers(1, 9))
        R = int(rng.integers(1, 2000))
        offsets = np.concatenate([[int(rng.integers(-300, 300))],
                                  int(rng.integers(-300, 300)) + np.cumsum(rng.integers(-300, 900, E))])
        _, bad, _, _ = model(R, 256, 256, offsets)
        assert not bad, (R, offsets.tolist(), bad[:4])
    # the case that motivated the clamp: offsets[E] 200,000 rows past R
    R = 1 << 20
    _, bad, _, _ = model(R, 256, 8192, np.concatenate([[0], np.cumsum([200_000, 1, 500_000, R - 500_001])]))
    assert not bad
