"""The allocation-free sort entry point (smoe_route_sort_noalloc, workspace
in a static device array) against smoe_route_sort with a caller workspace,
both through the C ABI: bit-identical maps, counts and offsets on two calls
in a row, the second smaller than the first (the static array keeps the
first call's contents), and an oversized request rejected on the host."""
import sys

import numpy as np
import pytest
import torch

from smoe import _C

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def _outs(T, K, E, dev):
    R = T * K
    return [torch.full((R,), -7, dtype=torch.int32, device=dev),
            torch.full((R,), -7, dtype=torch.int32, device=dev),
            torch.full((E,), -7, dtype=torch.int32, device=dev),
            torch.full((E + 1,), -7, dtype=torch.int32, device=dev)]


def _sort_both(idx, E, dev):
    lib = _C.lib()
    T, K = idx.shape
    stream = torch.cuda.current_stream().cuda_stream
    ref = _outs(T, K, E, dev)
    nbytes = int(lib.smoe_route_sort_workspace_size(T, K, E))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    st = lib.smoe_route_sort(idx.data_ptr(), T, K, E, *[t.data_ptr() for t in ref],
                             ws.data_ptr(), nbytes, stream)
    assert st == 0, st
    got = _outs(T, K, E, dev)
    st = lib.smoe_route_sort_noalloc(idx.data_ptr(), T, K, E, *[t.data_ptr() for t in got],
                                     stream)
    assert st == 0, st
    torch.cuda.synchronize()
    for n, r, g in zip(("row_map", "inv_map", "counts", "offsets"), ref, got):
        assert torch.equal(r, g), n
    return got


def test_noalloc_sort_matches_workspace_sort(dev):
    g = torch.Generator(device="cpu").manual_seed(21)
    # first call: config-2 size; second: smaller, other E and K
    for T, K, E in ((16384, 8, 256), (3001, 3, 37), (5, 2, 8)):
        say("noalloc sort", T, K, E)
        idx = torch.randint(0, E, (T, K), generator=g, dtype=torch.int32).to(dev)
        _sort_both(idx, E, dev)
    # a sorted expert histogram: the second call's maps must not see the first's
    idx = torch.randint(0, 4, (64, 2), generator=g, dtype=torch.int32).to(dev)
    rm, im, cnt, off = _sort_both(idx, 4, dev)
    flat = idx.reshape(-1).cpu().numpy()
    assert np.array_equal(rm.cpu().numpy(), np.argsort(flat, kind="stable"))
    assert int(off[-1]) == 128


def test_noalloc_sort_rejects_oversized(dev):
    lib = _C.lib()
    cap = int(lib.smoe_route_sort_noalloc_max_bytes())
    assert cap >= 1 << 22
    T, K, E = 1 << 20, 8, 1024  # 1024 * 16384 histogram words = 64 MiB
    assert int(lib.smoe_route_sort_workspace_size(T, K, E)) > cap
    FAKE = 0x100000  # never dereferenced: rejected before any launch
    st = lib.smoe_route_sort_noalloc(FAKE, T, K, E, FAKE, FAKE, FAKE, FAKE, None)
    assert st == -5


def test_noalloc_sort_status_readable(dev):
    """Out-of-range ids through the allocation-free sort: the maps equal the
    workspace sort's, and the routing status (pairs dropped) is readable
    through ops.last_route_status / check_route_status, also with an
    index-less device name."""
    from smoe import ops
    g = torch.Generator(device="cpu").manual_seed(23)
    T, K, E = 1000, 4, 16
    idx = torch.randint(0, E, (T, K), generator=g, dtype=torch.int32)
    bad = torch.randperm(T * K, generator=g)[:37]
    idx.view(-1)[bad[:20]] = E + 3
    idx.view(-1)[bad[20:]] = -1
    idx = idx.to(dev)
    say("noalloc sort status", T, K, E)
    ref = ops.route_sort(idx, E)
    got = _outs(T, K, E, dev)
    ops.route_sort_noalloc(idx, *got)
    # rows past offsets[E] belong to no pair and are left unwritten
    assert int(ref[3][-1]) == T * K - 37
    assert torch.equal(ref[0][:T * K - 37], got[0][:T * K - 37])
    assert bool((got[0][T * K - 37:] == -7).all())
    for n, r, g_ in zip(("inv_map", "counts", "offsets"), ref[1:], got[1:]):
        assert torch.equal(r, g_), n
    assert int(ops.last_route_status("cuda").item()) == 37
    assert int(ops.last_route_status(torch.device("cuda", torch.cuda.current_device())).item()) == 37
    with pytest.raises(ValueError, match="37"):
        ops.check_route_status()
    # a clean call clears it
    ops.route_sort_noalloc(idx.clamp(0, E - 1), *got)
    assert int(ops.last_route_status().item()) == 0
