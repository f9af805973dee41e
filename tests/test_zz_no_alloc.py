"""
The allocation-free graph build (mh_graph_build_noalloc: scratch in a device array the library owns) against the
allocating one (mh_graph_build with a caller-owned work buffer) through the C ABI: both CSRs, the clamped keys and
the out-of-range flag bitwise equal, on two calls in a row whose second is smaller (the array keeps the first call's
contents, so whatever must start at zero has to be cleared by the kernels), a graph with hub nodes (the long-segment
sort runs in the scratch too), and an out-of-range index.
"""
import numpy as np
import pytest
import torch

from mace_hip_kernels import _native
from mace_hip_kernels import conv as hconv
from oracle import conv as oconv

pytestmark = pytest.mark.gpu


def _noalloc(ei, n):
    dev = ei.device
    E = ei.shape[1]
    keys = torch.full((2, E), -7, device=dev, dtype=torch.int32)
    rowptr = torch.full((2, n + 1), -7, device=dev, dtype=torch.int32)
    eids = torch.full((2, E), -7, device=dev, dtype=torch.int32)
    bad = torch.full((1,), -7, device=dev, dtype=torch.int32)
    P = _native.ptr
    _native.launch('graph_build_noalloc', _native.load().mh_graph_build_noalloc, hconv._graph_module(dev).handle,
                   P(ei), E, n, P(keys), P(rowptr), P(eids), P(bad), _native.stream_of(ei))
    return keys, rowptr, eids, bad


def test_graph_build_noalloc_matches_graph_build():
    assert torch.cuda.is_available(), 'GPU test needs a GPU'
    dev = torch.device('cuda:0')
    rng = np.random.default_rng(21)
    cases = [(2533, 96000, False), (300, 5000, False), (3000, 60000, True), (40, 700, False)]
    for n, e, hubs in cases:
        print(f'[case] noalloc graph build n={n} e={e} hubs={hubs}', flush=True)
        s, r = rng.integers(0, n, e), rng.integers(0, n, e)
        if hubs:
            perm = rng.permutation(e)
            r[perm[:20000]] = 5
            s[perm[20000:26000]] = 9
        ei = torch.tensor(np.stack([s, r]), device=dev)
        want = hconv.build_graph(ei, n)
        got = _noalloc(ei, n)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b), (n, e)
        rp_o, ei_o = oconv.csr_by(r, n)
        assert np.array_equal(got[1][1].cpu().numpy(), rp_o) and np.array_equal(got[2][1].cpu().numpy(), ei_o)
    print('[case] noalloc graph build, out-of-range index', flush=True)
    ei = torch.tensor([[0, 1, 7, 2], [1, -1, 0, 2]], device=dev)
    got, want = _noalloc(ei, 3), hconv.build_graph(ei, 3)
    torch.cuda.synchronize()
    assert int(got[3].item()) == 1
    for a, b in zip(got, want):
        assert torch.equal(a, b)
