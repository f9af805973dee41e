"""
The species order kernel (``mh_species_order``) against torch's argmax / stable argsort and the contraction's slot
layout built from them, on one-hot attributes (every element mix, including elements absent and a single element)
and on rows with ties (the first maximum wins, as torch.argmax), with N crossing the kernel's 1024-node chunks.
"""
import numpy as np
import pytest
import torch

from mace_hip_kernels import species

pytestmark = pytest.mark.gpu


def _want(attrs, group):
    n, ne = attrs.shape
    elem = torch.argmax(attrs, dim=1)
    order = torch.argsort(elem, stable=True)
    slots = torch.full((species.slot_count(n, ne, group),), -1, dtype=torch.int64)
    cnt = torch.bincount(elem, minlength=ne)
    pos = 0
    for e in range(ne):
        members = order[elem[order] == e]
        slots[pos:pos + len(members)] = members
        pos += (int(cnt[e]) + group - 1) // group * group
    return elem.int(), order.int(), slots.int()


@pytest.mark.parametrize('n,ne', [(1, 4), (79, 4), (2533, 4), (4000, 89), (20000, 4), (3000, 1)])
def test_species_order_matches_torch(n, ne):
    dev = torch.device('cuda:0')
    print(f'[case] species order n={n} ne={ne}', flush=True)
    rng = np.random.default_rng(n + ne)
    used = rng.choice(ne, size=max(1, ne // 3), replace=False) if ne > 3 else np.arange(ne)
    idx = rng.choice(used, size=n)
    attrs = np.zeros((n, ne), dtype=np.float32)
    attrs[np.arange(n), idx] = 1.0
    if n > 10:
        attrs[5, :] = 0.5                 # a tie: the first maximum wins
    a = torch.tensor(attrs)
    for group in (8, 4):
        elem, order, slots = species.species_order(a.to(dev), group)
        we, wo, ws = _want(a, group)
        assert torch.equal(elem.cpu(), we) and torch.equal(order.cpu(), wo) and torch.equal(slots.cpu(), ws)
