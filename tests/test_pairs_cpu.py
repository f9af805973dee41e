"""
The premise of the shared radial-MLP rows (``conv.support_pairs`` / ``mh_edge_pairs``), on the CPU: in a MACE
neighbour list every edge inside the cutoff has a reverse edge (receiver and sender swapped, shift negated) whose
length, and so whose radial-embedding row, is bitwise equal to its own, because the reverse vector is the exact
negation of the edge's (p_s - p_r - S = -(p_r - p_s + S) in IEEE arithmetic).  Checked on config 2's padded graph with
the restated model's float32 geometry and embedding.  The GPU kernel's pairing itself is pinned against its
definition in tests/test_deferred_radial_gpu.py.
"""
import numpy as np
import torch

from mace_lite import factory
from mace_lite.models import get_edge_vectors_and_lengths


def test_reverse_edges_have_bitwise_equal_embedding_rows():
    model, batch, _ = factory.workload(2)
    s, r = (batch['edge_index'][i].numpy() for i in range(2))
    with torch.no_grad():
        vec, length = get_edge_vectors_and_lengths(batch['positions'], batch['edge_index'], batch['shifts'])
        ef, cut = model.radial_embedding(length)
    ef, cut = ef.numpy(), cut.numpy().reshape(-1)
    sh = batch['shifts'].numpy()
    inside = cut != 0
    def k(a, b, shift):                  # (+ 0.0: -0.0 and 0.0 are one key)
        return (int(a), int(b), *(np.round(shift.astype(np.float64), 6) + 0.0).tolist())
    key = {}
    for e in np.nonzero(inside)[0]:
        key[k(s[e], r[e], sh[e])] = e
    paired = 0
    for e in np.nonzero(inside)[0]:
        e2 = key.get(k(r[e], s[e], -sh[e]))
        assert e2 is not None, f'edge {e} has no reverse inside the cutoff'
        assert np.array_equal(vec[e2].numpy(), -vec[e].numpy())
        assert ef[e2].tobytes() == ef[e].tobytes() and cut[e2] == cut[e]
        paired += 1
    assert paired == int(inside.sum()) and paired > 70000
    # a planted mistake: a reverse vector off by one unit in the last place no longer gives an equal row
    e = int(np.nonzero(inside)[0][0])
    v = vec[e].numpy().copy()
    v[0] = np.nextafter(v[0], np.float32(np.inf))
    with torch.no_grad():
        l2 = torch.linalg.vector_norm(torch.tensor(v)).reshape(1, 1)
        ef2, _ = model.radial_embedding(l2)
    assert ef2.numpy()[0].tobytes() != ef[e].tobytes() or l2.item() == length[e].item()
