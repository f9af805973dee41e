"""
The radial MLP run inside the convolution's autograd node (``HipConvTP.defer_mlp``, ``conv_mlp.ConvRadialFn``, the
patched model's default) against the two modules run separately, and the edge compaction behind it
(``mh_edge_compact``) against numpy.  With the cutoff marked as the patched radial embedding's (-0.0 outside the
envelope's support), the deferred node lists the edges inside the support first, the MLP computes W0 rows for those
only, the convolution's backward leaves the other dL/dW0 rows unwritten (MH_CUT_NOZERO) and the MLP's backward
writes zero dL/d(edge features) rows there: every output and gradient must equal the separate modules' bitwise.
"""
import copy

import numpy as np
import pytest
import torch

from mace_hip_kernels import HipConvTP, HipRadialMLP, _native, patch_model
from mace_hip_kernels import conv as hconv
from mace_hip_kernels.conv_mlp import FusedWeights
from mace_lite import data as D
from mace_lite import factory

pytestmark = pytest.mark.gpu


def _dev():
    assert torch.cuda.is_available(), 'GPU test needs a GPU'
    return torch.device('cuda:0')


@pytest.mark.parametrize('E', [0, 1, 4095, 4096, 4097, 100003])
def test_edge_compact_vs_numpy(E):
    dev = _dev()
    print(f'[case] edge compaction E={E}', flush=True)
    rng = np.random.default_rng(E + 1)
    c = rng.uniform(0.0, 1.0, size=E).astype(np.float32)
    c[rng.uniform(size=E) < 0.3] = -0.0
    c[rng.uniform(size=E) < 0.05] = 0.0          # +0.0 is inside the support: only -0.0 marks an edge outside
    if E > 9000:
        c[4096:8192] = -0.0                      # one compaction workgroup wholly outside
    ct = torch.tensor(c, device=dev)
    rows, count = hconv.support_rows(ct)
    keep = ~(np.signbit(c) & (c == 0))
    K = int(keep.sum())
    assert int(count.item()) == K
    got = rows.cpu().numpy()
    assert np.array_equal(got[:K], np.nonzero(keep)[0])
    assert np.array_equal(np.sort(got[K:]), np.nonzero(~keep)[0])
    again = hconv.support_rows(ct)               # cached for the tensor's version
    assert again[0] is rows


def _modules(dev):
    model = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    blk = model.interactions[1]
    return HipConvTP(blk.conv_tp, device=dev), HipRadialMLP(blk.conv_tp_weights, device=dev)


@pytest.mark.parametrize('E,marked,want_x', [(40000, True, True), (40000, True, False), (40000, False, True),
                                             (3000, True, True)])
def test_deferred_mlp_equals_separate_modules(E, marked, want_x):
    dev = _dev()
    print(f'[case] deferred radial MLP E={E} marked={marked} want_x={want_x}', flush=True)
    op, mlp = _modules(dev)
    rng = np.random.default_rng(3)
    n = max(64, E // 30)
    s = rng.integers(0, n, size=E)
    r = rng.integers(0, n, size=E)
    c = rng.uniform(0.05, 1.0, size=(E, 1)).astype(np.float32)
    out_mask = rng.uniform(size=E) < 0.2
    if E > 30000:
        out_mask[12000:17000] = True             # whole MLP workgroups and compaction workgroups outside
    c[out_mask] = -0.0
    x = rng.normal(size=(n, op.spec.x_dim)).astype(np.float32)
    Y = rng.normal(size=(E, op.spec.y_dim)).astype(np.float32)
    ef = rng.normal(size=(E, mlp.spec.hs[0])).astype(np.float32)
    g = torch.tensor(rng.normal(size=(n, op.spec.out_dim)).astype(np.float32), device=dev)
    ei = torch.tensor(np.stack([s, r]), device=dev)

    def run(deferred):
        op.defer_mlp(mlp if deferred else None)
        mlp.fuse = deferred
        t = lambda a, rg=True: torch.tensor(a, device=dev, requires_grad=rg)  # noqa: E731
        xt, Yt, eft, ct = t(x, want_x), t(Y), t(ef), t(c)
        if marked:
            ct._mh_support_mask = ct._version
        W = mlp(eft) * ct
        assert isinstance(W, FusedWeights) == deferred
        with _native.timing() as tm:
            out = op(xt, Yt, W, ei)
            out.backward(g)
        torch.cuda.synchronize()
        return out.detach(), xt.grad, Yt.grad, eft.grad, ct.grad, tm.symbols

    try:
        sep = run(False)
        dfr = run(True)
    finally:
        op.defer_mlp(None)
        mlp.fuse = False
    names = ('out', 'gx', 'gY', 'gef', 'gcut')
    for nm, a, b in zip(names, sep[:5], dfr[:5]):
        if nm == 'gx' and not want_x:
            assert a is None and b is None
            continue
        assert torch.equal(a, b), (nm, float((a - b).abs().max()))
    compacted = 'edge_compact' in dfr[5] or 'edge_pairs' in dfr[5]     # (pairing lists the support as well)
    assert compacted == (marked and E >= hconv.EDGE_COMPACT_MIN), dfr[5]
    for tag in ('mlp_fwd[radial_mlp]', 'mlp_bwd[radial_mlp]', 'conv_fwd[conv]', 'conv_bwd[conv]'):
        assert tag in dfr[5], (tag, dfr[5])
    if marked:                                   # the masked edges' gradients are exact zeros
        m = torch.from_numpy(out_mask).to(dev)
        assert not dfr[3][m].any() and not dfr[4][m].any()


def test_patched_model_defers_and_matches(monkeypatch):
    """config 2 (padded: 18% of the edges outside the cutoff): the patched model with the MLPs inside the
    convolutions' nodes (the default) against the same model with them as separate nodes: E and F equal."""
    dev = _dev()
    print('[case] patched model, deferred radial MLP vs separate (config 2)', flush=True)
    model, batch, _ = factory.workload(2)
    b = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in batch.items()}
    outs = []
    for defer in (False, True):
        monkeypatch.setattr(hconv, 'DEFER_RADIAL', defer)
        m = copy.deepcopy(model).to(dev)
        patch_model(m, verbose=False)
        assert all((blk.conv_tp.deferred_mlp() is not None) == defer for blk in m.interactions)
        with _native.timing() as tm:
            o = m(D.fresh(b), compute_force=True)
        torch.cuda.synchronize()
        assert ('edge_compact' in tm.symbols or 'edge_pairs' in tm.symbols) == defer, tm.symbols
        outs.append((o['energy'].detach(), o['forces'].detach()))
    (e0, f0), (e1, f1) = outs
    assert float((e0 - e1).abs().max()) <= 1e-5 and float((f0 - f1).abs().max()) <= 1e-6
    print(f'[case] forces bitwise equal: {torch.equal(f0, f1)}', flush=True)


def _pair_graph(rng, n, m, nf):
    """A graph holding both directions of m node pairs with equal feature rows (as a neighbour list does), plus
    self-loops, reverse edges whose rows differ in one bit, a second image of some pairs at the same length, and
    edges outside the cutoff's support (-0.0).  Edge ids shuffled."""
    a = rng.integers(0, n, size=m)
    b = rng.integers(0, n, size=m)
    f = rng.normal(size=(m, nf)).astype(np.float32)
    s = np.concatenate([a, b, a[:m // 8]])
    r = np.concatenate([b, a, b[:m // 8]])
    ef = np.concatenate([f, f, f[:m // 8]])
    flip = rng.uniform(size=m) < 0.1                 # the reverse row differs by one bit: no sharing
    ef[m:2 * m][flip, 0] = np.nextafter(ef[m:2 * m][flip, 0], np.float32(np.inf))
    c = rng.uniform(0.05, 1.0, size=len(s)).astype(np.float32)
    c[rng.uniform(size=len(s)) < 0.1] = -0.0
    perm = rng.permutation(len(s))
    return s[perm], r[perm], ef[perm], c[perm]


def _pairs_numpy(s, r, ef, c):
    """The pairing's definition: an edge s -> r inside the support with r < s takes the W0 row of the first edge
    r -> s (by edge id) inside the support whose feature row is bitwise equal; every other edge keeps its own."""
    E = len(s)
    inside = ~(np.signbit(c) & (c == 0))
    bits = ef.view(np.uint32)
    wrow, keep = np.arange(E), inside.copy()
    for e in range(E):
        if inside[e] and r[e] < s[e]:
            for e2 in np.nonzero((s == r[e]) & (r == s[e]) & inside)[0]:
                if np.array_equal(bits[e2], bits[e]):
                    wrow[e], keep[e] = e2, False
                    break
    return wrow, keep


@pytest.mark.parametrize('n,m', [(50, 3000), (400, 20000)])
def test_edge_pairs_vs_definition(n, m):
    dev = _dev()
    print(f'[case] edge pairs n={n} m={m}', flush=True)
    rng = np.random.default_rng(n)
    s, r, ef, c = _pair_graph(rng, n, m, 8)
    ei = torch.tensor(np.stack([s, r]), device=dev)
    gr = hconv.graph_for(ei, n)
    eft, ct = torch.tensor(ef, device=dev), torch.tensor(c, device=dev)
    wrow, rows, count, partner = hconv.support_pairs(eft, ct, gr)
    assert partner is None
    want_w, keep = _pairs_numpy(s, r, ef, c)
    assert np.array_equal(wrow.cpu().numpy(), want_w)
    K = int(keep.sum())
    assert int(count.item()) == K and K < int((~(np.signbit(c) & (c == 0))).sum())
    got = rows.cpu().numpy()
    assert np.array_equal(got[:K], np.nonzero(keep)[0])
    assert np.array_equal(np.sort(got[K:]), np.nonzero(~keep)[0])
    # every row read through the map is one the MLP computes
    assert keep[want_w[~(np.signbit(c) & (c == 0))]].all()
    assert hconv.support_pairs(eft, ct, gr)[0] is wrow          # cached for the tensor's version and graph
    # the same pass listed the support (mh_edge_compact's list): cached for the cutoff, no launch
    inside = ~(np.signbit(c) & (c == 0))
    with _native.timing() as tm:
        srows, scount = hconv.support_rows(ct)
    assert not tm.symbols, tm.symbols
    S = int(inside.sum())
    assert int(scount.item()) == S
    got = srows.cpu().numpy()
    assert np.array_equal(got[:S], np.nonzero(inside)[0]) and np.array_equal(np.sort(got[S:]), np.nonzero(~inside)[0])


def _reverse_graph(rng, n, m, nf, hub=0):
    """Both directions of m node pairs with exactly negated vectors and equal feature rows, plus: reverse rows that
    differ in one bit, pairs whose reverse vector is -0.0 where the edge's is +0.0 (equal values), a second image of
    some pairs with its own vectors, edges with a pair's features but no reverse at all, exact duplicates of some
    edges in both directions, self-loops, edges outside the cutoff's support, and (hub > 0) a last node with hub
    incoming and outgoing edges.  Edge ids shuffled."""
    a = rng.integers(0, n, size=m)
    b = rng.integers(0, n, size=m)
    f = rng.normal(size=(m, nf)).astype(np.float32)
    v = rng.normal(size=(m, 3)).astype(np.float32)
    v[: m // 10, 2] = 0.0
    w = -v
    w[: m // 20, 2] = 0.0                                 # +0.0 on both sides: still the exact reverse
    k2, k3, kd = m // 8, m // 16, m // 32
    v2 = (v[:k2] + np.float32(1.5)).astype(np.float32)   # a second image: the same features, other vectors
    s = [a, b, a[:k2], b[:k2], a[:k3], a[:kd], b[:kd]]
    r = [b, a, b[:k2], a[:k2], b[:k3], b[:kd], a[:kd]]
    ef = [f, f, f[:k2], f[:k2], f[:k3], f[:kd], f[:kd]]
    vec = [v, w, v2, -v2, rng.normal(size=(k3, 3)).astype(np.float32), v[:kd], w[:kd]]
    if hub:
        h = n - 1
        src = rng.integers(0, n - 1, size=hub)
        fh = rng.normal(size=(hub, nf)).astype(np.float32)
        vh = rng.normal(size=(hub, 3)).astype(np.float32)
        s += [src, np.full(hub, h)]
        r += [np.full(hub, h), src]
        ef += [fh, fh]
        vec += [vh, -vh]
    s, r, ef, vec = (np.concatenate(x) for x in (s, r, ef, vec))
    flip = np.zeros(len(s), bool)
    flip[m:2 * m] = rng.uniform(size=m) < 0.1
    ef[flip, 0] = np.nextafter(ef[flip, 0], np.float32(np.inf))
    c = rng.uniform(0.05, 1.0, size=len(s)).astype(np.float32)
    c[rng.uniform(size=len(s)) < 0.1] = -0.0
    loops = rng.uniform(size=len(s)) < 0.01
    r[loops] = s[loops]
    perm = rng.permutation(len(s))
    return s[perm], r[perm], ef[perm], c[perm], vec[perm]


def _reverse_pairs_numpy(s, r, ef, c, vec, deg_max):
    """The exact-reverse pairing's definition: edges in id order; an edge s -> r inside the support with r < s (and s
    with at most deg_max incoming edges) takes the first edge r -> s (by id) inside the support, not taken yet, whose
    feature row is bitwise equal and whose vector is the negation of its own; partner[that edge] = the edge."""
    E = len(s)
    inside = ~(np.signbit(c) & (c == 0))
    bits = ef.view(np.uint32)
    indeg = np.bincount(r, minlength=max(s.max(), r.max()) + 1)
    wrow, keep, partner = np.arange(E), inside.copy(), np.full(E, -1)
    taken = np.zeros(E, bool)
    for e in range(E):
        if inside[e] and r[e] < s[e] and indeg[s[e]] <= deg_max:
            for e2 in np.nonzero((s == r[e]) & (r == s[e]) & inside)[0]:
                if not taken[e2] and np.array_equal(bits[e2], bits[e]) and np.all(vec[e2] == -vec[e]):
                    wrow[e], keep[e], partner[e2], taken[e2] = e2, False, e, True
                    break
    return wrow, keep, partner


@pytest.mark.parametrize('n,m,hub', [(50, 3000, 0), (400, 20000, 0), (300, 6000, 2100)])
def test_edge_pairs_exact_reverses(n, m, hub):
    """mh_edge_pairs with the edge vectors: partners are exact reverses, each row is shared by one edge at most,
    and partner[] names that edge; against the definition, edge for edge."""
    dev = _dev()
    print(f'[case] exact-reverse edge pairs n={n} m={m} hub={hub}', flush=True)
    rng = np.random.default_rng(n + m)
    s, r, ef, c, vec = _reverse_graph(rng, n, m, 8, hub)
    ei = torch.tensor(np.stack([s, r]), device=dev)
    gr = hconv.graph_for(ei, n)
    eft, ct, vt = (torch.tensor(a, device=dev) for a in (ef, c, vec))
    wrow, rows, count, partner = hconv.support_pairs(eft, ct, gr, vt)
    want_w, keep, want_p = _reverse_pairs_numpy(s, r, ef, c, vec, hconv.PAIR_DEG_MAX)
    got_w, got_p = wrow.cpu().numpy(), partner.cpu().numpy()
    assert np.array_equal(got_w, want_w) and np.array_equal(got_p, want_p)
    K = int(keep.sum())
    assert int(count.item()) == K
    assert np.array_equal(rows.cpu().numpy()[:K], np.nonzero(keep)[0])
    mapped = np.nonzero(want_w != np.arange(len(s)))[0]
    assert len(mapped) > m // 3 and np.array_equal(want_p[want_w[mapped]], mapped)
    # a duplicate pair shares rows with the duplicate reverse, one each; the hub's edges share none
    if hub:
        h = n - 1
        assert (got_w[(s == h) | (r == h)] == np.nonzero((s == h) | (r == h))[0]).all()
    # the same inputs without vectors: the pairing by feature rows alone, cached separately
    w2, _, _, p2 = hconv.support_pairs(eft, ct, gr)
    assert p2 is None and np.array_equal(w2.cpu().numpy(), _pairs_numpy(s, r, ef, c)[0])


@pytest.mark.parametrize('want_x', [True, False])
def test_paired_gradients_sum_per_pair(monkeypatch, want_x):
    """ConvRadialFn when the features are marked as a function of the lengths of exact-reverse edges
    (conv.PAIR_GRADS): the MLP's backward projects each shared row once from the pair's summed dL/dW0
    (mh_mlp_bwd_pairs).  Against the per-edge backward: output and every other gradient bitwise equal, dL/d(edge
    features) equal on unpaired edges, the pair's sum on the kept edge (fp32 rounding) and zero on its partner."""
    dev = _dev()
    print(f'[case] paired radial gradients want_x={want_x}', flush=True)
    op, mlp = _modules(dev)
    rng = np.random.default_rng(11)
    n = 900
    s, r, ef, c, vec = _reverse_graph(rng, n, 20000, mlp.spec.hs[0])
    E = len(s)
    x = rng.normal(size=(n, op.spec.x_dim)).astype(np.float32)
    Y = rng.normal(size=(E, op.spec.y_dim)).astype(np.float32)
    g = torch.tensor(rng.normal(size=(n, op.spec.out_dim)).astype(np.float32), device=dev)
    ei = torch.tensor(np.stack([s, r]), device=dev)
    vt = torch.tensor(vec, device=dev)

    def run(paired):
        monkeypatch.setattr(hconv, 'PAIR_GRADS', paired)
        op.defer_mlp(mlp)
        mlp.fuse = True
        t = lambda a, rg=True: torch.tensor(a, device=dev, requires_grad=rg)  # noqa: E731
        xt, Yt, eft, ct = t(x, want_x), t(Y), t(ef), t(c[:, None])
        ct._mh_support_mask = ct._version
        eft._mh_vec = (eft._version, vt, vt._version)       # as the patched embedding marks its features
        with _native.timing() as tm:
            out = op(xt, Yt, mlp(eft) * ct, ei)
            out.backward(g)
        torch.cuda.synchronize()
        return out.detach(), xt.grad, Yt.grad, eft.grad, ct.grad, tm.symbols

    try:
        one = run(False)
        two = run(True)
    finally:
        op.defer_mlp(None)
        mlp.fuse = False
    for nm, a, b in zip(('out', 'gx', 'gY', 'gcut'), (one[0], one[1], one[2], one[4]), (two[0], two[1], two[2], two[4])):
        if nm == 'gx' and not want_x:
            assert a is None and b is None
            continue
        assert torch.equal(a, b), (nm, float((a - b).abs().max()))
    assert one[5]['mlp_bwd[radial_mlp]'][0].startswith('mlp_bwd_'), one[5]
    assert two[5]['mlp_bwd[radial_mlp]'][0].startswith('mlp_bwdp_'), two[5]
    g1, g2 = one[3].cpu().numpy(), two[3].cpu().numpy()
    gr = hconv.graph_for(ei, n)
    wrow, _, _, partner = hconv.support_pairs(torch.tensor(ef, device=dev), torch.tensor(c[:, None], device=dev),
                                              gr, vt)
    p = partner.cpu().numpy()
    kept = np.nonzero(p >= 0)[0]
    part = p[kept]
    assert len(kept) > 5000
    scale = float(np.abs(g1).max())
    assert np.abs(g2[kept] - (g1[kept] + g1[part])).max() <= 2e-6 * scale
    assert (g2[part] == 0).all()
    rest = np.setdiff1d(np.arange(E), np.concatenate([kept, part]))
    assert np.array_equal(g2[rest], g1[rest])


@pytest.mark.parametrize('want_x', [True, False])
def test_paired_rows_equal_unpaired_bitwise(monkeypatch, want_x):
    """ConvRadialFn with the W0 rows of reverse edges shared (conv.PAIR_RADIAL) against one row per edge: every
    output and gradient bitwise equal, and the MLP's forward computes fewer rows."""
    dev = _dev()
    print(f'[case] paired radial rows want_x={want_x}', flush=True)
    op, mlp = _modules(dev)
    rng = np.random.default_rng(7)
    n = 900
    s, r, ef, c = _pair_graph(rng, n, 20000, mlp.spec.hs[0])
    E = len(s)
    x = rng.normal(size=(n, op.spec.x_dim)).astype(np.float32)
    Y = rng.normal(size=(E, op.spec.y_dim)).astype(np.float32)
    g = torch.tensor(rng.normal(size=(n, op.spec.out_dim)).astype(np.float32), device=dev)
    ei = torch.tensor(np.stack([s, r]), device=dev)

    def run(paired):
        monkeypatch.setattr(hconv, 'PAIR_RADIAL', paired)
        op.defer_mlp(mlp)
        mlp.fuse = True
        t = lambda a, rg=True: torch.tensor(a, device=dev, requires_grad=rg)  # noqa: E731
        xt, Yt, eft, ct = t(x, want_x), t(Y), t(ef), t(c[:, None])
        ct._mh_support_mask = ct._version
        with _native.timing() as tm:
            out = op(xt, Yt, mlp(eft) * ct, ei)
            out.backward(g)
        torch.cuda.synchronize()
        return out.detach(), xt.grad, Yt.grad, eft.grad, ct.grad, tm.symbols

    try:
        one = run(False)
        two = run(True)
    finally:
        op.defer_mlp(None)
        mlp.fuse = False
    for nm, a, b in zip(('out', 'gx', 'gY', 'gef', 'gcut'), one[:5], two[:5]):
        if nm == 'gx' and not want_x:
            assert a is None and b is None
            continue
        assert torch.equal(a, b), (nm, float((a - b).abs().max()))
    assert 'edge_pairs' in two[5] and 'edge_pairs' not in one[5], two[5]


def test_patched_model_pairs_bitwise(monkeypatch):
    """config 2 (a neighbour list holding both directions of every pair): E and F with the radial MLP rows of
    reverse edges shared equal the unshared ones bit for bit."""
    dev = _dev()
    print('[case] patched model, paired radial rows (config 2)', flush=True)
    model, batch, _ = factory.workload(2)
    b = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in batch.items()}
    outs = []
    monkeypatch.setattr(hconv, 'PAIR_GRADS', False)       # the per-edge backward: bitwise equal forces
    for paired in (False, True):
        monkeypatch.setattr(hconv, 'PAIR_RADIAL', paired)
        m = copy.deepcopy(model).to(dev)
        patch_model(m, verbose=False)
        o = m(D.fresh(b), compute_force=True)
        torch.cuda.synchronize()
        outs.append((o['energy'].detach(), o['forces'].detach()))
    (e0, f0), (e1, f1) = outs
    assert torch.equal(e0, e1) and torch.equal(f0, f1), (float((e0 - e1).abs().max()), float((f0 - f1).abs().max()))


def test_patched_model_paired_gradients(monkeypatch):
    """config 2: the MLP backward over the pairs of exact reverses (conv.PAIR_GRADS, the default) against the
    per-edge backward: energies bitwise equal, forces to fp32 rounding, and the paired kernel runs for both layers
    with E+F but not with stress (the shifts then need a gradient of their own)."""
    dev = _dev()
    print('[case] patched model, paired radial gradients (config 2)', flush=True)
    model, batch, _ = factory.workload(2)
    b = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in batch.items()}
    outs = []
    for paired in (False, True):
        monkeypatch.setattr(hconv, 'PAIR_GRADS', paired)
        m = copy.deepcopy(model).to(dev)
        patch_model(m, verbose=False)
        with _native.timing() as tm:
            o = m(D.fresh(b), compute_force=True)
        torch.cuda.synchronize()
        names = [nm for tag, nms in tm.symbols.items() if tag.startswith('mlp_bwd[') for nm in nms]
        assert len(names) == 2 and all(nm.startswith('mlp_bwdp_' if paired else 'mlp_bwd_') for nm in names), names
        outs.append((o['energy'].detach(), o['forces'].detach()))
        if paired:
            with _native.timing() as tm:
                m(D.fresh(b), compute_force=True, compute_stress=True)
            torch.cuda.synchronize()
            names = [nm for tag, nms in tm.symbols.items() if tag.startswith('mlp_bwd[') for nm in nms]
            assert names and all(nm.startswith('mlp_bwd_') for nm in names), names
    (e0, f0), (e1, f1) = outs
    assert torch.equal(e0, e1), float((e0 - e1).abs().max())
    assert float((f0 - f1).abs().max()) <= 1e-6 * max(1.0, float(f0.abs().max())), float((f0 - f1).abs().max())
