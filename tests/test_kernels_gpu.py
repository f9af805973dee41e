"""
Kernel-level parity of the HIP path against the oracle (float64 CPU restatement), through the C ABI.

Every case prints its name before launching.  Tolerance: fp32 kernels vs fp64 oracle, max relative error
(normalised by the largest reference magnitude) < 2e-6 for the convolution and < 1e-5 for the symmetric contraction
(hundreds of fp32 terms per output); determinism is bitwise.
"""
import copy
import ctypes

import numpy as np
import pytest
import torch

from mace_hip_kernels import (HipConvTP, HipNodeLinear, HipRadialEmbedding, HipRadialMLP, HipSphericalHarmonics,
                              HipSymmetricContraction, _native, patch_model)
from mace_hip_kernels import conv as hconv
from mace_lite import blocks as B
from mace_lite import factory
from mace_lite import o3
from mace_lite.o3 import Irreps, TensorProduct
from oracle import conv as oconv
from oracle import sc as osc
from oracle import wigner

pytestmark = pytest.mark.gpu
CONV_TOL = 2e-6
SC_TOL = 1e-5


def _dev():
    assert torch.cuda.is_available(), 'GPU test needs a GPU'
    return torch.device('cuda:0')


def _tp(hidden, lmax):
    sh = Irreps.spherical_harmonics(lmax)
    hid = Irreps(hidden)
    target = (sh * hid.count((0, 1))).sort()[0].simplify()
    irreps_mid, ins = B.tp_out_irreps_with_instructions(hid, sh, target)
    return TensorProduct(hid, sh, irreps_mid, ins, shared_weights=False, internal_weights=False)


def _graph(rng, n, e):
    """Random multigraph with isolated nodes, self loops, and one receiver and one sender with > 64 edges."""
    s, r = oconv.random_graph(rng, n, e)
    r[:150] = 0                    # receiver 0: >64 edges (several CSR chunks)
    s[150:230] = 1                 # sender 1: >64 edges
    s[s == n - 1] = 0              # node n-1 never sends ...
    r[r == n - 1] = 1              # ... nor receives
    return s, r


def _rel(got, want):
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


CONV_CASES = [('32x0e+32x1o', 2), ('128x0e', 3), ('128x0e+128x1o', 3), ('128x0e+128x1o+128x2e', 3),
              ('64x0e', 2), ('96x0e+96x1o', 3), ('32x0e', 2)]


@pytest.mark.parametrize('order', ['recv', 'send'])
@pytest.mark.parametrize('hidden,lmax', CONV_CASES)
def test_conv_fwd_bwd_vs_oracle(hidden, lmax, order):
    """Forward and all three gradients against the oracle, with the backward in receiver order (g rows read once
    per receiver, dX through per-edge messages) and in sender order (fused kernel)."""
    dev = _dev()
    print(f'[case] conv {hidden} l{lmax} bwd={order}', flush=True)
    tp = _tp(hidden, lmax)
    op = HipConvTP(tp, device=dev)
    op.bwd_recv = order == 'recv'
    desc = oconv.describe_tp(tp)
    coef = oconv.path_terms(desc)
    rng = np.random.default_rng(1)
    n, e = 41, 700
    s, r = _graph(rng, n, e)
    nw = len(desc['ins']) * desc['mul']
    x, Y, W = rng.normal(size=(n, desc['x_dim'])), rng.normal(size=(e, desc['y_dim'])), rng.normal(size=(e, nw))
    g = rng.normal(size=(n, desc['out_dim']))
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=dev, requires_grad=True)  # noqa: E731
    xt, Yt, Wt = t(x), t(Y), t(W)
    ei = torch.tensor(np.stack([s, r]), device=dev)
    out = op(xt, Yt, Wt, ei)
    out.backward(torch.tensor(g, dtype=torch.float32, device=dev))
    want = oconv.conv_fwd(desc, coef, x, Y, W, s, r, n)
    assert _rel(out.detach().double().cpu().numpy(), want) < CONV_TOL
    assert _rel(xt.grad.double().cpu().numpy(), oconv.conv_bwd_x(desc, coef, g, Y, W, s, r, n)) < CONV_TOL
    assert _rel(Wt.grad.double().cpu().numpy(), oconv.conv_bwd_w(desc, coef, x, g, Y, s, r)) < CONV_TOL
    assert _rel(Yt.grad.double().cpu().numpy(), oconv.conv_bwd_y(desc, coef, x, g, W, s, r)) < CONV_TOL
    assert float(out[n - 1].abs().max()) == 0.0 and float(xt.grad[n - 1].abs().max()) == 0.0


@pytest.mark.parametrize('order', ['recv', 'send'])
def test_conv_bwd_without_dx(order):
    """x not requiring grad (the first interaction layer under forces): gW and gY only, no dX messages."""
    dev = _dev()
    print(f'[case] conv bwd gW/gY only bwd={order}', flush=True)
    tp = _tp('128x0e+128x1o', 3)
    op = HipConvTP(tp, device=dev)
    op.bwd_recv = order == 'recv'
    desc = oconv.describe_tp(tp)
    coef = oconv.path_terms(desc)
    rng = np.random.default_rng(5)
    n, e = 29, 400
    s, r = _graph(rng, n, e)
    x, Y, W = (rng.normal(size=sh) for sh in ((n, desc['x_dim']), (e, desc['y_dim']), (e, 10 * 128)))
    g = rng.normal(size=(n, desc['out_dim']))
    xt = torch.tensor(x, dtype=torch.float32, device=dev)
    Yt, Wt = (torch.tensor(a, dtype=torch.float32, device=dev, requires_grad=True) for a in (Y, W))
    out = op(xt, Yt, Wt, torch.tensor(np.stack([s, r]), device=dev))
    out.backward(torch.tensor(g, dtype=torch.float32, device=dev))
    assert _rel(Wt.grad.double().cpu().numpy(), oconv.conv_bwd_w(desc, coef, x, g, Y, s, r)) < CONV_TOL
    assert _rel(Yt.grad.double().cpu().numpy(), oconv.conv_bwd_y(desc, coef, x, g, W, s, r)) < CONV_TOL


@pytest.mark.parametrize('masked', [False, True])
@pytest.mark.parametrize('want_x,hidden', [(True, '128x0e+128x1o'), (False, '128x0e+128x1o'),
                                           (True, '128x0e+128x1o+128x2e')])
def test_conv_factored_cutoff_weights(want_x, hidden, masked):
    """tp_weights = W0 * cutoff (MACE's form): the backward kernel returns d/dW0 and d/dcutoff itself.  Against the
    oracle: d/dW0 = gW * c, d/dc = sum_k gW * W0 (gW the oracle's d/dW), with some cutoffs exactly zero (padding).
    ``masked``: the cutoff is marked as a patched radial embedding's (-0.0 outside the envelope's support), and
    every third edge holds -0.0: the backward skips those edges (MH_CUT_MASKED), so d/dcutoff is 0 there while
    +0.0 edges keep the exact partial; every other gradient equals the unmasked call's.  The 17-instruction layer
    (l = 0, 1, 2 features) walks its receivers in chunks of 32 edges instead of 64 (its coupling products would
    not fit the LDS budget at 64)."""
    dev = _dev()
    print(f'[case] conv factored cutoff weights want_x={want_x} hidden={hidden} masked={masked}', flush=True)
    tp = _tp(hidden, 3)
    op = HipConvTP(tp, device=dev)
    desc = oconv.describe_tp(tp)
    coef = oconv.path_terms(desc)
    rng = np.random.default_rng(6)
    n, e = 41, 700
    s, r = _graph(rng, n, e)
    x, Y, W0 = (rng.normal(size=sh) for sh in ((n, desc['x_dim']), (e, desc['y_dim']), (e, op.spec.nins * 128)))
    c = rng.uniform(0.0, 1.0, size=(e, 1))
    c[::7] = 0.0
    c[r == 2] = 0.0                  # a receiver whose every edge is skipped by the forward
    neg = np.zeros(e, dtype=bool)
    if masked:
        neg[1::3] = True
        neg[r == 3] = True           # a receiver whose every edge is masked
        c[neg] = -0.0
    g = rng.normal(size=(n, desc['out_dim']))
    t = lambda a, rg=True: torch.tensor(a, dtype=torch.float32, device=dev, requires_grad=rg)  # noqa: E731
    ei = torch.tensor(np.stack([s, r]), device=dev)
    gt = torch.tensor(g, dtype=torch.float32, device=dev)

    def run(mark):
        xt, Yt, W0t, ct = t(x, want_x), t(Y), t(W0), t(c)
        if mark:
            ct._mh_support_mask = ct._version
        W = W0t * ct
        assert hconv._factored_weights(W) is not None
        with _native.timing() as tm:
            out = op(xt, Yt, W, ei)
            out.backward(gt)
        assert tm.symbols['conv_bwd[conv]'][0].startswith('conv_bwdrc_'), tm.symbols
        return out, xt, Yt, W0t, ct

    out, xt, Yt, W0t, ct = run(masked)
    assert (torch.signbit(ct.detach()).cpu().numpy()[:, 0] == neg).all()
    Wd = (W0.astype(np.float32) * c.astype(np.float32)).astype(np.float64)     # the fp32 product the kernel reads
    assert _rel(out.detach().double().cpu().numpy(), oconv.conv_fwd(desc, coef, x, Y, Wd, s, r, n)) < CONV_TOL
    gW = oconv.conv_bwd_w(desc, coef, x, g, Y, s, r)
    assert _rel(W0t.grad.double().cpu().numpy(), gW * c) < CONV_TOL
    gc_want = (gW * W0).sum(1, keepdims=True)
    gc_want[neg] = 0.0
    assert _rel(ct.grad.double().cpu().numpy(), gc_want) < CONV_TOL
    assert _rel(Yt.grad.double().cpu().numpy(), oconv.conv_bwd_y(desc, coef, x, g, Wd, s, r)) < CONV_TOL
    if want_x:
        assert _rel(xt.grad.double().cpu().numpy(), oconv.conv_bwd_x(desc, coef, g, Y, Wd, s, r, n)) < CONV_TOL
    else:
        assert xt.grad is None
    if masked:                       # the skipped edges change nothing but d/dcutoff there
        out_u, xu, Yu, W0u, cu = run(False)
        assert torch.equal(out, out_u) and torch.equal(Yt.grad, Yu.grad) and torch.equal(W0t.grad, W0u.grad)
        assert torch.equal(ct.grad[~torch.from_numpy(neg).to(dev)], cu.grad[~torch.from_numpy(neg).to(dev)])
        if want_x:
            assert torch.equal(xt.grad, xu.grad)


FUSED_TOL = 1e-5      # the MLP's fp32 hidden layers and the fp32-accurate output layer add ~1e-6 to the conv's error


@pytest.mark.parametrize('hidden,lmax,want_x', [('128x0e+128x1o', 3, True), ('128x0e+128x1o', 3, False),
                                                ('32x0e+32x1o', 2, True), ('96x0e+96x1o', 3, True)])
def test_conv_mlp_fused_vs_oracle(hidden, lmax, want_x):
    """The convolution with the radial MLP's output layer inside it (W = cutoff * MLP(ef) formed by the kernels,
    never stored) against the oracle's convolution on W from a float64 copy of the MLP: output, and the gradients
    of x, Y, the edge features (the oracle's dL/dW times the cutoff, through float64 autograd of the MLP) and the
    cutoff (sum over k of dL/dW * W0).  Both layers of each model; some cutoffs exactly zero, a receiver whose every
    edge has zero cutoff, rows longer than 64 edges, isolated nodes."""
    from mace_hip_kernels.conv_mlp import FusedWeights
    dev = _dev()
    model = factory.make_model(hidden, lmax, 3, elements=factory.ELEMENTS_PTCOH)
    rng = np.random.default_rng(17)
    for li, blk in enumerate(model.interactions):
        print(f'[case] fused conv+MLP {hidden} l{lmax} layer {li} want_x={want_x}', flush=True)
        op = HipConvTP(blk.conv_tp, device=dev)
        mlp = HipRadialMLP(blk.conv_tp_weights, device=dev)
        ok, why = op.attach_mlp(mlp)
        assert ok, why
        mlp.fuse = True
        desc = oconv.describe_tp(blk.conv_tp)
        coef = oconv.path_terms(desc)
        n, e = 43, 900
        s, r = _graph(rng, n, e)
        x, Y = rng.normal(size=(n, desc['x_dim'])), rng.normal(size=(e, desc['y_dim']))
        ef = rng.normal(size=(e, mlp.spec.hs[0]))
        c = rng.uniform(0.0, 1.0, size=(e, 1))
        c[::7] = 0.0
        c[r == 2] = 0.0
        g = rng.normal(size=(n, desc['out_dim']))
        t = lambda a, rg=True: torch.tensor(a, dtype=torch.float32, device=dev, requires_grad=rg)  # noqa: E731
        xt, Yt, eft, ct = t(x, want_x), t(Y), t(ef), t(c)
        W = mlp(eft) * ct
        assert isinstance(W, FusedWeights)
        out = op(xt, Yt, W, torch.tensor(np.stack([s, r]), device=dev))
        out.backward(torch.tensor(g, dtype=torch.float32, device=dev))
        m64 = copy.deepcopy(blk.conv_tp_weights).to(torch.float64)
        ef64 = torch.tensor(ef, requires_grad=True)
        W0 = m64(ef64)
        W0n = W0.detach().numpy()
        Wd = W0n * c
        assert _rel(out.detach().double().cpu().numpy(), oconv.conv_fwd(desc, coef, x, Y, Wd, s, r, n)) < FUSED_TOL
        gW = oconv.conv_bwd_w(desc, coef, x, g, Y, s, r)
        W0.backward(torch.tensor(gW * c))
        assert _rel(eft.grad.double().cpu().numpy(), ef64.grad.numpy()) < FUSED_TOL
        assert _rel(ct.grad.double().cpu().numpy(), (gW * W0n).sum(1, keepdims=True)) < FUSED_TOL
        assert _rel(Yt.grad.double().cpu().numpy(), oconv.conv_bwd_y(desc, coef, x, g, Wd, s, r)) < FUSED_TOL
        if want_x:
            assert _rel(xt.grad.double().cpu().numpy(), oconv.conv_bwd_x(desc, coef, g, Y, Wd, s, r, n)) < FUSED_TOL
        else:
            assert xt.grad is None
        # bitwise repeatable
        out2 = op(xt, Yt, mlp(eft) * ct, torch.tensor(np.stack([s, r]), device=dev))
        assert torch.equal(out, out2)


@pytest.mark.parametrize('hidden', ['128x0e', '128x0e+128x1o'])
def test_conv_row_map_entry_points(hidden):
    """mh_conv_fwd_cut_rows / mh_conv_bwd_recv_rows (W0 rows read through a row map, the shared radial-MLP rows of
    an edge and its reverse) through the C ABI: bitwise equal to mh_conv_fwd_cut / mh_conv_bwd_recv run on the
    gathered rows W0[wrow], forward and every gradient (dL/dW0 one row per edge), with the masked-edge flags the
    model uses; and a NULL map is the identity."""
    dev = _dev()
    print(f'[case] conv row map {hidden}', flush=True)
    op = HipConvTP(_tp(hidden, 3), device=dev)
    spec = op.spec
    rng = np.random.default_rng(21)
    n, e, P = 57, 900, 333
    s, r = _graph(rng, n, e)
    f32 = lambda a: torch.tensor(a, dtype=torch.float32, device=dev)  # noqa: E731
    x, Y = f32(rng.normal(size=(n, spec.x_dim))), f32(rng.normal(size=(e, spec.y_dim)))
    W0 = f32(rng.normal(size=(P, spec.nins * spec.mul)))
    wrow = torch.tensor(rng.integers(0, P, size=e), dtype=torch.int32, device=dev)
    c = rng.uniform(0.0, 1.0, size=e).astype(np.float32)
    c[::5] = -0.0                                       # outside the support: skipped by both directions
    c[1::11] = 0.0
    cut = f32(c)
    g = f32(rng.normal(size=(n, spec.out_dim)))
    ei = torch.tensor(np.stack([s, r]), device=dev)
    gr = hconv.graph_for(ei, n)
    (rp_r, ei_r), (rp_s, ei_s) = gr.by_recv(), gr.by_send()
    lib, Pp, st = _native.load(), _native.ptr, _native.stream_of(x)
    Wg = W0[wrow.long()].contiguous()                   # the rows each edge reads, gathered
    flags = _native.MH_WANT_GX | _native.MH_WANT_GWY | _native.MH_CUT_MASKED

    def run(W, m):
        out = torch.empty(n, spec.out_dim, device=dev)
        gx, gY, gW = torch.empty_like(x), torch.empty_like(Y), torch.zeros(e, spec.nins * spec.mul, device=dev)
        gc, work = torch.empty_like(cut), torch.empty(e, spec.x_dim, device=dev)
        _native.check(lib.mh_conv_fwd_cut_rows(op.module.handle, Pp(x), Pp(Y), Pp(W), Pp(rp_r), Pp(ei_r),
                                               Pp(gr.send), Pp(cut), Pp(m), Pp(out), n, st), 'fwd_cut_rows')
        _native.check(lib.mh_conv_bwd_recv_rows(op.module.handle, Pp(x), Pp(g), Pp(Y), Pp(W), Pp(rp_r), Pp(ei_r),
                                                Pp(gr.send), Pp(rp_s), Pp(ei_s), Pp(work), Pp(gx), Pp(gW), Pp(gY),
                                                Pp(cut), Pp(gc), Pp(m), n, flags, st), 'bwd_recv_rows')
        torch.cuda.synchronize()
        return out, gx, gY, gW, gc

    mapped, gathered = run(W0, wrow), run(Wg, None)
    for nm, a, b in zip(('out', 'gx', 'gY', 'gW0', 'gcut'), mapped, gathered):
        assert torch.equal(a, b), (nm, float((a - b).abs().max()))
    assert gathered[0].abs().max() > 0 and gathered[3].abs().max() > 0
    # the row map without a cutoff is refused before any launch
    gx, gY, gW = torch.empty_like(x), torch.empty_like(Y), torch.empty(e, spec.nins * spec.mul, device=dev)
    assert lib.mh_conv_bwd_recv_rows(op.module.handle, Pp(x), Pp(g), Pp(Y), Pp(W0), Pp(rp_r), Pp(ei_r), Pp(gr.send),
                                     None, None, None, None, Pp(gW), Pp(gY), None, None, Pp(wrow), n,
                                     _native.MH_WANT_GWY, st) != 0


def test_conv_c_abi_bwd_x_and_bwd_wy():
    """The reference-shaped entry points mh_conv_bwd_x / mh_conv_bwd_wy against the oracle and the fused kernel."""
    dev = _dev()
    print('[case] conv C-ABI bwd_x / bwd_wy', flush=True)
    tp = _tp('128x0e+128x1o', 3)
    op = HipConvTP(tp, device=dev)
    desc = oconv.describe_tp(tp)
    coef = oconv.path_terms(desc)
    rng = np.random.default_rng(2)
    n, e = 33, 500
    s, r = _graph(rng, n, e)
    f = lambda a: torch.tensor(a, dtype=torch.float32, device=dev)  # noqa: E731
    x, Y, W, g = (rng.normal(size=sh) for sh in ((n, desc['x_dim']), (e, desc['y_dim']), (e, 10 * 128),
                                                  (n, desc['out_dim'])))
    xt, Yt, Wt, gt = f(x), f(Y), f(W), f(g)
    st, rt = torch.tensor(s, dtype=torch.int32, device=dev), torch.tensor(r, dtype=torch.int32, device=dev)
    _, rowptr2, eids2, _ = hconv.build_graph(torch.tensor(np.stack([s, r]), device=dev), n)
    rowptr_s, eids_s = rowptr2[0], eids2[0]
    lib, P, st_ = _native.load(), _native.ptr, _native.stream_of(xt)
    gx = torch.zeros_like(xt)
    _native.check(lib.mh_conv_bwd_x(op.module.handle, P(gt), P(Yt), P(Wt), P(rowptr_s), P(eids_s), P(rt), P(gx), n,
                                    st_), 'bwd_x')
    gW, gY = torch.zeros_like(Wt), torch.zeros_like(Yt)
    _native.check(lib.mh_conv_bwd_wy(op.module.handle, P(xt), P(gt), P(Yt), P(Wt), P(st), P(rt), P(gW), P(gY), e,
                                     st_), 'bwd_wy')
    gW2, gY2, gx2 = torch.zeros_like(Wt), torch.zeros_like(Yt), torch.zeros_like(xt)
    _native.check(lib.mh_conv_bwd(op.module.handle, P(xt), P(gt), P(Yt), P(Wt), P(rowptr_s), P(eids_s), P(rt),
                                  P(gx2), P(gW2), P(gY2), n, 3, st_), 'bwd')
    torch.cuda.synchronize()
    assert _rel(gx.double().cpu().numpy(), oconv.conv_bwd_x(desc, coef, g, Y, W, s, r, n)) < CONV_TOL
    assert _rel(gW.double().cpu().numpy(), oconv.conv_bwd_w(desc, coef, x, g, Y, s, r)) < CONV_TOL
    assert _rel(gY.double().cpu().numpy(), oconv.conv_bwd_y(desc, coef, x, g, W, s, r)) < CONV_TOL
    # receiver-ordered backward through its own entry point (dX via per-edge messages)
    rowptr_r, eids_r = rowptr2[1], eids2[1]
    gW3, gY3, gx3 = torch.zeros_like(Wt), torch.zeros_like(Yt), torch.zeros_like(xt)
    work = torch.empty(e, desc['x_dim'], device=dev)
    _native.check(lib.mh_conv_bwd_recv(op.module.handle, P(xt), P(gt), P(Yt), P(Wt), P(rowptr_r), P(eids_r), P(st),
                                       P(rowptr_s), P(eids_s), P(work), P(gx3), P(gW3), P(gY3), None, None, n, 3, st_),
                  'bwd_recv')
    assert lib.mh_conv_bwd_recv(op.module.handle, P(xt), P(gt), P(Yt), P(Wt), P(rowptr_r), P(eids_r), P(st),
                                None, None, None, P(gx3), P(gW3), P(gY3), None, None, n, 3, st_) != 0   # GX without scratch
    assert b'NULL' in lib.mh_last_error()
    assert lib.mh_conv_bwd_recv(op.module.handle, P(xt), P(gt), P(Yt), P(Wt), P(rowptr_r), P(eids_r), P(st),
                                None, None, None, None, P(gW3), P(gY3), P(Yt), None, n, 2, st_) != 0  # no g_cutoff
    assert b'g_cutoff' in lib.mh_last_error()
    torch.cuda.synchronize()
    assert _rel(gx3.double().cpu().numpy(), oconv.conv_bwd_x(desc, coef, g, Y, W, s, r, n)) < CONV_TOL
    assert _rel(gW3.double().cpu().numpy(), oconv.conv_bwd_w(desc, coef, x, g, Y, s, r)) < CONV_TOL
    assert _rel(gY3.double().cpu().numpy(), oconv.conv_bwd_y(desc, coef, x, g, W, s, r)) < CONV_TOL
    assert torch.equal(gx, gx2)                  # same kernel (fused backward), different flags: bitwise
    # different kernels (per-edge vs fused): same formulas, possibly different fp32 contraction order
    assert _rel(gW2.double().cpu().numpy(), gW.double().cpu().numpy()) < 1e-6
    assert _rel(gY2.double().cpu().numpy(), gY.double().cpu().numpy()) < 1e-6


def test_graph_build_vs_oracle():
    """Both CSRs of an edge list built on the GPU (mh_graph_build) against the oracle's stable-argsort CSR: random
    multigraphs with isolated nodes, a node with 300 edges, one node, no edges, hub nodes of 129, 5,000 and 20,000
    edges (segments past the counting kernel's limit, sorted in LDS and in global memory); bitwise the same on a
    second run; out-of-range indices flagged (and reported by the graph cache's check) or, unvalidated, clamped."""
    dev = _dev()
    rng = np.random.default_rng(12)
    cases = [(37, 900), (2533, 96000), (1, 5), (50, 0), (5000, 300), (3000, 60000)]
    for n, e in cases:
        print(f'[case] graph build n={n} e={e}', flush=True)
        s, r = (rng.integers(0, n, e) for _ in range(2))
        if e >= 900:
            r[:300] = n // 2                     # a long segment
        if e == 60000:                           # hubs, edge ids of each hub scattered over the list
            hub = rng.permutation(e)
            r[hub[:20000]] = 7
            s[hub[20000:25000]] = 11
            s[hub[25000:25129]] = 12
        ei = torch.tensor(np.stack([s, r]), device=dev)
        keys, rowptr, eids, bad = hconv.build_graph(ei, n)
        keys2, rowptr2, eids2, _ = hconv.build_graph(ei, n)
        torch.cuda.synchronize()
        assert int(bad.item()) == 0
        for row, idx in enumerate((s, r)):
            rp_o, ei_o = oconv.csr_by(idx, n)
            assert np.array_equal(rowptr[row].cpu().numpy(), rp_o), (n, e, row)
            assert np.array_equal(eids[row].cpu().numpy(), ei_o), (n, e, row)
            assert np.array_equal(keys[row].cpu().numpy(), idx)
        assert torch.equal(rowptr, rowptr2) and torch.equal(eids, eids2) and torch.equal(keys, keys2)
    print('[case] graph build out of range', flush=True)
    ei = torch.tensor([[0, 1, 7, 2], [1, -1, 0, 2]], device=dev)
    keys, rowptr, eids, bad = hconv.build_graph(ei, 3)
    assert int(bad.item()) == 1 and keys.min() >= 0 and keys.max() <= 2
    hconv.check_graphs()
    hconv._Graph(ei, 3)                          # reported by the next check (GRAPH_CHECK 'deferred')
    with pytest.raises(ValueError, match='outside'):
        hconv.check_graphs()
    gr = hconv._Graph(ei, 3, validate=False)
    assert gr.send.tolist() == [0, 1, 2, 2] and gr.recv.tolist() == [1, 0, 0, 2]
    with pytest.raises(ValueError):
        hconv.build_graph(ei, 0)


def test_conv_deterministic_and_empty():
    dev = _dev()
    print('[case] conv determinism + empty graph', flush=True)
    tp = _tp('128x0e+128x1o', 3)
    op = HipConvTP(tp, device=dev)
    rng = np.random.default_rng(3)
    n, e = 60, 900
    s, r = _graph(rng, n, e)
    ei = torch.tensor(np.stack([s, r]), device=dev)
    f = lambda *sh: torch.randn(*sh, device=dev, requires_grad=True)  # noqa: E731
    x, Y, W = f(n, 512), f(e, 16), f(e, 1280)
    outs = []
    for _ in range(2):
        o = op(x, Y, W, ei)
        gx, gY, gW = torch.autograd.grad(o.square().sum(), (x, Y, W))
        outs.append((o.detach(), gx, gY, gW))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    # no edges at all: zero messages, zero node gradient, empty edge gradients
    ei0 = torch.zeros(2, 0, dtype=torch.int64, device=dev)
    Y0, W0 = f(0, 16), f(0, 1280)
    o = op(x, Y0, W0, ei0)
    assert o.shape == (n, 5120) and float(o.abs().max()) == 0.0
    gx, = torch.autograd.grad(o.sum(), (x,))
    assert float(gx.abs().max()) == 0.0


SC_MODELS = [('32x0e+32x1o', 2, 2), ('128x0e+128x1o', 3, 3), ('64x0e', 2, 2), ('128x0e+128x1o+128x2e', 3, 3)]


SC_FAMILIES = ['node', 'grouped', 'staged', 'staged2']


def _family(op, fam):
    """Force a kernel family of a HipSymmetricContraction."""
    op.split = fam == 'staged2'
    op.staged, op.grouped = (True, None) if fam.startswith('staged') else (False, fam == 'grouped')
    return op


@pytest.mark.parametrize('family', SC_FAMILIES)
@pytest.mark.parametrize('hidden,lmax,corr', SC_MODELS)
def test_sc_fwd_bwd_vs_oracle(hidden, lmax, corr, family):
    """Every kernel family: one node per workgroup; element-grouped (GROUP nodes per workgroup, mixed groups at
    element boundaries, a partial last group); LDS-staged (SLOT_GROUP slots of one element per workgroup, padded
    element runs, coefficient rows through LDS in chunks); the split LDS-staged kernels (the same with two groups of
    waves per workgroup, each walking part of the polynomial)."""
    dev = _dev()
    model = factory.make_model(hidden, lmax, corr, elements=factory.ELEMENTS_PTCOH)
    rng = np.random.default_rng(4)
    for li, prod in enumerate(model.products):
        print(f'[case] sc {hidden} l{lmax} c{corr} layer {li} family={family}', flush=True)
        sc = prod.symmetric_contractions
        op = _family(HipSymmetricContraction(sc, device=dev), family)
        C, n_ell = op.spec.C, op.spec.n_ell
        n = 37
        x = rng.normal(size=(n, C, n_ell)) * 0.7
        elem = rng.integers(0, 4, n)
        attrs = np.eye(4)[elem]
        g = rng.normal(size=(n, op.spec.out_dim))
        xt = torch.tensor(x, dtype=torch.float32, device=dev, requires_grad=True)
        out = op(xt, torch.tensor(attrs, dtype=torch.float32, device=dev))
        out.backward(torch.tensor(g, dtype=torch.float32, device=dev))
        # oracle: dense evaluation per contraction, outputs concatenated as [b, c*M]
        xo = torch.tensor(x, dtype=torch.float64, requires_grad=True)
        parts = []
        for ct in sc.contractions:
            U = {nu: getattr(ct, f'U_matrix_{nu}').double() for nu in range(1, ct.correlation + 1)}
            U = {nu: (u if u.dim() == nu + 2 else u.unsqueeze(0)) for nu, u in U.items()}
            U = {nu: u.reshape(u.shape[0], -1, u.shape[-1]) for nu, u in U.items()}
            Wd = {ct.correlation: ct.weights_max.detach().double()}
            for j, w in enumerate(ct.weights):
                Wd[ct.correlation - 1 - j] = w.detach().double()
            parts.append(osc.sc_dense(U, Wd, xo, elem).reshape(n, -1))
        want = torch.cat(parts, dim=-1)
        want.backward(torch.tensor(g, dtype=torch.float64))
        assert _rel(out.detach().double().cpu().numpy(), want.detach().numpy()) < SC_TOL
        assert _rel(xt.grad.double().cpu().numpy(), xo.grad.numpy()) < SC_TOL


@pytest.mark.parametrize('redundant', [0, 2])
def test_sc_basis_independent(redundant):
    """The kernels see a contraction only through sum_p U W: every contraction of the product rewritten in another
    path basis (a random well-conditioned change of basis, or a redundant one with extra paths; tests/test_oracle_sc
    ``rebased``, in float64) gives the outputs and input gradients of the original, in every kernel family, and
    all match the oracle on the original U and W."""
    from test_oracle_sc import rebased
    dev = _dev()
    model = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    rng = np.random.default_rng(8)
    for li, prod in enumerate(model.products):
        sc = copy.deepcopy(prod.symmetric_contractions).double()
        sc2 = copy.deepcopy(sc)
        for i, ct in enumerate(sc2.contractions):
            sc2.contractions[i] = rebased(ct, seed=10 + i, redundant=redundant)
        n = 41
        elem = rng.integers(0, 4, n)
        attrs = torch.tensor(np.eye(4)[elem], dtype=torch.float32, device=dev)
        for family in SC_FAMILIES:
            print(f'[case] sc basis change layer {li} redundant={redundant} family={family}', flush=True)
            res = []
            for mod in (sc, sc2):
                op = _family(HipSymmetricContraction(mod, device=dev), family)
                x = rng.normal(size=(n, op.spec.C, op.spec.n_ell)) * 0.7 if not res else res[0][0]
                g = rng.normal(size=(n, op.spec.out_dim)) if not res else res[0][1]
                xt = torch.tensor(x, dtype=torch.float32, device=dev, requires_grad=True)
                out = op(xt, attrs)
                out.backward(torch.tensor(g, dtype=torch.float32, device=dev))
                res.append((x, g, out.detach().double().cpu().numpy(), xt.grad.double().cpu().numpy()))
            (x, g, o1, g1), (_, _, o2, g2) = res
            assert _rel(o2, o1) < SC_TOL and _rel(g2, g1) < SC_TOL
            xo = torch.tensor(x, dtype=torch.float64, requires_grad=True)
            parts = []
            for ct in sc.contractions:
                U = {nu: getattr(ct, f'U_matrix_{nu}').double() for nu in range(1, ct.correlation + 1)}
                U = {nu: (u if u.dim() == nu + 2 else u.unsqueeze(0)) for nu, u in U.items()}
                U = {nu: u.reshape(u.shape[0], -1, u.shape[-1]) for nu, u in U.items()}
                Wd = {ct.correlation: ct.weights_max.detach().double()}
                for j, w in enumerate(ct.weights):
                    Wd[ct.correlation - 1 - j] = w.detach().double()
                parts.append(osc.sc_dense(U, Wd, xo, elem).reshape(n, -1))
            want = torch.cat(parts, dim=-1)
            want.backward(torch.tensor(g, dtype=torch.float64))
            assert _rel(o2, want.detach().numpy()) < SC_TOL and _rel(g2, xo.grad.numpy()) < SC_TOL


def test_sc_grouped_matches_per_node():
    """The element-grouped kernels (mh_sc_*_sorted) against the per-node ones (mh_sc_fwd / mh_sc_bwd, the reference's
    launch shape): sorted order (mostly single-element groups) and a random permutation (mostly mixed groups), with a
    node count that leaves a partial last group."""
    dev = _dev()
    print('[case] sc grouped vs per-node', flush=True)
    model = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    op = HipSymmetricContraction(model.products[0].symmetric_contractions, device=dev)
    s, h = op.spec, op.module.handle
    rng = np.random.default_rng(9)
    n = 4 * 13 + 3
    elem_np = rng.integers(0, 4, n)
    f = lambda a: torch.tensor(a, dtype=torch.float32, device=dev)  # noqa: E731
    X, G = f(rng.normal(size=(n, s.C, s.n_ell)) * 0.7), f(rng.normal(size=(n, s.out_dim)))
    elem = torch.tensor(elem_np, dtype=torch.int32, device=dev)
    lib, P, st = _native.load(), _native.ptr, _native.stream_of(X)
    out1, gx1 = torch.empty(n, s.out_dim, device=dev), torch.empty_like(X)
    _native.check(lib.mh_sc_fwd(h, P(X), P(elem), P(op.T), P(out1), n, st), 'sc_fwd')
    _native.check(lib.mh_sc_bwd(h, P(X), P(elem), P(op.T), P(G), P(gx1), n, st), 'sc_bwd')
    sorted_order = torch.argsort(elem, stable=True).to(torch.int32)
    perm = torch.tensor(rng.permutation(n), dtype=torch.int32, device=dev)
    for order in (sorted_order, perm):
        out2, gx2 = torch.full_like(out1, float('nan')), torch.full_like(gx1, float('nan'))
        _native.check(lib.mh_sc_fwd_sorted(h, P(X), P(elem), P(order), P(op.T), P(out2), n, st), 'sc_fwd_sorted')
        _native.check(lib.mh_sc_bwd_sorted(h, P(X), P(elem), P(order), P(op.T), P(G), P(gx2), n, st), 'sc_bwd_sorted')
        torch.cuda.synchronize()
        assert _rel(out2.double().cpu().numpy(), out1.double().cpu().numpy()) < 1e-6
        assert _rel(gx2.double().cpu().numpy(), gx1.double().cpu().numpy()) < 1e-6


@pytest.mark.parametrize('layout', [0, 1])
def test_sc_staged_matches_per_node(layout):
    """The LDS-staged kernels (mh_sc_fwd_staged / mh_sc_bwd_staged), unsplit and split, against the per-node ones
    through the C ABI: element runs of every length mod SLOT_GROUP (a single-node element, a run of exactly
    SLOT_GROUP, a long run with a partial last group), an element with no nodes, both layouts, and slots from
    group_slots; then a second, smaller call on the same module."""
    from mace_hip_kernels import symmetric as hsym
    dev = _dev()
    model = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    for li, prod in enumerate(model.products):
        op = HipSymmetricContraction(prod.symmetric_contractions, device=dev)
        s, h = op.spec, op.module.handle
        rng = np.random.default_rng(20 + li)
        gs = hsym.SLOT_GROUP
        for counts in ([1, gs, 3 * gs + 5, 0], [2, 0, 1, 1]):
            print(f'[case] sc staged vs per-node layer {li} layout {layout} counts {counts}', flush=True)
            elem_np = rng.permutation(np.repeat(np.arange(4), counts))
            n = elem_np.size
            f = lambda a: torch.tensor(a, dtype=torch.float32, device=dev)  # noqa: E731
            X, G = f(rng.normal(size=(n, s.C, s.n_ell)) * 0.7), f(rng.normal(size=(n, s.out_dim)))
            attrs = f(np.eye(4)[elem_np])
            elem = torch.tensor(elem_np, dtype=torch.int32, device=dev)
            slots = hsym.group_slots(attrs)
            Xl = X
            if layout:        # e3nn's irreps layout: block k of dimension d holds channel c at C o_k + c d + m
                parts, o = [], 0
                for d in s.dims:
                    parts.append(X[:, :, o:o + d].reshape(n, -1))
                    o += d
                Xl = torch.cat(parts, dim=1).contiguous()
            lib, P, st = _native.load(), _native.ptr, _native.stream_of(X)
            out1, gx1 = torch.empty(n, s.out_dim, device=dev), torch.empty_like(Xl)
            _native.check(lib.mh_sc_fwd_irreps(h, P(Xl), P(elem), None, P(op.T), P(out1), n, st) if layout else
                          lib.mh_sc_fwd(h, P(X), P(elem), P(op.T), P(out1), n, st), 'sc_fwd')
            _native.check(lib.mh_sc_bwd_irreps(h, P(Xl), P(elem), None, P(op.T), P(G), P(gx1), n, st) if layout else
                          lib.mh_sc_bwd(h, P(X), P(elem), P(op.T), P(G), P(gx1), n, st), 'sc_bwd')
            ms, TS2 = op.split_module()
            for hs, TS in ((h, op.TS), (ms.handle, TS2)):
                out2, gx2 = torch.full_like(out1, float('nan')), torch.full_like(gx1, float('nan'))
                _native.check(lib.mh_sc_fwd_staged(hs, P(Xl), P(slots), slots.numel(), P(elem), P(TS), P(out2), n,
                                                   layout, st), 'sc_fwd_staged')
                _native.check(lib.mh_sc_bwd_staged(hs, P(Xl), P(slots), slots.numel(), P(elem), P(TS), P(G),
                                                   P(gx2), n, layout, st), 'sc_bwd_staged')
                torch.cuda.synchronize()
                assert _rel(out2.double().cpu().numpy(), out1.double().cpu().numpy()) < 1e-6
                assert _rel(gx2.double().cpu().numpy(), gx1.double().cpu().numpy()) < 1e-6
        bad = lib.mh_sc_fwd_staged(h, P(Xl), P(slots), slots.numel() - 1, P(elem), P(op.TS), P(out2), n, layout, st)
        assert bad != 0 and b'multiple' in lib.mh_last_error()


SH_TOL = 5e-6        # absolute on Y (|Y| <= ~4 in component normalisation)


@pytest.mark.parametrize('lmax,norm', [(1, 'component'), (2, 'component'), (3, 'component'), (3, 'norm')])
def test_sh_fwd_bwd_vs_oracle(lmax, norm):
    """Edge spherical harmonics: forward against the oracle's harmonics (fp64), backward against float64 autograd of
    the host model's e3nn module; a ragged edge count (not a multiple of the 256-edge block), a zero vector, a
    leading batch shape, and no edges at all."""
    dev = _dev()
    print(f'[case] spherical harmonics l_max {lmax} {norm}', flush=True)
    mod = o3.SphericalHarmonics(Irreps.spherical_harmonics(lmax), normalize=True, normalization=norm)
    op = HipSphericalHarmonics(mod, device=dev)
    rng = np.random.default_rng(lmax)
    e = 70001
    v = rng.normal(size=(e, 3)) * rng.uniform(0.3, 6.0, size=(e, 1))
    v[0] = 0.0
    vt = torch.tensor(v, dtype=torch.float32, device=dev, requires_grad=True)
    Y = op(vt)
    g = rng.normal(size=(e, op.spec.dim))
    gv, = torch.autograd.grad(Y, vt, torch.tensor(g, dtype=torch.float32, device=dev))
    torch.cuda.synchronize()
    vd = vt.detach().double().cpu()
    ref = wigner.spherical_harmonics(lmax, vd.numpy()[1:]) * np.array(op.spec.scale)
    assert np.abs(Y.detach().double().cpu().numpy()[1:] - ref).max() < SH_TOL
    vr = vd.clone().requires_grad_(True)
    mod64 = o3.SphericalHarmonics(Irreps.spherical_harmonics(lmax), normalize=True, normalization=norm).double()
    Yr = mod64(vr)
    assert np.abs(Y.detach().double().cpu().numpy() - Yr.detach().numpy()).max() < SH_TOL
    gr, = torch.autograd.grad(Yr, vr, torch.tensor(g))
    gv_, gr_ = gv.double().cpu().numpy(), gr.numpy()
    assert np.abs(gv_[0] - gr_[0]).max() <= 1e-5 * np.abs(gr_[0]).max()     # zero vector: |v| clamped, ~1e30
    assert _rel(gv_[1:], gr_[1:]) < 1e-5
    # leading batch dimensions, and the empty edge list
    Y2 = op(vt.detach()[:1000].reshape(10, 100, 3))
    assert Y2.shape == (10, 100, op.spec.dim) and torch.equal(Y2.reshape(1000, -1), Y.detach()[:1000])
    v0 = torch.zeros(0, 3, device=dev, requires_grad=True)
    Y0 = op(v0)
    assert Y0.shape == (0, op.spec.dim)
    g0, = torch.autograd.grad(Y0.sum(), v0)
    assert g0.shape == (0, 3)


def test_sh_c_abi_and_golden():
    """mh_sh_fwd / mh_sh_bwd through the C ABI on the committed golden vectors (tests/golden/coupling.npz), and the
    entry points' errors for a negative edge count and an unbound module."""
    import os
    dev = _dev()
    print('[case] spherical harmonics C-ABI + golden', flush=True)
    gold = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'coupling.npz'))
    lmax = int(round(np.sqrt(gold['sh_values'].shape[1]))) - 1
    op = HipSphericalHarmonics(o3.SphericalHarmonics(Irreps.spherical_harmonics(lmax)), device=dev)
    v = torch.tensor(gold['sh_vectors'], dtype=torch.float32, device=dev)
    Y = torch.empty(v.shape[0], op.spec.dim, device=dev)
    lib, P, st = _native.load(), _native.ptr, _native.stream_of(v)
    _native.check(lib.mh_sh_fwd(op.module.handle, P(v), P(Y), v.shape[0], st), 'sh_fwd')
    gv = torch.empty_like(v)
    _native.check(lib.mh_sh_bwd(op.module.handle, P(v), P(Y), P(gv), v.shape[0], st), 'sh_bwd')
    torch.cuda.synchronize()
    assert np.abs(Y.double().cpu().numpy() - gold['sh_values']).max() < SH_TOL
    # d/dv of |Y(v/|v|)|^2 / 2 = 0 (|Y_l| is constant on the sphere): the backward with gY = Y gives ~0
    assert float(gv.abs().max()) < 1e-4 * float(Y.abs().max()) / float(v.norm(dim=1).min())
    assert lib.mh_sh_fwd(op.module.handle, P(v), P(Y), -1, st) != 0
    assert b'negative' in lib.mh_last_error()
    conv = HipConvTP(_tp('32x0e+32x1o', 2), device=dev)            # a module with no spherical-harmonics kernels
    assert lib.mh_sh_fwd(conv.module.handle, P(v), P(Y), v.shape[0], st) != 0
    assert b'not bound' in lib.mh_last_error()


LIN_TOL = 1e-5       # relative to the largest |component| of the float64 result


def _lin_modules():
    """(name, module) of every patchable node linear of the config-2 and config-4 models and of a 48-channel one."""
    from mace_hip_kernels import lin_supported
    out = []
    for tag, m in (('c2', factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)),
                   ('c4', factory.make_model('128x0e+128x1o+128x2e', 3, 3, elements=factory.ELEMENTS_PTCOH)),
                   ('c48', factory.make_model('48x0e+48x1o', 2, 2))):
        for name, mod in m.named_modules():
            if type(mod).__name__ in ('Linear', 'FullyConnectedTensorProduct') and lin_supported(mod)[0]:
                out.append((f'{tag}.{name}', mod))
    return out


@pytest.mark.parametrize('attrs_kind', ['one_hot', 'dense'])
def test_node_linears_vs_float64(attrs_kind):
    """Every node linear (o3.Linear and skip_tp) of three models: forward and input gradient against float64 runs of
    the e3nn module (autograd for the gradient), on a ragged node count; skip_tp with one-hot element attributes
    (zero terms skipped per tile) and with dense random attributes (every term live)."""
    dev = _dev()
    rng = np.random.default_rng(5)
    n = 1237
    for name, mod in _lin_modules():
        print(f'[case] node linear {name} attrs={attrs_kind}', flush=True)
        op = HipNodeLinear(mod, device=dev)
        s = op.spec
        x = rng.normal(size=(n, s.Din))
        a = None
        if s.V:
            a = (np.eye(s.V)[rng.integers(0, s.V, size=n)] if attrs_kind == 'one_hot' else rng.normal(size=(n, s.V)))
        g = rng.normal(size=(n, s.Dout))
        # every module but the node embedding of one-hot attributes has the tiled backward; that one has the plain
        # one-thread-per-value kernel
        assert s.tiled_bwd == (not name.endswith('node_embedding.linear')), name
        xt = torch.tensor(x, dtype=torch.float32, device=dev, requires_grad=True)
        at = None if a is None else torch.tensor(a, dtype=torch.float32, device=dev)
        out = op(xt, at)
        m64 = copy.deepcopy(mod).double()
        x64 = torch.tensor(x, requires_grad=True)
        ref = m64(x64, torch.tensor(a)) if s.V else m64(x64)
        assert _rel(out.detach().double().cpu().numpy(), ref.detach().numpy()) < LIN_TOL
        gx, = torch.autograd.grad(out, xt, torch.tensor(g, dtype=torch.float32, device=dev))
        gr, = torch.autograd.grad(ref, x64, torch.tensor(g))
        assert _rel(gx.double().cpu().numpy(), gr.numpy()) < LIN_TOL
        if attrs_kind == 'dense':
            continue
        # no nodes at all, and a leading batch shape
        x0 = torch.zeros(0, s.Din, device=dev, requires_grad=True)
        o0 = op(x0, None if at is None else at[:0])
        assert o0.shape == (0, s.Dout)
        o2 = op(xt.detach()[:60].reshape(3, 20, s.Din), None if at is None else at[:60].reshape(3, 20, s.V))
        assert torch.equal(o2.reshape(60, -1), out.detach()[:60])


def test_skip_tp_on_both_families(monkeypatch):
    """skip_tp (attribute terms, species-ordered nodes) generated by the bf16 family (what a 2048-wide skip_tp gets)
    and by the fp32 family (what the narrow ones get): both against float64, forward and input gradient."""
    from mace_hip_kernels import linear as hlin
    dev = _dev()
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    mod = m.interactions[0].skip_tp
    rng = np.random.default_rng(9)
    n = 1001
    x = rng.normal(size=(n, hlin.LinSpec(mod).Din))
    a = np.eye(4)[rng.integers(0, 4, size=n)]
    g = rng.normal(size=(n, hlin.LinSpec(mod).Dout))
    m64 = copy.deepcopy(mod).double()
    x64 = torch.tensor(x, requires_grad=True)
    ref = m64(x64, torch.tensor(a))
    gref, = torch.autograd.grad(ref, x64, torch.tensor(g))
    for fam in ('fp32', 'bf16'):
        print(f'[case] skip_tp on the {fam} family', flush=True)
        monkeypatch.setattr(hlin, 'use_bf16', lambda spec, backward=False, f=fam: f == 'bf16')
        op = HipNodeLinear(mod, device=dev)
        xt = torch.tensor(x, dtype=torch.float32, device=dev, requires_grad=True)
        out = op(xt, torch.tensor(a, dtype=torch.float32, device=dev))
        gx, = torch.autograd.grad(out, xt, torch.tensor(g, dtype=torch.float32, device=dev))
        assert _rel(out.detach().double().cpu().numpy(), ref.detach().numpy()) < LIN_TOL
        assert _rel(gx.double().cpu().numpy(), gref.numpy()) < LIN_TOL


def test_composed_linear_then_skip_tp():
    """MACE's first block, skip_tp(linear(x) / avg, attrs), as one composed launch per direction (compose_after):
    output and input gradient against float64 e3nn; any other use of the quotient forms it as usual."""
    from mace_hip_kernels import linear as hlin
    dev = _dev()
    print('[case] composed linear + skip_tp', flush=True)
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    blk = m.interactions[0]
    lin, skp = HipNodeLinear(blk.linear, device=dev), HipNodeLinear(blk.skip_tp, device=dev)
    lin.div_hint, avg = 7.5, 7.5
    skp.compose_after(lin)
    rng = np.random.default_rng(11)
    n = 1001
    x = rng.normal(size=(n, lin.spec.Din))
    a = np.eye(4)[rng.integers(0, 4, size=n)]
    g = rng.normal(size=(n, skp.spec.Dout))
    x64 = torch.tensor(x, requires_grad=True)
    ref = blk.skip_tp.double()(blk.linear.double()(x64) / avg, torch.tensor(a))
    gref, = torch.autograd.grad(ref, x64, torch.tensor(g))
    xt = torch.tensor(x, dtype=torch.float32, device=dev, requires_grad=True)
    at = torch.tensor(a, dtype=torch.float32, device=dev)
    q = lin(xt) / avg
    assert isinstance(q, hlin.PendingLinear) and q.shape == (n, lin.spec.Dout)
    with _native.timing() as tm:
        out = skp(q, at)
        gx, = torch.autograd.grad(out, xt, torch.tensor(g, dtype=torch.float32, device=dev))
    torch.cuda.synchronize()
    lins = {k: v for k, v in tm.symbols.items() if k.startswith('lin_')}      # (and the element order)
    assert lins == {'lin_fwd[linear+linear]': ['lin_fwd_i2048_o2048_v4c'],
                    'lin_bwd[linear+linear]': ['lin_bwd_i2048_o2048_v4c']}, tm.symbols
    assert _rel(out.detach().double().cpu().numpy(), ref.detach().numpy()) < LIN_TOL
    assert _rel(gx.double().cpu().numpy(), gref.numpy()) < LIN_TOL
    # another consumer of the quotient gets the plain tensor: the linear's kernel with the division folded in
    q2 = lin(xt) / avg
    plain = q2 * 1.0
    with torch.no_grad():
        ref_q = (blk.linear.double()(torch.tensor(x)) / avg).numpy()
    assert _rel(plain.detach().double().cpu().numpy(), ref_q) < LIN_TOL
    # the same skip_tp module on a plain tensor takes its own map
    out2 = skp(torch.tensor(ref_q, dtype=torch.float32, device=dev), at)
    assert _rel(out2.detach().double().cpu().numpy(), ref.detach().numpy()) < LIN_TOL


def test_node_linear_c_abi_and_errors():
    """mh_lin_fwd / mh_lin_bwd through the C ABI against the module, and their errors (NULL operands, a module
    without the kernel)."""
    dev = _dev()
    print('[case] node linear C-ABI', flush=True)
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    op = HipNodeLinear(m.interactions[0].skip_tp, device=dev)
    s = op.spec
    n = 300
    x = torch.randn(n, s.Din, device=dev)
    a = torch.eye(s.V, device=dev)[torch.randint(0, s.V, (n,), device=dev)]
    out, gx = torch.empty(n, s.Dout, device=dev), torch.empty(n, s.Din, device=dev)
    lib, P, st = _native.load(), _native.ptr, _native.stream_of(x)
    _native.check(lib.mh_lin_fwd(op.module.handle, P(x), P(a), P(op.W), P(out), None, 1.0, n, st), 'lin_fwd')
    _native.check(lib.mh_lin_bwd(op.module.handle, P(out), P(a), P(op.Wt), P(gx), None, 1.0, n, st), 'lin_bwd')
    torch.cuda.synchronize()
    ref = op(x, a)
    assert torch.equal(out, ref)
    # <out, out> = <gx, x> for gx = L^T out
    assert abs(_dot(gx, x) - _dot(out, out)) <= 1e-5 * abs(_dot(out, out))
    # the node order is a walking order only: any permutation gives the same numbers (zero terms add exactly 0)
    perm = torch.randperm(n, device=dev).to(torch.int32)
    out_p, gx_p = torch.empty_like(out), torch.empty_like(gx)
    _native.check(lib.mh_lin_fwd(op.module.handle, P(x), P(a), P(op.W), P(out_p), P(perm), 1.0, n, st), 'lin_fwd')
    _native.check(lib.mh_lin_bwd(op.module.handle, P(out), P(a), P(op.Wt), P(gx_p), P(perm), 1.0, n, st), 'lin_bwd')
    torch.cuda.synchronize()
    assert torch.equal(out_p, out) and torch.equal(gx_p, gx)
    # alpha scales every output (a power of two: exactly)
    _native.check(lib.mh_lin_fwd(op.module.handle, P(x), P(a), P(op.W), P(out_p), None, 0.25, n, st), 'lin_fwd')
    _native.check(lib.mh_lin_bwd(op.module.handle, P(out), P(a), P(op.Wt), P(gx_p), None, 0.25, n, st), 'lin_bwd')
    torch.cuda.synchronize()
    assert torch.equal(out_p, 0.25 * out) and torch.equal(gx_p, 0.25 * gx)
    assert lib.mh_lin_fwd(op.module.handle, None, P(a), P(op.W), P(out), None, 1.0, n, st) != 0
    assert b'NULL' in lib.mh_last_error()
    conv = HipConvTP(_tp('32x0e+32x1o', 2), device=dev)
    assert lib.mh_lin_fwd(conv.module.handle, P(x), P(a), P(op.W), P(out), None, 1.0, n, st) != 0
    assert b'not bound' in lib.mh_last_error()


def test_linear_residual_in_the_store():
    """mh_lin_fwd_res (out = alpha L(x) + res, the addition in the kernel's store) equals mh_lin_fwd's output plus
    res added apart, bitwise, on both kernel families (fp32: the product linears and skip_tp, with attributes;
    bf16: the 5120 -> 2048 interaction linear) and for alpha != 1; the pending output of a linear with pend_hint plus
    a same-shape tensor runs it (either operand order), with the residual's gradient g itself and the input's the
    plain map's; other shapes form the plain output first."""
    dev = _dev()
    print('[case] node linear with a residual in its store', flush=True)
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    lib, P = _native.load(), _native.ptr
    n = 611
    for mod in (m.products[0].linear, m.products[1].linear, m.interactions[1].skip_tp, m.interactions[1].linear):
        op = HipNodeLinear(mod, device=dev)
        s = op.spec
        x = torch.randn(n, s.Din, device=dev)
        a = torch.eye(s.V, device=dev)[torch.randint(0, s.V, (n,), device=dev)] if s.V else None
        res = torch.randn(n, s.Dout, device=dev)
        st = _native.stream_of(x)
        for alpha in (1.0, 0.3):
            plain, got = torch.empty(n, s.Dout, device=dev), torch.empty(n, s.Dout, device=dev)
            _native.check(lib.mh_lin_fwd(op.module.handle, P(x), P(a), P(op.W), P(plain), None, alpha, n, st), 'fwd')
            _native.check(lib.mh_lin_fwd_res(op.module.handle, P(x), P(a), P(op.W), P(got), None, alpha, P(res), n,
                                             st), 'fwd_res')
            torch.cuda.synchronize()
            assert torch.equal(got, plain + res), (mod.__class__.__name__, s.Din, s.Dout, alpha)
    op = HipNodeLinear(m.products[1].linear, device=dev)
    x = torch.randn(n, op.spec.Din, device=dev, requires_grad=True)
    res = torch.randn(n, op.spec.Dout, device=dev, requires_grad=True)
    g = torch.randn(n, op.spec.Dout, device=dev)
    plain = op(x)
    ref = plain + res
    gx_ref, = torch.autograd.grad(ref, x, g)
    op.pend_hint = True
    for order in (0, 1):
        pend = op(x)
        assert type(pend).__name__ == 'PendingLinear'
        y = pend + res if order == 0 else res + pend
        assert type(y) is torch.Tensor and torch.equal(y, ref)
        gx, gr = torch.autograd.grad(y, (x, res), g)
        assert torch.equal(gx, gx_ref) and torch.equal(gr, g)
    y = op(x) + res[:1]                          # broadcast: the plain output first, then torch's add
    assert torch.equal(y, plain + res[:1])


def test_linear_backward_over_three_gradients():
    """mh_lin_bwd_sum (lin_bwds: the backward over (g + g2) + g3, added as loaded) equals mh_lin_bwd on that sum
    formed apart, bitwise, for the fp32-family product linear; NULL gradients are rejected."""
    dev = _dev()
    print('[case] node linear backward over three gradients', flush=True)
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    op = HipNodeLinear(m.products[0].linear, device=dev)
    s = op.spec
    lib, P = _native.load(), _native.ptr
    for n in (611, 5):
        g = [torch.randn(n, s.Dout, device=dev) for _ in range(3)]
        got, want = torch.empty(n, s.Din, device=dev), torch.empty(n, s.Din, device=dev)
        st = _native.stream_of(g[0])
        _native.check(lib.mh_lin_bwd_sum(op.sum_module().handle, P(g[0]), P(g[1]), P(g[2]), None, P(op.Wt), P(got),
                                         None, 1.0, n, st), 'bwd_sum')
        tot = (g[0] + g[1]) + g[2]
        _native.check(lib.mh_lin_bwd(op.module.handle, P(tot), None, P(op.Wt), P(want), None, 1.0, n, st), 'bwd')
        torch.cuda.synchronize()
        assert torch.equal(got, want), n
    assert lib.mh_lin_bwd_sum(op.sum_module().handle, P(g[0]), None, P(g[2]), None, P(op.Wt), P(got), None, 1.0, 5,
                              st) != 0
    assert b'NULL' in lib.mh_last_error()


def test_linear_division_folded():
    """The interaction linear's output divided by avg_num_neighbors (MACE's block code) is computed with the division
    folded into the kernels: same values and input gradient as dividing the plain output, and any other use of the
    pending output sees the plain output."""
    dev = _dev()
    print('[case] folded avg_num_neighbors division', flush=True)
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    mod = m.interactions[1].linear
    op = HipNodeLinear(mod, device=dev)
    n = 777
    x = torch.randn(n, op.spec.Din, device=dev, requires_grad=True)
    g = torch.randn(n, op.spec.Dout, device=dev)
    ref = op(x) / 20.0
    gref, = torch.autograd.grad(ref, x, g)
    op.div_hint = 20.0
    pend = op(x)
    assert type(pend).__name__ == 'PendingLinear' and pend.shape == (n, op.spec.Dout)
    got = pend / 20.0
    assert type(got) is torch.Tensor
    ggot, = torch.autograd.grad(got, x, g)
    assert torch.allclose(got, ref, rtol=1e-6, atol=1e-6 * float(ref.abs().max()))
    assert torch.allclose(ggot, gref, rtol=1e-6, atol=1e-6 * float(gref.abs().max()))
    other = op(x) + 1.0                                   # not a division: the plain output
    assert torch.equal(other, ref * 20.0 + 1.0) or torch.allclose(other, ref * 20.0 + 1.0, rtol=1e-6, atol=1e-5)
    # the patched model folds it for both interaction blocks
    rep = patch_model(copy.deepcopy(m).to(dev), verbose=False)
    assert 'interactions.1.linear' in rep['patched']


def _dot(a, b):
    return float((a.double() * b.double()).sum())


MLP_TOL = 1e-5       # relative to the largest |component| of the float64 result


@pytest.mark.parametrize('hidden,lmax,elements', [('128x0e+128x1o', 3, 'ptcoh'), ('128x0e+128x1o+128x2e', 3, 'ptcoh'),
                                                  ('32x0e+32x1o', 2, 'ref')])
def test_radial_mlp_vs_float64(hidden, lmax, elements):
    """Each interaction block's radial MLP: forward and d/d(edge features) against float64 runs of the e3nn module,
    on a ragged edge count (not a multiple of the 64-edge block), with edge features of the model's radial
    embedding (Bessel basis times the cutoff envelope, so rows of zeros past the cutoff) and random ones."""
    dev = _dev()
    el = factory.ELEMENTS_PTCOH if elements == 'ptcoh' else factory.ELEMENTS_REF
    model = factory.make_model(hidden, lmax, 2, elements=el)
    rng = np.random.default_rng(9)
    e = 3001
    r = torch.tensor(rng.uniform(0.5, 6.0, size=(e, 1)))
    emb, _ = model.radial_embedding.double()(r)
    for kind, ef in (('embedding', emb.numpy()), ('random', rng.normal(size=(e, emb.shape[1])))):
        for li, blk in enumerate(model.interactions):
            print(f'[case] radial MLP {hidden} layer {li} ({kind} features)', flush=True)
            op = HipRadialMLP(blk.conv_tp_weights, device=dev)
            xt = torch.tensor(ef, dtype=torch.float32, device=dev, requires_grad=True)
            out = op(xt)
            g = rng.normal(size=tuple(out.shape))
            gx, = torch.autograd.grad(out, xt, torch.tensor(g, dtype=torch.float32, device=dev))
            m64 = copy.deepcopy(blk.conv_tp_weights).double()
            x64 = torch.tensor(ef, requires_grad=True)
            ref = m64(x64)
            gr, = torch.autograd.grad(ref, x64, torch.tensor(g))
            assert _rel(out.detach().double().cpu().numpy(), ref.detach().numpy()) < MLP_TOL
            assert _rel(gx.double().cpu().numpy(), gr.numpy()) < MLP_TOL
    # no edges, and a leading batch shape
    op = HipRadialMLP(model.interactions[0].conv_tp_weights, device=dev)
    x0 = torch.zeros(0, emb.shape[1], device=dev, requires_grad=True)
    o0 = op(x0)
    assert o0.shape == (0, op.hs[-1])
    assert torch.autograd.grad(o0.sum(), x0)[0].shape == (0, emb.shape[1])
    xb = torch.tensor(ef[:64], dtype=torch.float32, device=dev)
    assert torch.equal(op(xb.reshape(4, 16, -1)).reshape(64, -1), op(xb))


@pytest.mark.parametrize('hidden,lmax', [('128x0e+128x1o', 3), ('32x0e+32x1o', 2)])
def test_radial_mlp_double_backward_vs_float64(hidden, lmax):
    """The radial MLP's second derivatives (mlp_jvp, mlp_bwd2 behind patch's double backward) against float64
    autograd of the e3nn module: for the loss <u, dL/def> with dL/def = J(ef)^T g, the gradients with respect to g
    (J u, the forward-mode derivative) and to ef (the Hessian-vector product sum_k g_k d^2 W0_k/def^2 u), on a
    ragged edge count, embedding-like and random features."""
    dev = _dev()
    model = factory.make_model(hidden, lmax, 2, elements=factory.ELEMENTS_PTCOH)
    rng = np.random.default_rng(19)
    e = 1999
    r = torch.tensor(rng.uniform(0.5, 6.0, size=(e, 1)))
    emb, _ = model.radial_embedding.double()(r)
    for kind, ef in (('embedding', emb.numpy()), ('random', rng.normal(size=(e, emb.shape[1])))):
        for li, blk in enumerate(model.interactions):
            print(f'[case] radial MLP double backward {hidden} layer {li} ({kind} features)', flush=True)
            op = HipRadialMLP(blk.conv_tp_weights, device=dev)
            op.double_backward = True
            nw = op.hs[-1]
            g, u = rng.normal(size=(e, nw)), rng.normal(size=ef.shape)
            res = []
            for dt, m in ((torch.float32, op), (torch.float64, copy.deepcopy(blk.conv_tp_weights).double().to(dev))):
                xt = torch.tensor(ef, dtype=dt, device=dev, requires_grad=True)
                gt = torch.tensor(g, dtype=dt, device=dev, requires_grad=True)
                out = m(xt)
                gx, = torch.autograd.grad(out, xt, gt, create_graph=True)
                d_g, d_x = torch.autograd.grad((gx * torch.tensor(u, dtype=dt, device=dev)).sum(), (gt, xt))
                res.append((gx.detach().double().cpu().numpy(), d_g.double().cpu().numpy(),
                            d_x.double().cpu().numpy()))
            for got, want in zip(*res):
                assert _rel(got, want) < MLP_TOL


def test_radial_mlp_c_abi():
    dev = _dev()
    print('[case] radial MLP C-ABI', flush=True)
    model = factory.make_model('128x0e+128x1o', 3, 2, elements=factory.ELEMENTS_PTCOH)
    op = HipRadialMLP(model.interactions[1].conv_tp_weights, device=dev)
    e = 200
    x = torch.randn(e, op.hs[0], device=dev)
    out = torch.empty(e, op.hs[-1], device=dev)
    lib, P, st = _native.load(), _native.ptr, _native.stream_of(x)
    _native.check(lib.mh_mlp_fwd(op.module.handle, P(x), P(op.WhT), P(op.WlT), P(out), e, st), 'mlp_fwd')
    gx = torch.empty_like(x)
    _native.check(lib.mh_mlp_bwd(op.module.handle, P(x), P(op.Wh), P(op.Wl), P(out), P(gx), e, st), 'mlp_bwd')
    torch.cuda.synchronize()
    assert _rel(out.double().cpu().numpy(), op(x).double().cpu().numpy()) < 2e-6     # the module's forward (mlp_out)
    # the backward is the adjoint of the Jacobian: <gx, dx> = <out, J dx> for a small step dx (finite difference)
    dx = 1e-3 * torch.randn_like(x)
    jdx = (op(x + dx) - op(x - dx)) / 2
    lhs, rhs = _dot(gx, dx), _dot(out, jdx)
    assert abs(lhs - rhs) <= 1e-3 * abs(rhs)
    assert lib.mh_mlp_fwd(op.module.handle, None, P(op.WhT), P(op.WlT), P(out), e, st) != 0
    assert b'NULL' in lib.mh_last_error()


@pytest.mark.parametrize('hidden,lmax', [('128x0e+128x1o', 3), ('32x0e+32x1o', 2)])
def test_radial_mlp_weight_stationary_c_abi(hidden, lmax):
    """mh_mlp_fwd_ws (hidden activations into a slot-ordered scratch, then the output layer with each wave's 64-column
    block of split weights held in registers over the tiles of its XCD's share, four waves sharing each tile through
    LDS) against the single-kernel
    mh_mlp_fwd_rows and against float64 (MLPSpec.apply): every listed row to fp32 accuracy, every unlisted row left
    untouched (a NaN sentinel survives), on ragged counts and slot counts (0, 1, 15, 17 ... rows; tiles of 16), with
    and without a row list, for output widths with whole and partial 64-column blocks (1280, 512, 224, 96)."""
    dev = _dev()
    model = factory.make_model(hidden, lmax, 2, elements=factory.ELEMENTS_PTCOH)
    lib, P = _native.load(), _native.ptr
    rng = np.random.default_rng(29)
    for li, blk in enumerate(model.interactions):
        op = HipRadialMLP(blk.conv_tp_weights, device=dev)
        nw, hl = op.hs[-1], op.hs[-2]
        for e, cnt in ((1, 1), (17, 15), (17, 0), (1000, 1000), (3001, 1777), (3001, None)):
            print(f'[case] weight-stationary MLP forward {hidden} layer {li}: E={e} count={cnt} (NW={nw})', flush=True)
            x = torch.tensor(rng.normal(size=(e, op.hs[0])), dtype=torch.float32, device=dev)
            st = _native.stream_of(x)
            if cnt is None:
                rows = count = None
                listed = np.arange(e)
            else:
                perm = rng.permutation(e).astype(np.int32)
                rows = torch.tensor(perm, device=dev)
                count = torch.tensor([cnt], dtype=torch.int32, device=dev)
                listed = perm[:cnt]
            got = torch.full((e, nw), float('nan'), device=dev)
            old = torch.full((e, nw), float('nan'), device=dev)
            h3 = torch.empty(e, hl, device=dev)
            _native.check(lib.mh_mlp_fwd_ws(op.module.handle, P(x), P(op.WhT), P(op.Wo), P(h3), P(got), e, P(rows),
                                            P(count), op.ncb, st), 'mlp_fwd_ws')
            _native.check(lib.mh_mlp_fwd_rows(op.module.handle, P(x), P(op.WhT), P(op.WlT), P(old), e, P(rows),
                                              P(count), st), 'mlp_fwd_rows')
            torch.cuda.synchronize()
            g, o = got.cpu().numpy(), old.cpu().numpy()
            unl = np.setdiff1d(np.arange(e), listed)
            assert np.isnan(g[unl]).all()
            if len(listed):
                want = op.spec.apply(x.double().cpu().numpy()[listed])
                assert _rel(g[listed].astype(np.float64), want) < MLP_TOL
                assert _rel(g[listed].astype(np.float64), o[listed].astype(np.float64)) < 2e-6
    assert lib.mh_mlp_fwd_ws(op.module.handle, P(x), P(op.WhT), P(op.Wo), P(h3), P(got), 5, None, None, 0, st) != 0
    assert b'ncb' in lib.mh_last_error()
    assert lib.mh_mlp_fwd_ws(op.module.handle, P(x), P(op.WhT), None, P(h3), P(got), 5, None, None, 1, st) != 0
    assert b'NULL' in lib.mh_last_error()


def test_radial_embedding_vs_float64():
    """Bessel x polynomial-cutoff embedding of the edge lengths: both outputs against the module in float64, and
    dL/dr against float64 autograd with gradients on both outputs and on the features only; lengths on both sides of
    r_max and exactly at it, a ragged count, a leading batch shape and no edges."""
    dev = _dev()
    print('[case] radial embedding', flush=True)
    model = factory.make_model('128x0e+128x1o', 3, 2, elements=factory.ELEMENTS_PTCOH)
    emb = model.radial_embedding
    op = HipRadialEmbedding(emb, device=dev)
    rng = np.random.default_rng(4)
    e = 5001
    r = rng.uniform(0.4, 1.3 * op.spec.r_max, size=(e, 1))
    r[:7, 0] = op.spec.r_max
    rt = torch.tensor(r, dtype=torch.float32, device=dev, requires_grad=True)
    f, c = op(rt)
    m64 = copy.deepcopy(emb).double()
    r64 = torch.tensor(r, requires_grad=True)
    f64, c64 = m64(r64)
    assert _rel(f.detach().double().cpu().numpy(), f64.detach().numpy()) < 1e-5
    assert _rel(c.detach().double().cpu().numpy(), c64.detach().numpy()) < 1e-5
    assert float(c[:7].abs().max()) == 0.0 and float(f[:7].abs().max()) == 0.0
    gf, gc = rng.normal(size=(e, op.spec.n)), rng.normal(size=(e, 1))
    for with_cut in (True, False):
        outs, outs64 = (f, c) if with_cut else (f,), (f64, c64) if with_cut else (f64,)
        grads = (gf, gc) if with_cut else (gf,)
        got, = torch.autograd.grad(outs, rt, [torch.tensor(g, dtype=torch.float32, device=dev) for g in grads],
                                   retain_graph=True)
        want, = torch.autograd.grad(outs64, r64, [torch.tensor(g) for g in grads], retain_graph=True)
        assert _rel(got.double().cpu().numpy(), want.numpy()) < 1e-5
    f2, c2 = op(rt.detach()[:60].reshape(3, 20, 1))
    assert f2.shape == (3, 20, op.spec.n) and torch.equal(f2.reshape(60, -1), f.detach()[:60])
    f0, c0 = op(torch.zeros(0, 1, device=dev))
    assert f0.shape == (0, op.spec.n) and c0.shape == (0, 1)


def test_reshape_irreps_is_the_module_permutation():
    """reshape_irreps drop-in: forward and backward equal the PyTorch module bitwise (a permutation), for the
    config-2 and config-4 layouts and a ragged node count."""
    from mace_hip_kernels import HipReshapeIrreps
    dev = _dev()
    for hidden in ('128x0e+128x1o', '128x0e+128x1o+128x2e'):
        print(f'[case] reshape_irreps {hidden}', flush=True)
        model = factory.make_model(hidden, 3, 2, elements=factory.ELEMENTS_PTCOH)
        rs = model.interactions[0].reshape
        op = HipReshapeIrreps(rs, device=dev)
        n = 1001
        x = torch.randn(n, op.spec.dim, device=dev, requires_grad=True)
        y = op(x)
        y_ref = rs(x)
        assert y.shape == y_ref.shape and torch.equal(y, y_ref)
        g = torch.randn_like(y)
        gx, = torch.autograd.grad(y, x, g)
        gx_ref, = torch.autograd.grad(y_ref, x, g)
        assert torch.equal(gx, gx_ref)
        assert op(torch.zeros(0, op.spec.dim, device=dev)).shape == (0, op.spec.mul, op.spec.D)


@pytest.mark.parametrize('grouped', [False, True])
def test_sc_reads_the_irreps_layout(grouped):
    """The symmetric contraction on MACE's reshape_irreps left unformed (PendingReshape): it reads the irreps-layout
    tensor itself and returns its gradient in that layout.  Output and input gradient equal the reshape-then-contract
    path bitwise (the same arithmetic on the same numbers), per node and element-grouped, through the module and the
    C ABI; another consumer of the pending reshape sees the reshaped tensor."""
    from mace_hip_kernels import HipReshapeIrreps
    from mace_hip_kernels.layout import PendingReshape
    from mace_hip_kernels.symmetric import element_order
    dev = _dev()
    for hidden in ('128x0e+128x1o', '128x0e+128x1o+128x2e'):
        print(f'[case] SC on the irreps layout {hidden} grouped={grouped}', flush=True)
        model = factory.make_model(hidden, 3, 3, elements=factory.ELEMENTS_PTCOH)
        rs = HipReshapeIrreps(model.interactions[1].reshape, device=dev)
        sc = HipSymmetricContraction(model.products[1].symmetric_contractions, device=dev)
        sc.grouped = grouped
        n = 1237
        rng = np.random.default_rng(3)
        x = torch.randn(n, rs.spec.dim, device=dev, requires_grad=True)
        attrs = torch.tensor(np.eye(4)[rng.integers(0, 4, size=n)], dtype=torch.float32, device=dev)
        ref = sc(rs(x), attrs)
        g = torch.randn_like(ref)
        gref, = torch.autograd.grad(ref, x, g)
        rs.fuse = True
        pend = rs(x)
        assert isinstance(pend, PendingReshape) and pend.shape == (n, rs.spec.mul, rs.spec.D)
        out = sc(pend, attrs)
        gx, = torch.autograd.grad(out, x, g)
        assert torch.equal(out, ref) and torch.equal(gx, gref)
        assert torch.equal(rs(x) * 1.0, rs.original[0](x))          # any other use: the reshaped tensor
        # the C ABI entry point on the same input
        elem, order = element_order(attrs)
        lib, P, st = _native.load(), _native.ptr, _native.stream_of(x)
        o2, g2 = torch.empty_like(ref), torch.empty_like(x)
        ordp = P(order) if grouped else None
        xd = x.detach().contiguous()
        _native.check(lib.mh_sc_fwd_irreps(sc.module.handle, P(xd), P(elem), ordp, P(sc.T), P(o2), n, st), 'sc_fwd_i')
        _native.check(lib.mh_sc_bwd_irreps(sc.module.handle, P(xd), P(elem), ordp, P(sc.T), P(g.contiguous()), P(g2),
                                           n, st), 'sc_bwd_i')
        torch.cuda.synchronize()
        assert torch.equal(o2, ref) and torch.equal(g2, gref)


def test_readout_heads_vs_float64():
    """Both readout heads (linear on 128x0e+128x1o, SiLU MLP on 128x0e) of the config-2 model and of a 48-channel
    model: energies and input gradients against float64 runs of the e3nn modules on a ragged node count; the C ABI
    entry points equal the module."""
    from mace_hip_kernels import HipReadout
    dev = _dev()
    rng = np.random.default_rng(4)
    for hidden in ('128x0e+128x1o', '48x0e+48x1o'):
        m = factory.make_model(hidden, 3, 3, elements=factory.ELEMENTS_PTCOH)
        for i, ro in enumerate(m.readouts):
            print(f'[case] readout {hidden} {i}', flush=True)
            op = HipReadout(ro, device=dev)
            n = 1237
            x = rng.normal(size=(n, op.spec.Din))
            g = rng.normal(size=(n, 1))
            xt = torch.tensor(x, dtype=torch.float32, device=dev, requires_grad=True)
            out = op(xt)
            gx, = torch.autograd.grad(out, xt, torch.tensor(g, dtype=torch.float32, device=dev))
            m64 = copy.deepcopy(ro).double()
            x64 = torch.tensor(x, requires_grad=True)
            ref = m64(x64)
            gref, = torch.autograd.grad(ref, x64, torch.tensor(g))
            assert out.shape == (n, 1)
            assert _rel(out.detach().double().cpu().numpy(), ref.detach().numpy()) < 1e-5
            assert _rel(gx.double().cpu().numpy(), gref.numpy()) < 1e-5
            lib, P, st = _native.load(), _native.ptr, _native.stream_of(xt)
            o2, g2 = torch.empty(n, device=dev), torch.empty_like(xt)
            gg = torch.tensor(g[:, 0], dtype=torch.float32, device=dev)
            xd = xt.detach()
            _native.check(lib.mh_readout_fwd(op.module.handle, P(xd), P(o2), n, st), 'ro_fwd')
            _native.check(lib.mh_readout_bwd(op.module.handle, P(xd), P(gg), P(g2), n, st), 'ro_bwd')
            torch.cuda.synchronize()
            assert torch.equal(o2, out.detach()[:, 0]) and torch.equal(g2, gx)
            assert op(torch.zeros(0, op.spec.Din, device=dev)).shape == (0, 1)


def test_edge_geometry_vs_float64():
    """Edge vectors and lengths and their backward (atom CSR sums) against float64 autograd of the PyTorch gathers,
    with gradients on vectors and lengths, on positions and shifts (the stress path), and with zero-length edges."""
    from mace_hip_kernels import geometry
    dev = _dev()
    print('[case] edge geometry', flush=True)
    rng = np.random.default_rng(8)
    n, e = 700, 9000
    s, r = _graph(rng, n, e)
    s[:5] = r[:5]                                    # self edges with zero shift: zero length
    pos = rng.normal(size=(n, 3)) * 4.0
    sh = rng.normal(size=(e, 3))
    sh[:5] = 0.0
    ei = torch.tensor(np.stack([s, r]), device=dev)
    pt = torch.tensor(pos, dtype=torch.float32, device=dev, requires_grad=True)
    st = torch.tensor(sh, dtype=torch.float32, device=dev, requires_grad=True)
    v, ln = geometry.edge_vectors_and_lengths(pt, ei, st)
    p64 = torch.tensor(pos, requires_grad=True)
    s64 = torch.tensor(sh, requires_grad=True)
    ei64 = torch.tensor(np.stack([s, r]))
    v64 = p64[ei64[1]] - p64[ei64[0]] + s64
    l64 = torch.linalg.norm(v64, dim=-1, keepdim=True)
    assert _rel(v.detach().double().cpu().numpy(), v64.detach().numpy()) < 1e-6
    assert _rel(ln.detach().double().cpu().numpy(), l64.detach().numpy()) < 1e-6
    gv, gl = rng.normal(size=(e, 3)), rng.normal(size=(e, 1))
    got = torch.autograd.grad((v, ln), (pt, st), (torch.tensor(gv, dtype=torch.float32, device=dev),
                                                  torch.tensor(gl, dtype=torch.float32, device=dev)))
    want = torch.autograd.grad((v64, l64), (p64, s64), (torch.tensor(gv), torch.tensor(gl)))
    for a, b in zip(got, want):
        assert _rel(a.double().cpu().numpy(), b.numpy()) < 1e-5
    # lengths only, positions only
    got, = torch.autograd.grad(geometry.edge_vectors_and_lengths(pt, ei, st.detach())[1].sum(), pt)
    want, = torch.autograd.grad(torch.linalg.norm(p64[ei64[1]] - p64[ei64[0]] + s64.detach(), dim=-1).sum(), p64)
    assert _rel(got.double().cpu().numpy(), want.numpy()) < 1e-5


def test_fused_edge_pass_c_abi():
    """mh_edge_fwd / mh_edge_bwd (edge geometry, harmonics and embedding in one pass each way) against the separate
    entry points on the same inputs (mh_geom_fwd, then mh_sh_fwd on its vectors and mh_emb_fwd on its lengths;
    mh_sh_bwd and mh_emb_bwd): within 1e-6 relative, the cutoff's -0.0 marks in the same places, a zero-length
    self-loop and an edge exactly at r_max, a ragged edge count, with and without a cutoff gradient; NULL operands
    are rejected."""
    from mace_hip_kernels import HipRadialEmbedding, HipSphericalHarmonics, edgefeat, geometry
    dev = _dev()
    print('[case] fused edge pass through the C ABI', flush=True)
    model = factory.make_model('128x0e+128x1o', 3, 2, elements=factory.ELEMENTS_PTCOH)
    sh = HipSphericalHarmonics(model.spherical_harmonics, device=dev)
    emb = HipRadialEmbedding(model.radial_embedding, device=dev)
    m = edgefeat.module(sh, emb, dev)
    lib, P = _native.load(), _native.ptr
    rng = np.random.default_rng(12)
    N, E = 300, 40001
    f = lambda a: torch.tensor(a, dtype=torch.float32, device=dev)  # noqa: E731
    pos = f(rng.uniform(0.0, 12.0, size=(N, 3)))
    send = torch.tensor(rng.integers(0, N, E), dtype=torch.int32, device=dev)
    recv = torch.tensor(rng.integers(0, N, E), dtype=torch.int32, device=dev)
    shifts = (rng.integers(-1, 2, size=(E, 3)) * 12.0).astype(np.float32)
    send[0], recv[0] = 5, 5
    shifts[0] = 0.0
    send[1], recv[1] = 7, 7
    shifts[1] = (emb.spec.r_max, 0.0, 0.0)
    shifts = f(shifts)
    st = _native.stream_of(pos)
    out = [torch.empty(E, 3, device=dev), torch.empty(E, device=dev), torch.empty(E, sh.spec.dim, device=dev),
           torch.empty(E, emb.spec.n, device=dev), torch.empty(E, device=dev)]
    _native.check(lib.mh_edge_fwd(m.handle, P(pos), P(send), P(recv), P(shifts), *[P(t) for t in out], E, st),
                  'edge_fwd')
    vec, ln = torch.empty(E, 3, device=dev), torch.empty(E, device=dev)
    _native.check(lib.mh_geom_fwd(geometry._module(dev).handle, P(pos), P(send), P(recv), P(shifts), P(vec), P(ln),
                                  E, st), 'geom_fwd')
    Y = torch.empty(E, sh.spec.dim, device=dev)
    _native.check(lib.mh_sh_fwd(sh.module.handle, P(vec), P(Y), E, st), 'sh_fwd')
    feats, cut = torch.empty(E, emb.spec.n, device=dev), torch.empty(E, device=dev)
    _native.check(lib.mh_emb_fwd(emb.module.handle, P(ln), P(feats), P(cut), E, st), 'emb_fwd')
    torch.cuda.synchronize()

    def same(got, want):                  # NaN in the same places (the features of a zero-length edge: 0 / 0)
        gn, wn = torch.isnan(got), torch.isnan(want)
        assert torch.equal(gn, wn)
        return _rel(got[~gn].double().cpu().numpy(), want[~wn].double().cpu().numpy()) < 1e-6
    for got, want in zip(out, (vec, ln, Y, feats, cut)):
        assert same(got, want)
    assert torch.equal(torch.signbit(out[4]) & (out[4] == 0), torch.signbit(cut) & (cut == 0))
    assert bool(torch.signbit(out[4][1])) and float(out[4][1]) == 0.0 and float(out[1][0]) == 0.0
    gY, gf, gc = torch.randn(E, sh.spec.dim, device=dev), torch.randn(E, emb.spec.n, device=dev), \
        torch.randn(E, device=dev)
    for with_cut in (True, False):
        gv, gl = torch.empty(E, 3, device=dev), torch.empty(E, device=dev)
        _native.check(lib.mh_edge_bwd(m.handle, P(vec), P(ln), P(gY), P(gf), P(gc) if with_cut else None, P(gv),
                                      P(gl), E, st), 'edge_bwd')
        wv, wl = torch.empty(E, 3, device=dev), torch.empty(E, device=dev)
        _native.check(lib.mh_sh_bwd(sh.module.handle, P(vec), P(gY), P(wv), E, st), 'sh_bwd')
        _native.check(lib.mh_emb_bwd(emb.module.handle, P(ln), P(gf), P(gc) if with_cut else None, P(wl), E, st),
                      'emb_bwd')
        torch.cuda.synchronize()
        assert same(gv, wv) and same(gl, wl)
    # a second consumer's gradients (mh_edge_bwd2): bitwise what mh_edge_bwd gives on the sums, each second operand
    # also absent on its own (then the first one alone)
    print('[case] fused edge backward with two gradient sets', flush=True)
    nz = lambda t: t.nan_to_num(7.0)  # noqa: E731  (the zero-length self-loop's NaNs compared as a number)
    g2 = (torch.randn(E, sh.spec.dim, device=dev), torch.randn(E, emb.spec.n, device=dev), torch.randn(E, device=dev))
    for keep in ((1, 1, 1), (1, 0, 1), (0, 1, 0), (0, 0, 0)):
        sec = [t if k else None for t, k in zip(g2, keep)]
        gv, gl = torch.empty(E, 3, device=dev), torch.empty(E, device=dev)
        _native.check(lib.mh_edge_bwd2(m.handle, P(vec), P(ln), P(gY), P(gf), P(gc), *[P(t) for t in sec], P(gv),
                                       P(gl), E, st), 'edge_bwd2')
        tot = [a if b is None else a + b for a, b in zip((gY, gf, gc), sec)]
        wv, wl = torch.empty(E, 3, device=dev), torch.empty(E, device=dev)
        _native.check(lib.mh_edge_bwd(m.handle, P(vec), P(ln), *[P(t) for t in tot], P(wv), P(wl), E, st),
                      'edge_bwd')
        torch.cuda.synchronize()
        assert torch.equal(nz(gv), nz(wv)) and torch.equal(nz(gl), nz(wl)), keep
    # the cutoff gradient given only as the second operand
    gv, gl = torch.empty(E, 3, device=dev), torch.empty(E, device=dev)
    _native.check(lib.mh_edge_bwd2(m.handle, P(vec), P(ln), P(gY), P(gf), None, None, None, P(gc), P(gv), P(gl), E,
                                   st), 'edge_bwd2')
    wv, wl = torch.empty(E, 3, device=dev), torch.empty(E, device=dev)
    _native.check(lib.mh_edge_bwd(m.handle, P(vec), P(ln), P(gY), P(gf), P(gc), P(wv), P(wl), E, st), 'edge_bwd')
    torch.cuda.synchronize()
    assert torch.equal(nz(gv), nz(wv)) and torch.equal(nz(gl), nz(wl))
    assert lib.mh_edge_fwd(m.handle, P(pos), P(send), P(recv), P(shifts), P(out[0]), None, P(out[2]), P(out[3]),
                           P(out[4]), E, st) != 0
    assert b'NULL' in lib.mh_last_error()


def test_edge_geometry_only_while_a_patched_model_runs():
    """The edge-geometry route is taken inside a patched model's forward and nowhere else: an unpatched copy of the
    same model, run in the same process, launches no geometry kernel."""
    from mace_hip_kernels import patch_model, unpatch_model
    dev = _dev()
    print('[case] edge geometry scoping', flush=True)
    from mace_lite import data as D
    model = factory.make_model('32x0e+32x1o', 2, 2, elements=factory.ELEMENTS_PTCOH)
    plain = copy.deepcopy(model).to(dev)
    patched = copy.deepcopy(model).to(dev)
    assert 'edge_geometry' in patch_model(patched, verbose=False)['patched']
    st = factory.make_structure(seed=1)
    batch = D.batch_graphs([D.graph_of(st, 5.0)], factory.ELEMENTS_REF)
    b = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in batch.items()}
    for mdl, expect in ((plain, False), (patched, True), (plain, False)):
        with _native.timing() as tm:
            mdl(D.fresh(b), compute_force=True)
        tags = {t for t, *_ in tm.records}
        fwd = 'geom_fwd' in tags or any(t.startswith('edge_fwd') for t in tags)   # alone, or in the fused edge pass
        assert fwd == expect and ('geom_bwd' in tags) == expect, tags
    assert 'edge_geometry' in unpatch_model(patched)
    with _native.timing() as tm:
        patched(D.fresh(b), compute_force=True)
    assert not any(t.startswith(('geom', 'edge_fwd', 'edge_bwd')) for t, *_ in tm.records)


def test_structure_energy_sums():
    """MACE's per-structure energy sums as segmented sums over ptr (geometry.structure_sum, geom_segsum1): against
    float64 index_add with an empty structure and one of more than 256 atoms, the backward (a gather) and its own
    backward; in a patched model both sums take this path, and two calls give bitwise-equal energies."""
    from mace_hip_kernels import geometry, patch_model
    from mace_lite import data as D
    dev = _dev()
    print('[case] per-structure energy sums', flush=True)
    counts = [3, 0, 300, 1, 57]
    ptr = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), device=dev)
    batch = torch.repeat_interleave(torch.arange(len(counts), device=dev), torch.tensor(counts, device=dev))
    src = torch.randn(int(ptr[-1]), device=dev, dtype=torch.float32, requires_grad=True)
    out = geometry.structure_sum(src, batch, ptr)
    want = torch.zeros(len(counts), dtype=torch.float64, device=dev).index_add_(0, batch, src.detach().double())
    assert float((out.double() - want).abs().max()) <= 1e-5 * float(want.abs().max())
    assert float(out[1]) == 0.0
    w = torch.randn(len(counts), device=dev, requires_grad=True)
    g, = torch.autograd.grad((out * w).sum(), src, create_graph=True)
    assert torch.equal(g.detach(), w.detach()[batch])
    v = torch.randn_like(src)
    gw, = torch.autograd.grad((g * v).sum(), w)                   # d/dw of <v, w[batch]> = per-structure sums of v
    want_gw = torch.zeros(len(counts), dtype=torch.float64, device=dev).index_add_(0, batch, v.double())
    assert float((gw.double() - want_gw).abs().max()) <= 1e-5 * float(want_gw.abs().max())
    model, b, _ = factory.workload(2)
    met = model.to(dev)
    patch_model(met, verbose=False)
    b = {k: (t.to(dev) if torch.is_tensor(t) else t) for k, t in b.items()}
    es = []
    for _ in range(2):
        with _native.timing() as tm:
            es.append(met(D.fresh(b), compute_force=True)['energy'].detach())
        assert tm.summary()['geom_segsum1'][0] == 2, tm.symbols
    assert torch.equal(es[0], es[1])


@pytest.mark.parametrize('factored', [False, True])
def test_conv_double_backward_vs_oracle(factored):
    """Second derivatives through the convolution (patched with double_backward): the first-order gradients taken
    with create_graph, contracted with random directions, and differentiated again with respect to g and every
    input.  Against the oracle's conv_double_bwd (first-order formulas with substituted arguments, pinned by finite
    differences).  Factored: the weights are W0 * cutoff (some cutoffs 0), which the convolution reads as its two
    factors; the oracle side applies the product rule by hand."""
    dev = _dev()
    print(f'[case] conv double backward factored={factored}', flush=True)
    tp = _tp('32x0e+32x1o', 2)
    op = HipConvTP(tp, device=dev)
    op.double_backward = True
    desc = oconv.describe_tp(tp)
    coef = oconv.path_terms(desc)
    rng = np.random.default_rng(11)
    n, e = 23, 300
    s, r = _graph(rng, n, e)
    nw = len(desc['ins']) * desc['mul']
    x, Y, g = rng.normal(size=(n, desc['x_dim'])), rng.normal(size=(e, desc['y_dim'])), rng.normal(size=(n, desc['out_dim']))
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=dev, requires_grad=True)  # noqa: E731
    ei = torch.tensor(np.stack([s, r]), device=dev)
    xt, Yt, gt = t(x), t(Y), t(g)
    if factored:
        W0, cut = rng.normal(size=(e, nw)), rng.uniform(0.1, 1.0, size=(e, 1))
        cut[::7] = 0.0
        W0t, ct = t(W0), t(cut)
        ins, Wt = (xt, Yt, W0t, ct), W0t * ct
    else:
        W = rng.normal(size=(e, nw))
        Wt = t(W)
        ins = (xt, Yt, Wt)
    out = op(xt, Yt, Wt, ei)
    firsts = torch.autograd.grad(out, ins, gt, create_graph=True)
    dirs = [rng.normal(size=f.shape) for f in firsts]
    sval = sum((f * torch.tensor(d, dtype=torch.float32, device=dev)).sum() for f, d in zip(firsts, dirs))
    seconds = torch.autograd.grad(sval, (gt,) + ins)
    if factored:
        ggx, ggY, ggW0, ggc = dirs
        og, ox, oY, oW = oconv.conv_double_bwd(desc, coef, x, Y, W0 * cut, g, ggx, ggY, ggW0 * cut + ggc * W0, s, r, n)
        A = oconv.conv_bwd_w(desc, coef, x, g, Y, s, r)
        want = [og, ox, oY, oW * cut + ggc * A, (oW * W0).sum(1, keepdims=True) + (ggW0 * A).sum(1, keepdims=True)]
    else:
        want = oconv.conv_double_bwd(desc, coef, x, Y, W, g, *dirs, s, r, n)
    for i, (got, w) in enumerate(zip(seconds, want)):
        assert _rel(got.double().cpu().numpy(), w) < 1e-5, i
    # the module as patched by default refuses, with the reference's message
    op.double_backward = False
    out = op(xt, Yt, Wt, ei)
    with pytest.raises(RuntimeError, match='double backward'):
        torch.autograd.grad(out, ins, gt, create_graph=True)


def _sc_oracle_tables(sc):
    tabs = []
    for ct in sc.contractions:
        U = {}
        for nu in range(1, ct.correlation + 1):
            u = getattr(ct, f'U_matrix_{nu}').double()
            u = u if u.dim() == nu + 2 else u.unsqueeze(0)
            U[nu] = u.reshape(u.shape[0], -1, u.shape[-1]).numpy()
        Wd = {ct.correlation: ct.weights_max.detach().double().numpy()}
        for j, w in enumerate(ct.weights):
            Wd[ct.correlation - 1 - j] = w.detach().double().numpy()
        tabs.append(osc.poly_table(U, Wd))
    return tabs


@pytest.mark.parametrize('layout', ['mace', 'irreps'])
def test_sc_double_backward_vs_oracle(layout):
    """Second derivatives through the symmetric contraction (the sc_jvp / sc_bwd2 kernels): d<v, gx>/dg and
    d<v, gx>/dx against the oracle's directional derivatives, both layers of the config-2 model, on x as
    [N, C, n_ell] and in e3nn's irreps layout; the C ABI's layout argument is checked on the host."""
    from mace_hip_kernels import symmetric as hsym
    dev = _dev()
    model = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    rng = np.random.default_rng(6)
    for li, prod in enumerate(model.products):
        print(f'[case] sc double backward layer {li} layout={layout}', flush=True)
        sc = prod.symmetric_contractions
        op = HipSymmetricContraction(sc, device=dev)
        op.double_backward = True
        sp = op.spec
        n = 29
        x, v = rng.normal(size=(n, sp.C, sp.n_ell)) * 0.7, rng.normal(size=(n, sp.C, sp.n_ell))
        elem_np = rng.integers(0, 4, n)
        g = rng.normal(size=(n, sp.out_dim))
        attrs = torch.tensor(np.eye(4)[elem_np], dtype=torch.float32, device=dev)

        def irreps(a):
            parts, o = [], 0
            for d in sp.dims:
                parts.append(a[:, :, o:o + d].reshape(n, -1))
                o += d
            return np.concatenate(parts, axis=1)
        lay = (lambda a: a) if layout == 'mace' else irreps
        t = lambda a: torch.tensor(a, dtype=torch.float32, device=dev, requires_grad=True)  # noqa: E731
        xt, gt = t(lay(x)), t(g)
        if layout == 'mace':
            out = op(xt, attrs)
        else:
            elem, order = hsym.element_order(attrs)
            out = hsym._SCIrrepsFn.apply(xt, elem, order, hsym.group_slots(attrs), op)
        gx, = torch.autograd.grad(out, xt, gt, create_graph=True)
        d_g, d_x = torch.autograd.grad((gx * torch.tensor(lay(v), dtype=torch.float32, device=dev)).sum(), (gt, xt))
        want_g, want_x, off = [], np.zeros_like(x), 0
        for tab in _sc_oracle_tables(sc):
            M = next(iter(tab.values())).shape[1]
            want_g.append(osc.poly_jvp(tab, x, elem_np, v).reshape(n, -1))
            want_x += osc.poly_grad_jvp(tab, x, elem_np, g[:, off:off + sp.C * M].reshape(n, sp.C, M), v)
            off += sp.C * M
        assert _rel(d_g.double().cpu().numpy(), np.concatenate(want_g, axis=1)) < SC_TOL
        assert _rel(d_x.double().cpu().numpy(), lay(want_x)) < SC_TOL
    lib = _native.load()
    m2 = op.second_module()
    assert lib.mh_sc_jvp(m2.handle, None, None, None, None, None, 0, 2, None) != 0
    assert b'layout' in lib.mh_last_error()


def test_linear_double_backward():
    """Node linears (o3.Linear and skip_tp) patched with double_backward: the input gradient does not depend on x,
    and its derivative with respect to g along v is the map applied to v (checked against float64 runs of the
    e3nn module); the readout heads likewise (the SiLU head's second-order kernels against float64 double
    backward)."""
    from mace_hip_kernels import HipReadout
    dev = _dev()
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    rng = np.random.default_rng(8)
    n = 301
    for name in ('interactions.1.linear', 'interactions.0.skip_tp', 'products.0.linear'):
        print(f'[case] linear double backward {name}', flush=True)
        mod = m.get_submodule(name)
        op = HipNodeLinear(mod, device=dev)
        op.double_backward = True
        s = op.spec
        a = np.eye(s.V)[rng.integers(0, s.V, size=n)] if s.V else None
        at = None if a is None else torch.tensor(a, dtype=torch.float32, device=dev)
        xt = torch.tensor(rng.normal(size=(n, s.Din)), dtype=torch.float32, device=dev, requires_grad=True)
        gt = torch.tensor(rng.normal(size=(n, s.Dout)), dtype=torch.float32, device=dev, requires_grad=True)
        v = rng.normal(size=(n, s.Din))
        gx, = torch.autograd.grad(op(xt, at), xt, gt, create_graph=True)
        d_g, d_x = torch.autograd.grad((gx * torch.tensor(v, dtype=torch.float32, device=dev)).sum(), (gt, xt),
                                       allow_unused=True)
        m64 = copy.deepcopy(mod).double()
        want = m64(torch.tensor(v), torch.tensor(a)) if s.V else m64(torch.tensor(v))
        assert d_x is None
        assert _rel(d_g.double().cpu().numpy(), want.detach().numpy()) < LIN_TOL
    print('[case] SiLU readout double backward', flush=True)
    ro = HipReadout(m.readouts[1], device=dev)
    ro.double_backward = True
    xt = torch.tensor(rng.normal(size=(n, ro.spec.Din)), dtype=torch.float32, device=dev, requires_grad=True)
    gt = torch.tensor(rng.normal(size=(n, 1)), dtype=torch.float32, device=dev, requires_grad=True)
    v = rng.normal(size=(n, ro.spec.Din))
    gx, = torch.autograd.grad(ro(xt), xt, gt, create_graph=True)
    d_g, d_x = torch.autograd.grad((gx * torch.tensor(v, dtype=torch.float32, device=dev)).sum(), (gt, xt))
    r64 = copy.deepcopy(m.readouts[1]).double()
    x64, g64 = xt.detach().double().cpu().requires_grad_(True), gt.detach().double().cpu().requires_grad_(True)
    gx64, = torch.autograd.grad(r64(x64), x64, g64, create_graph=True)
    w_g, w_x = torch.autograd.grad((gx64 * torch.tensor(v)).sum(), (g64, x64))
    assert _rel(d_g.double().cpu().numpy(), w_g.numpy()) < LIN_TOL
    assert _rel(d_x.double().cpu().numpy(), w_x.numpy()) < LIN_TOL
    print('[case] linear readout double backward', flush=True)
    ro = HipReadout(m.readouts[0], device=dev)
    ro.double_backward = True
    xt = torch.tensor(rng.normal(size=(n, ro.spec.Din)), dtype=torch.float32, device=dev, requires_grad=True)
    gt = torch.tensor(rng.normal(size=(n, 1)), dtype=torch.float32, device=dev, requires_grad=True)
    v = rng.normal(size=(n, ro.spec.Din))
    gx, = torch.autograd.grad(ro(xt), xt, gt, create_graph=True)
    d_g, = torch.autograd.grad((gx * torch.tensor(v, dtype=torch.float32, device=dev)).sum(), gt)
    want = copy.deepcopy(m.readouts[0]).double()(torch.tensor(v))
    assert _rel(d_g.double().cpu().numpy(), want.detach().numpy()) < LIN_TOL


def test_sh_and_embedding_double_backward():
    """The spherical harmonics' and radial embedding's second derivatives on the GPU (sh_jvp / sh_bwd2, emb_jvp /
    emb_bwd2): d<v, dL/dinput>/d(incoming gradients) and /d(input) against float64 double backward of the e3nn
    modules, lengths on both sides of r_max; relative error < 1e-5 (2e-5 for the embedding's Hessian term)."""
    from mace_hip_kernels import HipRadialEmbedding, HipSphericalHarmonics
    dev = _dev()
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    rng = np.random.default_rng(14)
    n = 3001
    print('[case] SH double backward', flush=True)
    op = HipSphericalHarmonics(m.spherical_harmonics, device=dev)
    op.double_backward = True
    v = rng.normal(size=(n, 3)) * rng.uniform(0.5, 5.0, size=(n, 1))
    dv, g = rng.normal(size=(n, 3)), rng.normal(size=(n, op.spec.dim))
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=dev, requires_grad=True)  # noqa: E731
    vt, gt = t(v), t(g)
    gv, = torch.autograd.grad(op(vt), vt, gt, create_graph=True)
    d_g, d_v = torch.autograd.grad((gv * torch.tensor(dv, dtype=torch.float32, device=dev)).sum(), (gt, vt))
    m64 = copy.deepcopy(m.spherical_harmonics).double()
    v64, g64 = torch.tensor(v, requires_grad=True), torch.tensor(g, requires_grad=True)
    gv64, = torch.autograd.grad(m64(v64), v64, g64, create_graph=True)
    w_g, w_v = torch.autograd.grad((gv64 * torch.tensor(dv)).sum(), (g64, v64))
    assert _rel(d_g.double().cpu().numpy(), w_g.numpy()) < 1e-5
    assert _rel(d_v.double().cpu().numpy(), w_v.numpy()) < 1e-5
    print('[case] radial embedding double backward', flush=True)
    op = HipRadialEmbedding(m.radial_embedding, device=dev)
    op.double_backward = True
    r = rng.uniform(0.7, 6.0, size=(n, 1))
    dl, gf, gc = rng.normal(size=(n, 1)), rng.normal(size=(n, op.spec.n)), rng.normal(size=(n, 1))
    rt, gft, gct = t(r), t(gf), t(gc)
    f, c = op(rt)
    gr, = torch.autograd.grad((f, c), rt, (gft, gct), create_graph=True)
    d_f, d_c, d_r = torch.autograd.grad((gr * torch.tensor(dl, dtype=torch.float32, device=dev)).sum(), (gft, gct, rt))
    e64 = copy.deepcopy(m.radial_embedding).double()
    r64, gf64, gc64 = (torch.tensor(a, requires_grad=True) for a in (r, gf, gc))
    f64, c64 = e64(r64)
    gr64, = torch.autograd.grad((f64, c64), r64, (gf64, gc64), create_graph=True)
    w_f, w_c, w_r = torch.autograd.grad((gr64 * torch.tensor(dl)).sum(), (gf64, gc64, r64))
    assert _rel(d_f.double().cpu().numpy(), w_f.numpy()) < 1e-5
    assert _rel(d_c.double().cpu().numpy(), w_c.numpy()) < 1e-5
    assert _rel(d_r.double().cpu().numpy(), w_r.numpy()) < 2e-5


def test_edge_geometry_double_backward():
    """The edge geometry's second derivatives (geom_jvp + the first-order atom sums), with shifts and zero-length
    edges absent: d<(ggpos, ggshifts), (dL/dpos, dL/dshifts)>/d(g_vec, g_len, positions, shifts) against float64
    double backward of the plain PyTorch expressions; relative error < 1e-5."""
    from mace_hip_kernels import geometry as geo
    dev = _dev()
    print('[case] edge geometry double backward', flush=True)
    rng = np.random.default_rng(15)
    n, e = 61, 900
    s, r = _graph(rng, n, e)
    keep = s != r
    s, r = s[keep], r[keep]
    e = len(s)
    pos, sh = rng.normal(size=(n, 3)) * 3.0, rng.normal(size=(e, 3))
    gv, gl = rng.normal(size=(e, 3)), rng.normal(size=(e, 1))
    ggp, ggs = rng.normal(size=(n, 3)), rng.normal(size=(e, 3))
    ei = torch.tensor(np.stack([s, r]), device=dev)
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=dev, requires_grad=True)  # noqa: E731
    pt, st, gvt, glt = t(pos), t(sh), t(gv), t(gl)
    vec, ln = geo._GeomFn.apply(pt, st, ei, True)
    gp, gs = torch.autograd.grad((vec, ln), (pt, st), (gvt, glt), create_graph=True)
    sval = (gp * torch.tensor(ggp, dtype=torch.float32, device=dev)).sum() + \
        (gs * torch.tensor(ggs, dtype=torch.float32, device=dev)).sum()
    got = torch.autograd.grad(sval, (gvt, glt, pt, st))
    p64, s64, gv64, gl64 = (torch.tensor(a, requires_grad=True) for a in (pos, sh, gv, gl))
    v64 = p64[torch.tensor(r)] - p64[torch.tensor(s)] + s64
    l64 = torch.linalg.norm(v64, dim=-1, keepdim=True)
    gp64, gs64 = torch.autograd.grad((v64, l64), (p64, s64), (gv64, gl64), create_graph=True)
    want = torch.autograd.grad((gp64 * torch.tensor(ggp)).sum() + (gs64 * torch.tensor(ggs)).sum(),
                               (gv64, gl64, p64, s64))
    for i, (a, w) in enumerate(zip(got, want)):
        assert _rel(a.double().cpu().numpy(), w.numpy()) < 1e-5, i
    vec, ln = geo._GeomFn.apply(pt, st, ei, False)
    with pytest.raises(RuntimeError, match='double backward'):
        torch.autograd.grad((vec, ln), (pt, st), (gvt, glt), create_graph=True)


def test_kernels_match_golden_fixtures():
    """Kernels against the committed oracle fixtures (tests/golden/make_golden.py)."""
    import os
    dev = _dev()
    print('[case] golden fixtures', flush=True)
    gdir = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')
    model = factory.make_model('32x0e+32x1o', 3, 3)
    g = np.load(os.path.join(gdir, 'conv_small.npz'))
    op = HipConvTP(model.interactions[1].conv_tp, device=dev)
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=dev, requires_grad=True)  # noqa: E731
    xt, Yt, Wt = t(g['x']), t(g['Y']), t(g['W'])
    out = op(xt, Yt, Wt, torch.tensor(np.stack([g['sender'], g['receiver']]), device=dev))
    out.backward(torch.tensor(g['g'], dtype=torch.float32, device=dev))
    for got, want in ((out, g['out']), (xt.grad, g['gx']), (Wt.grad, g['gW']), (Yt.grad, g['gY'])):
        assert _rel(got.detach().double().cpu().numpy(), want) < CONV_TOL
    f = np.load(os.path.join(gdir, 'sc_small.npz'))
    op = HipSymmetricContraction(model.products[0].symmetric_contractions, device=dev)
    xt = torch.tensor(f['x'], dtype=torch.float32, device=dev, requires_grad=True)
    out = op(xt, torch.tensor(np.eye(4)[f['elem']], dtype=torch.float32, device=dev))
    out.backward(torch.tensor(f['g'], dtype=torch.float32, device=dev))
    assert _rel(out.detach().double().cpu().numpy(), f['out']) < SC_TOL
    assert _rel(xt.grad.double().cpu().numpy(), f['gx']) < SC_TOL


def test_library_runtime_is_torchs():
    dev = _dev()
    print('[case] runtime binding', flush=True)
    lib = _native.load()
    assert 'torch' in lib.mh_hip_runtime_path().decode()
    assert lib.mh_version() == _native.ABI_VERSION
    del dev
