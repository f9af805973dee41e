"""
Parity at BASELINE config 4's full size (20,000-atom bulk Pt, 820,110 edges, hidden 128x0e+128x1o+128x2e, l_max 3,
correlation 3), where the float64 oracle is too slow, through size-independent properties:

* the convolution is linear in each of x, W and Y, so for any g:  <g, out> = <gx, x> = <gW, W> = <gY, Y>  (each
  product of the backward is the adjoint of the forward; a dropped term, a wrong sign or a wrong index breaks it);
* the receiver-ordered and the sender-ordered backward, and the factored-weight (W0 * cutoff) and plain paths, agree;
* the LDS-staged and the element-grouped symmetric contraction agree with the one-node-per-workgroup kernels.

Tolerances are relative, sized for fp32 sums over ~10^8 terms: 1e-4 on the inner products, 1e-5 between kernels.
"""
import pytest
import torch

from mace_hip_kernels import HipConvTP, HipSymmetricContraction
from mace_hip_kernels import conv as hconv
from mace_lite import factory

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def cfg4():
    assert torch.cuda.is_available(), 'GPU test needs a GPU'
    model, batch, meta = factory.workload(4)
    return model, batch, meta


def _rel(a, b):
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def _dot(a, b):
    return float((a.double() * b.double()).sum())


@pytest.mark.parametrize('layer', [0, 1])
def test_conv_adjoint_identities_full_size(cfg4, layer):
    model, batch, meta = cfg4
    dev = torch.device('cuda:0')
    print(f'[case] config 4 conv layer {layer} adjoint identities', flush=True)
    op = HipConvTP(model.interactions[layer].conv_tp, device=dev)
    s = op.spec
    N, E = batch['positions'].shape[0], batch['edge_index'].shape[1]
    ei = batch['edge_index'].to(dev)
    gen = torch.Generator(device='cpu').manual_seed(10 + layer)
    r = lambda *sh: torch.randn(*sh, generator=gen).to(dev).requires_grad_(True)  # noqa: E731
    x, Y, W = r(N, s.x_dim), r(E, s.y_dim), r(E, s.nins * s.mul)
    g = torch.randn(N, s.out_dim, generator=gen).to(dev)
    results = {}
    for order in ('recv', 'send'):
        op.bwd_recv = order == 'recv'
        out = op(x, Y, W, ei)
        gx, gY, gW = torch.autograd.grad(out, (x, Y, W), g)
        lhs = _dot(g, out.detach())
        for name, gr_, inp in (('x', gx, x), ('W', gW, W), ('Y', gY, Y)):
            rhs = _dot(gr_, inp.detach())
            print(f'  {order}: <g,out> = {lhs:.6e}  <g{name},{name}> = {rhs:.6e}', flush=True)
            assert abs(lhs - rhs) <= 1e-4 * abs(lhs)
        results[order] = (out.detach(), gx, gY, gW)
        del out
    a, b = results['recv'], results['send']
    assert torch.equal(a[0], b[0])
    for u, v in zip(a[1:], b[1:]):
        assert _rel(u, v) < 1e-5


def test_conv_factored_matches_plain_full_size(cfg4):
    model, batch, meta = cfg4
    dev = torch.device('cuda:0')
    print('[case] config 4 conv layer 1 factored weights vs plain', flush=True)
    op = HipConvTP(model.interactions[1].conv_tp, device=dev)
    s = op.spec
    N, E = batch['positions'].shape[0], batch['edge_index'].shape[1]
    ei = batch['edge_index'].to(dev)
    gen = torch.Generator(device='cpu').manual_seed(20)
    x = torch.randn(N, s.x_dim, generator=gen).to(dev).requires_grad_(True)
    Y = torch.randn(E, s.y_dim, generator=gen).to(dev).requires_grad_(True)
    W0 = torch.randn(E, s.nins * s.mul, generator=gen).to(dev).requires_grad_(True)
    c = torch.rand(E, 1, generator=gen).to(dev)
    c[::5] = 0.0
    c.requires_grad_(True)
    g = torch.randn(N, s.out_dim, generator=gen).to(dev)
    got = {}
    for fuse in (True, False):
        op.fuse_cutoff = fuse
        W = W0 * c
        assert (hconv._factored_weights(W) is not None) or not fuse
        out = op(x, Y, W, ei)
        got[fuse] = (out.detach(),) + torch.autograd.grad(out, (x, Y, W0, c), g)
        del out, W
    for u, v in zip(got[True], got[False]):
        assert _rel(u, v) < 1e-5


def test_sc_families_match_per_node_full_size(cfg4):
    """The four symmetric-contraction families at N = 20,000: the LDS-staged kernels (what the patched model
    launches at this size), the split LDS-staged ones and the element-grouped ones against one node per workgroup
    (itself against the oracle at small sizes), outputs and input gradients."""
    model, batch, meta = cfg4
    dev = torch.device('cuda:0')
    N = batch['positions'].shape[0]
    attrs = batch['node_attrs'].to(dev)
    gen = torch.Generator(device='cpu').manual_seed(30)
    for li, prod in enumerate(model.products):
        op = HipSymmetricContraction(prod.symmetric_contractions, device=dev)
        assert op.use_grouped(N, dev)
        assert op.kernel_family(N, dev) == 'staged'
        x = (0.5 * torch.randn(N, op.spec.C, op.spec.n_ell, generator=gen)).to(dev).requires_grad_(True)
        g = torch.randn(N, op.spec.out_dim, generator=gen).to(dev)
        got = {}
        for fam, (staged, grouped, split) in (('staged', (True, None, None)), ('staged2', (None, None, True)),
                                              ('grouped', (False, True, None)), ('node', (False, False, None))):
            print(f'[case] config 4 symmetric contraction {li}: {fam} kernels', flush=True)
            op.staged, op.grouped, op.split = staged, grouped, split
            assert op.kernel_family(N, dev) == fam
            out = op(x, attrs)
            got[fam] = (out.detach(), torch.autograd.grad(out, x, g)[0])
            del out
        for fam in ('staged', 'staged2', 'grouped'):
            for u, v in zip(got[fam], got['node']):
                assert _rel(u, v) < 1e-5, fam


def test_patched_model_full_size(cfg4):
    """The patched model with every drop-in at config 4's full size (20,000 atoms) against the same model with only
    the reference's two ops patched (convolution and symmetric contraction on the HIP kernels, everything else on the
    e3nn path), both fp32: energy and forces.  The unpatched e3nn path would materialise per-edge tensor products of
    tens of GB at this size; each drop-in is checked against float64 at small sizes elsewhere."""
    import copy
    from mace_hip_kernels import patch_model
    from mace_lite import data as D
    model, batch, meta = cfg4
    dev = torch.device('cuda:0')
    print('[case] config 4 patched model E+F, every drop-in vs conv+SC only', flush=True)
    b = {k: (v.to(dev, torch.float32) if torch.is_tensor(v) and v.is_floating_point() else
             v.to(dev) if torch.is_tensor(v) else v) for k, v in batch.items()}
    outs = []
    for full in (True, False):
        met = copy.deepcopy(model).to(dev, torch.float32)
        kw = {} if full else dict(spherical_harmonics=False, linears=False, radial_mlp=False, radial_embedding=False,
                                  layouts=False, edge_geometry=False)
        report = patch_model(met, verbose=False, **kw)
        assert not report['skipped'], report['skipped']
        out = met(D.fresh(b), compute_force=True)
        outs.append((out['energy'].detach().double(), out['forces'].detach().double()))
        del met, out
        torch.cuda.empty_cache()
    (ea, fa), (eb, fb) = outs
    n = batch['positions'].shape[0]
    de = float((ea - eb).abs().max())
    df = float((fa - fb).abs().max())
    print(f'  |dE| {de:.3e} eV ({de / n:.2e} eV/atom)  max|dF| {df:.2e} eV/A  (max|F| {float(fb.abs().max()):.2f})',
          flush=True)
    assert de / n < 1e-6 and df < 1e-5
