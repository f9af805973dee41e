"""
Pins of the convolution oracle (CPU, float64).

* the fused per-term forward (reference conv.py:109-141) equals the unfused e3nn-style path (dense CG einsum on
  x[sender], scatter-summed) — two different evaluation orders of one sum;
* each backward formula (conv.py:144-222) equals central finite differences of the unfused forward;
* the probed coefficient table of the product (ConvSpec) equals the oracle's table built from sympy's CG;
* the (0e ⊗ l → l) path coefficient is 1 (identity), as e3nn's normalisation implies for a single path;
* CSR construction equals brute-force grouping (the GPU build is checked against it in test_kernels_gpu.py);
* planted mistakes (a dropped term, a wrong sign) are caught by the fused-vs-unfused comparison.
"""
import numpy as np
import pytest
import torch

from mace_hip_kernels import conv as hconv
from mace_lite import blocks as B
from mace_lite.o3 import Irreps, TensorProduct
from oracle import conv as oconv


def _tp(hidden, lmax):
    sh = Irreps.spherical_harmonics(lmax)
    hid = Irreps(hidden)
    target = (sh * hid.count((0, 1))).sort()[0].simplify()
    irreps_mid, ins = B.tp_out_irreps_with_instructions(hid, sh, target)
    return TensorProduct(hid, sh, irreps_mid, ins, shared_weights=False, internal_weights=False)


CASES = [('4x0e+4x1o', 3), ('3x0e', 2), ('2x0e+2x1o+2x2e', 3), ('128x0e+128x1o', 3)]


def _inputs(desc, rng, n, e):
    s, r = oconv.random_graph(rng, n, e)
    nw = len(desc['ins']) * desc['mul']
    return (s, r, rng.normal(size=(n, desc['x_dim'])), rng.normal(size=(e, desc['y_dim'])),
            rng.normal(size=(e, nw)), rng.normal(size=(n, desc['out_dim'])))


@pytest.mark.parametrize('hidden,lmax', CASES)
def test_fused_forward_equals_unfused(hidden, lmax):
    desc = oconv.describe_tp(_tp(hidden, lmax))
    coef = oconv.path_terms(desc)
    rng = np.random.default_rng(0)
    s, r, x, Y, W, _ = _inputs(desc, rng, 9, 40)
    a = oconv.conv_fwd(desc, coef, x, Y, W, s, r, 9)
    b = oconv.conv_unfused(desc, x, Y, W, s, r, 9)
    assert np.abs(a - b).max() < 1e-12 * max(1.0, np.abs(b).max())


def test_unfused_equals_harness_tensor_product():
    """The oracle's unfused path equals mace_lite's TensorProduct + scatter_sum (the unpatched model path)."""
    tp = _tp('4x0e+4x1o', 3).double()
    desc = oconv.describe_tp(tp)
    rng = np.random.default_rng(1)
    s, r, x, Y, W, _ = _inputs(desc, rng, 7, 30)
    t = lambda a: torch.tensor(a, dtype=torch.float64)  # noqa: E731
    mji = tp(t(x)[torch.tensor(s)], t(Y), t(W))
    got = B.scatter_sum(mji, torch.tensor(r), 0, 7).numpy()
    assert np.abs(got - oconv.conv_unfused(desc, x, Y, W, s, r, 7)).max() < 1e-12


@pytest.mark.parametrize('hidden,lmax', CASES[:3])
def test_backward_formulas_equal_finite_differences(hidden, lmax):
    desc = oconv.describe_tp(_tp(hidden, lmax))
    coef = oconv.path_terms(desc)
    rng = np.random.default_rng(2)
    n, e = 5, 14
    s, r, x, Y, W, g = _inputs(desc, rng, n, e)
    f = lambda x_, Y_, W_: (oconv.conv_unfused(desc, x_, Y_, W_, s, r, n) * g).sum()  # noqa: E731
    h = 1e-6

    def fd(arr, which):
        out = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            p, m = arr.copy(), arr.copy()
            p[idx] += h
            m[idx] -= h
            args_p = [x, Y, W]
            args_m = [x, Y, W]
            args_p[which], args_m[which] = p, m
            out[idx] = (f(*args_p) - f(*args_m)) / (2 * h)
        return out

    assert np.abs(oconv.conv_bwd_x(desc, coef, g, Y, W, s, r, n) - fd(x, 0)).max() < 1e-6
    assert np.abs(oconv.conv_bwd_y(desc, coef, x, g, W, s, r) - fd(Y, 1)).max() < 1e-6
    assert np.abs(oconv.conv_bwd_w(desc, coef, x, g, Y, s, r) - fd(W, 2)).max() < 1e-6


@pytest.mark.parametrize('hidden,lmax', [('128x0e', 3), ('128x0e+128x1o', 3), ('128x0e+128x1o+128x2e', 3),
                                         ('32x0e+32x1o', 2), ('64x0e', 2), ('32x0e+32x1o+32x2e', 3)])
def test_probed_coefficients_equal_oracle_table(hidden, lmax):
    tp = _tp(hidden, lmax)
    spec = hconv.ConvSpec(tp)
    want = oconv.path_terms(oconv.describe_tp(tp))
    assert len(spec.coef) == len(want)
    for a, b in zip(spec.coef, want):
        assert (a['l1'], a['l2'], a['l3'], a['o1'], a['o2'], a['o3']) == \
               (b['l1'], b['l2'], b['l3'], b['o1'], b['o2'], b['o3'])
        ta = {(i, j, k): v for i, j, k, v in a['terms']}
        tb = {(i, j, k): v for i, j, k, v in b['terms']}
        assert ta.keys() == tb.keys()
        assert max(abs(ta[k] - tb[k]) for k in ta) < 1e-14


def test_scalar_path_is_identity():
    desc = oconv.describe_tp(_tp('3x0e', 3))
    for co in oconv.path_terms(desc):
        assert co['l1'] == 0
        d = 2 * co['l3'] + 1
        assert sorted((b, c) for _, b, c, _ in co['terms']) == [(m, m) for m in range(d)]
        assert all(abs(v - 1.0) < 1e-14 for *_, v in co['terms'])


def test_double_backward_equals_finite_differences():
    """conv_double_bwd (first-order formulas with substituted arguments) against central differences of
    s = <ggx, gx> + <ggY, gY> + <ggW, gW> in each of g, x, Y, W, with the first-order formulas themselves pinned
    against the unfused forward above.  s is linear in each argument, so differences are exact up to rounding."""
    desc = oconv.describe_tp(_tp('2x0e+2x1o', 2))
    coef = oconv.path_terms(desc)
    rng = np.random.default_rng(5)
    n, e = 4, 9
    s, r, x, Y, W, g = _inputs(desc, rng, n, e)
    ggx, ggY, ggW = rng.normal(size=x.shape), rng.normal(size=Y.shape), rng.normal(size=W.shape)

    def sfun(g_, x_, Y_, W_):
        return ((ggx * oconv.conv_bwd_x(desc, coef, g_, Y_, W_, s, r, n)).sum()
                + (ggY * oconv.conv_bwd_y(desc, coef, x_, g_, W_, s, r)).sum()
                + (ggW * oconv.conv_bwd_w(desc, coef, x_, g_, Y_, s, r)).sum())

    args = [g, x, Y, W]
    got = oconv.conv_double_bwd(desc, coef, x, Y, W, g, ggx, ggY, ggW, s, r, n)
    h = 1e-3
    for which, want_shape in enumerate((g.shape, x.shape, Y.shape, W.shape)):
        fd = np.zeros(want_shape)
        for idx in np.ndindex(want_shape):
            p, m = [a.copy() for a in args], [a.copy() for a in args]
            p[which][idx] += h
            m[which][idx] -= h
            fd[idx] = (sfun(*p) - sfun(*m)) / (2 * h)
        assert np.abs(got[which] - fd).max() < 1e-8 * max(1.0, np.abs(fd).max()), which
    # a direction left out (None) is a zero direction
    part = oconv.conv_double_bwd(desc, coef, x, Y, W, g, ggx, None, None, s, r, n)
    assert np.abs(part[1]).max() == 0.0 and np.abs(part[0]).max() > 0


def test_planted_mistakes_are_caught():
    desc = oconv.describe_tp(_tp('4x0e+4x1o', 3))
    coef = oconv.path_terms(desc)
    rng = np.random.default_rng(3)
    s, r, x, Y, W, _ = _inputs(desc, rng, 8, 30)
    ref = oconv.conv_unfused(desc, x, Y, W, s, r, 8)
    dropped = [dict(c) for c in coef]
    dropped[5] = dict(dropped[5], terms=dropped[5]['terms'][1:])
    flipped = [dict(c) for c in coef]
    a, b, cc, v = flipped[7]['terms'][0]
    flipped[7] = dict(flipped[7], terms=[(a, b, cc, -v)] + flipped[7]['terms'][1:])
    for bad in (dropped, flipped):
        assert np.abs(oconv.conv_fwd(desc, bad, x, Y, W, s, r, 8) - ref).max() > 1e-3


def test_csr_matches_bruteforce():
    rng = np.random.default_rng(4)
    idx = rng.integers(0, 10, 200)
    idx[idx == 3] = 4                          # an empty row
    rowptr, eids = oconv.csr_by(idx, 12)
    for n in range(12):
        rows = eids[rowptr[n]:rowptr[n + 1]]
        assert list(rows) == [e for e in range(200) if idx[e] == n]
