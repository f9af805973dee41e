"""
Oracle for the interaction convolution (test infrastructure only; see oracle/__init__.py).

Restates, in float64 numpy, with coupling tables built from ``oracle.wigner`` (never from the product):
  * ``path_terms``     the effective coefficient table the reference probes from an e3nn 'uvu' TensorProduct
                       (reference conv.py:57-88): sqrt(alpha)·C[a,b,c], alpha = (2 l3 + 1) / Σ fan-in of the
                       instructions feeding the same output block (e3nn "component" irreps, "element" paths);
  * ``conv_unfused``   MACE's unpatched path: message_e = TP(x[sender_e], Y_e, W_e), scatter-summed to receivers;
  * ``conv_fwd`` / ``conv_bwd_x`` / ``conv_bwd_w`` / ``conv_bwd_y``
                       the per-term formulas of the reference's three kernels (conv.py:109-141, 144-176, 179-222);
  * ``csr_by``         the receiver/sender CSR (conv.py:229-235) with numpy's stable argsort.
  * ``conv_double_bwd`` the second derivatives of <g, out> as first-order formulas with substituted arguments.

Pinned by (tests/test_oracle_conv.py): fused forward == unfused forward on random graphs; each backward formula ==
central finite differences of the unfused forward; conv_double_bwd == central
finite differences of the first-order formulas; probed coefficients == path_terms; path (0e ⊗ l → l) is
δ/√(2l+1)·√(2l+1) = identity; CSR == brute-force grouping.
"""
import math

import numpy as np

from . import wigner


def describe_tp(tp):
    """Plain-data description of an e3nn-style TensorProduct: blocks of in1/in2/out as (l, mul, offset) and the
    instruction list (i_in1, i_in2, i_out).  Reads only irreps and instructions (data), never calls the TP."""
    def blocks(irreps):
        res, off = [], 0
        for mul, ir in irreps:
            res.append((ir.l, mul, off))
            off += mul * (2 * ir.l + 1)
        return res, off
    in1, x_dim = blocks(tp.irreps_in1)
    in2, y_dim = blocks(tp.irreps_in2)
    outb, out_dim = blocks(tp.irreps_out)
    ins = [(i.i_in1, i.i_in2, i.i_out) for i in tp.instructions]
    return dict(in1=in1, in2=in2, out=outb, x_dim=x_dim, y_dim=y_dim, out_dim=out_dim, ins=ins, mul=in1[0][1])


def path_terms(desc, tol=1e-12):
    """Per instruction: dict(l1, l2, l3, o1, o2, o3, terms=[(a, b, c, coefficient)])."""
    fan = {}
    for i1, i2, io in desc['ins']:
        fan[io] = fan.get(io, 0) + desc['in2'][i2][1]           # 'uvu' fan-in: mul of input 2
    out = []
    for k, (i1, i2, io) in enumerate(desc['ins']):
        l1, _, o1 = desc['in1'][i1]
        l2, _, o2 = desc['in2'][i2]
        l3, _, o3 = desc['out'][io]
        c = wigner.wigner_3j(l1, l2, l3) * math.sqrt((2 * l3 + 1) / fan[io])
        terms = [(a, b, cc, float(c[a, b, cc])) for a in range(2 * l1 + 1) for b in range(2 * l2 + 1)
                 for cc in range(2 * l3 + 1) if abs(c[a, b, cc]) > tol]
        out.append(dict(k=k, l1=l1, l2=l2, l3=l3, o1=o1, o2=o2, o3=o3, terms=terms))
    return out


def conv_unfused(desc, x, Y, W, sender, receiver, n):
    """scatter_sum over receivers of the dense uvu tensor product of (x[sender], Y, W)."""
    mul = desc['mul']
    xs = x[sender]
    E = len(sender)
    out = np.zeros((n, desc['out_dim']))
    fan = {}
    for i1, i2, io in desc['ins']:
        fan[io] = fan.get(io, 0) + desc['in2'][i2][1]
    for k, (i1, i2, io) in enumerate(desc['ins']):
        l1, _, o1 = desc['in1'][i1]
        l2, _, o2 = desc['in2'][i2]
        l3, _, o3 = desc['out'][io]
        d1, d2, d3 = 2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1
        c = wigner.wigner_3j(l1, l2, l3) * math.sqrt(d3 / fan[io])
        a = xs[:, o1:o1 + mul * d1].reshape(E, mul, d1)
        b = Y[:, o2:o2 + d2]
        w = W[:, k * mul:(k + 1) * mul]
        m = np.einsum('eui,ej,ijk,eu->euk', a, b, c, w, optimize=True).reshape(E, mul * d3)
        np.add.at(out[:, o3:o3 + mul * d3], receiver, m)
    return out


def conv_fwd(desc, coef, x, Y, W, sender, receiver, n):
    """out[n, o3+u·d3+c] = Σ_{e→n} Σ_terms v·W[e, k·mul+u]·x[s, o1+u·d1+a]·Y[e, o2+b] (reference conv.py:109-141)."""
    mul = desc['mul']
    out = np.zeros((n, desc['out_dim']))
    u = np.arange(mul)
    for co in coef:
        k, o1, o2, o3 = co['k'], co['o1'], co['o2'], co['o3']
        d1, d3 = 2 * co['l1'] + 1, 2 * co['l3'] + 1
        w = W[:, k * mul + u]
        for a, b, c, v in co['terms']:
            msg = v * w * x[sender][:, o1 + u * d1 + a] * Y[:, o2 + b][:, None]
            np.add.at(out, (receiver[:, None], (o3 + u * d3 + c)[None, :]), msg)
    return out


def conv_bwd_x(desc, coef, g, Y, W, sender, receiver, n):
    """gx[s, o1+u·d1+a] = Σ_{e: s→} Σ_terms v·W·Y[e, o2+b]·g[r, o3+u·d3+c] (reference conv.py:144-176)."""
    mul = desc['mul']
    gx = np.zeros((n, desc['x_dim']))
    u = np.arange(mul)
    for co in coef:
        k, o1, o2, o3 = co['k'], co['o1'], co['o2'], co['o3']
        d1, d3 = 2 * co['l1'] + 1, 2 * co['l3'] + 1
        w = W[:, k * mul + u]
        for a, b, c, v in co['terms']:
            msg = v * w * Y[:, o2 + b][:, None] * g[receiver][:, o3 + u * d3 + c]
            np.add.at(gx, (sender[:, None], (o1 + u * d1 + a)[None, :]), msg)
    return gx


def conv_bwd_w(desc, coef, x, g, Y, sender, receiver):
    """gW[e, k·mul+u] = Σ_terms v·x[s, o1+u·d1+a]·Y[e, o2+b]·g[r, o3+u·d3+c] (reference conv.py:205-209)."""
    mul = desc['mul']
    gW = np.zeros((len(sender), len(coef) * mul))
    u = np.arange(mul)
    for co in coef:
        k, o1, o2, o3 = co['k'], co['o1'], co['o2'], co['o3']
        d1, d3 = 2 * co['l1'] + 1, 2 * co['l3'] + 1
        for a, b, c, v in co['terms']:
            gW[:, k * mul + u] += v * x[sender][:, o1 + u * d1 + a] * Y[:, o2 + b][:, None] * \
                g[receiver][:, o3 + u * d3 + c]
    return gW


def conv_bwd_y(desc, coef, x, g, W, sender, receiver):
    """gY[e, o2+b] = Σ_u Σ_terms v·W[e, k·mul+u]·x[s, o1+u·d1+a]·g[r, o3+u·d3+c] (reference conv.py:210-220)."""
    mul = desc['mul']
    gY = np.zeros((len(sender), desc['y_dim']))
    u = np.arange(mul)
    for co in coef:
        k, o1, o2, o3 = co['k'], co['o1'], co['o2'], co['o3']
        d1, d3 = 2 * co['l1'] + 1, 2 * co['l3'] + 1
        w = W[:, k * mul + u]
        for a, b, c, v in co['terms']:
            gY[:, o2 + b] += (v * w * x[sender][:, o1 + u * d1 + a] * g[receiver][:, o3 + u * d3 + c]).sum(1)
    return gY


def conv_double_bwd(desc, coef, x, Y, W, g, ggx, ggY, ggW, sender, receiver, n):
    """Gradients of s = <ggx, gx> + <ggY, gY> + <ggW, gW> (gx, gY, gW the first-order gradients of <g, out>) with
    respect to (g, x, Y, W).  The product is linear in each of x, Y, W, so every term is a first-order formula with
    one argument replaced by a direction: d s/d g = out(ggx, Y, W) + out(x, ggY, W) + out(x, Y, ggW), and e.g.
    d s/d x = gx(g; ggY, W) + gx(g; Y, ggW) (the second derivatives the reference's backward guard refuses,
    conv.py:254-256).  Any direction may be None (zero)."""
    z = lambda a, shape: np.zeros(shape) if a is None else a             # noqa: E731
    E = len(sender)
    ggx, ggY, ggW = z(ggx, x.shape), z(ggY, Y.shape), z(ggW, W.shape)
    f = lambda xx, yy, ww: conv_fwd(desc, coef, xx, yy, ww, sender, receiver, n)    # noqa: E731
    gg = f(ggx, Y, W) + f(x, ggY, W) + f(x, Y, ggW)
    gx = conv_bwd_x(desc, coef, g, ggY, W, sender, receiver, n) + conv_bwd_x(desc, coef, g, Y, ggW, sender, receiver, n)
    gY = conv_bwd_y(desc, coef, ggx, g, W, sender, receiver) + conv_bwd_y(desc, coef, x, g, ggW, sender, receiver)
    gW = conv_bwd_w(desc, coef, ggx, g, Y, sender, receiver) + conv_bwd_w(desc, coef, x, g, ggY, sender, receiver)
    assert gY.shape == (E, desc['y_dim'])
    return gg, gx, gY, gW


def csr_by(index, n):
    """(rowptr[n+1], edge ids sorted stably by index) as int32."""
    index = np.asarray(index)
    order = np.argsort(index, kind='stable')
    rowptr = np.zeros(n + 1, dtype=np.int64)
    rowptr[1:] = np.cumsum(np.bincount(index, minlength=n))
    return rowptr.astype(np.int32), order.astype(np.int32)


def random_graph(rng, n, e, max_deg=None):
    """Random multigraph (self-loops and repeated pairs allowed) with n nodes and e edges, as sender/receiver."""
    s = rng.integers(0, n, e)
    r = rng.integers(0, n, e)
    return s.astype(np.int64), r.astype(np.int64)
