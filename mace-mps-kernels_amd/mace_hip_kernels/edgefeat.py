"""
The edge geometry, the spherical harmonics and the radial embedding of one E+F call as one pass per edge, each way.

MACE forms, per edge, vectors and lengths (``get_edge_vectors_and_lengths``), then the spherical harmonics of the
vectors and the radial embedding of the lengths, in three calls.  Patched, each is a kernel of its own, and a kernel
costs a few microseconds of dispatch and drain however little it does.  When a patched model's geometry, harmonics
and embedding are all drop-ins, the geometry's forward runs ``edge_fwd`` instead: one thread per edge computes the
vector, the length, the harmonics and the embedding (the statements of ``geom_fwd``, ``sh_fwd`` and ``emb_fwd``) and
leaves the three later outputs on the vectors tensor.  The harmonics module, called next on that tensor, returns them
through one autograd node of the vectors and the lengths (``_EdgeFeatFn``), which hands the embedding's outputs on to
the embedding module through the lengths tensor.  Its backward is ``edge_bwd``: dL/dvectors from the harmonics'
gradient and dL/dlengths from the embedding's, in one pass (the statements of ``sh_bwd`` and ``emb_bwd``).

Outputs left on a tensor are taken only by the module they were made for, only once, and only while the tensor is
unmodified (same version); any other call computes as before.
"""
import torch

from . import _native
from . import edge as _edge
from . import embedding as _emb
from .pending import set_slots, slot  # noqa: F401  (slot: the joint node's aliases, handed out)

BLOCK = 256
FUSE = True            # run the three forwards (and the two backwards) as one pass where a model allows it


def kname(sh_spec, emb_spec, base):
    return f'{base}_l{sh_spec.lmax}_{"norm" if sh_spec.norm else "comp"}_n{emb_spec.n}_p{emb_spec.p}'


def source(sh_spec, emb_spec):
    """HIP source of ``edge_fwd`` and ``edge_bwd`` for one (harmonics, embedding) pair."""
    sh, em = _edge.math_lines(sh_spec), _emb.math_lines(emb_spec)
    ind = lambda lines, k=2: [' ' * k + ln for ln in lines]  # noqa: E731
    n, dim = emb_spec.n, sh_spec.dim
    idx = ['  const long long e = (long long)mh_xcd_block(blockIdx.x, gridDim.x) * BLOCK + threadIdx.x;',
           '  if (e >= E) return;']
    L = [_native.device_header(), f'#define BLOCK {BLOCK}', f'#define DIM {dim}']
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {kname(sh_spec, emb_spec, "edge_fwd")}(',
          '    const float* __restrict__ pos, const int* __restrict__ send, const int* __restrict__ recv,',
          '    const float* __restrict__ shifts, float* __restrict__ vec, float* __restrict__ len,',
          '    float* __restrict__ Y, float* __restrict__ feats, float* __restrict__ cutoff, long long E) {'] + idx
    L += ['  float vx, vy, vz;',
          '  {                                         // the edge vector and its length (geom_fwd)',
          '    const long long s = send[e], r = recv[e];',
          '    vx = (pos[3 * r] - pos[3 * s]) + shifts[3 * e];',
          '    vy = (pos[3 * r + 1] - pos[3 * s + 1]) + shifts[3 * e + 1];',
          '    vz = (pos[3 * r + 2] - pos[3 * s + 2]) + shifts[3 * e + 2];',
          '  }',
          '  vec[3 * e] = vx; vec[3 * e + 1] = vy; vec[3 * e + 2] = vz;',
          '  const float le = sqrtf(vx * vx + vy * vy + vz * vz);',
          '  len[e] = le;',
          '  {                                         // the spherical harmonics of the vector (sh_fwd)']
    L += ind(sh['head'] + sh['fwd'], 4)
    L += ['    float* __restrict__ ye = Y + e * DIM;'] + [f'    ye[{c}] = Y{c};' for c in range(dim)]
    L += ['  }',
          '  {                                         // the radial embedding of the length (emb_fwd)',
          '    const float x = le;']
    L += ind(em['head'], 4) + ['    cutoff[e] = cut;'] + ind(em['fwd'], 4)
    L += [f'    feats[e * {n} + {k}] = f{k};' for k in range(n)]
    L += ['  }', '}', '']
    # gY2 / gfeats2 / gcut2 (each may be NULL): a second consumer's gradients of the same outputs, added to the
    # first's per element as autograd would (a + b), so that no separate sum runs
    L += [f'extern "C" __global__ __launch_bounds__(BLOCK) void {kname(sh_spec, emb_spec, "edge_bwd")}(',
          '    const float* __restrict__ vec, const float* __restrict__ len, const float* __restrict__ gY,',
          '    const float* __restrict__ gfeats, const float* __restrict__ gcut, float* __restrict__ gvec,',
          '    float* __restrict__ glen, long long E, const float* __restrict__ gY2,',
          '    const float* __restrict__ gfeats2, const float* __restrict__ gcut2) {'] + idx
    L += ['  {                                         // dL/dvec from the harmonics\' gradient (sh_bwd)',
          '    const float vx = vec[3 * e], vy = vec[3 * e + 1], vz = vec[3 * e + 2];']
    L += ind(sh['head'], 4)
    # one wave-uniform test per operand, each branch straight-line loads (a test per element would wait per element)
    L += ['    const float* __restrict__ ge = gY + e * DIM;', f'    float {", ".join(f"g{c}" for c in range(dim))};',
          '    if (gY2) {', '      const float* __restrict__ ge2 = gY2 + e * DIM;']
    L += [f'      g{c} = ge[{c}] + ge2[{c}];' for c in range(dim)]
    L += ['    } else {'] + [f'      g{c} = ge[{c}];' for c in range(dim)] + ['    }']
    L += ind(sh['bwd'], 4) + ['    gvec[3 * e] = ox; gvec[3 * e + 1] = oy; gvec[3 * e + 2] = oz;', '  }']
    L += ['  {                                         // dL/dlen from the embedding\'s gradients (emb_bwd)',
          '    const float x = len[e];']
    L += [f'    float {", ".join(f"gf{k}" for k in range(n))};', '    if (gfeats2) {']
    L += [f'      gf{k} = gfeats[e * {n} + {k}] + gfeats2[e * {n} + {k}];' for k in range(n)]
    L += ['    } else {'] + [f'      gf{k} = gfeats[e * {n} + {k}];' for k in range(n)] + ['    }']
    L += ['    const bool hc = gcut || gcut2;',
          '    float gc = 0.f;',
          '    if (gcut && gcut2) gc = gcut[e] + gcut2[e];',
          '    else if (gcut) gc = gcut[e];',
          '    else if (gcut2) gc = gcut2[e];']
    # the embedding's statements read gfeats[e * n + k] and gcut; here they read the summed values
    bwd, hits = [], 0
    for ln_ in em['bwd']:
        new_ = ln_.replace('gcut ? gcut[e] * dcut : 0.f', 'hc ? gc * dcut : 0.f')
        for k in range(n):
            new_ = new_.replace(f'gfeats[e * {n} + {k}]', f'gf{k}')
        hits += new_ != ln_
        bwd.append(new_)
    if hits != n + 1 or any('gfeats' in b or 'gcut' in b for b in bwd):
        raise RuntimeError('edgefeat: the embedding\'s backward statements changed form')
    L += ind(em['head'] + bwd, 4) + ['    glen[e] = acc;', '  }', '}', '']
    return '\n'.join(L)


def module(sh_op, emb_op, device):
    """The module of the fused kernels for a (harmonics, embedding) pair of drop-ins (their constants are compiled
    in), compiled on first use and kept on the harmonics drop-in per (embedding drop-in, device)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    cache = sh_op.__dict__.setdefault('_mh_edge_modules', {})
    hit = cache.get((id(emb_op), idx))
    if hit is not None and hit[0] is emb_op:
        return hit[1]
    code = _native.compile_source(source(sh_op.spec, emb_op.spec))
    with torch.cuda.device(idx):
        m = _native.Module(code, {
            _native.MH_EDGE_FWD: (kname(sh_op.spec, emb_op.spec, 'edge_fwd'), BLOCK, BLOCK),
            _native.MH_EDGE_BWD: (kname(sh_op.spec, emb_op.spec, 'edge_bwd'), BLOCK, BLOCK)})
    cache[(id(emb_op), idx)] = (emb_op, m)
    return m


def forward_all(pos, gr, shifts, vec, ln, ops):
    """Fill vec [E, 3] and ln [E, 1] as ``geom_fwd`` does and leave the harmonics and the embedding of the same edges
    on ``vec`` for the modules of ``ops`` = (harmonics, embedding)."""
    sh_op, emb_op = ops
    E = vec.shape[0]
    dev = vec.device
    Y = torch.empty(E, sh_op.spec.dim, device=dev, dtype=torch.float32)
    feats = torch.empty(E, emb_op.spec.n, device=dev, dtype=torch.float32)
    cut = torch.empty(E, 1, device=dev, dtype=torch.float32)
    P = _native.ptr
    _native.launch(f'edge_fwd[{sh_op.tag}+{emb_op.tag}]', _native.load().mh_edge_fwd,
                   module(sh_op, emb_op, dev).handle, P(pos), P(gr.send), P(gr.recv), P(shifts), P(vec), P(ln), P(Y),
                   P(feats), P(cut), E, _native.stream_of(pos))
    vec._mh_edge = (sh_op, emb_op, ln, Y, feats, cut, vec._version, ln._version)


def _two(gs, shape):
    """The gradients ``gs`` (Nones dropped) as at most two contiguous tensors of ``shape``; a third and further ones
    (three or more consumers) are added to the second."""
    gs = [g.reshape(shape).contiguous() for g in gs if g is not None]
    if len(gs) > 2:
        gs = [gs[0], sum(gs[2:], gs[1])]
    return gs + [None] * (2 - len(gs))


def _edge_bwd(sh_op, emb_op, vec, ln, gYs, gfs, gcs):
    """(gvec, glen) of the joint node from the gradients its consumers gave each output (lists; None: none)."""
    E = vec.shape[0]
    dev = vec.device
    gY, gY2 = _two(gYs, (E, sh_op.spec.dim))
    gf, gf2 = _two(gfs, (E, emb_op.spec.n))
    gc, gc2 = _two(gcs, (E,))
    gY = torch.zeros(E, sh_op.spec.dim, device=dev) if gY is None else gY
    gf = torch.zeros(E, emb_op.spec.n, device=dev) if gf is None else gf
    gv = torch.empty(E, 3, device=dev, dtype=torch.float32)
    gl = torch.empty(E, 1, device=dev, dtype=torch.float32)
    P = _native.ptr
    two = gY2 is not None or gf2 is not None or gc2 is not None
    _native.launch(f'edge_bwd[{sh_op.tag}+{emb_op.tag}{"+slots" if two else ""}]', _native.load().mh_edge_bwd2,
                   module(sh_op, emb_op, dev).handle, P(vec), P(ln), P(gY), P(gf), P(gc), P(gY2), P(gf2), P(gc2),
                   P(gv), P(gl), E, _native.stream_of(vec))
    return gv, gl


class _EdgeFeatFn(torch.autograd.Function):
    """(harmonics, features, cutoff) of (vectors, lengths), made by ``edge_fwd``: one node for the two modules, so
    that their gradients arrive together and one ``edge_bwd`` serves both.  With ``nslot`` > 0 the node also returns
    ``nslot`` aliases of the three (the same storage, outputs of their own) for the other patched consumers
    (``slot``): each consumer's gradients then reach the node separately, and ``edge_bwd`` adds them as it loads them
    instead of autograd summing each output's gradients in kernels of their own.  Under create_graph the gradient is
    the two modules' own differentiable functions (``_SHAdjFn``, ``_EmbAdjFn``) of the summed gradients."""

    @staticmethod
    def forward(ctx, vec, ln, made, nslot):
        sh_op, emb_op, _, Y, feats, cut = made[:6]
        ctx.save_for_backward(vec, ln)
        ctx.sh_op, ctx.emb_op = sh_op, emb_op
        extra = []
        for _ in range(nslot):
            extra += [Y.detach(), feats.detach(), cut.detach()]
        return (Y, feats, cut, *extra)

    @staticmethod
    def backward(ctx, gY, gf, gc, *extra):
        vec, ln = ctx.saved_tensors
        sh_op, emb_op = ctx.sh_op, ctx.emb_op
        gYs, gfs, gcs = [gY, *extra[0::3]], [gf, *extra[1::3]], [gc, *extra[2::3]]
        if torch.is_grad_enabled():          # only true under create_graph=True
            if not sh_op.double_backward:
                raise RuntimeError(_edge._DOUBLE_BACKWARD)
            if not emb_op.double_backward:
                raise RuntimeError(_emb._DOUBLE_BACKWARD)
            total = lambda gs: None if all(g is None for g in gs) else sum(g for g in gs if g is not None)  # noqa
            gY, gf, gc = total(gYs), total(gfs), total(gcs)
            gv = None if gY is None else _edge._SHAdjFn.apply(gY, vec, sh_op)
            gl = None if gf is None and gc is None else _emb._EmbAdjFn.apply(gf, gc, ln, emb_op)
            return gv, gl, None, None
        gv, gl = _edge_bwd(sh_op, emb_op, vec, ln, gYs, gfs, gcs)
        return gv, gl.reshape(ln.shape), None, None




def take_harmonics(sh_op, vec):
    """The harmonics ``edge_fwd`` left on ``vec`` for ``sh_op`` (through the joint node, which leaves the embedding's
    outputs on the lengths tensor), or None."""
    made = getattr(vec, '_mh_edge', None)
    if made is None or made[0] is not sh_op or made[6] != vec._version:
        return None
    del vec._mh_edge
    ln = made[2]
    if ln._version != made[7]:
        return None
    nslot = max(0, int(getattr(sh_op, 'slots', 0)))
    outs = _EdgeFeatFn.apply(vec, ln, made, nslot)
    Y, feats, cut = outs[:3]
    if nslot:
        for k, t in enumerate((Y, feats, cut)):
            set_slots(t, outs[3 + k::3])
    ln._mh_emb = (made[1], feats, cut, ln._version)
    return Y


def take_embedding(emb_op, ln):
    """The (features, cutoff) the joint node left on the lengths ``ln`` for ``emb_op``, or None."""
    made = getattr(ln, '_mh_emb', None)
    if made is None or made[0] is not emb_op or made[3] != ln._version:
        return None
    del ln._mh_emb
    return made[1], made[2]
