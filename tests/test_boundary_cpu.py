"""
The drop-in boundary on the CPU (no GPU calls): the C-ABI library, the supports-checks and skip reasons of
patch_model (reference __init__.py:34-79, conv.py:31-51, symmetric.py:42-49), code generation for gfx950, the graph
cache, and the golden kernel fixtures.
"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

import mace_hip_kernels as mhk
from mace_hip_kernels import _native, conv, symmetric
from mace_lite import factory
from mace_lite.o3 import FullyConnectedTensorProduct, TensorProduct
from oracle import conv as oconv

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'mace_hip.h')
GOLDEN = os.path.join(ROOT, 'tests', 'golden')


def test_library_loads_and_exports_header_symbols():
    lib = _native.load()
    declared = set(re.findall(r'\b(mh_\w+)\s*\(', open(HEADER).read()))
    assert declared == set(_native.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.mh_version() == _native.ABI_VERSION
    assert lib.mh_last_error() is not None


_CTYPE_OF = {
    'int': ctypes.c_int, 'int32_t': ctypes.c_int32, 'int64_t': ctypes.c_int64, 'size_t': ctypes.c_size_t,
    'float': ctypes.c_float, 'double': ctypes.c_double,
}


def _header_prototypes():
    """{name: [parameter C type]} of every function declared in include/mace_hip.h."""
    text = re.sub(r'/\*.*?\*/', ' ', open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r'\b(mh_\w+)\s*\(([^()]*)\)\s*;', text):
        params = [p.strip() for p in m.group(2).split(',') if p.strip() and p.strip() != 'void']
        types = []
        for p in params:
            p = re.sub(r'\s+', ' ', p)
            if '*' in p:
                types.append('ptr')
            else:
                types.append(p.rsplit(' ', 1)[0].replace('const ', '').strip())
        out[m.group(1)] = types
    return out


def test_ctypes_signatures_match_the_header():
    """Every ctypes binding has the header's arity, and each scalar parameter the header's width (a missing trailing
    argument or an int32 bound as int64 would still "work" through ctypes' default conversions)."""
    protos = _header_prototypes()
    assert set(protos) == set(_native.EXPORTS)
    for name, (_, argtypes) in _native._SIGS.items():
        want = protos[name]
        assert len(argtypes) == len(want), (name, len(argtypes), len(want))
        for i, (ct, c) in enumerate(zip(argtypes, want)):
            if c == 'ptr':
                assert ct is ctypes.c_void_p or ct is ctypes.c_char_p or issubclass(ct, ctypes._Pointer), (name, i, ct)
            else:
                assert ctypes.sizeof(ct) == ctypes.sizeof(_CTYPE_OF[c]), (name, i, ct, c)
                assert (ct is ctypes.c_float) == (c == 'float'), (name, i, ct, c)
                assert (ct is ctypes.c_double) == (c == 'double'), (name, i, ct, c)


def test_launch_log_is_off_by_default_and_clears():
    lib = _native.load()
    assert lib.mh_launch_log(1) == 0
    assert _native.launch_log_take() == []
    assert lib.mh_launch_log(0) == 1
    assert lib.mh_launch_log_take(None, 0) == 0


def test_c_abi_rejects_bad_arguments_before_any_launch():
    """Argument errors of the entry points come back as a status and a message, checked before anything reaches the
    GPU (so this runs without one)."""
    lib = _native.load()
    cases = [
        (lambda: lib.mh_graph_build(None, None, 5, 0, None, None, None, None, None, None), 'zero nodes'),
        (lambda: lib.mh_graph_build(None, None, 5, 3, None, None, None, None, None, None), 'NULL'),
        (lambda: lib.mh_graph_build(None, None, -1, 3, None, None, None, None, None, None), 'bad sizes'),
        (lambda: lib.mh_graph_build_noalloc(None, None, 3_000_000, 1000, None, None, None, None, None), 'scratch'),
        (lambda: lib.mh_graph_build_noalloc(None, None, -4, 1000, None, None, None, None, None), 'bad sizes'),
        (lambda: lib.mh_sc_jvp(None, None, None, None, None, None, 4, 2, None), 'layout'),
        (lambda: lib.mh_sc_bwd2(None, None, None, None, None, None, None, 4, 7, None), 'layout'),
        (lambda: lib.mh_sh_jvp(None, None, None, None, 10, None), 'NULL'),
        (lambda: lib.mh_sh_bwd2(None, None, None, None, None, 10, None), 'NULL'),
        (lambda: lib.mh_emb_jvp(None, None, None, None, None, 10, None), 'NULL'),
        (lambda: lib.mh_emb_bwd2(None, None, None, None, None, None, 10, None), 'NULL'),
        (lambda: lib.mh_geom_jvp(None, *([None] * 10), 10, None), 'NULL'),
        (lambda: lib.mh_lin_fwd(None, None, None, None, None, None, 1.0, 10, None), 'NULL'),
        (lambda: lib.mh_readout_bwd(None, None, None, None, 10, None), 'NULL'),
    ]
    for call, msg in cases:
        assert call() != 0
        assert msg in lib.mh_last_error().decode(), (msg, lib.mh_last_error())


def test_compile_errors_are_reported():
    with pytest.raises(RuntimeError, match='hipRTC compile'):
        _native.compile_source('extern "C" __global__ void k() { this is not HIP; }')


@pytest.mark.parametrize('hidden,lmax,corr', [('32x0e+32x1o', 2, 2), ('128x0e+128x1o', 3, 3),
                                              ('64x0e', 2, 2), ('96x0e+96x1o', 3, 2)])
def test_generated_kernels_compile_for_gfx950(hidden, lmax, corr):
    m = factory.make_model(hidden, lmax, corr, elements=factory.ELEMENTS_PTCOH)
    for blk in m.interactions:
        code = _native.compile_source(conv.source(conv.ConvSpec(blk.conv_tp)))
        assert code[:4] == b'\x7fELF'
    for prod in m.products:
        code = _native.compile_source(symmetric.source(symmetric.SCSpec(prod.symmetric_contractions)))
        assert code[:4] == b'\x7fELF'


def test_conv_supported_reasons():
    m = factory.make_model('48x0e+48x1o', 3, 3)
    ok, why = conv.conv_supported(m.interactions[1].conv_tp)
    assert not ok and 'multiple of 32' in why
    ok, why = conv.conv_supported(m.interactions[1].skip_tp)          # uvw, internal shared weights
    assert not ok and 'uvu' in why
    tp = m.interactions[1].conv_tp
    shared = TensorProduct(tp.irreps_in1, tp.irreps_in2, tp.irreps_out,
                           [(i.i_in1, i.i_in2, i.i_out, 'uvu', True) for i in tp.instructions])
    ok, why = conv.conv_supported(shared)
    assert not ok and 'per-edge' in why
    ok, why = conv.conv_supported(object())
    assert not ok and 'not an e3nn TensorProduct' in why
    ok, why = conv.conv_supported(factory.make_model('32x0e+32x1o', 3, 3).interactions[1].conv_tp)
    assert ok and why == ''
    assert not symmetric.sc_supported(object())[0]
    assert symmetric.sc_supported(m.products[0].symmetric_contractions) == (True, '')
    assert isinstance(FullyConnectedTensorProduct('2x0e', '1x0e', '2x0e'), TensorProduct)


def test_patch_model_refuses_cpu_and_float64():
    m = factory.make_model('32x0e+32x1o', 2, 2)
    with pytest.raises(RuntimeError, match='ROCm GPU'):
        mhk.patch_model(m)
    with pytest.raises(RuntimeError):
        mhk.patch_model(m.double())


def test_block_conv_fusion_detection():
    m = factory.make_model('32x0e+32x1o', 2, 2)
    assert all(mhk._block_has_conv_fusion(b) for b in m.interactions)
    assert not mhk._block_has_conv_fusion(torch.nn.Linear(2, 2))


def _oracle_build(edge_index, n):
    """CPU stand-in for the GPU graph build (conv.build_graph) from the oracle's CSR, so that the cache and
    validation logic around it runs here; the GPU build itself is checked against the same oracle on the GPU."""
    ei = edge_index.to(torch.int64)
    bad = torch.tensor([int(bool(((ei < 0) | (ei >= n)).any()))], dtype=torch.int32)
    k = ei.clamp(0, max(n - 1, 0)).to(torch.int32)
    rows = [oconv.csr_by(k[r].numpy(), n) for r in range(2)]
    return (k, torch.stack([torch.tensor(rp) for rp, _ in rows]), torch.stack([torch.tensor(e) for _, e in rows]),
            bad)


def test_graph_cache_and_validation(monkeypatch):
    """Cache and out-of-range report (the synchronous check; the deferred one reads a pinned copy of the flag behind
    a HIP event and is covered on the GPU, tests/test_neighbours_gpu.py)."""
    monkeypatch.setattr(conv, 'build_graph', _oracle_build)
    monkeypatch.setattr(conv, 'GRAPH_CHECK', 'sync')
    conv.clear_graph_cache()
    ei = torch.tensor([[0, 1, 2, 2], [1, 2, 0, 1]])
    g1 = conv.graph_for(ei, 3)
    assert conv.graph_for(ei, 3) is g1                       # same tensor object, same version: cached
    rp, eids = g1.by_recv()
    assert rp.tolist() == [0, 1, 3, 4] and eids.tolist() == [2, 0, 3, 1]
    rp, eids = g1.by_send()
    assert rp.tolist() == [0, 1, 2, 4] and eids.tolist() == [0, 1, 2, 3]
    ei[1, 0] = 2                                              # in-place change bumps the version
    g2 = conv.graph_for(ei, 3)
    assert g2 is not g1 and g2.by_recv()[0].tolist() == [0, 1, 2, 4]
    assert conv.graph_for(ei.clone(), 3) is not g2           # a different tensor object
    with pytest.raises(ValueError, match='outside'):
        conv.graph_for(torch.tensor([[0, 5], [1, 0]]), 3)
    with pytest.raises(ValueError):
        conv.graph_for(torch.tensor([0, 1, 2]), 3)


def test_graph_build_source_compiles():
    assert _native.compile_source(conv.graph_source())[:4] == b'\x7fELF'


def test_neighbour_and_species_sources_compile():
    from mace_hip_kernels import neighbours, species
    assert _native.compile_source(neighbours.source())[:4] == b'\x7fELF'
    assert _native.compile_source(species.source())[:4] == b'\x7fELF'


def test_neighbour_list_work_size_and_argument_checks():
    """The scratch layout grows with atoms, structures and edges; bad arguments fail before any launch."""
    lib = _native.load()
    a, b = lib.mh_neighbour_list_work_size(1, 100, 0), lib.mh_neighbour_list_work_size(1, 100, 5000)
    assert 0 < a < b and b - a >= 8 * 5000 and lib.mh_neighbour_list_work_size(-1, 0, 0) == 0
    cases = [
        ((None, None, None, None, None, 2, 10, 5.0, 100, 150, None, None, None, 0, None, None, None), 'B \\* e_pad'),
        ((None, None, None, None, None, 2, 10, -1.0, 0, 0, None, None, None, 0, None, None, None), 'r_max'),
        ((None, None, None, None, None, 2, 10, 5.0, 0, 0, None, None, None, 0, None, None, None), 'NULL'),
        ((None, None, None, None, None, -1, 10, 5.0, 0, 0, None, None, None, 0, None, None, None), 'bad sizes'),
    ]
    for args, msg in cases:
        assert lib.mh_neighbour_list(*args) != 0
        assert re.search(msg, lib.mh_last_error().decode()), lib.mh_last_error()
    assert lib.mh_species_order(None, None, 10, 200, None, None, None, 0, 8, None) != 0
    assert b'ne <=' in lib.mh_last_error()
    assert lib.mh_species_order(None, None, 10, 4, None, None, None, 8, 8, None) != 0
    assert b'nslots' in lib.mh_last_error()


def test_edge_compaction_and_row_list_argument_checks():
    """mh_edge_compact's scratch is one int32 per 4096 edges (one for none); bad arguments and a row list without
    its count fail before any launch."""
    lib = _native.load()
    assert [lib.mh_edge_compact_work_size(e) for e in (0, 1, 4096, 4097, 100000)] == [4, 4, 4, 8, 100]
    P = ctypes.c_void_p
    assert lib.mh_edge_compact(None, None, -1, None, None, None, None) != 0
    assert b'bad edge count' in lib.mh_last_error()
    assert lib.mh_edge_compact(None, None, 10, None, P(8), P(8), None) != 0
    assert b'NULL' in lib.mh_last_error()
    assert lib.mh_edge_compact(None, P(8), 10, P(8), P(8), P(8), None) != 0
    assert b'null module' in lib.mh_last_error()
    assert lib.mh_mlp_fwd_rows(None, P(8), P(8), P(8), P(8), 10, P(8), None, None) != 0
    assert b'go together' in lib.mh_last_error()
    assert lib.mh_mlp_bwd_rows(None, P(8), P(8), P(8), P(8), P(8), 10, None, P(8), None) != 0
    assert b'go together' in lib.mh_last_error()
    # the paired backward needs its row list, count and partner map
    assert lib.mh_mlp_bwd_pairs(None, P(8), P(8), P(8), P(8), P(8), 10, P(8), P(8), None, None) != 0
    assert b'mh_mlp_bwd_pairs: NULL' in lib.mh_last_error()
    assert lib.mh_mlp_bwd_pairs(None, P(8), P(8), P(8), P(8), P(8), 10, P(8), None, P(8), None) != 0
    assert b'NULL count' in lib.mh_last_error()
    # the pairing's vectors and partner map go together
    ops = [P(8)] * 7
    assert lib.mh_edge_pairs(None, P(8), 8, *ops, 5, 10, P(8), P(8), None, P(8), P(8), P(8), P(8), P(8), None) != 0
    assert b'vec and partner go together' in lib.mh_last_error()
    assert lib.mh_conv_bwd_recv(None, P(8), P(8), P(8), P(8), None, None, None, None, None, None, None, P(8), P(8),
                                P(8), P(8), 10, _native.MH_WANT_GWY | _native.MH_CUT_NOZERO, None) != 0
    assert b'MH_CUT_NOZERO needs MH_CUT_MASKED' in lib.mh_last_error()
    # the edge pass's backward with a second consumer's gradients: those may be NULL, the first ones may not
    assert lib.mh_edge_bwd2(None, P(8), P(8), None, P(8), None, P(8), P(8), P(8), P(8), P(8), 10, None) != 0
    assert b'mh_edge_bwd: NULL' in lib.mh_last_error()
    assert lib.mh_edge_bwd2(None, P(8), P(8), P(8), P(8), None, None, None, None, P(8), P(8), 10, None) != 0
    assert b'null module' in lib.mh_last_error()
    # the node linear with a residual: NULL x, W or out is an error (res may be NULL)
    assert lib.mh_lin_fwd_res(None, None, None, P(8), P(8), None, 1.0, P(8), 10, None) != 0
    assert b'mh_lin_fwd: NULL x, W or out' in lib.mh_last_error()
    assert lib.mh_lin_bwd_sum(None, P(8), None, P(8), None, P(8), P(8), None, 1.0, 10, None) != 0
    assert b'mh_lin_bwd_sum: NULL' in lib.mh_last_error()


def test_species_order_fallback_on_large_tables():
    """More elements than the kernel's LDS tables: the torch expressions (they run on the CPU too)."""
    from mace_hip_kernels import species
    rng = np.random.default_rng(0)
    n, ne, group = 300, 150, 8
    idx = rng.integers(0, ne, n)
    a = torch.zeros(n, ne)
    a[torch.arange(n), torch.from_numpy(idx)] = 1.0
    elem, order, slots = species.species_order(a, group)
    assert torch.equal(elem.long(), torch.from_numpy(idx)) and torch.equal(order.long(), torch.argsort(elem, stable=True))
    assert slots.numel() == species.slot_count(n, ne, group)
    live = slots[slots >= 0]
    assert torch.equal(live, order)                               # the runs in element order, -1 between them
    starts = (torch.nonzero(slots >= 0).reshape(-1))
    run_elem = elem[slots[starts].long()]
    assert bool((starts[1:][run_elem[1:] != run_elem[:-1]] % group == 0).all())


def test_golden_fixtures_reproduce():
    """The oracle still produces the committed fixtures that the GPU tests compare the kernels with."""
    g = np.load(os.path.join(GOLDEN, 'conv_small.npz'))
    tp = factory.make_model('32x0e+32x1o', 3, 3).interactions[1].conv_tp
    desc = oconv.describe_tp(tp)
    coef = oconv.path_terms(desc)
    s, r, n = g['sender'], g['receiver'], int(g['n'])
    assert np.abs(oconv.conv_fwd(desc, coef, g['x'], g['Y'], g['W'], s, r, n) - g['out']).max() < 1e-12
    assert np.abs(oconv.conv_bwd_x(desc, coef, g['g'], g['Y'], g['W'], s, r, n) - g['gx']).max() < 1e-12
    assert np.abs(oconv.conv_bwd_w(desc, coef, g['x'], g['g'], g['Y'], s, r) - g['gW']).max() < 1e-12
    assert np.abs(oconv.conv_bwd_y(desc, coef, g['x'], g['g'], g['W'], s, r) - g['gY']).max() < 1e-12


def test_grad_needed_follows_the_engine():
    """The backward asks the autograd engine which input gradients the current pass uses (host logic, CPU)."""
    seen = []

    class Probe(torch.autograd.Function):
        @staticmethod
        def forward(ctx, a, b):
            return a * b

        @staticmethod
        def backward(ctx, g):
            seen.append((conv._grad_needed(ctx, 0), conv._grad_needed(ctx, 1)))
            return g, g

    x, p = torch.randn(3, requires_grad=True), torch.randn(3, requires_grad=True)
    cases = [
        (lambda: torch.autograd.grad(Probe.apply(x * 2, p * 3).sum(), [p]), (False, True)),   # branch unused
        (lambda: torch.autograd.grad(Probe.apply(x, p * 3).sum(), [x]), (True, False)),       # leaf is an input
        (lambda: Probe.apply(x * 2, p * 3).sum().backward(), (True, True)),
        (lambda: Probe.apply(torch.randn(3), p * 3).sum().backward(), (False, True)),           # no grad at all
    ]
    for run, want in cases:
        seen.clear()
        run()
        assert seen == [want]
    a = x * 2                                                                                    # non-leaf input
    seen.clear()
    torch.autograd.grad(Probe.apply(a, p * 3).sum(), [a])
    assert seen == [(True, False)]


def test_grad_needed_without_the_engine_query(monkeypatch):
    """A torch without the engine query answers conservatively: every input gradient autograd asks for counts as
    needed, and the gradients are still right (host logic, CPU)."""
    monkeypatch.delattr(torch._C, '_will_engine_execute_node')
    seen = []

    class Probe(torch.autograd.Function):
        @staticmethod
        def forward(ctx, a, b):
            ctx.save_for_backward(a, b)
            return a * b

        @staticmethod
        def backward(ctx, g):
            a, b = ctx.saved_tensors
            seen.append((conv._grad_needed(ctx, 0), conv._grad_needed(ctx, 1)))
            return g * b, g * a

    x, p = torch.randn(3, requires_grad=True), torch.randn(3, requires_grad=True)
    (gp,) = torch.autograd.grad(Probe.apply(x * 2, p * 3).sum(), [p])
    assert seen == [(True, True)]                       # the unused branch is computed, not skipped
    assert torch.allclose(gp, 3 * (x * 2).detach())
    seen.clear()
    Probe.apply(torch.randn(3), p * 3).sum().backward()
    assert seen == [(False, True)]                      # needs_input_grad still decides first


def test_factored_weights_or_the_plain_path():
    """``W0 * cutoff`` is read from its autograd node; any other producer, or a node whose saved tensors are gone,
    keeps the plain path (None) instead of failing (host logic, CPU)."""
    E, nw = 5, 8
    W0 = torch.randn(E, nw, requires_grad=True)
    cut = torch.rand(E, 1, requires_grad=True)
    W = W0 * cut
    got = conv._factored_weights(W)
    assert got is not None and torch.equal(got[0], W0) and torch.equal(got[1], cut)
    assert conv._factored_weights(cut.reshape(E, 1) * W0) is not None          # either operand order
    assert conv._factored_weights(W0 * 2.0) is None                          # scalar product
    assert conv._factored_weights(W0 + cut) is None                          # another op
    assert conv._factored_weights(W0.detach() * cut.detach()) is None        # no graph
    assert conv._factored_weights(W0 * torch.rand(E, nw)) is None            # factor of the wrong shape
    W2 = W0 * cut
    W2.sum().backward()                                                      # saved tensors freed
    assert conv._factored_weights(W2) is None
