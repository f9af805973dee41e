"""
Host side of the radial MLP drop-in (mace_hip_kernels.radial), on the CPU: the restated layers against the e3nn
module in float64, the refusal of modules it does not cover, and the generated HIP source compiling for gfx950.
"""
import numpy as np
import pytest
import torch

from mace_hip_kernels import radial
from mace_lite import factory
from mace_lite import nn as enn


def test_restated_layers_match_every_block():
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    rng = np.random.default_rng(2)
    for blk in m.interactions:
        spec = radial.MLPSpec(blk.conv_tp_weights)
        x = rng.normal(size=(11, spec.hs[0]))
        with torch.no_grad():
            ref = blk.conv_tp_weights.double()(torch.tensor(x)).numpy()
        assert np.abs(spec.apply(x) - ref).max() < 1e-12 * np.abs(ref).max()
        pw = radial.packed_weights(spec)
        assert pw['fwd'][0].dtype == np.float32
        # both hidden layouts hold the same numbers
        assert np.isclose(np.abs(pw['fwd'][0]).sum(), np.abs(pw['bwd'][0]).sum(), rtol=1e-6)
        # both output-layer layouts rebuild the float32 weights exactly from their three bf16 parts
        want = spec.A[-1].astype(np.float32)
        assert np.array_equal(_unpack(pw['fwd'][1], spec, fwd=True), want)
        assert np.array_equal(_unpack(pw['bwd'][1], spec, fwd=False), want)


def _bf16(u16):
    return (u16.astype(np.uint32) << np.uint32(16)).view(np.float32)


def _unpack(buf, spec, fwd):
    """Sum of the three bf16 parts of a packed output layer, back in [HL, NW] order (the forward layout walks K in
    the MFMA-operand order 32 s + 8 q + 4 t + r <-> hidden feature 32 s + 16 t + 4 q + r)."""
    HL, NW = spec.A[-1].shape
    CH = radial.CH_FWD if fwd else radial.CH_BWD
    nch = -(-NW // CH)
    if fwd:
        p = buf.reshape(nch, 3, HL // 8, CH, 8).transpose(0, 1, 3, 2, 4).reshape(nch, 3, CH, HL)
        w = _bf16(p[:, 0]) + _bf16(p[:, 1]) + _bf16(p[:, 2])          # exact: the parts do not overlap
        out = np.zeros((HL, nch * CH), dtype=np.float32)
        for pos in range(HL):
            s_, rem = divmod(pos, 32)
            q, j = divmod(rem, 8)
            t, r = divmod(j, 4)
            out[32 * s_ + 16 * t + 4 * q + r] = w[:, :, pos].reshape(-1)
    else:
        p = buf.reshape(nch, 3, CH // 8, HL, 8).transpose(0, 1, 3, 2, 4).reshape(nch, 3, HL, CH)
        w = _bf16(p[:, 0]) + _bf16(p[:, 1]) + _bf16(p[:, 2])
        out = w.transpose(1, 0, 2).reshape(HL, nch * CH)
    assert not np.any(out[:, NW:]), 'padding columns must be zero'
    return out[:, :NW]


def test_bf16_split_is_exact_and_six_products_reach_fp32_accuracy():
    """The output layer's arithmetic, restated in numpy: each fp32 operand split exactly into three bf16 parts, the
    six leading partial products summed.  Against a float64 dot product the error must be at the level of an fp32
    dot product; dropping one of the six (a planted mistake) must show up."""
    rng = np.random.default_rng(5)
    a = (rng.normal(size=(200, 64)) * np.exp(rng.normal(size=(200, 64)))).astype(np.float32)
    b = rng.normal(size=(64,)).astype(np.float32)
    pa, pb = radial.bf16_split3(a), radial.bf16_split3(b)
    assert np.array_equal(_bf16(pa[0]) + _bf16(pa[1]) + _bf16(pa[2]), a)
    for x in pa:        # every part is a bf16 value: no bits below the top 16
        assert x.dtype == np.uint16
    exact = a.astype(np.float64) @ b.astype(np.float64)
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)

    def dot(pairs):
        return sum(_bf16(pa[i]).astype(np.float64) @ _bf16(pb[j]).astype(np.float64) for i, j in pairs)
    six = [(0, 0), (0, 1), (1, 0), (0, 2), (1, 1), (2, 0)]
    assert (np.abs(dot(six) - exact) / scale).max() < 2 ** -22
    assert (np.abs(dot(six[:3] + six[4:]) - exact) / scale).max() > 2 ** -20      # hi*lo dropped


def test_unsupported_networks_are_refused():
    assert not radial.mlp_supported(enn.FullyConnectedNet([8, 64, 100], torch.nn.functional.silu))[0]   # output
    assert not radial.mlp_supported(enn.FullyConnectedNet([8, 40, 128], torch.nn.functional.silu))[0]   # hidden
    assert not radial.mlp_supported(enn.FullyConnectedNet([8, 48, 128], torch.nn.functional.silu))[0]   # last hidden
    assert radial.mlp_supported(enn.FullyConnectedNet([8, 64, 144], torch.nn.functional.silu))[0]       # 16 mod 32
    assert not radial.mlp_supported(enn.FullyConnectedNet([8, 64, 128], torch.tanh))[0]                 # activation
    assert not radial.mlp_supported(enn.FullyConnectedNet([8, 128]))[0]                                 # no hidden
    assert radial.mlp_supported(enn.FullyConnectedNet([8, 64, 64, 128], torch.nn.functional.silu))[0]


def test_mismatched_module_is_rejected():
    """A planted mistake: a network whose forward is not the stack of its layers."""
    class Scaled(enn.FullyConnectedNet):
        def forward(self, x):
            return 1.001 * super().forward(x)
    with pytest.raises(ValueError, match='does not match'):
        radial.MLPSpec(Scaled([8, 64, 64, 128], torch.nn.functional.silu))


@pytest.mark.parametrize('widths', [[8, 64, 64, 64, 1280], [8, 64, 64, 144]])
def test_generated_source_compiles(widths):
    from mace_hip_kernels import _native
    spec = radial.MLPSpec(enn.FullyConnectedNet(widths, torch.nn.functional.silu))
    assert len(_native.compile_source(radial.source(spec))) > 1000


def test_fused_output_layer_packing():
    """The fused convolution's two packings of the MLP's output layer A [HL, NINS·MUL] (conv_mlp.FusedSpec.pack_fwd,
    conv_mlp.pack_bwd): summing the three bf16 parts at every documented (lane, position) gives float32(A) back
    exactly (forward: K position 8 q + t of step s is hidden feature 32 s + 16 (t / 4) + 4 q + t % 4), every element of
    A appears (forward) and the padding of an odd instruction count is zero (backward)."""
    from mace_hip_kernels import conv as hconv, conv_mlp, radial
    from mace_lite import factory
    for hidden, lmax in (('128x0e+128x1o', 3), ('32x0e+32x1o', 2)):
        m = factory.make_model(hidden, lmax, 3, elements=factory.ELEMENTS_PTCOH)
        for blk in m.interactions:
            cs, ms = hconv.ConvSpec(blk.conv_tp), radial.MLPSpec(blk.conv_tp_weights)
            fs = conv_mlp.FusedSpec(cs, ms)
            A = np.asarray(ms.A[-1], dtype=np.float32).astype(np.float64)
            HL, mul, nk = fs.HL, cs.mul, len(fs.korder)

            def val(parts_u16):
                return sum((p.astype(np.uint32) << 16).view(np.float32).astype(np.float64) for p in parts_u16)
            f = fs.pack_fwd().reshape(fs.nct, nk, fs.S, 3, 64, 8)
            seen = np.zeros_like(A, dtype=bool)
            for ct in range(fs.nct):
                for ki, k in enumerate(fs.korder):
                    for s in range(fs.S):
                        for lane in range(64):
                            q, i16 = divmod(lane, 16)
                            rows = 32 * s + 16 * (np.arange(8) // 4) + 4 * q + np.arange(8) % 4
                            col = k * mul + 16 * ct + i16
                            got = val([f[ct, ki, s, p, lane] for p in range(3)])
                            assert np.array_equal(got, A[rows, col])
                            seen[rows, col] = True
            assert seen.all()
            b = conv_mlp.pack_bwd(fs).reshape(fs.nct, (nk + 1) // 2, 3, HL // 16, 64, 8)
            for ct in range(fs.nct):
                for kp in range((nk + 1) // 2):
                    for mt in range(HL // 16):
                        for lane in range(64):
                            q, i16 = divmod(lane, 16)
                            got = val([b[ct, kp, p, mt, lane] for p in range(3)])
                            for t in range(2):
                                ki = 2 * kp + t
                                want = (A[16 * mt + i16, fs.korder[ki] * mul + 16 * ct + 4 * q + np.arange(4)]
                                        if ki < nk else np.zeros(4))
                                assert np.array_equal(got[4 * t:4 * t + 4], want)


def _kernel_params(src, name):
    """Parameter names of the generated kernel ``name`` (in order)."""
    i = src.index(f'void {name}(')
    sig = src[i + len(name) + 6:src.index(')', i)]
    return [p.strip().split()[-1].lstrip('*') for p in sig.split(',')]


def _launcher_args(fn, array='args'):
    """Argument names, in order, of the kernel-argument array ``array`` of the C entry point ``fn`` in
    csrc/mace_hip.cpp."""
    import os
    import re
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    cpp = open(os.path.join(root, 'mace-mps-kernels_amd', 'csrc', 'mace_hip.cpp')).read()
    i = cpp.index(f'\nint {fn}(')
    body = cpp[i:cpp.index('\n}\n', i)]
    return re.findall(r'&(\w+)', re.search(r'void\* ' + array + r'\[\] = \{([^}]*)\}', body).group(1))


def test_kernel_parameters_follow_the_launchers_arguments():
    """Every radial-MLP entry point passes its kernel arguments in the order of the generated kernel's parameters
    (names as in the C source; gW0 is the kernels' gW, W0's WhT / Wh / Wl the weight buffers in order)."""
    spec = radial.MLPSpec(factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
                          .interactions[1].conv_tp_weights)
    src = radial.source(spec)
    alias = {'gW0': 'gW'}
    for fn, kern in (('mh_mlp_fwd_rows', 'mlp_fwd'), ('mh_mlp_bwd_rows', 'mlp_bwd'), ('mh_mlp_bwd_pairs', 'mlp_bwdp')):
        got = [alias.get(a, a) for a in _launcher_args(fn)]
        want = _kernel_params(src, spec.kname(kern))
        assert len(got) == len(want), (fn, got, want)
        for g, w in zip(got, want):
            assert g == w or {g, w} <= {'Wh', 'WhT', 'Wl'}, (fn, got, want)


def test_edge_pair_parameters_follow_the_launcher():
    """mh_edge_pairs passes edge_pair's arguments in the kernel's parameter order (cutoff is the kernel's cut)."""
    from mace_hip_kernels import conv
    got = [{'cutoff': 'cut'}.get(a, a) for a in _launcher_args('mh_edge_pairs', 'a0')]
    assert got == _kernel_params(conv.graph_source(), 'edge_pair'), got
