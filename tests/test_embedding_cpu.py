"""
Host side of the radial-embedding drop-in (mace_hip_kernels.embedding), on the CPU: the restated formulas against the
module in float64, refusal of other embeddings, and the generated HIP source compiling for gfx950.
"""
import numpy as np
import pytest
import torch

from mace_hip_kernels import embedding
from mace_lite import blocks, factory


def test_restated_formulas_match_the_module():
    m = factory.make_model('128x0e+128x1o', 3, 3, elements=factory.ELEMENTS_PTCOH)
    spec = embedding.EmbSpec(m.radial_embedding)
    r = np.linspace(0.2, 7.0, 301).reshape(-1, 1)
    with torch.no_grad():
        f, c = m.radial_embedding.double()(torch.tensor(r))
    ff, cc = spec.apply(r)
    assert np.abs(ff - f.numpy()).max() < 1e-12 and np.abs(cc - c.numpy()).max() < 1e-12
    assert (cc[r[:, 0] >= spec.r_max] == 0).all()


def test_other_embeddings_are_refused():
    class Gaussian(torch.nn.Module):
        pass
    mod = blocks.RadialEmbeddingBlock(5.0, 8, 5)
    mod.bessel_fn = Gaussian()
    assert not embedding.emb_supported(mod)[0]


def test_mismatched_module_is_rejected():
    """A planted mistake: an embedding whose forward is not Bessel x envelope."""
    class Off(blocks.RadialEmbeddingBlock):
        def forward(self, x):
            f, c = super().forward(x)
            return f * 1.0001, c
    with pytest.raises(ValueError, match='does not match'):
        embedding.EmbSpec(Off(5.0, 8, 5))


def test_generated_source_compiles():
    from mace_hip_kernels import _native
    spec = embedding.EmbSpec(blocks.RadialEmbeddingBlock(5.0, 8, 6))
    assert len(_native.compile_source(embedding.source(spec))) > 1000
