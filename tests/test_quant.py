"""The product's torch quantizers agree bit for bit with the oracle's numpy
restatement (CPU tensors)."""

import numpy as np
import pytest
import torch

from gfx950_gluon_tutorials_amd import quant as Q
from oracle import gemm_ref as R


@pytest.mark.parametrize("seed,shape,scale", [(3, (64, 1024), 1.0), (5, (33, 256), 1e-3), (7, (8, 4096), 300.0)])
def test_mxfp4_matches_oracle(seed, shape, scale):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g) * scale
    x[0, :32] = 0.0
    x[1, :32] = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.0] * 4)
    x[2, :32] = -x[1, :32]
    p, s = Q.quantize_mxfp4(x)
    po, so = R.quant_mxfp4(x.numpy())
    np.testing.assert_array_equal(p.numpy(), po)
    np.testing.assert_array_equal(s.numpy(), so)
    np.testing.assert_array_equal(Q.dequantize_mxfp4(p, s).numpy(), R.mxfp4_dequant(po, so))


@pytest.mark.parametrize("seed,scale", [(2, 1.0), (9, 1e-4), (11, 1e3)])
def test_e5m2_matches_oracle(seed, scale):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(128, 512, generator=g) * scale
    q, s = Q.quantize_e5m2(x)
    qo, so = R.quant_e5m2_per_tensor(x.numpy())
    np.testing.assert_array_equal(q.view(torch.uint8).numpy(), qo)
    assert float(s) == float(so)


def test_mxfp4_rejects_ragged_k():
    with pytest.raises(ValueError):
        Q.quantize_mxfp4(torch.zeros(4, 40))
