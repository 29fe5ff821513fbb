"""Host-side pieces of the phi backward (nsa_hip_ops): the weight gradient
dW1 from shifted chunk views of the sequence and the split tall product,
against their direct forms on the CPU (float64)."""

import pytest
import torch

import nsa_hip_ops as ops


@pytest.mark.parametrize("shape", [(1, 4, 300, 64, 32, 16, 32), (2, 2, 200, 64, 16, 16, 64),
                                   (1, 2, 257, 64, 48, 16, 32), (1, 3, 130, 64, 24, 16, 32),
                                   (1, 1, 32, 64, 32, 16, 32)],
                         ids=["l2d", "l=d", "l3d", "l-not-multiple", "one-span"])
def test_phi_dw1_matches_unfolded_spans(shape):
    B, H, T, D, l, d, Hd = shape
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, H, T, D, generator=g, dtype=torch.float64)
    n = (T - l) // d + 1
    dpre = torch.randn(B * H * n, Hd, generator=g, dtype=torch.float64)
    spans = x.as_strided((B * H, n, l * D), (T * D, d * D, 1)).reshape(B * H * n, l * D)
    torch.testing.assert_close(ops._phi_dw1(x, dpre, B * H, n, l, d), dpre.t() @ spans, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("M", [1, 15, 16, 1001])
def test_sum_of_products_matches_direct(M):
    g = torch.Generator().manual_seed(1)
    a = torch.randn(M, 64, generator=g, dtype=torch.float64)
    b = torch.randn(M, 32, generator=g, dtype=torch.float64)
    torch.testing.assert_close(ops._sum_of_products(a, b), a.t() @ b, rtol=1e-12, atol=1e-12)
