"""MFMA scoring vs a float64 contraction of the same bf16 operands."""
import pytest
import torch

from glsdm.memory.backends import hip

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,T,H,dk,half", [(2, 512, 1, 64, 64), (2, 100, 8, 128, 256), (1, 70, 2, 32, 32),
                                           (1, 64, 1, 128, 1024)])
def test_score_matches_float64(device, B, T, H, dk, half):
    g = torch.Generator().manual_seed(B * T + half)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, dk, generator=g), dim=-1).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(H, 2 * half, dk, generator=g), dim=-1).bfloat16()
    out = hip.score(q.to(device), k.to(device)).cpu()
    ref = torch.einsum("bthe,hce->bthc", q.double(), k.double())
    torch.testing.assert_close(out.double(), ref, atol=1e-5, rtol=1e-5)
