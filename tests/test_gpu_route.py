"""HIP route vs the CPU oracle: indices bit-exact for both tie rules, weights
within the reference's route tolerance (P/tests/test_layer_stack.py:170-172)."""
import pytest
import torch

from oracle import c_oracle, torch_oracle
from glsdm.memory.backends import hip
from _util import known_answers, route_scores

pytestmark = pytest.mark.gpu

SHAPES = [  # (rows, half, width)
    (37, 1, 1), (64, 4, 4), (64, 3, 5), (48, 8, 64), (40, 64, 8), (300, 64, 16),
    (513, 256, 16), (200, 256, 8), (96, 1024, 32), (50, 512, 8), (33, 7, 3), (20, 100, 2), (17, 300, 64),
]


@pytest.mark.parametrize("tie", ["highest", "lowest"])
@pytest.mark.parametrize("kind", ["randn", "bf16", "mixed"])
@pytest.mark.parametrize("rows,half,width", SHAPES)
def test_route_matches_oracle(device, tie, kind, rows, half, width):
    s = route_scores(kind, (rows, 2 * half), seed=rows * 7 + half + width)
    idx, w = hip.route(s.to(device), width, tie)
    ridx, rw = c_oracle.route(s, width, tie)
    assert torch.equal(idx.cpu(), ridx)
    torch.testing.assert_close(w.cpu(), rw, atol=2e-7, rtol=2e-6, equal_nan=True)


@pytest.mark.parametrize("tie", ["highest", "lowest"])
@pytest.mark.parametrize("kind", ["floor", "zeros", "signed_zero"])
@pytest.mark.parametrize("rows,half,width", [(64, 4, 4), (64, 3, 5), (40, 64, 8), (70, 256, 16), (9, 1024, 32)])
def test_route_ties_match_oracle(device, tie, kind, rows, half, width):
    s = route_scores(kind, (rows, 2 * half), seed=half + width)
    idx, w = hip.route(s.to(device), width, tie)
    ridx, rw = torch_oracle.route(s, width, tie)
    assert torch.equal(idx.cpu(), ridx)
    torch.testing.assert_close(w.cpu(), rw, atol=2e-7, rtol=2e-6)


def test_route_known_answers(device):
    ka = known_answers()
    c = ka["route_highest_zero_scores"]
    idx, w = hip.route(torch.zeros(c["scores_shape"], device=device), c["width"], "highest")
    assert (idx.cpu() == torch.tensor(c["expect_index_row"])).all()
    assert torch.equal(w.cpu(), torch.full_like(w.cpu(), 0.25))
    for half, count in ka["route_lowest_signed_zero"]["cases"]:
        s = torch.randn(3, 2, 2 * half, generator=torch.Generator().manual_seed(13))
        s[0].zero_()
        s[0, :, 0] = -0.0
        idx, _ = hip.route(s.to(device), count, "lowest")
        idx = idx.cpu()
        assert idx[0, 0].tolist() == list(range(count))
        assert (idx[..., 1:] > idx[..., :-1]).all()


def test_route_large_bank_zero_and_floored_rows(device):
    """P/tests/test_layer_stack.py:143-176 shapes: S = 262144 (half 512), width 8."""
    g = torch.Generator().manual_seed(7)
    s = torch.randn(1, 3, 1, 1024, generator=g)
    s[:, 0].zero_()
    s[:, 2].floor_()
    idx, w = hip.route(s.to(device), 8, "highest")
    ridx, rw = torch_oracle.route(s, 8, "highest")
    assert torch.equal(idx.cpu(), ridx)
    torch.testing.assert_close(w.cpu(), rw, atol=2e-7, rtol=2e-6)


def test_route_empty(device):
    idx, w = hip.route(torch.zeros(0, 16, device=device), 4)
    assert idx.shape == (0, 4) and w.shape == (0, 4)
