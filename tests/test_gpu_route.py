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


def _route_raw(scores, width, tie, workspace):
    """glsdm_route through the C ABI, with or without the split path's workspace."""
    from glsdm import _native as N
    rows, L = scores.numel() // scores.shape[-1], scores.shape[-1]
    index = torch.empty(rows, width, dtype=torch.int64, device=scores.device)
    weights = torch.empty(rows, width, dtype=torch.float32, device=scores.device)
    ws = hip.route_workspace(rows, L // 2, width, scores.device) if workspace else None
    N.call("glsdm_route", N.ptr(scores), N.dtype_code(scores), rows, L // 2, width, N.TIES[tie], N.ptr(index),
           N.ptr(weights), N.ptr(ws), 0 if ws is None else ws.numel(), N.stream(scores.device))
    return index, weights


def _bf16_rows(kind, rows, L, seed):
    s = route_scores("randn" if kind in ("nan", "specials") else kind, (rows, L), seed=seed).bfloat16()
    if kind == "nan":
        s[::3, 5 % L] = float("nan")
    if kind == "specials":
        s[::4] = 0.0
        s[1::4, ::2] = -0.0
        s[2::5, 0] = float("inf")
        s[3::7, -1] = float("-inf")
    return s


@pytest.mark.parametrize("tie", ["highest", "lowest"])
@pytest.mark.parametrize("kind", ["randn", "floor", "zeros", "specials", "nan"])
@pytest.mark.parametrize("rows,half,width", [(64, 4, 4), (300, 64, 16), (70, 256, 16), (1024, 1024, 16),
                                             (33, 512, 8), (20, 100, 2), (17, 300, 64), (96, 1024, 32),
                                             (5000, 256, 16), (20000, 64, 16)])
def test_route_bf16_scores_equal_their_fp32_widening(device, tie, kind, rows, half, width):
    """bf16 scores (32-bit keys) route bit for bit as the same values widened to
    fp32 (64-bit keys), which the oracle pins."""
    s16 = _bf16_rows(kind, rows, 2 * half, seed=rows + half + width).to(device)
    idx, w = hip.route(s16, width, tie)
    fidx, fw = hip.route(s16.float(), width, tie)
    assert torch.equal(idx, fidx)
    torch.testing.assert_close(w, fw, atol=0, rtol=0, equal_nan=True)
    if kind != "nan":
        ridx, rw = torch_oracle.route(s16.cpu().float(), width, tie)
        assert torch.equal(idx.cpu(), ridx)
        torch.testing.assert_close(w.cpu(), rw, atol=2e-7, rtol=2e-6, equal_nan=True)   # inf rows: NaN weights


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind", ["randn", "floor", "mixed"])
@pytest.mark.parametrize("rows,half,width", [(1024, 1024, 16), (1, 1024, 16), (64, 512, 8), (200, 256, 32),
                                             (7, 2048, 64), (100, 300, 4), (3, 65, 1)])
def test_route_split_path_equals_single_kernel(device, dtype, kind, rows, half, width):
    """Few rows: the column-range split (part lists + merge) gives the single
    kernel's results bit for bit."""
    s = route_scores(kind, (rows, 2 * half), seed=rows * 3 + half).to(dtype).to(device)
    a_idx, a_w = _route_raw(s, width, "highest", workspace=True)
    b_idx, b_w = _route_raw(s, width, "highest", workspace=False)
    assert torch.equal(a_idx, b_idx)
    torch.testing.assert_close(a_w, b_w, atol=0, rtol=0, equal_nan=True)
    ridx, _ = torch_oracle.route(s.cpu().float(), width, "highest")
    assert torch.equal(a_idx.cpu(), ridx)
