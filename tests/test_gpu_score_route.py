"""Fused MFMA scoring + route: the route is bit-exact against the oracle on the
exported scores, the exported scores match a float64 contraction, and the
result does not depend on whether scores are exported, nor on whether small
launches take the split path (per-range partial lists in a workspace, then a
merge kernel) or the single kernel."""
import pytest
import torch

from oracle import c_oracle, torch_oracle
from glsdm.memory.backends import hip

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, dk, half, seed, clusters=False):
    g = torch.Generator().manual_seed(seed)
    norm = torch.nn.functional.normalize
    k = norm(torch.randn(H, 2 * half, dk, generator=g), dim=-1)
    if clusters:   # near-duplicate sub-keys: many close and equal scores
        k = norm(k[:, :4].repeat(1, half // 2, 1) + 1e-3 * torch.randn(H, 2 * half, dk, generator=g), dim=-1)
    q = norm(torch.randn(B, T, H, dk, generator=g), dim=-1)
    return q.bfloat16(), k.bfloat16()


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("tie", ["highest", "lowest"])
@pytest.mark.parametrize("B,T,H,dk,half,width", [
    (8, 64, 8, 128, 256, 16),      # config 2 geometry
    (2, 100, 1, 64, 64, 8),        # config 1 geometry, ragged token count
    (1, 40, 1, 128, 1024, 32),     # config 3 geometry
    (2, 17, 2, 32, 16, 4), (1, 33, 3, 96, 48, 5), (1, 20, 1, 256, 32, 64), (1, 9, 2, 64, 16, 1),
    (1, 18, 2, 64, 32, 2), (1, 70, 1, 128, 512, 8),
])
def test_fused_route_matches_oracle_on_exported_scores(device, split, tie, B, T, H, dk, half, width):
    q, k = _inputs(B, T, H, dk, half, seed=B * T + half + width)
    idx, w, scores = hip.score_route(q.to(device), k.to(device), width, tie, export_scores=True, split=split)
    ref = torch.einsum("bthe,hce->bthc", q.double(), k.double())
    torch.testing.assert_close(scores.cpu().double(), ref, atol=1e-5, rtol=1e-5)
    ridx, rw = c_oracle.route(scores.cpu(), width, tie)
    assert torch.equal(idx.cpu(), ridx)
    torch.testing.assert_close(w.cpu(), rw, atol=2e-7, rtol=2e-6)
    idx2, w2, none = hip.score_route(q.to(device), k.to(device), width, tie, split=not split)
    assert none is None and torch.equal(idx2, idx) and torch.equal(w2, w)


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("tie", ["highest", "lowest"])
def test_fused_route_with_duplicate_subkeys(device, split, tie):
    q, k = _inputs(2, 64, 2, 64, 64, seed=5, clusters=True)
    idx, w, scores = hip.score_route(q.to(device), k.to(device), 16, tie, export_scores=True, split=split)
    ridx, rw = torch_oracle.route(scores.cpu(), 16, tie)
    assert torch.equal(idx.cpu(), ridx)
    torch.testing.assert_close(w.cpu(), rw, atol=2e-7, rtol=2e-6)


def test_fused_route_equals_unfused(device):
    q, k = _inputs(4, 128, 8, 128, 256, seed=9)
    idx, w, _ = hip.score_route(q.to(device), k.to(device), 16)
    s = hip.score(q.to(device), k.to(device))
    idx2, w2 = hip.route(s, 16, "highest")
    assert torch.equal(idx, idx2) and torch.equal(w, w2)


def test_split_plan_uses_workspace_only_for_small_launches():
    assert hip.score_route_workspace_bytes(8, 512, 8, 256, 16) == 0           # config 2: 512 blocks already
    need = hip.score_route_workspace_bytes(4, 512, 1, 1024, 32)               # config 3: 64 blocks
    assert need > 0 and need % (4 * 512 * 2 * 32 * 8) == 0


@pytest.mark.parametrize("tie", ["highest", "lowest"])
def test_split_route_config3_epoch(device, tie):
    """A full config-3 epoch (B=4, 512 tokens, one head, 1024 sub-keys per factor,
    k=32) on the split path equals the single kernel and the oracle."""
    q, k = _inputs(4, 512, 1, 128, 1024, seed=31)
    idx, w, scores = hip.score_route(q.to(device), k.to(device), 32, tie, export_scores=True)
    idx1, w1, _ = hip.score_route(q.to(device), k.to(device), 32, tie, split=False)
    assert torch.equal(idx, idx1) and torch.equal(w, w1)
    ridx, rw = c_oracle.route(scores.cpu(), 32, tie)
    assert torch.equal(idx.cpu(), ridx)
    torch.testing.assert_close(w.cpu(), rw, atol=2e-7, rtol=2e-6)


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("B,T,H,half,width,offset,chunk,layers,layer", [
    (8, 512, 8, 256, 16, 0, 512, 1, 0), (2, 100, 3, 64, 8, 37, 512, 16, 6), (4, 512, 1, 1024, 32, 0, 512, 2, 1),
    (1, 33, 2, 128, 64, 480, 512, 8, 7),
])
def test_score_route_keys_equals_route_then_keys(device, split, B, T, H, half, width, offset, chunk, layers, layer):
    """glsdm_score_route_keys = glsdm_score_route + glsdm_proposal_keys, bit for bit
    (both the single kernel and the split path)."""
    q, k = _inputs(B, T, H, 128, half, seed=T + half + width)
    qd, kd = q.to(device), k.to(device)
    idx, w, addr, keys = hip.score_route_keys(qd, kd, width, offset, chunk, layers, layer, split=split)
    ridx, rw, _ = hip.score_route(qd, kd, width, split=split)
    assert torch.equal(idx, ridx) and torch.equal(w, rw)
    bank = torch.empty(B, H, half * half, 1, device=device)
    raddr, rkeys = hip.proposal_keys(bank, ridx, offset, chunk, layers, layer)
    assert torch.equal(addr, raddr) and torch.equal(keys, rkeys)
    pos = torch.arange(offset, offset + T, device=device).view(1, T, 1, 1)
    assert torch.equal(keys, addr * (chunk * layers) + pos * layers + layer)


def _check_filtered(device, q, k, width, tie):
    """The filtered K = 16 kernel (taken without score export) against the
    unfiltered kernel's exported scores and the oracle routing them."""
    qd, kd = q.to(device), k.to(device)
    idx, w, none = hip.score_route(qd, kd, width, tie, split=False)
    assert none is None
    ridx, rw, scores = hip.score_route(qd, kd, width, tie, export_scores=True, split=False)
    assert torch.equal(idx, ridx)
    torch.testing.assert_close(w, rw, atol=0, rtol=0, equal_nan=True)     # bitwise; NaN rows stay NaN
    oidx, ow = c_oracle.route(scores.cpu(), width, tie)
    assert torch.equal(idx.cpu(), oidx)
    torch.testing.assert_close(w.cpu(), ow, atol=2e-7, rtol=2e-6, equal_nan=True)


@pytest.mark.parametrize("tie", ["highest", "lowest"])
@pytest.mark.parametrize("B,T,H,dk,half,width", [
    (8, 512, 8, 128, 256, 16),     # config 2's epoch
    (1, 77, 3, 64, 64, 9),         # one chunk per factor, ragged tokens
    (2, 45, 2, 256, 128, 12),
    (2, 33, 1, 64, 128, 16),       # two chunks per factor, scores held in registers
    (1, 100, 2, 128, 192, 16),     # three chunks per factor, scores held in registers
    (1, 130, 1, 128, 320, 16),     # five chunks: a partial group of maxima
    (1, 64, 2, 64, 512, 15),
])
def test_filtered_route_matches_unfiltered_and_oracle(device, tie, B, T, H, dk, half, width):
    q, k = _inputs(B, T, H, dk, half, seed=3 * T + half + width + dk)
    _check_filtered(device, q, k, width, tie)


@pytest.mark.parametrize("tie", ["highest", "lowest"])
def test_filtered_route_overflow_falls_back_exactly(device, tie):
    """Near-duplicate sub-keys (many equal and close scores), zero queries (every
    score ties) and a block mixing both with ordinary tokens: tokens whose
    survivors overflow the buffer make the block select unfiltered."""
    q, k = _inputs(2, 96, 2, 128, 256, seed=41, clusters=True)
    _check_filtered(device, q, k, 16, tie)
    q, k = _inputs(1, 64, 1, 128, 256, seed=42)
    _check_filtered(device, torch.zeros_like(q), k, 16, tie)
    q[0, 10:20] = 0
    _check_filtered(device, q, k, 16, tie)


def test_filtered_route_non_finite_rows(device):
    """Rows whose queries hold NaN (every score NaN) or huge values (infinite
    scores) route as the unfiltered kernel and the oracle do (NaN ranks highest)."""
    q, k = _inputs(1, 70, 2, 128, 256, seed=43)
    q = q.float()
    q[0, 3, 0, 5] = float("nan")
    q[0, 7, 1] *= 1e38
    q[0, 9, 0, :4] = float("inf")
    _check_filtered(device, q.bfloat16(), k, 16, "highest")
