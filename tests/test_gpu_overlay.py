"""Overlay snapshots (shared base + per-request touched rows) vs the dense
replicated bank: reads, commits and the materialised bank are bitwise equal
after every commit of a sequence (keyed and unkeyed, collisions, dropped
out-of-range addresses, fp32 and bf16), including across pool growth."""
import pytest
import torch

from glsdm.memory import OverlayView
from glsdm.memory.backends import hip
from oracle import torch_oracle
from _util import gen

pytestmark = pytest.mark.gpu


def _routes(g, B, T, H, S, width):
    index = torch.stack([torch.randperm(S, generator=g)[:width].sort().values for _ in range(B * T * H)])
    weights = torch.randn(B * T * H, width, generator=g).softmax(-1)
    return index.view(B, T, H, width), weights.view(B, T, H, width)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("keyed", [False, True])
def test_overlay_matches_dense_over_commits(device, dtype, keyed):
    B, H, S, D, T, width = 3, 2, 256, 64, 40, 8
    g = gen(21)
    base = (torch.randn(H, S, D, generator=g) * 0.1).to(dtype).to(device)
    dense = base.unsqueeze(0).expand(B, -1, -1, -1).contiguous()
    ov = OverlayView.from_base(base, B, capacity=64)            # small: forces growth
    base_before = base.cpu()
    ref_bank = base.cpu().float().unsqueeze(0).expand(B, -1, -1, -1).reshape(-1, D)   # oracle's bank, fp32
    touched = set()
    for step in range(4):
        idx, w = _routes(g, B, T, H, S, width)
        ref_read = torch_oracle.read(ref_bank.view(B, H, S, D), idx, w)
        idx, w = idx.to(device), w.to(device)
        got = ov.read(idx, w)
        assert torch.equal(got, hip.snapshot_read(dense, idx, w))
        tol = dict(atol=1e-6, rtol=1e-5) if dtype == torch.float32 else dict(atol=1e-5, rtol=2e-2)
        torch.testing.assert_close(got.cpu(), ref_read, **tol)
        E = 700
        addr = torch.randint(0, B * H * S // 4, (E,), generator=g)        # collisions
        addr[::97] = B * H * S + 5                                         # dropped
        delta = (torch.randn(E, D, generator=g) * 0.01).to(dtype)
        keys = addr * (E + 1) + torch.randperm(E, generator=g) if keyed else None
        touched.update(a for a in addr.tolist() if a < B * H * S)
        ref = torch_oracle.commit(ref_bank, addr[addr < B * H * S], delta[addr < B * H * S].float(),
                                  None if keys is None else keys[addr < B * H * S])
        ref_bank = ref if dtype == torch.float32 else ref.bfloat16().float()   # bf16: one rounding per commit
        addr, delta = addr.to(device), delta.to(device)
        keys = None if keys is None else keys.to(device)
        dense = hip.commit(dense, addr, delta, keys)
        ov.commit(addr, delta, keys)
        assert ov.version == step + 1
        assert torch.equal(ov.materialise(), dense)
        assert torch.equal(ov.materialise().cpu().float().reshape(-1, D), ref_bank)
    assert ov.mapped_rows() == len(touched)                                # one pool row per touched row
    assert ov.pool.shape[0] >= ov.pool_rows() == 4 * 700 > 64              # reserved per commit; the pool grew
    assert torch.equal(base.cpu(), base_before)                            # the base is never written


def test_overlay_used_rows_and_copy(device):
    B, H, S, D = 2, 1, 64, 16
    base = torch.randn(H, S, D, generator=gen(22)).to(device)
    ov = OverlayView.from_base(base, B, capacity=8)
    addr = torch.tensor([3, 3, 70, 5, 3, 127], device=device)            # 4 distinct rows of 128
    delta = torch.ones(6, D, device=device)
    ov.commit(addr, delta)
    assert ov.mapped_rows() == 4 and ov.pool_rows() == 6
    twin = ov.copy()
    ov.commit(torch.tensor([3], device=device), torch.ones(1, D, device=device))
    dense = twin.materialise()
    row3 = base[0, 3].cpu()
    assert torch.equal(dense.reshape(-1, D)[3].cpu(), row3 + torch.full((D,), 3.0))     # fp32: old + (1+1+1)
    assert torch.equal(ov.materialise().reshape(-1, D)[3].cpu(), (row3 + 3.0) + 1.0)    # second commit on top
    assert torch.equal(dense.reshape(-1, D)[0], base[0, 0])                # untouched: the base row


def test_overlay_routed_read(device):
    B, H, half, D, T, width = 2, 2, 16, 32, 24, 8
    g = gen(23)
    base = torch.randn(H, half * half, D, generator=g).to(device)
    ov = OverlayView.from_base(base, B)
    scores = torch.randn(B, T, H, 2 * half, generator=g).to(device)
    out, idx, w = ov.routed_read(scores, width)
    dense = base.unsqueeze(0).expand(B, -1, -1, -1).contiguous()
    ref, ridx, rw = hip.routed_snapshot_read(dense, scores, width)
    assert torch.equal(idx, ridx) and torch.equal(w, rw) and torch.equal(out, ref)
    # against the oracle on the materialised bank (routing.py:10-28)
    o_out, o_idx, o_w = torch_oracle.routed_read(ov.materialise().cpu(), scores.cpu(), width)
    assert torch.equal(idx.cpu(), o_idx)
    torch.testing.assert_close(w.cpu(), o_w, atol=2e-7, rtol=2e-6)
    torch.testing.assert_close(out.cpu(), o_out, atol=1e-6, rtol=1e-5)
