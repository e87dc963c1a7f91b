"""The glsdm.memory mirror end to end at the config-1 shape (B=2, T=512, M=4096,
dk=64, D=256, k=8, one head, fp32): scores -> routed read -> proposal keys ->
merge -> commit, each step compared with the CPU oracle on identical inputs."""
import pytest
import torch

from oracle import c_oracle, torch_oracle
from glsdm.memory import MemoryView, WriteProposal, merge, commit
from glsdm.memory import routing
from glsdm.memory.backends import hip

pytestmark = pytest.mark.gpu


class _Attn:
    backend, reference = "hip", False


class _Block:
    attn = _Attn()


def _config1(seed=0):
    g = torch.Generator("cpu").manual_seed(seed)
    B, T, H, half, dk, D, k = 2, 512, 1, 64, 64, 256, 8
    keys = torch.nn.functional.normalize(torch.randn(H, 2 * half, dk, generator=g), dim=-1)
    bank = torch.randn(H, half * half, D, generator=g) * 0.02
    qr = torch.randn(B, T, H, dk, generator=g)
    qw = torch.randn(B, T, H, dk, generator=g)
    delta = torch.randn(B, T, H, k, D, generator=g) * 0.02
    return dict(B=B, T=T, H=H, half=half, dk=dk, D=D, k=k, keys=keys, bank=bank, qr=qr, qw=qw, delta=delta)


def test_config1_pipeline(device):
    c = _config1()
    values = c["bank"].unsqueeze(0).expand(c["B"], -1, -1, -1).contiguous()
    view = MemoryView(values.to(device))
    scores = torch.einsum("bthe,hce->bthc", c["qr"], c["keys"])       # fp32 factor scores on the CPU
    out, idx, w = routing.routed_read(_Block(), view.values, scores.to(device), c["k"])
    ref_out, ref_idx, ref_w = torch_oracle.routed_read(values, scores, c["k"])
    assert torch.equal(idx.cpu(), ref_idx)
    torch.testing.assert_close(w.cpu(), ref_w, atol=2e-7, rtol=2e-6)
    torch.testing.assert_close(out.cpu(), ref_out, atol=1e-6, rtol=1e-5)

    wscores = torch.einsum("bthe,hce->bthc", c["qw"], c["keys"])
    _, widx, _ = routing.routed_read(_Block(), view.values, wscores.to(device), c["k"])
    ridx, _ = torch_oracle.route(wscores, c["k"])
    assert torch.equal(widx.cpu(), ridx)
    addr, keys = hip.proposal_keys(view.values, widx, 0, 512, 1, 0)
    p = WriteProposal(view.version, addr.reshape(-1), c["delta"].reshape(-1, c["D"]).to(device), view.lineage,
                      keys.reshape(-1))
    new = commit(view, merge(view, [p]))
    raddr = torch_oracle.absolute_addresses(values, ridx).reshape(-1)
    rkeys = raddr * 512 + torch.arange(512).view(1, 512, 1, 1).expand(2, 512, 1, 8).reshape(-1)
    ref_bank = torch_oracle.commit(values.reshape(-1, c["D"]), raddr, c["delta"].reshape(-1, c["D"]), rkeys)
    assert torch.equal(new.values.cpu().reshape(-1, c["D"]), ref_bank)
    assert new.version == 1
    assert torch.equal(view.values.cpu(), values)         # snapshot frozen
    donated = commit(view, merge(view, [p]), donate=True)
    assert torch.equal(donated.values, new.values) and donated.values.data_ptr() == view.values.data_ptr()


def test_five_dim_scores(device):
    g = torch.Generator().manual_seed(1)
    mem = torch.randn(2, 2, 16, 8, generator=g)
    scores = torch.randn(2, 3, 17, 2, 8, generator=g)
    out, idx, w = routing.routed_read(_Block(), mem.to(device), scores.to(device), 2)
    r_out, r_idx, r_w = torch_oracle.routed_read(mem, scores, 2)
    assert out.shape == (2, 3, 17, 2, 8) and torch.equal(idx.cpu(), r_idx)
    torch.testing.assert_close(out.cpu(), r_out, atol=1e-6, rtol=1e-5)


def test_scored_route_is_bit_exact_on_exported_scores(device):
    """The MFMA scores are exported; routing them on the GPU equals the oracle on the same scores."""
    g = torch.Generator().manual_seed(2)
    q = torch.nn.functional.normalize(torch.randn(2, 256, 8, 128, generator=g), dim=-1).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(8, 512, 128, generator=g), dim=-1).bfloat16()
    s = hip.score(q.to(device), k.to(device))
    idx, w = hip.route(s, 16, "highest")
    ridx, rw = c_oracle.route(s.cpu(), 16, "highest")
    assert torch.equal(idx.cpu(), ridx)
    torch.testing.assert_close(w.cpu(), rw, atol=2e-7, rtol=2e-6)
