"""Backward of the HIP route, read and commit vs torch autograd through the CPU
oracle (the reference's torch ops), on the same inputs.

Route and read gradients are sums whose order differs from the reference's
reductions, so they are compared within fp32 tolerance: rtol 1e-5 and an
absolute 2e-6 of the gradient's largest magnitude (unit-normal banks make
the weights' gradients dot products of size ~sqrt(D), whose rounding
cancels into near-zero score gradients); the commit's delta gradient is a
pure gather and is bitwise.  The routes themselves are bit-exact, so both sides differentiate
the same chosen slots, tie-heavy rows included.
"""
import pytest
import torch

from oracle import torch_oracle
from glsdm.memory.backends import hip
from _util import gen, route_scores

pytestmark = pytest.mark.gpu

def close(got, ref):
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=2e-6 * max(1.0, ref.abs().max().item()))


@pytest.mark.parametrize("tie", ["highest", "lowest"])
@pytest.mark.parametrize("kind,rows,half,width", [
    ("randn", 300, 16, 8), ("randn", 64, 64, 16), ("floor", 97, 32, 16), ("randn", 40, 256, 32),
    ("zeros", 9, 8, 4), ("randn", 33, 8, 64), ("randn", 50, 5, 1),
])
def test_route_backward(device, tie, kind, rows, half, width):
    s = route_scores(kind, (rows, 2 * half), seed=rows + half)
    upstream = torch.randn(rows, width, generator=gen(3))
    ref_s = s.clone().requires_grad_()
    _, rw = torch_oracle.route(ref_s, width, tie)
    (rw * upstream).sum().backward()
    dev_s = s.to(device).requires_grad_()
    idx, w = hip.route(dev_s, width, tie)
    (w * upstream.to(device)).sum().backward()
    close(dev_s.grad.cpu(), ref_s.grad)
    assert idx.requires_grad is False


@pytest.mark.parametrize("tie", ["highest", "lowest"])
@pytest.mark.parametrize("B,T,H,half,D,width", [
    (2, 40, 2, 16, 64, 8), (1, 64, 1, 32, 256, 16), (2, 17, 3, 8, 37, 4), (1, 128, 2, 16, 128, 16),
])
def test_routed_read_backward(device, tie, B, T, H, half, D, width):
    S = half * half
    g = gen(B * T + D)
    bank = torch.randn(B, H, S, D, generator=g)
    scores = torch.randn(B, T, H, 2 * half, generator=g)
    go = torch.randn(B, T, H, D, generator=g)
    gw = torch.randn(B, T, H, width, generator=g)
    rb, rs = bank.clone().requires_grad_(), scores.clone().requires_grad_()
    out, ridx, rw = torch_oracle.routed_read(rb, rs, width, tie)
    ((out * go).sum() + (rw * gw).sum()).backward()
    db, ds = bank.to(device).requires_grad_(), scores.to(device).requires_grad_()
    dout, didx, dw = hip.routed_snapshot_read(db, ds, width, tie=tie)
    ((dout * go.to(device)).sum() + (dw * gw.to(device)).sum()).backward()
    assert torch.equal(didx.cpu(), ridx)
    close(db.grad.cpu(), rb.grad)
    close(ds.grad.cpu(), rs.grad)


def test_routed_read_backward_bank_only_and_scores_only(device):
    B, T, H, half, D, width = 2, 32, 2, 16, 64, 8
    g = gen(11)
    bank = torch.randn(B, H, half * half, D, generator=g)
    scores = torch.randn(B, T, H, 2 * half, generator=g)
    go = torch.randn(B, T, H, D, generator=g)
    rb = bank.clone().requires_grad_()
    out, _, _ = torch_oracle.routed_read(rb, scores, width)
    (out * go).sum().backward()
    db = bank.to(device).requires_grad_()
    dout, _, _ = hip.routed_snapshot_read(db, scores.to(device), width)
    (dout * go.to(device)).sum().backward()
    close(db.grad.cpu(), rb.grad)
    rs = scores.clone().requires_grad_()
    out, _, _ = torch_oracle.routed_read(bank, rs, width)
    (out * go).sum().backward()
    ds = scores.to(device).requires_grad_()
    dout, _, _ = hip.routed_snapshot_read(bank.to(device), ds, width)
    (dout * go.to(device)).sum().backward()
    close(ds.grad.cpu(), rs.grad)


def test_snapshot_read_backward_collisions(device):
    """Many tokens reading the same few rows: the rows' gradient accumulates every
    w * grad_out term (entry order), checked against the oracle's index backward."""
    B, T, H, S, D, width = 2, 200, 2, 8, 48, 4
    g = gen(12)
    bank = torch.randn(B, H, S, D, generator=g)
    index = torch.stack([torch.randperm(S, generator=g)[:width].sort().values for _ in range(B * T * H)])
    index = index.view(B, T, H, width)
    weights = torch.randn(B, T, H, width, generator=g).softmax(-1)
    go = torch.randn(B, T, H, D, generator=g)
    rb, rw = bank.clone().requires_grad_(), weights.clone().requires_grad_()
    (torch_oracle.read(rb, index, rw) * go).sum().backward()
    db, dw = bank.to(device).requires_grad_(), weights.to(device).requires_grad_()
    (hip.snapshot_read(db, index.to(device), dw) * go.to(device)).sum().backward()
    close(db.grad.cpu(), rb.grad)
    close(dw.grad.cpu(), rw.grad)


def test_read_backward_rows_entry_order_is_sequential(device):
    """Rows' gradient = old + the entry-order sum of w * g: bitwise equal to a
    sequential fp32 accumulation (the reference's accumulating index backward)."""
    rows, D, E, width = 50, 16, 400, 4
    g = gen(13)
    grad_bank = torch.randn(rows, D, generator=g)
    addr = torch.randint(0, rows, (E,), generator=g)
    w = torch.randn(E, generator=g)
    go = torch.randn(E // width, D, generator=g)
    out = hip.read_backward_rows(grad_bank.to(device), addr.to(device), w.to(device), go.to(device)).cpu()
    terms = go.repeat_interleave(width, 0) * w[:, None]
    sums = torch.zeros(rows, D)
    for e in range(E):
        sums[addr[e]] = sums[addr[e]] + terms[e]
    assert torch.equal(out, grad_bank + sums)


@pytest.mark.parametrize("keyed", [False, True])
def test_commit_backward(device, keyed):
    rows, D, E = 300, 32, 900
    g = gen(14)
    flat = torch.randn(rows, D, generator=g)
    addr = torch.randint(0, rows // 3, (E,), generator=g)
    delta = torch.randn(E, D, generator=g) * 0.1
    keys = addr * (E + 1) + torch.randperm(E, generator=g) if keyed else None
    upstream = torch.randn(rows, D, generator=g)
    rf, rd = flat.clone().requires_grad_(), delta.clone().requires_grad_()
    (torch_oracle.commit(rf, addr, rd, keys) * upstream).sum().backward()
    df, dd = flat.to(device).requires_grad_(), delta.to(device).requires_grad_()
    out = hip.commit(df, addr.to(device), dd, None if keys is None else keys.to(device))
    (out * upstream.to(device)).sum().backward()
    assert torch.equal(df.grad.cpu(), rf.grad)
    assert torch.equal(dd.grad.cpu(), rd.grad)
    with pytest.raises(ValueError, match="donate"):
        hip.commit(df, addr.to(device), dd, donate=True)
