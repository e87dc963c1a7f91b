"""Failure reporting of the commit family, through the C ABI: the device status
words of glsdm_commit_status (dropped out-of-range entries counted; a sort that
gave up leaves every bank row untouched and is reported), the host-forced
look-back timeout that drives that path, and the debug bounds checks, which
raise IndexError where the reference's torch indexing does (flat[index],
S/memory/routing.py:42 and S/memory/transactions.py:96)."""
import pytest
import torch

from glsdm import _native as N
from glsdm.memory.backends import hip
from oracle import torch_oracle
from _util import gen

pytestmark = pytest.mark.gpu


def _commit_capi(bank, addr, delta, ws):
    rows, D = bank.shape
    N.call("glsdm_commit", N.ptr(bank), N.dtype_code(bank), rows, D, N.ptr(addr), N.ptr(delta),
           N.dtype_code(delta), None, addr.numel(), N.ptr(ws), ws.numel(), None, N.stream(bank.device))


@pytest.mark.parametrize("rows", [4000, 1 << 18])        # look-back passes; bucket path
def test_dropped_entries_are_counted(device, rows):
    g = gen(41)
    D, E = 32, 30000
    bank = torch.randn(rows, D, generator=g)
    addr = torch.randint(0, rows, (E,), generator=g)
    oor = torch.zeros(E, dtype=torch.bool)
    oor[::37] = True
    oor[5::101] = True
    addr[oor] = rows + torch.arange(int(oor.sum())) % 5
    addr[5::101] = -3
    delta = torch.randn(E, D, generator=g) * 0.01
    dev_bank = bank.to(device)
    ws = torch.empty(hip.commit_workspace_bytes(E, rows), dtype=torch.uint8, device=device)
    _commit_capi(dev_bank, addr.to(device), delta.to(device), ws)
    err, dropped = hip.commit_status(ws, E, rows)
    assert err == 0 and dropped == int(oor.sum())
    assert torch.equal(dev_bank.cpu(), torch_oracle.commit(bank, addr[~oor], delta[~oor]))
    # a clean commit with the same workspace reports no drop
    addr = addr.clamp(0, rows - 1)
    _commit_capi(dev_bank, addr.to(device), delta.to(device), ws)
    assert hip.commit_status(ws, E, rows) == (0, 0)


def test_forced_lookback_timeout_leaves_bank_untouched(device):
    rows, D, E = 4000, 32, 20000                           # five sort tiles: tiles 1..4 look back
    g = gen(42)
    bank = torch.randn(rows, D, generator=g)
    addr = torch.randint(0, rows, (E,), generator=g)
    delta = torch.randn(E, D, generator=g) * 0.01
    dev_bank, addr_d, delta_d = bank.to(device), addr.to(device), delta.to(device)
    ws = torch.empty(hip.commit_workspace_bytes(E, rows), dtype=torch.uint8, device=device)
    lib = N.lib()
    lib.glsdm_debug_force_lookback_timeout(1)
    try:
        _commit_capi(dev_bank, addr_d, delta_d, ws)
        err, _ = hip.commit_status(ws, E, rows)
        assert err & 1
        assert torch.equal(dev_bank.cpu(), bank)           # the segment step wrote nothing
        with N.checks(status=True):
            with pytest.raises(N.NativeError, match="sort failed"):
                hip.commit(dev_bank, addr_d, delta_d, donate=True)
        assert torch.equal(dev_bank.cpu(), bank)
    finally:
        lib.glsdm_debug_force_lookback_timeout(0)
    out = hip.commit(dev_bank, addr_d, delta_d, workspace=ws)
    assert hip.commit_status(ws, E, rows) == (0, 0)
    assert torch.equal(out.cpu(), torch_oracle.commit(bank, addr, delta))


def test_bounds_checks_raise_like_torch_indexing(device):
    g = gen(43)
    bank = torch.randn(2, 2, 16, 8, generator=g).to(device)
    idx = torch.randint(0, 16, (2, 3, 2, 4), generator=g)
    idx[1, 2, 0, 3] = 16
    idx = idx.to(device)
    w = torch.randn(2, 3, 2, 4, generator=g).softmax(-1).to(device)
    flat = bank.view(-1, 8)
    addr = torch.tensor([0, 5, 64], device=device)
    before = flat.clone()
    with pytest.raises(IndexError):                         # the reference's own indexing, on the CPU
        before.cpu()[addr.cpu()]
    with N.checks(bounds=True):
        with pytest.raises(IndexError):
            hip.snapshot_read(bank, idx, w)
        with pytest.raises(IndexError):
            hip.commit(flat, addr, torch.ones(3, 8, device=device), donate=True)
        with pytest.raises(IndexError):
            hip.gather_flat(flat, addr)
        with pytest.raises(IndexError):
            hip.absolute_addresses(bank, idx)
    assert torch.equal(flat, before)                        # nothing was written
    # unchecked: the documented behaviour (out-of-range routes contribute nothing,
    # out-of-range commit entries are dropped)
    hip.snapshot_read(bank, idx, w)
    out = hip.commit(flat, addr, torch.ones(3, 8, device=device))
    assert torch.equal(out[:64].cpu(), torch_oracle.commit(before.cpu(), addr[:2].cpu(), torch.ones(2, 8)))
