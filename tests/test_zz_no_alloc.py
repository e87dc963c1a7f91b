"""glsdm_commit_noalloc -- the commit whose workspace is the library's static
device scratch, for callers that cannot allocate -- against glsdm_commit with a
caller workspace, through the C ABI: bitwise equal banks and unique-row counts
on two calls in a row (the second with a smaller input, on the other sort
path), its status through glsdm_commit_status with a NULL workspace, and the
scratch's size limit reported as an error before any launch."""
import pytest
import torch

from glsdm import _native as N
from glsdm.memory.backends import hip

pytestmark = pytest.mark.gpu

MAX_ENTRIES = 1 << 19


def _noalloc_fn():
    return N.lib().glsdm_commit_noalloc


def _operands(device, seed, rows, D, dtype, E, keyed):
    g = torch.Generator(device).manual_seed(seed)
    bank = (torch.randn(rows, D, generator=g, device=device) * 0.02).to(dtype)
    addr = torch.randint(0, rows, (E,), generator=g, device=device)
    addr[::5] = addr[1::5][: addr[::5].numel()]                        # collisions
    delta = (torch.randn(E, D, generator=g, device=device) * 0.02).to(dtype)
    keys = addr * 4096 + torch.randperm(E, generator=g, device=device) if keyed else None
    return bank, addr, delta, keys


def test_noalloc_commit_matches_commit(device):
    fn = _noalloc_fn()
    # first the largest input the scratch takes (config 2's epoch: 2^22 bf16 rows, bucket
    # sort path), then a smaller one (fp32, fewer than 2^16 rows: look-back passes)
    cases = [(1 << 22, 128, torch.bfloat16, MAX_ENTRIES, True, 1),
             (40000, 64, torch.float32, 30000, False, 2)]
    for rows, D, dtype, E, keyed, seed in cases:
        print(f"noalloc case rows={rows} D={D} dtype={dtype} E={E} keyed={keyed}", flush=True)
        bank, addr, delta, keys = _operands(device, seed, rows, D, dtype, E, keyed)
        a, b = bank.clone(), bank.clone()
        ua = torch.zeros(1, dtype=torch.int64, device=device)
        ub = torch.zeros(1, dtype=torch.int64, device=device)
        ws = torch.empty(hip.commit_workspace_bytes(E, rows), dtype=torch.uint8, device=device)
        st = N.stream(device)
        N.call("glsdm_commit", N.ptr(a), N.dtype_code(a), rows, D, N.ptr(addr), N.ptr(delta), N.dtype_code(delta),
               N.ptr(keys), E, N.ptr(ws), ws.numel(), N.ptr(ua), st)
        with torch.cuda.device(device):
            rc = fn(N.ptr(b), N.dtype_code(b), rows, D, N.ptr(addr), N.ptr(delta), N.dtype_code(delta), N.ptr(keys),
                    E, N.ptr(ub), st)
        assert rc == N.OK, N.lib().glsdm_last_error().decode()
        status = torch.full((2,), -1, dtype=torch.int64, device=device)
        N.call("glsdm_commit_status", None, 0, E, rows, N.ptr(status), st)
        torch.cuda.synchronize(device)
        assert status.tolist() == [0, 0]
        assert not torch.equal(b, bank)
        assert torch.equal(a, b)
        assert ua.item() == ub.item() == addr.unique().numel()


def test_noalloc_commit_rejects_sizes_beyond_its_scratch(device):
    fn = _noalloc_fn()
    bank = torch.zeros(16, 8, device=device)
    addr = torch.zeros(4, dtype=torch.int64, device=device)
    delta = torch.zeros(4, 8, device=device)
    with torch.cuda.device(device):
        rc = fn(N.ptr(bank), N.F32, 16, 8, N.ptr(addr), N.ptr(delta), N.F32, None, MAX_ENTRIES + 1, None,
                N.stream(device))
    assert rc == N.ERR_UNSUPPORTED
    assert "scratch" in N.lib().glsdm_last_error().decode()
