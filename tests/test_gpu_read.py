"""HIP snapshot read vs the oracle: fp32 within 1e-5 relative, bf16 banks
within 1e-5 of the fp32 read of the widened bank (bf16 outputs: 2e-2)."""
import pytest
import torch

from oracle import c_oracle, torch_oracle
from glsdm.memory.backends import hip

pytestmark = pytest.mark.gpu


def _case(B, H, S, D, T, k, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    mem = (torch.randn(B, H, S, D, generator=g) * 0.02).to(dtype)
    idx = torch.randint(0, S, (B, T, H, k), generator=g)
    w = torch.randn(B, T, H, k, generator=g).softmax(-1)
    return mem, idx, w


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,S,D,T,k", [
    (2, 1, 4096, 256, 64, 8),      # config 1 geometry
    (2, 8, 256, 128, 33, 16),      # config 2 geometry, small bank
    (1, 1, 1024, 512, 20, 32),     # config 3 geometry
    (3, 2, 67, 37, 4, 3),          # odd D (P/tests/test_native_memory.py:52-92 shapes)
    (2, 2, 16, 8, 17, 2),
    (1, 2, 64, 1024, 5, 4),
    (1, 1, 16, 2048, 3, 4),
])
def test_read_matches_oracle(device, dtype, B, H, S, D, T, k):
    mem, idx, w = _case(B, H, S, D, T, k, dtype, seed=S + D)
    out = hip.snapshot_read(mem.to(device), idx.to(device), w.to(device))
    ref = c_oracle.read(mem, idx, w)
    torch.testing.assert_close(out.cpu(), ref, atol=1e-6, rtol=1e-5)
    torch.testing.assert_close(out.cpu(), torch_oracle.read(mem.float(), idx, w), atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,S,D,T,k", [
    (2, 8, 256, 128, 33, 16),      # config 2 geometry: four entries per lane group in flight
    (1, 1, 1024, 512, 20, 32),     # config 3 geometry: one lane group per wave
    (2, 2, 16, 8, 17, 3),          # ragged: the last batch of entries is partial
    (1, 1, 16, 2048, 3, 5),        # two pieces per lane: two entries in flight
    (3, 2, 67, 37, 4, 3),          # scalar pieces
])
def test_read_narrow_equals_wide(device, dtype, B, H, S, D, T, k):
    """glsdm_read (several entries per lane group in flight) and glsdm_read_narrow
    (one) add the same products in the same order: bitwise equal, and the oracle's."""
    mem, idx, w = _case(B, H, S, D, T, k, dtype, seed=7 * S + D + k)
    idx[0, 0, 0, k - 1] = S                       # an out-of-range slot adds nothing in both
    args = (mem.to(device), idx.to(device), w.to(device), torch.float32)
    wide, narrow = hip._read(*args), hip._read(*args, narrow=True)
    keep = (idx >= 0) & (idx < S)
    ref = c_oracle.read(mem, idx.clamp(0, S - 1), w * keep)
    torch.testing.assert_close(wide.cpu(), ref, atol=1e-6, rtol=1e-5)
    torch.testing.assert_close(narrow.cpu(), ref, atol=1e-6, rtol=1e-5)
    assert torch.equal(wide, narrow)


def test_read_bf16_output(device):
    mem, idx, w = _case(2, 8, 256, 128, 16, 16, torch.bfloat16, seed=1)
    out = hip.snapshot_read(mem.to(device), idx.to(device), w.to(device), out_dtype=torch.bfloat16)
    ref = c_oracle.read(mem, idx, w)
    torch.testing.assert_close(out.cpu().float(), ref, atol=1e-4, rtol=2e-2)
    # the fp32 sums rounded once: the bits of an fp32 read followed by .to(bfloat16)
    # (the stack's global layers read straight into bf16 on this)
    wide = hip.snapshot_read(mem.to(device), idx.to(device), w.to(device), out_dtype=torch.float32)
    assert torch.equal(out, wide.to(torch.bfloat16))


def test_read_out_of_range_slots_contribute_nothing(device):
    mem, idx, w = _case(1, 1, 16, 8, 4, 4, torch.float32, seed=2)
    idx[0, 0, 0, 1] = -1
    idx[0, 1, 0, 2] = 16
    out = hip.snapshot_read(mem.to(device), idx.to(device), w.to(device)).cpu()
    keep = (idx >= 0) & (idx < 16)
    ref = c_oracle.read(mem, idx.clamp(0, 15), w * keep)
    torch.testing.assert_close(out, ref, atol=1e-6, rtol=1e-5)


def test_gather_and_addresses(device):
    mem, idx, _ = _case(2, 3, 40, 12, 5, 4, torch.float32, seed=3)
    addr = hip.absolute_addresses(mem.to(device), idx.to(device)).cpu()
    assert torch.equal(addr, torch_oracle.absolute_addresses(mem, idx))
    rows = hip.gather_rows(mem.to(device), idx.to(device)).cpu()
    assert torch.equal(rows, torch_oracle.gather_rows(mem, idx))
    a, keys = hip.proposal_keys(mem.to(device), idx.to(device), 3, 16, 4, 2)
    pos = torch.arange(3, 3 + 5).view(1, 5, 1, 1)
    assert torch.equal(a.cpu(), addr)
    assert torch.equal(keys.cpu(), addr * (16 * 4) + pos * 4 + 2)
