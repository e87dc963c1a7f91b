"""HIP commit vs the oracle: bitwise for fp32 and bf16 banks (the summation
order is the reference's), the reference's golden cancellation fixtures, and
the commit invariants (untouched rows, repeatability, donation)."""
import pytest
import torch

from oracle import c_oracle, torch_oracle
from glsdm.memory import MemoryView, WriteProposal, merge, commit
from glsdm.memory.backends import hip
from _util import known_answers

pytestmark = pytest.mark.gpu


def test_commit_golden_fixtures(device):
    ka = known_answers()
    c = ka["commit_stable_collisions"]
    view = MemoryView(torch.zeros(1, 1, c["rows"], 1, device=device))
    p = WriteProposal(0, torch.tensor(c["addresses"], device=device),
                      torch.tensor(c["deltas"], device=device)[:, None], view.lineage)
    out = commit(view, merge(view, [p]))
    assert out.values.flatten().tolist() == c["expect"]
    assert out.version == 1 and out.lineage is view.lineage
    assert view.values.abs().sum().item() == 0          # the old view is unchanged
    with pytest.raises(ValueError, match="stale"):
        commit(out, merge(view, [p]))

    c = ka["commit_keyed_arrival_order"]
    view = MemoryView(torch.zeros(1, 1, c["rows"], 1, device=device))
    props = [WriteProposal(0, torch.tensor([a], device=device), torch.tensor([[d]], device=device),
                           view.lineage, torch.tensor([k], device=device))
             for a, d, k in zip(c["addresses"], c["deltas"], c["keys"])]
    a = commit(view, merge(view, props))
    b = commit(view, merge(view, [props[i] for i in c["permutation"]]))
    assert torch.equal(a.values, b.values) and a.values.flatten()[3].item() == c["expect_row3"]

    c = ka["commit_unrelated_addresses"]
    view = MemoryView(torch.zeros(1, 1, c["rows"], 1, device=device))
    p = WriteProposal(0, torch.tensor(c["addresses"], device=device),
                      torch.tensor(c["deltas"], device=device)[:, None], view.lineage)
    assert commit(view, merge(view, [p])).values[0, 0, 3, 0].item() == c["expect_row3"]


def _case(rows, D, E, spread, seed, bank_dtype=torch.float32, delta_dtype=torch.float32, keyed=True):
    g = torch.Generator().manual_seed(seed)
    flat = torch.randn(rows, D, generator=g).to(bank_dtype)
    addr = torch.randint(0, spread, (E,), generator=g)
    delta = (torch.randn(E, D, generator=g) * 0.02).to(delta_dtype)
    keys = addr * (E + 1) + torch.randperm(E, generator=g) if keyed else None
    return flat, addr, delta, keys


@pytest.mark.parametrize("keyed", [False, True])
@pytest.mark.parametrize("rows,D,E,spread", [
    (64, 8, 5, 4), (4096, 256, 8192, 4096), (1000, 128, 20000, 300), (50000, 128, 70000, 50000),
    (67, 37, 300, 67), (10, 16, 3000, 3), (1, 4, 1, 1), (2048, 512, 4096, 64), (300, 2048, 600, 300),
])
def test_commit_fp32_bitwise(device, keyed, rows, D, E, spread):
    flat, addr, delta, keys = _case(rows, D, E, spread, seed=rows + E, keyed=keyed)
    unique = torch.zeros(1, dtype=torch.int64, device=device)
    out = hip.commit(flat.to(device), addr.to(device), delta.to(device),
                     None if keys is None else keys.to(device), unique=unique)
    ref, n = c_oracle.commit(flat, addr, delta, keys)
    assert torch.equal(out.cpu(), ref)
    assert unique.item() == n


@pytest.mark.parametrize("bank_dtype,delta_dtype", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                                    (torch.float32, torch.bfloat16)])
def test_commit_mixed_precision_bitwise(device, bank_dtype, delta_dtype):
    flat, addr, delta, keys = _case(8192, 128, 40000, 8192, seed=11, bank_dtype=bank_dtype, delta_dtype=delta_dtype)
    out = hip.commit(flat.to(device), addr.to(device), delta.to(device), keys.to(device))
    ref = torch_oracle.commit(flat.float(), addr, delta.float(), keys).to(bank_dtype)
    assert out.dtype == bank_dtype
    assert torch.equal(out.cpu(), ref)


def test_commit_donate_repeat_and_untouched(device):
    flat, addr, delta, keys = _case(5000, 64, 9000, 3000, seed=3)
    base = flat.to(device)
    first = hip.commit(base, addr.to(device), delta.to(device), keys.to(device))
    for _ in range(3):
        again = hip.commit(base, addr.to(device), delta.to(device), keys.to(device))
        assert torch.equal(again, first)
    assert torch.equal(base.cpu(), flat)                  # functional by default
    donated = base.clone()
    out = hip.commit(donated, addr.to(device), delta.to(device), keys.to(device), donate=True)
    assert out.data_ptr() == donated.data_ptr() and torch.equal(out, first)
    untouched = torch.ones(5000, dtype=torch.bool)
    untouched[addr] = False
    assert torch.equal(first.cpu()[untouched], flat[untouched])


def test_commit_negative_and_interleaved_keys(device):
    flat, addr, delta, _ = _case(700, 16, 5000, 700, seed=8)
    keys = addr * 5000 + torch.arange(5000) - 12345          # negative keys are ordinary int64 keys
    out = hip.commit(flat.to(device), addr.to(device), delta.to(device), keys.to(device))
    ref, _ = c_oracle.commit(flat, addr, delta, keys)
    assert torch.equal(out.cpu(), ref)
    # two proposals (layers) concatenated: within an address the key order interleaves them
    pos = torch.randint(0, 512, (5000,))
    layer = (torch.arange(5000) >= 2500).long()
    keys2 = addr * (512 * 2) + pos * 2 + layer
    out2 = hip.commit(flat.to(device), addr.to(device), delta.to(device), keys2.to(device))
    ref2, _ = c_oracle.commit(flat, addr, delta, keys2)
    assert torch.equal(out2.cpu(), ref2)


def test_commit_long_unordered_run(device):
    """One hot row with 3000 deltas in scrambled key order (a skewed, multi-layer commit)."""
    g = torch.Generator().manual_seed(12)
    flat = torch.randn(64, 32, generator=g)
    addr = torch.full((3000,), 17)
    addr[::7] = torch.randint(0, 64, (429,), generator=g)
    delta = torch.randn(3000, 32, generator=g) * 0.5
    keys = addr * 100000 + torch.randperm(3000, generator=g)
    out = hip.commit(flat.to(device), addr.to(device), delta.to(device), keys.to(device))
    ref, _ = c_oracle.commit(flat, addr, delta, keys)
    assert torch.equal(out.cpu(), ref)


def test_commit_drops_out_of_range_addresses(device):
    flat, addr, delta, _ = _case(100, 8, 500, 100, seed=4, keyed=False)
    bad = addr.clone()
    bad[::50] = 100                      # one past the end; keys = addresses, so they sort last
    out = hip.commit(flat.to(device), bad.to(device), delta.to(device))
    keep = bad < 100
    ref, _ = c_oracle.commit(flat, bad[keep], delta[keep])
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("keyed", [False, True])
@pytest.mark.parametrize("rows,D,E,lo,hi", [
    (1 << 18, 32, 30000, 0, 1 << 18),        # three address digits: tile bucketing + per-bucket LDS sort
    (1 << 20, 16, 60000, 0, 4096),           # one bucket holds every entry: chunked global bucket sort
    (1 << 20, 16, 50000, (1 << 20) - 3000, 1 << 20),   # a crowded last bucket plus the out-of-range run
    ((1 << 17) + 5, 8, 20000, 0, (1 << 17) + 5),
])
def test_commit_bucket_sort_paths(device, keyed, rows, D, E, lo, hi):
    g = torch.Generator().manual_seed(rows + E)
    flat = torch.randn(rows, D, generator=g)
    addr = torch.randint(lo, hi, (E,), generator=g)
    addr[::501] = rows + 7                                  # out of range: dropped
    delta = torch.randn(E, D, generator=g) * 0.02
    keys = addr * (E + 1) + torch.randperm(E, generator=g) if keyed else None
    out = hip.commit(flat.to(device), addr.to(device), delta.to(device), None if keys is None else keys.to(device))
    keep = addr < rows                                      # the oracle takes in-range entries only
    ref, _ = c_oracle.commit(flat, addr[keep], delta[keep], None if keys is None else keys[keep])
    assert torch.equal(out.cpu(), ref)


def test_commit_bucket_sort_more_tiles_than_threads(device):
    """Over 1024 sort tiles of 4096 entries: each bucket gathers its pieces in
    several rounds, and every bucket (~17k words) takes the global-memory sort."""
    rows, D, E = 1 << 20, 4, (1 << 22) + 200_003
    g = torch.Generator().manual_seed(11)
    flat = torch.randn(rows, D, generator=g)
    addr = torch.randint(0, rows, (E,), generator=g)
    addr[::9973] = rows + 1                                 # out of range: dropped
    delta = torch.randn(E, D, generator=g) * 0.02
    out = hip.commit(flat.to(device), addr.to(device), delta.to(device))
    keep = addr < rows
    ref, _ = c_oracle.commit(flat, addr[keep], delta[keep])
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("E", [70_000, 100_000, 200_000])
def test_commit_long_runs_past_windows(device, dtype, E):
    """Commits of ~1e5 entries use windows of 8-32 sorted positions per wave, so
    runs that continue past their window go to the long-run kernel: hot
    addresses with thousands of entries (keys in arrival order), warm ones whose
    keys run against arrival order (the selection path), and out-of-range
    entries.  Bitwise equal to the oracle's sequential per-address sums."""
    g = torch.Generator().manual_seed(E)
    rows, D = 4096, 64
    addr = torch.randint(0, rows, (E,), generator=g)
    pick = torch.rand(E, generator=g)
    hot = torch.randint(0, rows, (16,), generator=g)
    warm = torch.randint(0, rows, (64,), generator=g)
    h = pick < 0.5
    addr[h] = hot[torch.randint(0, 16, (int(h.sum()),), generator=g)]
    w = (pick >= 0.5) & (pick < 0.52)
    addr[w] = warm[torch.randint(0, 64, (int(w.sum()),), generator=g)]
    addr[::997] = rows + 3                                   # out of range: dropped
    ent = torch.arange(E)
    keys = addr * (E + 1) + ent
    rev = torch.isin(addr, warm)
    keys[rev] = addr[rev] * (E + 1) + (E - ent[rev])
    flat = torch.randn(rows, D, generator=g).to(dtype)
    delta = torch.randn(E, D, generator=g) * 0.02
    out = hip.commit(flat.to(device), addr.to(device), delta.to(device), keys.to(device))
    keep = addr < rows
    if dtype == torch.float32:
        ref = torch_oracle.commit(flat, addr[keep], delta[keep], keys[keep])
    else:
        ref = torch_oracle.commit_bf16(flat, addr[keep], delta[keep], keys[keep])
    assert torch.equal(out.cpu(), ref)


def test_overlay_commit_long_runs_equal_dense(device):
    """The overlay row store through the long-run kernel: same bits as the dense bank."""
    from glsdm.memory import OverlayView
    g = torch.Generator().manual_seed(5)
    B, H, S, D, E = 2, 2, 1024, 32, 90_000
    base = torch.randn(H, S, D, generator=g)
    rows = B * H * S
    addr = torch.randint(0, rows, (E,), generator=g)
    addr[: E // 2] = torch.randint(0, 8, (E // 2,), generator=g) * 97     # 8 hot rows, long runs
    keys = addr * (E + 1) + torch.arange(E)
    delta = torch.randn(E, D, generator=g) * 0.02
    ov = OverlayView.from_base(base.to(device), B)
    ov.commit(addr.to(device), delta.to(device), keys.to(device))
    dense = base.unsqueeze(0).expand(B, -1, -1, -1).reshape(rows, D).clone()
    ref = torch_oracle.commit(dense, addr, delta, keys)
    assert torch.equal(ov.materialise().cpu().reshape(rows, D), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,D,E", [(5000, 32, 3000), (1 << 22, 128, 60_000), (70_000, 16, 100_000),
                                      (1 << 20, 64, 250_000)])
def test_commit_prepare_apply_equals_commit(device, dtype, rows, D, E):
    """glsdm_commit_prepare then glsdm_commit_apply (here with other work and
    another epoch's prepare in between, on another stream) equals glsdm_commit
    bit for bit, on the LSD path (few address digits) and the top-digit + bucket
    path, with keys."""
    from glsdm import _native as N
    g = torch.Generator().manual_seed(rows + E)
    flat = (torch.randn(rows, D, generator=g)).to(dtype)
    addr = torch.randint(0, rows, (E,), generator=g)
    addr[: E // 10] = addr[E // 10: 2 * (E // 10)]                    # collisions
    delta = (torch.randn(E, D, generator=g) * 0.02).to(dtype)
    keys = addr * (E + 1) + torch.randperm(E, generator=g)
    ref = hip.commit(flat.to(device), addr.to(device), delta.to(device), keys.to(device))
    need = hip.commit_workspace_bytes(E, rows)
    ws = torch.empty(need, dtype=torch.uint8, device=device)
    ws2 = torch.empty(need, dtype=torch.uint8, device=device)
    bank, a, d, k = flat.to(device), addr.to(device), delta.to(device), keys.to(device)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        N.call("glsdm_commit_prepare", rows, N.ptr(a), E, N.ptr(ws), need, N.stream(device))
        N.call("glsdm_commit_prepare", rows, N.ptr(a.flip(0).contiguous()), E, N.ptr(ws2), need, N.stream(device))
    torch.cuda.current_stream(device).wait_stream(side)
    N.call("glsdm_commit_apply", N.ptr(bank), N.dtype_code(bank), rows, D, N.ptr(d), N.dtype_code(d), N.ptr(k), E,
           N.ptr(ws), need, None, N.stream(device))
    assert torch.equal(bank, ref)
