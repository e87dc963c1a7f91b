"""Host-side logic of the glsdm.memory mirror (no GPU): validation, staleness,
lineage and backend checks, with the reference's error messages
(P/tests/test_global_memory.py:49-54,128-131; P/tests/test_native_memory.py:141-144)."""
import pytest
import torch

from glsdm.memory import MemoryView, WriteProposal, MemoryBank, merge, commit
from glsdm.memory import routing
from glsdm.memory.backends import hip


def _view():
    return MemoryView(torch.zeros(1, 1, 4, 2))


def test_view_validation():
    with pytest.raises(ValueError):
        MemoryView(torch.zeros(1, 4, 2))
    with pytest.raises(ValueError):
        MemoryView(torch.zeros(1, 1, 4, 2, dtype=torch.float16))
    with pytest.raises(ValueError):
        MemoryView(torch.zeros(1, 1, 4, 2), version=-1)
    assert MemoryView(torch.zeros(1, 1, 4, 2, dtype=torch.bfloat16)).version == 0


def test_merge_and_stale_commit_errors():
    view = _view()
    p = WriteProposal(0, torch.tensor([1]), torch.ones(1, 2), view.lineage)
    buf = merge(view, [p])
    with pytest.raises(ValueError, match="snapshot"):
        merge(view, [])
    with pytest.raises(ValueError, match="snapshot"):
        merge(MemoryView(view.values, 1, view.lineage), [p])
    with pytest.raises(ValueError, match="stale"):
        commit(MemoryView(view.values, 1, view.lineage), buf)
    with pytest.raises(ValueError, match="stale"):
        commit(MemoryView(view.values), buf)             # other lineage
    q = WriteProposal(0, torch.tensor([2]), torch.ones(1, 2), view.lineage, torch.tensor([5]))
    with pytest.raises(ValueError, match="mix"):
        commit(view, merge(view, [p, q]))


def test_backend_and_device_checks():
    view = _view()
    buf = merge(view, [WriteProposal(0, torch.tensor([1]), torch.ones(1, 2), view.lineage)])
    with pytest.raises(ValueError, match="backend"):
        commit(view, buf, backend="torch")
    with pytest.raises(ValueError, match="oracle"):
        commit(view, buf, reference=True)
    with pytest.raises(ValueError, match="CUDA"):       # never a silent CPU fallback
        commit(view, buf)
    with pytest.raises(ValueError, match="CUDA"):
        hip.route(torch.zeros(2, 8), 2)
    with pytest.raises(ValueError, match="CUDA"):
        hip.routed_snapshot_read(torch.zeros(1, 1, 16, 4), torch.zeros(1, 3, 1, 8), 2)

    class Attn:
        backend, reference = "torch", False

    class Block:
        attn = Attn()

    with pytest.raises(ValueError, match="hip"):
        routing.routed_read(Block(), torch.zeros(1, 1, 16, 4), torch.zeros(1, 3, 1, 8), 2)


def test_forward_only_guard():
    # scoring, proposals and the fused commit are forward-only
    q = torch.zeros(1, 2, 1, 32, dtype=torch.bfloat16, requires_grad=True)
    k = torch.zeros(1, 64, 32, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        hip.score(q, k)
    # the differentiable route still never falls back to the CPU
    s = torch.zeros(2, 8, requires_grad=True)
    with pytest.raises(ValueError, match="CUDA"):
        hip.route(s, 2)
    # the proposal arithmetic under autograd (training with writes) runs on the device only
    from glsdm.runtime import proposal_delta
    rows = torch.zeros(1, 2, 1, 2, 4, requires_grad=True)
    with pytest.raises(ValueError, match="CUDA"):
        proposal_delta(rows, torch.zeros(1, 2, 1, 2), torch.zeros(1, 2, 1, 4), torch.zeros(1, 2, 1, 4),
                       torch.zeros(1, 2, 1, 1), torch.zeros(1, 2, 1, 1), torch.ones(1, 2))
    with pytest.raises(ValueError, match="CUDA"):
        hip.gather_rows(torch.zeros(1, 1, 4, 2, requires_grad=True), torch.zeros(1, 1, 1, 1, dtype=torch.int64))


def test_bank_stays_fp32_and_caches_validate():
    bank = MemoryBank(2, 16, 4)
    bank = bank.bfloat16()
    assert bank.memory.dtype == torch.float32
    cache = bank.new_cache(3)
    assert cache.view.values.shape == (3, 2, 16, 4)
    bank.validate_cache(cache, 3)
    with pytest.raises(ValueError, match="cache belongs"):
        bank.validate_cache(cache, 2)
    with pytest.raises(ValueError, match="cache belongs"):
        MemoryBank(2, 16, 4).validate_cache(cache, 3)
    b16 = MemoryBank(2, 16, 4, state_dtype=torch.bfloat16)
    c16 = b16.new_cache(2)
    assert c16.view.values.dtype == torch.bfloat16
    assert torch.equal(c16.view.values[1].float(), b16.memory.detach().bfloat16().float())


def test_route_size_validation():
    with pytest.raises(ValueError):
        hip._square_root(15)
    assert hip._square_root(65536) == 256


def test_bounds_check_helper():
    """The debug bounds check raises IndexError (as torch indexing does) only when on."""
    from glsdm import _native as N
    idx = torch.tensor([0, 3, 7])
    N.check_range(idx, 7, "x")                              # off by default: no check
    with N.checks(bounds=True):
        N.check_range(idx, 8, "x")
        with pytest.raises(IndexError, match="index 7 is out of bounds for size 7"):
            N.check_range(idx, 7, "x")
        with pytest.raises(IndexError):
            N.check_range(torch.tensor([-1]), 7, "x")
    assert not N.checking("bounds")
