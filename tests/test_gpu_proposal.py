"""HIP write-proposal arithmetic and the fused proposal -> commit vs the oracle.

The exponential is the only operation whose rounding may differ between the
device and the CPU (each is within an ulp of exp): it is checked against
float64 exp, and every later operation is compared bit for bit with the
oracle evaluated on the device's decay values.  The fused commit must equal
the unfused path (gather rows, materialise deltas, commit) bit for bit, and
both must equal the oracle's commit of the oracle's deltas.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import torch_oracle
from glsdm.memory import (DeferredProposal, MemoryView, WriteProposal, commit, layer_proposal, merge)
from glsdm.memory.backends import hip
from glsdm.runtime import proposal_delta as dense_proposal_delta
from _util import gen

pytestmark = pytest.mark.gpu


def _operands(seed, lead, H, k, D, S, target_dtype=torch.float32, mass="ones"):
    """Stack-shaped proposal operands on the CPU (S/layers/global_layer.py:42-50)."""
    g = gen(seed)
    index = torch.randint(0, S, (*lead, H, k), generator=g)
    weights = torch.randn(*lead, H, k, generator=g).softmax(-1)
    prediction = torch.randn(*lead, H, D, generator=g) * 0.1
    target = (torch.randn(*lead, H, D, generator=g) * 0.1).to(target_dtype)
    beta = torch.randn(*lead, H, generator=g).sigmoid().unsqueeze(-1)
    log_decay = -F.softplus(torch.randn(*lead, H, generator=g) - 4).unsqueeze(-1)
    m = torch.ones(lead) if mass == "ones" else torch.rand(*lead, generator=g)
    return index, weights, prediction, target, beta, log_decay, m


def _to(device, *ts):
    return [None if t is None else t.to(device) for t in ts]


def _ulps(a, b):
    a64, b64 = a.double().numpy(), b.double().numpy()
    spacing = np.spacing(np.abs(b.float().numpy())).astype(np.float64)
    return np.abs(a64 - b64) / spacing


@pytest.mark.parametrize("D,target_dtype", [(128, torch.float32), (128, torch.bfloat16), (37, torch.float32),
                                            (512, torch.bfloat16), (2048, torch.float32), (4, torch.float32)])
def test_proposal_error(device, D, target_dtype):
    _, _, pred, tgt, beta, ld, _ = _operands(D, (3, 50), 4, 1, D, 16, target_dtype)
    error, decay = hip.proposal_error(*_to(device, pred, tgt, beta, ld))
    decay = decay.cpu()
    assert _ulps(decay, ld[..., 0].double().exp()).max() <= 1.0
    ref = torch_oracle.proposal_error(pred, tgt, beta, decay[..., None])
    assert torch.equal(error.cpu(), ref)


@pytest.mark.parametrize("lead,H,k,D,rows_dtype,target_dtype,mass", [
    ((2, 64), 8, 16, 128, torch.bfloat16, torch.bfloat16, "ones"),
    ((2, 64), 8, 16, 128, torch.float32, torch.float32, "rand"),
    ((1, 33), 1, 8, 256, torch.float32, torch.bfloat16, "rand"),
    ((2, 3, 5), 2, 3, 37, torch.float32, torch.float32, "rand"),     # chunk path lead [B, R, length]; scalar D
    ((1, 7), 1, 32, 512, torch.bfloat16, torch.float32, "ones"),
    ((1, 5), 3, 2, 2048, torch.float32, torch.float32, "rand"),
    ((4,), 1, 1, 4, torch.float32, torch.float32, "rand"),
])
def test_proposal_delta_bitwise(device, lead, H, k, D, rows_dtype, target_dtype, mass):
    index, w, pred, tgt, beta, ld, m = _operands(sum(lead) + D, lead, H, k, D, 64, target_dtype, mass)
    rows = (torch.randn(*lead, H, k, D, generator=gen(1)) * 0.02).to(rows_dtype)
    dev = _to(device, rows, w, pred, tgt, beta, ld, m)
    out = dense_proposal_delta(*dev)
    _, decay = hip.proposal_error(*dev[2:6])
    ref = torch_oracle.proposal_delta(rows.float(), w, pred, tgt, beta, ld, m, decay=decay.cpu()[..., None])
    assert out.dtype == torch.float32 and out.shape == rows.shape
    assert torch.equal(out.cpu(), ref)
    # against the oracle's own exp: within the tolerance the exponential allows
    torch.testing.assert_close(out.cpu(), torch_oracle.proposal_delta(rows.float(), w, pred, tgt, beta, ld, m),
                               atol=1e-6, rtol=1e-5)


def _flat_case(seed, B, T, H, k, D, S, bank_dtype, target_dtype=torch.float32, mass="ones", spread=None):
    g = gen(seed + 1000)
    bank = (torch.randn(B, H, S, D, generator=g) * 0.02).to(bank_dtype)
    index, w, pred, tgt, beta, ld, m = _operands(seed, (B, T), H, k, D, spread or S, target_dtype, mass)
    addr = ((torch.arange(B).view(B, 1, 1, 1) * H + torch.arange(H).view(1, 1, H, 1)) * S + index)
    keys = addr * (T * 1) + torch.arange(T).view(1, T, 1, 1)
    return bank, index, addr, keys, w, pred, tgt, beta, ld, m


def _oracle_commit(bank, addr, keys, w, pred, tgt, beta, ld, m, decay):
    flat = bank.reshape(-1, bank.shape[-1])
    rows = flat.float()[addr]
    delta = torch_oracle.proposal_delta(rows, w, pred, tgt, beta, ld, m, decay=decay[..., None])
    D = bank.shape[-1]
    out = torch_oracle.commit(flat.float(), addr.reshape(-1), delta.reshape(-1, D),
                              None if keys is None else keys.reshape(-1))
    return out.to(bank.dtype).reshape(bank.shape)


@pytest.mark.parametrize("B,T,H,k,D,S,bank_dtype,keyed,spread", [
    (2, 64, 8, 16, 128, 1024, torch.bfloat16, True, None),
    (2, 64, 8, 16, 128, 1024, torch.float32, True, None),
    (1, 128, 1, 8, 256, 4096, torch.float32, False, None),
    (1, 200, 2, 4, 64, 256, torch.float32, True, 5),          # long collision runs
    (1, 50, 1, 32, 512, 4096, torch.bfloat16, True, 64),
    (2, 9, 3, 2, 37, 49, torch.float32, True, None),          # scalar row path
])
def test_commit_proposals_bitwise(device, B, T, H, k, D, S, bank_dtype, keyed, spread):
    bank, index, addr, keys, w, pred, tgt, beta, ld, m = _flat_case(T + D, B, T, H, k, D, S, bank_dtype,
                                                                    mass="rand", spread=spread)
    keys = keys if keyed else None
    d_bank, d_addr, d_keys, d_w, d_pred, d_tgt, d_beta, d_ld, d_m = _to(device, bank, addr, keys, w, pred, tgt,
                                                                          beta, ld, m)
    error, decay = hip.proposal_error(d_pred, d_tgt, d_beta, d_ld)
    unique = torch.zeros(1, dtype=torch.int64, device=device)
    fused = hip.commit_proposals(d_bank, d_addr, d_keys, d_w, error, decay, d_m, unique=unique)
    # unfused device path: gather rows, materialise deltas, commit
    rows = hip.gather_rows(d_bank, index.to(device))
    delta = hip.proposal_delta(rows, d_w, d_pred, d_tgt, d_beta, d_ld, d_m)
    unfused = hip.commit(d_bank, d_addr.reshape(-1), delta.reshape(-1, D),
                         None if d_keys is None else d_keys.reshape(-1))
    assert torch.equal(fused, unfused)
    ref = _oracle_commit(bank, addr, keys, w, pred, tgt, beta, ld, m, decay.cpu())
    assert torch.equal(fused.cpu(), ref)
    assert unique.item() == addr.unique().numel()
    assert torch.equal(d_bank.cpu(), bank)                  # not donated: the snapshot is unchanged


def test_commit_proposals_drops_out_of_range(device):
    bank, index, addr, keys, w, pred, tgt, beta, ld, m = _flat_case(5, 1, 32, 2, 4, 64, 256, torch.float32)
    addr = addr.clone()
    addr[0, 3, 1, 2] = -1
    addr[0, 7, 0, 0] = bank.numel() // 64
    d = _to(device, bank, addr, keys, w, pred, tgt, beta, ld, m)
    error, decay = hip.proposal_error(*d[4:8])
    fused = hip.commit_proposals(d[0], d[1], d[2], d[3], error, decay, d[8])
    keep = (addr >= 0) & (addr < bank.numel() // 64)
    flat = bank.reshape(-1, 64)
    rows = flat[addr.clamp(0, flat.shape[0] - 1)]
    delta = torch_oracle.proposal_delta(rows, w, pred, tgt, beta, ld, m, decay=decay.cpu()[..., None])
    ref = torch_oracle.commit(flat, addr[keep], delta[keep], keys[keep]).reshape(bank.shape)
    assert torch.equal(fused.cpu(), ref)


def test_layer_proposals_through_transactions(device):
    """Two layers' deferred proposals merged and committed together equal the
    oracle's commit of both layers' materialised deltas under the stack keys;
    so do a deferred and a materialised proposal mixed in one buffer."""
    B, T, H, k, D, S = 2, 48, 4, 8, 64, 256
    C, L = 64, 2
    bank = (torch.randn(B, H, S, D, generator=gen(7)) * 0.02)
    view = MemoryView(bank.to(device))
    layers = [_operands(20 + l, (B, T), H, k, D, 16) for l in range(L)]   # 16 of 256 slots: collisions
    props, refs = [], []
    for l, (index, w, pred, tgt, beta, ld, m) in enumerate(layers):
        d = _to(device, index, w, pred, tgt, beta, ld)
        props.append(layer_proposal(view, *d, offset=3, layer_idx=l, chunk_size=C, num_layers=L))
        _, decay = hip.proposal_error(d[2], d[3], d[4], d[5])
        addr = ((torch.arange(B).view(B, 1, 1, 1) * H + torch.arange(H).view(1, 1, H, 1)) * S + index)
        keys = addr * (C * L) + (3 + torch.arange(T)).view(1, T, 1, 1) * L + l
        rows = bank.reshape(-1, D)[addr]
        delta = torch_oracle.proposal_delta(rows, w, pred, tgt, beta, ld, torch.ones(B, T),
                                            decay=decay.cpu()[..., None])
        refs.append((addr.reshape(-1), delta.reshape(-1, D), keys.reshape(-1)))
    assert all(isinstance(p, DeferredProposal) for p in props)
    out = commit(view, merge(view, props))
    ref = torch_oracle.commit(bank.reshape(-1, D), *[torch.cat(t) for t in zip(*refs)]).reshape(bank.shape)
    assert out.version == 1 and torch.equal(out.values.cpu(), ref)

    index, w, pred, tgt, beta, ld, _ = layers[1]
    plain = layer_proposal(view, *_to(device, index, w, pred, tgt, beta, ld), offset=3, layer_idx=1,
                           chunk_size=C, num_layers=L, deferred=False)
    assert isinstance(plain, WriteProposal) and plain.deltas.shape == (B * T * H * k, D)
    mixed = commit(view, merge(view, [props[0], plain]))
    assert torch.equal(mixed.values, out.values)


def test_delta_rule_fixed_point(device):
    """A single full-weight write with beta = 1 whose prediction is the row it
    writes moves that row to the target (row + (g-1) row + (t - g row) = t)."""
    B, T, H, D, S = 1, 64, 2, 128, 4096
    bank = torch.randn(B, H, S, D, generator=gen(9)) * 0.02
    slots = torch.randperm(S, generator=gen(10))[:T * H].view(B, T, H, 1)   # distinct rows: one write each
    addr = (torch.arange(H).view(1, 1, H, 1) * S + slots)
    pred = bank.reshape(-1, D)[addr[..., 0]]
    tgt = torch.randn(B, T, H, D, generator=gen(11))
    ld = -torch.rand(B, T, H, 1, generator=gen(12))
    d = _to(device, bank, addr, pred, tgt, torch.ones(B, T, H, 1), ld)
    error, decay = hip.proposal_error(d[2], d[3], d[4], d[5])
    out = hip.commit_proposals(d[0], d[1], None, torch.ones(B, T, H, 1, device=device), error, decay,
                               torch.ones(B, T, device=device))
    torch.testing.assert_close(out.reshape(-1, D)[addr.reshape(-1).to(device)].cpu(), tgt.reshape(-1, D),
                               atol=1e-6, rtol=1e-5)


def test_commit_proposals_config2_epoch(device):
    """One config-2 epoch at full size (B=8, C=512, H=8, k=16, D=128, 65,536
    slots per head, bf16 bank and target): the fused commit equals the unfused
    device path bit for bit, and a sample of rows equals the oracle."""
    B, T, H, k, D, S = 8, 512, 8, 16, 128, 65536
    torch.manual_seed(0)
    bank = (torch.randn(B, H, S, D, device=device) * 0.02).to(torch.bfloat16)
    index = torch.randint(0, S, (B, T, H, k), device=device)
    w = torch.randn(B, T, H, k, device=device).softmax(-1)
    pred = torch.randn(B, T, H, D, device=device) * 0.1
    tgt = (torch.randn(B, T, H, D, device=device) * 0.1).to(torch.bfloat16)
    beta = torch.randn(B, T, H, 1, device=device).sigmoid()
    ld = -F.softplus(torch.randn(B, T, H, 1, device=device) - 4)
    mass = torch.ones(B, T, device=device)
    addr, keys = hip.proposal_keys(bank, index, 0, T, 1, 0)
    error, decay = hip.proposal_error(pred, tgt, beta, ld)
    fused = hip.commit_proposals(bank, addr, keys, w, error, decay, mass)
    rows = hip.gather_rows(bank, index)
    delta = hip.proposal_delta(rows, w, pred, tgt, beta, ld, mass)
    unfused = hip.commit(bank, addr.reshape(-1), delta.reshape(-1, D), keys.reshape(-1))
    assert torch.equal(fused, unfused)
    # oracle on the rows written by the first 64 tokens of request 0, on a compact bank of those rows
    sel = addr[0, :64].reshape(-1).unique()                       # sorted
    all_addr, all_keys = addr.reshape(-1), keys.reshape(-1)
    e_idx = torch.isin(all_addr, sel).nonzero()[:, 0]
    r_idx = e_idx // k
    n = e_idx.numel()
    compact = bank.reshape(-1, D)[sel].float().cpu()
    local = torch.searchsorted(sel, all_addr[e_idx]).cpu()
    delta_c = torch_oracle.proposal_delta(
        compact[local].view(n, 1, 1, D), w.reshape(-1)[e_idx].cpu().view(n, 1, 1),
        pred.reshape(-1, D)[r_idx].cpu().view(n, 1, D), tgt.reshape(-1, D)[r_idx].cpu().view(n, 1, D),
        beta.reshape(-1)[r_idx].cpu().view(n, 1, 1), ld.reshape(-1)[r_idx].cpu().view(n, 1, 1),
        mass.reshape(-1)[r_idx // H].cpu(), decay=decay.reshape(-1)[r_idx].cpu().view(n, 1, 1))
    ref = torch_oracle.commit(compact, local, delta_c.view(n, D), all_keys[e_idx].cpu())
    assert torch.equal(fused.reshape(-1, D)[sel].cpu(), ref.to(torch.bfloat16))


def test_materialised_proposals_commit_gradients(device):
    """A read, two materialised proposals colliding at every address (the
    second with doubled targets and mass 1 - m) and their commit under
    autograd, with cotangents on both the reading and the committed bank: the
    values and the gradients of the bank, route weights, targets, gates and
    mass equal the reference's torch equations' (the protocol and tolerances
    of P/tests/test_native_memory.py:52-93)."""
    B, T, H, k, D, S = 2, 3, 2, 3, 37, 64
    g = gen(91)
    memory = torch.randn(B, H, S, D, generator=g)
    index = torch.randint(0, S, (B, T, H, k), generator=g)
    weights = torch.randn(B, T, H, k, generator=g).softmax(-1)
    target = torch.randn(B, T, H, D, generator=g)
    beta = torch.full((B, T, H, 1), 0.3)
    log_decay = torch.full((B, T, H, 1), -0.12)
    mass = torch.rand(B, T, generator=g)
    read_cot, bank_cot = torch.randn(B, T, H, D, generator=g), torch.randn(B, H, S, D, generator=g)

    def run(dev, native):
        leaves = [t.to(dev).requires_grad_() for t in (memory, weights, target, beta, log_decay, mass)]
        mem, w, tgt, b, ld, m = leaves
        idx = index.to(dev)
        if native:
            view = MemoryView(mem)
            read = hip.snapshot_read(mem, idx, w)
            p1 = layer_proposal(view, idx, w, read, tgt, b, ld, 0, 0, T, 2, mass=m, deferred=False)
            p2 = layer_proposal(view, idx, w, read, tgt * 2, b, ld, 0, 1, T, 2, mass=1 - m, deferred=False)
            new = commit(view, merge(view, [p1, p2])).values
        else:
            read = torch_oracle.read(mem, idx, w)
            rows = torch_oracle.gather_rows(mem, idx)
            addr = torch_oracle.absolute_addresses(mem, idx)
            pos = torch.arange(T).view(1, T, 1, 1)
            d1 = torch_oracle.proposal_delta(rows, w, read, tgt, b, ld, m)
            d2 = torch_oracle.proposal_delta(rows, w, read, tgt * 2, b, ld, 1 - m)
            keys = torch.cat([(addr * (T * 2) + pos * 2 + layer).reshape(-1) for layer in (0, 1)])
            new = torch_oracle.commit(mem.reshape(-1, D), torch.cat([addr.reshape(-1)] * 2),
                                      torch.cat([d1.reshape(-1, D), d2.reshape(-1, D)]), keys).reshape(mem.shape)
        loss = (read * read_cot.to(dev)).sum() + (new * bank_cot.to(dev)).sum()
        grads = torch.autograd.grad(loss, leaves)
        return [t.detach().cpu() for t in (read, new)], [t.cpu() for t in grads]

    (read, new), grads = run(device, True)
    (rread, rnew), rgrads = run("cpu", False)
    torch.testing.assert_close(read, rread, atol=5e-7, rtol=2e-6)
    torch.testing.assert_close(new, rnew, atol=1e-6, rtol=2e-6)
    for name, actual, expected in zip(("memory", "weights", "target", "beta", "log_decay", "mass"), grads, rgrads):
        torch.testing.assert_close(actual, expected, atol=2e-5, rtol=2e-5, msg=lambda m: f"{name}: {m}")
