"""The proposal log (the stack's inference write path) vs the unfused HIP steps
and the deferred-proposal path.

``glsdm_proposal_append`` must write, bit for bit, what the write gates,
``glsdm_proposal_keys`` and ``glsdm_proposal_error`` produce one after another
(the gates through ``write_gates``, whose tensor-op parity is
tests/test_gpu_stack_ops.py's); its gates are also checked against the
reference's torch formulas (S/layers/global_layer.py:48-49) within an ulp.  A
stack run with the log must equal the same run with deferred proposals bit
for bit (banks and logits), across prefill, decode and commits; the log's
misuse (stale rows, mixed kinds, overflow) raises.
"""
import copy

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from glsdm.model import create_model
from glsdm.layers.global_layer import write_gates
from glsdm.memory import LoggedProposal, MemoryView, ProposalLog, commit, layer_proposal, merge
from glsdm.memory.backends import hip
from _util import gen

pytestmark = pytest.mark.gpu


def _operands(seed, B, T, H, k, D, S, dtype):
    g = gen(seed)
    index = torch.randint(0, S, (B, T, H, k), generator=g)
    weights = torch.randn(B, T, H, k, generator=g).softmax(-1)
    prediction = torch.randn(B, T, H, D, generator=g) * 0.1
    target = (torch.randn(B, T, H, D, generator=g) * 0.1).to(dtype)
    # gate projections over a wide range: both softplus branches (d - 4 above and below 20)
    b_lin = (torch.randn(B, T, H, generator=g) * 4).to(dtype)
    d_lin = (torch.randn(B, T, H, generator=g) * 15).to(dtype)
    return index, weights, prediction, target, b_lin, d_lin


def _ulps(a, b):
    a64, b64 = a.double().numpy(), b.double().numpy()
    return np.abs(a64 - b64) / np.spacing(np.abs(b.float().numpy())).astype(np.float64)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float32, 128), (torch.float32, 37)])
def test_append_matches_unfused_steps(device, dtype, D):
    B, H, k, S, C, L = 3, 4, 8, 256, 16, 6
    values = torch.zeros(B, H, S, D, device=device)
    view = MemoryView(values)
    log = ProposalLog(2 * B * C * H, H, k, D, device)
    expect = []
    for n, (T, offset, layer) in enumerate([(5, 3, 2), (1, 9, 5), (C, 0, 0)]):
        ops = [t.to(device) for t in _operands(n, B, T, H, k, D, S, dtype)]
        index, weights, prediction, target, b_lin, d_lin = ops
        p = log.append(view, index, weights, prediction, target, b_lin, d_lin, offset, layer, C, L)
        assert isinstance(p, LoggedProposal) and p.rows == B * T * H
        beta, log_decay = write_gates(b_lin, d_lin)
        addresses, keys = hip.proposal_keys(values, index, offset, C, L, layer)
        error, decay = hip.proposal_error(prediction, target, beta, log_decay)
        expect.append((p, addresses, keys, weights, error, decay))
        # the gates against the reference's torch formulas
        ref_beta = b_lin.cpu().float().sigmoid()
        ref_ld = -F.softplus(d_lin.cpu().float() - 4)
        assert _ulps(beta[..., 0].cpu(), ref_beta).max() <= 2.0
        assert _ulps(log_decay[..., 0].cpu(), ref_ld).max() <= 2.0
    assert log.fill == sum(p.rows for p, *_ in expect)
    for p, addresses, keys, weights, error, decay in expect:
        a, kk, w, e, dc = log.terms(p.start, p.rows)
        n = p.rows // H
        assert torch.equal(a, addresses.view(n, H, k)) and torch.equal(kk, keys.view(n, H, k))
        assert torch.equal(w, weights.view(n, H, k))
        assert torch.equal(e, error.view(n, H, D)) and torch.equal(dc, decay.view(n, H))
        assert torch.equal(p.sort_keys, keys.reshape(-1))


def _logged_and_deferred(device, seed, B=2, T=3, H=4, k=8, D=64, S=256, dtype=torch.float32):
    """Three proposals on one snapshot, as a log and as deferred proposals."""
    g = gen(seed)
    values = (torch.randn(B, H, S, D, generator=g) * 0.1).to(device)
    view = MemoryView(values)
    log = ProposalLog(3 * B * T * H, H, k, D, device)
    logged, deferred = [], []
    for layer in range(3):
        ops = [t.to(device) for t in _operands(seed * 10 + layer, B, T, H, k, D, S, dtype)]
        index, weights, prediction, target, b_lin, d_lin = ops
        logged.append(log.append(view, index, weights, prediction, target, b_lin, d_lin, 0, layer, T, 3))
        beta, log_decay = write_gates(b_lin, d_lin)
        deferred.append(layer_proposal(view, index, weights, prediction, target, beta, log_decay, 0, layer, T, 3))
    return view, log, logged, deferred


@pytest.mark.parametrize("order", ["log", "reversed"])
def test_logged_commit_equals_deferred_commit(device, order):
    view, log, logged, deferred = _logged_and_deferred(device, 1)
    if order == "reversed":
        logged, deferred = logged[::-1], deferred[::-1]
    got = commit(view, merge(view, logged))
    ref = commit(view, merge(view, deferred))
    assert got.version == ref.version == 1
    assert torch.equal(got.values, ref.values)
    assert not torch.equal(got.values, view.values)


def test_logged_commit_misuse_raises(device):
    view, log, logged, deferred = _logged_and_deferred(device, 2)
    with pytest.raises(ValueError, match="same log"):
        commit(view, merge(view, logged[:1] + deferred[1:]))
    _, other, other_logged, _ = _logged_and_deferred(device, 3)
    with pytest.raises(ValueError, match="same log"):
        commit(view, merge(view, logged[:1] + [LoggedProposal(view.version, view.lineage, other, other.generation,
                                                              0, other_logged[0].rows)]))
    log.clear()
    with pytest.raises(ValueError, match="stale proposal"):
        commit(view, merge(view, logged))
    # a full log refuses the next proposal
    ops = [t.to(device) for t in _operands(9, 2, 3, 4, 8, 64, 256, torch.float32)]
    for layer in range(3):
        log.append(view, *ops, 0, layer, 3, 3)
    with pytest.raises(RuntimeError, match="proposal log full"):
        log.append(view, *ops, 0, 0, 3, 3)


def _stack_config(**changes):
    base = dict(arch_type="gl_sdm", vocab_size=64, hidden_size=64, head_dim=16, num_hidden_layers=8,
                dtype="float32", gl_layer_pattern=["local", "global"], gl_slots=256, gl_reads=4, gl_writes=4,
                gl_chunk_size=4, gl_local_window=6, gl_memory_backend="hip", seq_len=16)
    return {**base, **changes}


@pytest.mark.parametrize("cfg", [_stack_config(), _stack_config(dtype="bfloat16", gl_state_dtype="bfloat16",
                                                                 gl_slots=65536, gl_writes=16)],
                         ids=["fp32", "bf16"])
def test_stack_with_log_equals_deferred(device, cfg):
    torch.manual_seed(7)
    model = create_model(cfg).to(device).eval()
    plain = copy.deepcopy(model)
    plain.cfg = {**plain.cfg, "gl_proposal_log": False}
    x = torch.randint(cfg["vocab_size"], (3, 14), generator=gen(4)).to(device)
    outs = {}
    for name, m in (("log", model), ("deferred", plain)):
        parts = []
        first, cache = m.prefill(x[:, :6])        # one commit, two tokens pending
        parts.append(first)
        for t in range(6, 14):                    # decode across two more commits
            out, cache = m.decode(x[:, t:t + 1], cache)
            parts.append(out)
        outs[name] = (torch.cat(parts, 1), cache)
    (logits, cache), (ref_logits, ref_cache) = outs["log"], outs["deferred"]
    assert cache[0].view.version == ref_cache[0].view.version == 3
    assert cache[0].log is not None and ref_cache[0].log is None
    # two pending tokens x 3 requests x 4 global layers x heads
    assert cache[0].log.fill == 2 * 3 * 4 * (cfg["hidden_size"] // cfg["head_dim"])
    assert torch.equal(cache[0].view.values, ref_cache[0].view.values)
    assert torch.equal(logits, ref_logits)
