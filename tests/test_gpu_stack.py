"""The layer stack on the HIP memory operator vs the same stack with the CPU
oracle's memory steps (``tests/_stack_oracle.py``), and the stack properties
of P/tests/test_layer_stack.py:35-85 (P/ = projects/gl-sdm/): one snapshot
per chunk shared by every global layer, chunked prefill/decode equal to one
pass, causality, and proposals summed without averaging.

Tolerances: fp32 logits within the reference's fp32 verification bounds
(atol 5e-4, rtol 3e-3, S/experiments/verify.py:103); the committed bank
within fp32 rounding (the oracle and the kernels agree to a few ulp on the
reads that feed the deltas).  Routes are discrete: the first global layer's
routes are compared bit for bit, later ones through the outputs they feed.
bf16 stacks are bounded by relative L2 error (5%, verify.py:17-28), since a
rounding-level score difference can move a later layer's route.
"""
import copy
from unittest.mock import patch

import pytest
import torch

from glsdm.model import create_model
from glsdm.layers.global_layer import GlobalLayer
from glsdm.memory import DeferredProposal, routing
from glsdm.memory.backends import hip
from glsdm.memory.transactions import _materialise
from _stack_oracle import oracle_memory

pytestmark = pytest.mark.gpu


def config(**changes):
    base = dict(arch_type="gl_sdm", vocab_size=64, hidden_size=32, head_dim=16, num_hidden_layers=16,
                dtype="float32", gl_layer_pattern=["local", "local", "global", "local"], gl_slots=16, gl_reads=2,
                gl_writes=2, gl_chunk_size=4, gl_local_window=6, gl_memory_backend="hip", seq_len=9)
    return {**base, **changes}


def models(cfg, device, seed=1234):
    torch.manual_seed(seed)
    model = create_model(cfg).to(device).eval()
    return model, copy.deepcopy(model)


def rel_l2(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-12)).item()


@pytest.mark.parametrize("cfg", [
    config(),
    config(hidden_size=64, head_dim=32, gl_slots=64, gl_reads=4, gl_writes=4, gl_chunk_size=8,
           gl_local_window=8, num_hidden_layers=8, gl_layer_pattern=["local", "global"]),
    # P/tests/test_layer_stack.py:180-186: the large route (2^18 slots, 8 reads and writes)
    config(gl_slots=262144, gl_reads=8, gl_writes=8),
], ids=["tiny", "small", "large_route"])
def test_stack_prefill_matches_oracle_memory(device, cfg):
    model, oracle = models(cfg, device)
    x = torch.randint(cfg["vocab_size"], (2, 23), generator=torch.Generator().manual_seed(0)).to(device)
    with patch.object(hip, "routed_snapshot_read", wraps=hip.routed_snapshot_read) as reads, \
            patch.object(hip, "commit_proposals", wraps=hip.commit_proposals) as commits:
        logits, cache = model.prefill(x)
    assert reads.call_count > 0 and commits.call_count > 0      # the native operator ran
    with oracle_memory():
        ref_logits, ref_cache = oracle.prefill(x)
    torch.testing.assert_close(logits, ref_logits, atol=5e-4, rtol=3e-3)
    assert cache[0].view.version == ref_cache[0].view.version == 23 // cfg["gl_chunk_size"] + (
        23 % cfg["gl_chunk_size"] == 0)
    torch.testing.assert_close(cache[0].view.values, ref_cache[0].view.values, atol=2e-6, rtol=2e-5)


def test_first_global_layer_routes_are_bit_exact(device):
    cfg = config(gl_slots=256, gl_reads=8, gl_writes=8)
    model, _ = models(cfg, device)
    layer = model.blocks[2]
    view = model.bank.snapshot(2)
    x = torch.randn(2, 4, 32, device=device)
    with torch.no_grad():
        scores = layer.attn.q(layer.norm1(x)).float().view(2, 4, 2, -1)
        out, idx, w = routing.routed_read(layer, view.values, scores, 8)
        with oracle_memory():
            r_out, r_idx, r_w = routing.routed_read(layer, view.values, scores, 8)
    assert torch.equal(idx, r_idx)
    torch.testing.assert_close(w, r_w, atol=2e-7, rtol=2e-6)
    torch.testing.assert_close(out, r_out, atol=1e-6, rtol=1e-5)


def test_bf16_stack_matches_oracle_memory(device):
    cfg = config(dtype="bfloat16", residual_dtype="float32")
    model, oracle = models(cfg, device)
    x = torch.randint(64, (2, 23), generator=torch.Generator().manual_seed(1)).to(device)
    logits, cache = model.prefill(x)
    with oracle_memory():
        ref_logits, ref_cache = oracle.prefill(x)
    assert torch.isfinite(logits).all()
    assert rel_l2(logits, ref_logits) < 0.05
    assert rel_l2(cache[0].view.values, ref_cache[0].view.values) < 0.05


def test_chunk_snapshot_is_shared_across_depth_and_local_history_survives_commit(device):
    model, _ = models(config(), device)
    records = []
    original = GlobalLayer.forward

    def observe(layer, x, snapshot, physical=None):
        records.append((snapshot.version, id(snapshot)))
        return original(layer, x, snapshot, physical)

    x = torch.randint(64, (1, 9), generator=torch.Generator().manual_seed(2)).to(device)
    with patch.object(GlobalLayer, "forward", observe):
        full, full_cache = model.prefill(x)
        cache = model.new_cache(1)
        parts = []
        for start, end in [(0, 3), (3, 4), (4, 7), (7, 9)]:
            logits, cache = model.prefill(x[:, start:end], cache)
            parts.append(logits)
            if end == 4:
                assert cache[0].view.version == 1
                assert cache[0].local[0]["tokens"] == 4 and cache[0].local[0]["k"].shape[2] == 4
    for chunk in range(3):
        group = records[chunk * 4:(chunk + 1) * 4]
        assert len(set(group)) == 1 and group[0][0] == chunk
    torch.testing.assert_close(torch.cat(parts, 1), full, atol=1e-4, rtol=3e-3)
    torch.testing.assert_close(cache[0].view.values, full_cache[0].view.values, atol=2e-6, rtol=2e-5)
    assert cache[0].local[0]["tokens"] == 9 and cache[0].local[0]["k"].shape[2] == 5


@pytest.mark.parametrize("cfg", [config(), config(gl_slots=262144, gl_reads=8, gl_writes=8)],
                         ids=["tiny", "large_route"])
def test_decode_continues_prefill(device, cfg):
    model, _ = models(cfg, device)
    x = torch.randint(64, (2, 21), generator=torch.Generator().manual_seed(3)).to(device)
    full, full_cache = model.prefill(x)
    first, cache = model.prefill(x[:, :17])
    second, cache = model.prefill(x[:, 17:-2], cache)
    third, cache = model.decode(x[:, -2:-1], cache)
    fourth, cache = model.decode(x[:, -1:], cache)
    torch.testing.assert_close(torch.cat((first, second, third, fourth), 1), full, atol=1e-4, rtol=3e-3)
    assert cache[0].tokens == 21 and cache[0].view.version == full_cache[0].view.version == 5
    with pytest.raises(ValueError, match="one token"):
        model.decode(x[:, :2], cache)


def test_causality(device):
    model, _ = models(config(), device)
    x = torch.randint(64, (1, 9), generator=torch.Generator().manual_seed(4)).to(device)
    with torch.no_grad():
        full = model.head(model.hidden(x)[0])
        for start in (2, 4, 7):
            changed = x.clone()
            changed[:, start:] = (changed[:, start:] + 1) % 64
            out = model.head(model.hidden(changed)[0])
            torch.testing.assert_close(out[:, :start], full[:, :start], atol=1e-4, rtol=2e-3)


def test_identical_token_proposals_are_summed_without_chunk_averaging(device):
    model, _ = models(config(), device)
    layer = model.blocks[2]
    with torch.no_grad():
        view = model.bank.snapshot(1)
        x = torch.randn(1, 1, 32, device=device)
        single = layer.propose(x, view, 0, 2, 4, 16)
        repeated = layer.propose(x.expand(-1, 2, -1).contiguous(), view, 0, 2, 4, 16)
        longer = layer.propose(x, view, 0, 2, 128, 16)
        assert isinstance(single, DeferredProposal)
        d1, d2, d3 = (_materialise(view.values, p).reshape(p.addresses.shape[1], -1, 16)
                      for p in (single, repeated, longer))
    torch.testing.assert_close(d2[0], d1[0])
    torch.testing.assert_close(d2[1], d1[0])
    torch.testing.assert_close(d3, d1)
    assert torch.equal(repeated.sort_keys[0, 1] - repeated.sort_keys[0, 0],
                       torch.full_like(repeated.sort_keys[0, 0], 16))


def test_training_read_gradients_match_oracle(device):
    """One chunk (no commit inside the sequence): every parameter's gradient,
    the learned bank's included, through the HIP read backward."""
    cfg = config(gl_chunk_size=16)
    model, oracle = models(cfg, device)
    model.train()
    oracle.train()
    g = torch.Generator().manual_seed(5)
    x = torch.randint(64, (2, 12), generator=g).to(device)
    t = torch.randint(64, (2, 12), generator=g).to(device)
    loss, _, _ = model(x, t)
    loss.backward()
    with oracle_memory():
        ref_loss, _, _ = oracle(x, t)
        ref_loss.backward()
    torch.testing.assert_close(loss, ref_loss, atol=1e-4, rtol=1e-5)
    for (name, p), (_, r) in zip(model.named_parameters(), oracle.named_parameters()):
        # the write projections (k, v, beta, decay) get none: nothing commits inside the sequence
        parts = name.split(".")
        write_proj = (parts[0] == "blocks" and isinstance(model.blocks[int(parts[1])], GlobalLayer)
                      and parts[2] == "attn" and parts[3] in ("k", "v", "beta", "decay"))
        assert p.grad is None and r.grad is None if write_proj else p.grad is not None and r.grad is not None, name
        if p.grad is not None:
            torch.testing.assert_close(p.grad, r.grad, atol=1e-5, rtol=5e-3, msg=lambda m: f"{name}: {m}")
    assert model.bank.memory.grad.abs().sum() > 0


def test_delayed_write_gradients_for_every_global_layer(device):
    """P/tests/test_layer_stack.py:64-82: a loss on the last token's hidden
    state reaches the write projections of every global layer (through the
    commits of the earlier chunks) and the learned bank."""
    torch.manual_seed(7)
    model = create_model(config()).to(device).train()
    x = torch.randint(64, (1, 9), device=device)
    model.hidden(x)[0][:, -1].square().sum().backward()
    assert model.bank.memory.grad is not None
    for block in model.blocks:
        if isinstance(block, GlobalLayer):
            for name in ("k", "v", "beta", "decay"):
                gradient = getattr(block.attn, name).weight.grad
                assert gradient is not None and torch.isfinite(gradient).all() and gradient.abs().sum() > 0, name


@pytest.mark.parametrize("tokens", [12, 9])
def test_training_write_gradients_match_oracle(device, tokens):
    """Three chunks of 4 tokens (the last one partial for 9): the first two
    propose and commit, so every parameter's gradient -- the write projections'
    and the learned bank's included -- flows through the proposal deltas, the
    commit and the next chunk's reads, against the reference's torch
    equations."""
    model, oracle = models(config(), device)
    model.train()
    oracle.train()
    g = torch.Generator().manual_seed(6)
    x = torch.randint(64, (2, tokens), generator=g).to(device)
    t = torch.randint(64, (2, tokens), generator=g).to(device)
    loss, _, _ = model(x, t)
    loss.backward()
    with oracle_memory():
        ref_loss, _, _ = oracle(x, t)
        ref_loss.backward()
    torch.testing.assert_close(loss, ref_loss, atol=1e-4, rtol=1e-5)
    for (name, p), (_, r) in zip(model.named_parameters(), oracle.named_parameters()):
        assert (p.grad is None) == (r.grad is None), name
        if p.grad is not None:
            torch.testing.assert_close(p.grad, r.grad, atol=1e-5, rtol=5e-3, msg=lambda m: f"{name}: {m}")
    writes = [b.attn.v.weight.grad for b in model.blocks if isinstance(b, GlobalLayer)]
    assert all(w is not None and w.abs().sum() > 0 for w in writes)
    assert model.bank.memory.grad.abs().sum() > 0
