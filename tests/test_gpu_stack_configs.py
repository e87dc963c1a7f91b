"""The layer stack at the shapes of BASELINE configs[3] and configs[4] on the
GPU, against the oracle (S/ = projects/gl-sdm/src/gl_sdm/): 16 layers
alternating local (window 512) and global, d_model 1024, 16 memory heads of
64, top-k 16 reads and writes, the 512-token clock, 2^18 (config 4) and 2^20
bf16 (config 5) slots per head.  Batch and length are reduced where noted;
head, route and bank shapes are the configs' own.

* Shadow (``_stack_oracle.Shadow``): every memory step of the native stack --
  each routed read of every global layer and chunk, each proposal, each
  commit -- is re-run by the oracle on the native step's own inputs; routes
  must agree bit for bit, readings within fp32 rounding (1e-6 / 1e-5), the
  committed bank within the rounding of the deltas' exponential (fp32 bank
  2e-6 / 2e-5; bf16 bank one bf16 ulp).
* End to end: the stack against the same stack on the oracle's memory steps
  (P/tests/test_layer_stack.py:143-176 style; relative L2 as
  S/experiments/verify.py:17-28 bounds bf16, 5%), and decode against one
  prefill (S/model.py:84-96).
"""
import copy

import pytest
import torch

from glsdm.model import create_model
from _stack_oracle import RouteLog, Shadow, check_ties, compare_routes, oracle_memory

pytestmark = pytest.mark.gpu

STACK = dict(arch_type="gl_sdm", vocab_size=32000, hidden_size=1024, head_dim=64, num_hidden_layers=16,
             dtype="bfloat16", gl_layer_pattern=["local", "global"], gl_reads=16, gl_writes=16,
             gl_chunk_size=512, gl_local_window=512, gl_memory_backend="hip", residual_dtype="float32")
CONFIG4 = dict(STACK, gl_slots=262144)
CONFIG5 = dict(STACK, gl_slots=1048576, gl_state_dtype="bfloat16")
BF16_BANK = dict(atol=1e-5, rtol=2 ** -7)          # one bf16 ulp


def build(cfg, device, seed=0):
    torch.manual_seed(seed)
    return create_model(cfg).to(device).eval()


def tokens(B, T, seed):
    return torch.randint(32000, (B, T), generator=torch.Generator().manual_seed(seed))


def rel_l2(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-12)).item()


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_config4_every_memory_step_matches_the_oracle(device, dtype):
    """Config 4 (B = 1, T = 1024: two chunks, two commits of 2^20 entries)."""
    model = build(dict(CONFIG4, dtype=dtype), device)
    x = tokens(1, 1024, 10).to(device)
    with Shadow().watch() as shadow:
        logits, cache = model.prefill(x)
    print(f"config4 {dtype}: shadowed {shadow.reads} reads, {shadow.proposals} proposals, {shadow.commits} commits",
          flush=True)
    assert (shadow.reads, shadow.proposals, shadow.commits) == (32, 16, 2)
    assert torch.isfinite(logits).all() and cache[0].view.version == 2


FP32_LOGITS = dict(atol=5e-4, rtol=3e-3)           # S/experiments/verify.py:103


@pytest.mark.parametrize("dtype,tie_rel", [("float32", 1e-5), ("bfloat16", 2 ** -7)])
def test_config4_stack_matches_oracle_memory_stack(device, dtype, tie_rel):
    """The whole prefill against the same stack on the oracle's memory steps:
    routes agree bit for bit in the stack's causal order (chunk, layer, read
    before write) until the first disagreement, which must be a tie at the
    path's rounding level (fp32: 1e-5 relative; bf16 projections: one bf16
    ulp).  Past such a tie the two random-init stacks legitimately diverge
    (every later route and the committed bank of that request depend on it)."""
    model = build(dict(CONFIG4, dtype=dtype), device)
    oracle = copy.deepcopy(model)
    x = tokens(1, 1024, 11).to(device)
    a, b = RouteLog(512), RouteLog(512)
    with a.watch(model):
        logits, _ = model.prefill(x)
    with oracle_memory(), b.watch(oracle):
        ref_logits, _ = oracle.prefill(x)
    first, bad_rows, bad_requests, keys = compare_routes(a, b)
    check_ties(a, b, bad_rows, tie_rel)
    print(f"config4 {dtype}: first route disagreement in group {first} ({len(bad_rows)} tied rows of "
          f"{keys} positions x 16 heads); logits rel L2 {rel_l2(logits, ref_logits):.3e}", flush=True)
    assert torch.isfinite(logits).all()
    if not bad_requests:
        torch.testing.assert_close(logits, ref_logits, **FP32_LOGITS)


def test_config5_decode_every_memory_step_matches_the_oracle(device):
    """Config 5's bank (2^20 bf16 slots per head), 2 streams: an 8-token prompt,
    then 520 one-token decode steps, which cross the 512-token commit and the
    local layers' KV window buffer (512 rows of room: reallocated once); every
    memory step shadowed, then the decode logits against one prefill."""
    model = build(CONFIG5, device)
    B, P, steps = 2, 8, 520
    seq = tokens(B, P + steps, 12).to(device)
    with Shadow(bank_tol=BF16_BANK).watch() as shadow:
        _, cache = model.prefill(seq[:, :P])
        outs = [model.decode(seq[:, t:t + 1], cache)[0] for t in range(P, P + steps)]
    print(f"config5 decode: shadowed {shadow.reads} reads, {shadow.commits} commits", flush=True)
    assert shadow.commits == 1 and shadow.reads == (1 + steps) * 16
    assert cache[0].tokens == P + steps and cache[0].view.version == 1
    local = cache[0].local[0]
    assert local["kbuf"].shape[2] > 520 and local["k"].shape[2] == 511    # reallocated window buffer


def test_config5_decode_agrees_with_one_prefill(device):
    """Config 5's bank, 2 streams: 520 one-token decode steps after an 8-token
    prompt against one prefill of all 528 tokens (fp32 weights; the two runs'
    GEMMs differ in shape, so their scores differ by rounding): routes agree
    in causal order until the first disagreement, a rounding-level tie, and a
    stream whose routes all agree has the same logits and committed bank."""
    model = build(dict(CONFIG5, dtype="float32"), device)
    B, P, steps = 2, 8, 520
    seq = tokens(B, P + steps, 12).to(device)
    a, b = RouteLog(512), RouteLog(512)
    with a.watch(model):
        _, cache = model.prefill(seq[:, :P])
        outs = torch.cat([model.decode(seq[:, t:t + 1], cache)[0] for t in range(P, P + steps)], 1)
    with b.watch(model):
        full, full_cache = model.prefill(seq)
    first, bad_rows, bad_requests, keys = compare_routes(a, b)
    check_ties(a, b, bad_rows, 1e-5)
    same = [r for r in range(B) if r not in bad_requests]
    print(f"config5 decode vs prefill: first route disagreement in group {first} ({len(bad_rows)} tied rows); "
          f"streams with identical routes {same}", flush=True)
    assert torch.isfinite(outs).all()
    if same:
        torch.testing.assert_close(outs[same], full[same, P:], **FP32_LOGITS)
        torch.testing.assert_close(cache[0].view.values[same], full_cache[0].view.values[same], **BF16_BANK)


def test_config5_full_batch_decode_continues_prefill(device):
    """All 64 streams of config 5 (bf16 2^20-slot snapshots, 128 GiB): a
    510-token prompt then 4 decode steps across the 512-token commit against
    one prefill of the 514 tokens (fp32 weights).  Routes agree in causal
    order until a rounding-level tie (its scores recorded in a second,
    identical pass: all scores of both runs would be ~70 GB), and every stream
    whose routes all agree has the same logits and sampled bank rows."""
    model = build(dict(CONFIG5, dtype="float32"), device)
    B, P, T = 64, 510, 514
    seq = tokens(B, T, 13).to(device)
    g = torch.Generator().manual_seed(14)
    sample = torch.randperm(1 << 20, generator=g)[:4096].to(device)

    def runs(keep):
        a, b = RouteLog(512, keep_scores=keep), RouteLog(512, keep_scores=keep)
        with b.watch(model):
            full, cache = model.prefill(seq)
        full, full_rows = full[:, P:].clone(), cache[0].view.values[:, :, sample].clone()
        assert cache[0].view.version == 1
        del cache
        torch.cuda.empty_cache()
        with a.watch(model):
            _, cache = model.prefill(seq[:, :P])
            outs = torch.cat([model.decode(seq[:, t:t + 1], cache)[0] for t in range(P, T)], 1)
        assert cache[0].view.version == 1 and cache[0].tokens == T
        rows = cache[0].view.values[:, :, sample].clone()
        del cache
        torch.cuda.empty_cache()
        return a, b, outs, full, rows, full_rows

    a, b, outs, full, rows, full_rows = runs(False)
    first, bad_rows, bad_requests, keys = compare_routes(a, b)
    if first is not None:
        a2, b2, outs2, *_ = runs({first})
        assert torch.equal(outs2, outs)                    # the second pass repeats the first bit for bit
        assert compare_routes(a2, b2)[1] == bad_rows
        check_ties(a2, b2, bad_rows, 1e-5)
    same = [r for r in range(B) if r not in bad_requests]
    print(f"config5 x64 decode vs prefill: first route disagreement in group {first} ({len(bad_rows)} tied rows); "
          f"{len(same)} of {B} streams with identical routes", flush=True)
    assert len(same) > B // 2
    torch.testing.assert_close(outs[same], full[same], **FP32_LOGITS)
    torch.testing.assert_close(rows[same], full_rows[same], **BF16_BANK)
