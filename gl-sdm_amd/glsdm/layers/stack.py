"""The physical layer stack and its chunk clock (S/layers/stack.py:12-71,
S/ = projects/gl-sdm/src/gl_sdm/).

Every layer runs once per chunk of ``gl_chunk_size`` tokens.  All global layers
read and propose against the chunk-start snapshot (no write is visible between
layers); at each absolute multiple of the chunk size the pending proposals are
merged and committed, and local KV history survives the commit.  A request
cache carries the token count and the proposals of an unfinished chunk across
prefill/decode calls.  The last chunk of a stateless call proposes nothing.

Outside autograd the commit updates the cache's own snapshot storage in place
(``gl_commit_in_place``, default on): the snapshot of a chunk is dropped at
its commit anyway, and a full-bank copy per commit is the cost the fused
commit exists to avoid.  Outside autograd the global layers also append
their proposals to the cache's proposal log (``gl_proposal_log``, default
on): one chunk of preallocated device rows that the commit reads as one
proposal, so a decode chunk's thousands of one-token proposals are never
concatenated.
"""
import torch

from ..memory import LoggedProposal, commit, merge
from ..memory.proposals import ProposalLog
from .block import Block, zero
from .global_layer import GlobalLayer


def make_layers(cfg):
    pattern = cfg["gl_layer_pattern"]
    count = cfg["num_hidden_layers"]
    if (not pattern or any(kind not in {"local", "global"} for kind in pattern) or "global" not in pattern
            or count % len(pattern)):
        raise ValueError("gl_layer_pattern must include global and repeat to cover num_hidden_layers")
    if cfg.get("gl_max_steps", 1) != 1 or cfg.get("gl_reasoning", "fixed") != "fixed":
        raise ValueError("the physical GL-SDM stack has no reasoning loops")
    if cfg.get("gl_chunk_size", 512) < 1 or cfg.get("gl_local_window", 512) < 1:
        raise ValueError("positive GL-SDM chunk and local window required")
    if cfg.get("gl_cuda_graph", False):
        raise ValueError("physical GL-SDM stack currently uses ordinary training, not legacy loop CUDA graphs")
    local = {**cfg, "arch_type": "transformer", "attention_window": cfg.get("gl_local_window", 512)}
    return [GlobalLayer(cfg) if pattern[i % len(pattern)] == "global" else Block(local, i) for i in range(count)]


def _proposal_log(model, cache, batch, chunk):
    """The cache's proposal log, sized for one chunk of every global layer's
    proposals (a new one when the cache has none, or none of this shape)."""
    layers = [b for b in model.blocks if isinstance(b, GlobalLayer)]
    router = layers[0].attn
    H, k, D = router.heads, router.num_writes, cache.view.values.shape[-1]
    rows = len(layers) * chunk * batch * H
    device = cache.view.values.device
    if cache.log is None or (not cache.pending and not cache.log.fits(rows, H, k, D, device)):
        cache.log = ProposalLog(rows, H, k, D, device)
    return cache.log


def _all_logged(cache):
    """Whether every pending proposal of the cache is a ``LoggedProposal``.  The answer
    is kept with the pending tuple it was computed for (tuples are immutable, so the
    same object has the same contents): a decode step would otherwise walk the
    chunk's thousands of pending proposals every time."""
    memo = getattr(cache, "_all_logged", None)
    if memo is not None and memo[0] is cache.pending:
        return memo[1]
    flag = all(isinstance(p, LoggedProposal) for p in cache.pending)
    cache._all_logged = (cache.pending, flag)
    return flag


def forward(model, inputs, cache=None):
    """Run embedded ``inputs [B, T, dim]`` through the stack; returns
    ``(hidden [B, T, dim], reg, align)``.  ``cache`` is a request cache
    (``MemoryBank.new_cache``); without one the call is stateless."""
    B, T, _ = inputs.shape
    if min(B, T) < 1:
        raise ValueError("GL-SDM requires a nonempty token batch")
    retain = cache is not None
    cache = model.bank.new_cache(B) if cache is None else cache
    model.bank.validate_cache(cache, B)
    C = model.cfg.get("gl_chunk_size", 512)
    layers = len(model.blocks)
    in_place = model.cfg.get("gl_commit_in_place", True) and not torch.is_grad_enabled()
    # proposal log: inference on the device, and no pending proposal of another kind
    use_log = (model.cfg.get("gl_proposal_log", True) and not torch.is_grad_enabled() and cache.view.values.is_cuda
               and any(isinstance(b, GlobalLayer) for b in model.blocks)
               and _all_logged(cache))
    outputs = []
    reg = align = None          # sums of the blocks' terms that are not the shared zeros
    position = 0
    while position < T:
        offset = cache.tokens % C
        length = min(C - offset, T - position)
        snapshot = cache.view
        writes = retain or position + length < T
        proposals = list(cache.pending)
        log = _proposal_log(model, cache, B, C) if use_log and writes else None
        x = inputs[:, position:position + length]
        for i, block in enumerate(model.blocks):
            if isinstance(block, GlobalLayer):
                x, r, a = block(x, snapshot)
                if writes:
                    proposals.append(block.propose(x, snapshot, offset, i, C, layers, log=log))
            else:
                x, r, a = block(x, cache.local.setdefault(i, {}))
            if r is not zero(r) or a is not zero(a):     # the baseline's are the shared zeros: nothing to add
                term = r * (length / T)
                reg = term if reg is None else reg + term
                align = a if align is None else align + a
        cache.tokens += length
        if cache.tokens % C == 0 and writes:
            cache.view = commit(snapshot, merge(snapshot, proposals), donate=in_place)
            cache.pending = ()
            if cache.log is not None:
                cache.log.clear()          # its rows are committed: the next chunk reuses them
        else:
            logged = _all_logged(cache) and all(isinstance(p, LoggedProposal) for p in proposals[len(cache.pending):])
            cache.pending = tuple(proposals)
            cache._all_logged = (cache.pending, logged)
        outputs.append(x)
        position += length
    # one chunk (every decode step) needs no concatenation; with only zero terms the
    # regularisers are the shared read-only zero (no fill or division launches)
    hidden = outputs[0] if len(outputs) == 1 else torch.cat(outputs, 1)
    z = zero(inputs)
    return hidden, z if reg is None else reg / layers, z if align is None else align / layers
