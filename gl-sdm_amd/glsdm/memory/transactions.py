"""Buffered proposals and the deterministic commit (HIP backend).

Mirrors merge/commit of S/memory/transactions.py:62-97 (S/ =
projects/gl-sdm/src/gl_sdm/): same checks and error messages, same result
(stable key order, sequential fp32 sums per address, old + sum, version + 1).
The commit runs in libglsdm.so; ``donate=True`` updates the view's storage in
place instead of returning a new bank (the old view must not be used again).
"""
import torch

from .state import DeferredProposal, LoggedProposal, MemoryView, WriteBuffer
from .backends import hip
from .proposals import _ones

BACKENDS = ("hip",)


def _check_backend(backend, reference):
    if backend not in BACKENDS:
        raise ValueError("memory backend must be hip (the torch equations are the test oracle)")
    if reference:
        raise ValueError("reference=True selects the dense one-hot oracle, which is not part of the HIP package")


def merge(view, proposals):
    proposals = tuple(proposals)
    if not proposals or any(p.base_version != view.version or p.lineage is not view.lineage for p in proposals):
        raise ValueError("write buffers must be nonempty and use the same snapshot version")
    return WriteBuffer(view.version, proposals, view.lineage)


def _cat(tensors):
    return tensors[0] if len(tensors) == 1 else torch.cat(tensors)


def _materialise(values, p):
    """Deltas [E, D] of a deferred proposal against the snapshot ``values``."""
    D = values.shape[-1]
    rows = hip.gather_flat(values, p.addresses)
    return hip.proposal_delta(rows, p.weights, p.prediction, p.target, p.beta, p.log_decay,
                              p.mass).reshape(-1, D)


def _commit_deferred(view, props, keys, donate):
    """All proposals deferred with one (heads, width): one fused commit."""
    H, k = props[0].heads, props[0].width
    lead = lambda t, tail: t.reshape(-1, *tail)
    idx = _cat([lead(p.addresses, (H, k)) for p in props])
    weights = _cat([lead(p.weights, (H, k)) for p in props])
    pred = _cat([lead(p.prediction, (H, p.prediction.shape[-1])) for p in props])
    targets = [lead(p.target, (H, p.target.shape[-1])) for p in props]
    if len({t.dtype for t in targets}) > 1:
        targets = [t.float() for t in targets]
    beta = _cat([lead(p.beta, (H, 1)) for p in props])
    log_decay = _cat([lead(p.log_decay, (H, 1)) for p in props])
    mass = _cat([p.mass.reshape(-1) for p in props])
    error, decay = hip.proposal_error(pred.contiguous(), _cat(targets).contiguous(), beta.contiguous(),
                                      log_decay.contiguous())
    return hip.commit_proposals(view.values, idx.contiguous(), None if keys is None else keys.reshape(idx.shape),
                                weights.contiguous(), error, decay, mass.contiguous(), donate=donate)


def _commit_logged(view, props, donate):
    """Proposals of one proposal log: one fused commit of their rows.  When they
    are the log's rows in order from its start (the stack's chunk), the log's
    buffers are committed as they lie; else their rows are gathered in the
    buffer's order (which breaks ties of equal keys, as concatenation does)."""
    log = props[0].log
    if any(p.log is not log for p in props):
        raise ValueError("logged proposals commit only with proposals of the same log")
    if any(p.generation != log.generation for p in props):
        raise ValueError("stale proposal: its log's rows were reused after a commit")
    in_order, at = True, 0
    for p in props:
        in_order &= p.start == at
        at += p.rows
    if in_order:
        terms = log.terms(0, at)
    else:
        parts = [log.terms(p.start, p.rows) for p in props]
        terms = tuple(torch.cat(t) for t in zip(*parts))
    addresses, keys, weights, error, decay = terms
    mass = _ones(addresses.shape[:1], addresses.device)
    return hip.commit_proposals(view.values, addresses, keys, weights, error, decay, mass, donate=donate)


def commit(view, buffer, reference=False, backend="hip", donate=False):
    _check_backend(backend, reference)
    if buffer.base_version != view.version or buffer.lineage is not view.lineage:
        raise ValueError("stale memory transaction")
    props = buffer.proposals
    logged = [isinstance(p, LoggedProposal) for p in props]
    if any(logged):
        if not all(logged):
            raise ValueError("logged proposals commit only with proposals of the same log")
        return MemoryView(_commit_logged(view, props, donate), view.version + 1, view.lineage)
    keyed = [p.sort_keys is not None for p in props]
    if any(keyed) and not all(keyed):
        raise ValueError("cannot mix keyed and unkeyed proposals")
    # unkeyed proposals collide in arrival order: the reference sorts them by address
    # with a stable sort, which keeps arrival order within an address
    keys = _cat([p.sort_keys.reshape(-1) for p in props]).contiguous() if all(keyed) else None
    deferred = [isinstance(p, DeferredProposal) for p in props]
    if all(deferred) and len({(p.heads, p.width) for p in props}) == 1:
        updated = _commit_deferred(view, props, keys, donate)
        return MemoryView(updated, view.version + 1, view.lineage)
    idx = _cat([p.addresses.reshape(-1) for p in props])
    D = view.values.shape[-1]
    deltas = [_materialise(view.values, p) if d else p.deltas.reshape(-1, D) for p, d in zip(props, deferred)]
    if len({d.dtype for d in deltas}) > 1:
        deltas = [d.float() for d in deltas]
    delta = _cat(deltas)
    updated = hip.commit(view.values, idx.contiguous(), delta.contiguous(), keys, donate=donate)
    return MemoryView(updated, view.version + 1, view.lineage)
