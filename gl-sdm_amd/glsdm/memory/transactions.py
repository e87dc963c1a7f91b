"""Buffered proposals and the deterministic commit (HIP backend).

Mirrors merge/commit of S/memory/transactions.py:62-97 (S/ =
projects/gl-sdm/src/gl_sdm/): same checks and error messages, same result
(stable key order, sequential fp32 sums per address, old + sum, version + 1).
The commit runs in libglsdm.so; ``donate=True`` updates the view's storage in
place instead of returning a new bank (the old view must not be used again).
"""
import torch

from .state import MemoryView, WriteBuffer
from .backends import hip

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


def commit(view, buffer, reference=False, backend="hip", donate=False):
    _check_backend(backend, reference)
    if buffer.base_version != view.version or buffer.lineage is not view.lineage:
        raise ValueError("stale memory transaction")
    props = buffer.proposals
    keyed = [p.sort_keys is not None for p in props]
    if any(keyed) and not all(keyed):
        raise ValueError("cannot mix keyed and unkeyed proposals")
    idx = _cat([p.addresses.reshape(-1) for p in props])
    D = view.values.shape[-1]
    deltas = [p.deltas.reshape(-1, D) for p in props]
    if len({d.dtype for d in deltas}) > 1:
        deltas = [d.float() for d in deltas]
    delta = _cat(deltas)
    # unkeyed proposals collide in arrival order: the reference sorts them by address
    # with a stable sort, which keeps arrival order within an address
    keys = _cat([p.sort_keys.reshape(-1) for p in props]) if all(keyed) else None
    updated = hip.commit(view.values, idx.contiguous(), delta.contiguous(),
                         None if keys is None else keys.contiguous(), donate=donate)
    return MemoryView(updated, view.version + 1, view.lineage)
