"""Write proposals of one global layer on the HIP path.

Mirrors the proposal construction of ``GlobalLayer.propose``
(S/layers/global_layer.py:33-54, S/ = projects/gl-sdm/src/gl_sdm/) after its
write route: addresses and collision keys ``addr*(C*L) + position*L + layer``
(:45,52-53), ``mass = 1`` per token (:50), and the deltas of
S/runtime/dense.py:11-14 against the snapshot rows the route selected (:44).

``deferred=True`` (default) returns a :class:`DeferredProposal`, whose deltas
are evaluated inside the commit from the rows it touches (the ``[E, D]``
deltas and the row re-gather are never materialised); ``deferred=False``
returns the reference's :class:`WriteProposal` with fp32 deltas, which carry
gradients under autograd.
"""
import torch

from .state import DeferredProposal, WriteProposal
from .backends import hip


_ONES = {}


def _ones(shape, device):
    """A shared read-only fp32 ones tensor per (shape, device): the stack's mass
    (one per token) is the same for every proposal, and a fill per layer and
    chunk is a launch each.  Built outside inference mode so autograd may use it."""
    key = (tuple(shape), device)
    t = _ONES.get(key)
    if t is None:
        with torch.inference_mode(False), torch.no_grad():
            t = torch.ones(key[0], dtype=torch.float32, device=device)
        if len(_ONES) >= 64:
            _ONES.clear()
        _ONES[key] = t
    return t


def layer_proposal(snapshot, index, weights, prediction, target, beta, log_decay, offset, layer_idx,
                   chunk_size, num_layers, mass=None, deferred=True):
    """Proposal of the write route ``index``/``weights [B, T, H, k]`` with its routed
    read ``prediction [B, T, H, D]``, value ``target [B, T, H, D]`` and gates
    ``beta``/``log_decay [B, T, H, 1]`` (``mass [B, T]``, default ones)."""
    addresses, keys = hip.proposal_keys(snapshot.values, index, offset, chunk_size, num_layers, layer_idx)
    if mass is None:
        mass = _ones(index.shape[:2], index.device)
    if deferred:
        return DeferredProposal(snapshot.version, addresses, weights, prediction, target, beta, log_decay, mass,
                                snapshot.lineage, keys)
    from ..runtime.dense import proposal_delta          # autograd-aware (training with writes)
    rows = hip.gather_rows(snapshot.values, index)
    delta = proposal_delta(rows, weights, prediction, target, beta, log_decay, mass)
    return WriteProposal(snapshot.version, addresses.flatten(), delta.flatten(0, 3), snapshot.lineage,
                         keys.flatten())
