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

:class:`ProposalLog` is the stack's inference path: each proposal's terms go
straight into preallocated per-chunk buffers (one launch per proposal, gates
included), and the chunk's commit reads them as one proposal.
"""
import torch

from .. import _native as N
from .state import DeferredProposal, LoggedProposal, WriteProposal
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


def log_proposal(log, snapshot, index, weights, prediction, target, b_lin, d_lin, offset, layer_idx, chunk_size,
                 num_layers):
    """The inference proposal of a global layer, appended to ``log`` (see
    :class:`ProposalLog`): returns its :class:`LoggedProposal`."""
    return log.append(snapshot, index, weights, prediction, target, b_lin, d_lin, offset, layer_idx, chunk_size,
                      num_layers)


class ProposalLog:
    """Device storage for one chunk's deferred write proposals.

    Each proposal appends, at the log's fill, its per-entry terms (absolute
    addresses, collision keys ``addr*(C*L) + position*L + layer`` and route
    weights, ``width`` per proposal row) and its per-row terms (the error row
    ``beta * (target - exp(log_decay) * prediction)`` and ``exp(log_decay)``,
    S/runtime/dense.py:12-13, with the gates of S/layers/global_layer.py:48-49)
    in one launch (``glsdm_proposal_append``).  The chunk's commit reads the
    filled rows as one fused proposal, so the chunk's proposals are never
    concatenated or re-formed (the reference concatenates its list of
    proposals at the commit, S/memory/transactions.py:73-79).  ``rows``
    proposal rows (token-heads) of capacity: global layers x chunk tokens x
    requests x heads holds a whole chunk of the stack.  The owner clears it
    after each commit and reuses the storage; every operation runs on the
    current stream, so a commit's reads finish before the next chunk's
    appends overwrite them."""

    def __init__(self, rows, heads, width, D, device):
        if rows < 1 or heads < 1 or rows % heads or width < 1 or D < 1:
            raise ValueError("a proposal log needs whole tokens of rows and positive heads, width and D")
        self.rows, self.heads, self.width, self.D = rows, heads, width, D
        self.device = torch.device(device)
        self.addresses = torch.empty(rows * width, dtype=torch.int64, device=device)
        self.keys = torch.empty_like(self.addresses)
        self.weights = torch.empty(rows * width, dtype=torch.float32, device=device)
        self.error = torch.empty(rows, D, dtype=torch.float32, device=device)
        self.decay = torch.empty(rows, dtype=torch.float32, device=device)
        self.fill = 0
        self.generation = 0

    def fits(self, rows, heads, width, D, device):
        return (self.rows >= rows and (self.heads, self.width, self.D) == (heads, width, D)
                and self.device == torch.device(device))

    def clear(self):
        """Forget every appended proposal (after their commit): the rows are reused."""
        self.fill = 0
        self.generation += 1

    def append(self, snapshot, index, weights, prediction, target, b_lin, d_lin, offset, layer_idx, chunk_size,
               num_layers):
        """Append the proposal of the write route ``index``/``weights [B, T, H, k]``
        against ``snapshot``: routed read ``prediction [B, T, H, D]`` fp32, value
        ``target [B, T, H, D]`` and the beta/decay projections' outputs
        ``b_lin``/``d_lin [B, T, H]`` (fp32 or bf16); returns its LoggedProposal."""
        values = snapshot.values
        B, H, S, D = values.shape
        if (index.ndim != 4 or index.dtype != torch.int64 or index.shape[0] != B or index.shape[2] != H
                or weights.shape != index.shape or weights.dtype != torch.float32):
            raise ValueError("proposal_append needs a [B, T, H, width] int64 index and fp32 weights")
        T, k = index.shape[1], index.shape[3]
        if (prediction.shape != (B, T, H, D) or prediction.dtype != torch.float32 or target.shape != (B, T, H, D)
                or b_lin.shape != (B, T, H) or d_lin.shape != (B, T, H) or b_lin.dtype != d_lin.dtype):
            raise ValueError("proposal_append needs prediction/target [B, T, H, D] and gates [B, T, H]")
        if (H, k, D) != (self.heads, self.width, self.D):
            raise ValueError("proposal does not match the log's heads, width and value dim")
        R = B * T * H
        if self.fill + R > self.rows:
            raise RuntimeError(f"proposal log full: {self.fill} + {R} rows exceed its {self.rows}")
        device = hip.require_cuda(values, index, weights, prediction, target, b_lin, d_lin)
        if device != self.device:
            raise ValueError("proposal log and proposal on different devices")
        N.check_range(index, S, "proposal_append")
        f = self.fill
        at = lambda t, n: N.ctypes.c_void_p(t.data_ptr() + n * t.element_size())
        N.call("glsdm_proposal_append", N.ptr(index), N.ptr(weights), N.ptr(prediction), N.ptr(target),
               N.dtype_code(target), N.ptr(b_lin), N.ptr(d_lin), N.dtype_code(b_lin), B, T, H, k, S, D, offset,
               chunk_size, num_layers, layer_idx, at(self.addresses, f * k), at(self.keys, f * k),
               at(self.weights, f * k), at(self.error, f * D), at(self.decay, f), N.stream(device))
        self.fill = f + R
        return LoggedProposal(snapshot.version, snapshot.lineage, self, self.generation, f, R)

    def terms(self, start, rows):
        """Views of rows ``[start, start + rows)``: addresses, keys and weights
        ``[n, H, k]``, error ``[n, H, D]`` and decay ``[n, H]`` (n = rows / H)."""
        H, k, D = self.heads, self.width, self.D
        n = rows // H
        e = slice(start * k, (start + rows) * k)
        return (self.addresses[e].view(n, H, k), self.keys[e].view(n, H, k), self.weights[e].view(n, H, k),
                self.error[start:start + rows].view(n, H, D), self.decay[start:start + rows].view(n, H))
