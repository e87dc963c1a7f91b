"""Frozen views, buffered proposals, request caches and the learned bank.

Mirrors S/memory/state.py:7-70 (S/ = projects/gl-sdm/src/gl_sdm/) with one
extension: the transactional state may be bf16 as well as fp32 (the reference
is fp32-only); a bf16 bank commits as bf16_rne(fp32(old) + fp32 sum).
"""
from dataclasses import dataclass, field

import torch
from torch import nn

STATE_DTYPES = (torch.float32, torch.bfloat16)


@dataclass(frozen=True)
class MemoryView:
    values: torch.Tensor  # [requests, heads, slots, value_dim], fp32 or bf16
    version: int = 0
    lineage: object = field(default_factory=object)

    def __post_init__(self):
        v = self.values
        if v.ndim != 4 or v.dtype not in STATE_DTYPES or min(v.shape) < 1 or self.version < 0:
            raise ValueError("memory views require nonempty [batch, heads, slots, dim] FP32 or BF16 values "
                             "and a nonnegative version")


@dataclass(frozen=True)
class WriteProposal:
    base_version: int
    addresses: torch.Tensor  # flattened request/head/slot addresses, int64 [E]
    deltas: torch.Tensor     # [E, value_dim], already weighted (fp32 or bf16)
    lineage: object
    sort_keys: torch.Tensor | None = None  # optional address/token/depth order, int64 [E]


@dataclass(frozen=True)
class DeferredProposal:
    """A write proposal whose deltas are evaluated inside the commit.

    Holds the operands of S/runtime/dense.py:11-14 except the gathered rows:
    the commit reads each touched row once anyway, and that row (before the
    commit) is the snapshot row the reference gathers at
    S/layers/global_layer.py:44, so ``mass * ((exp(log_decay) - 1) * row +
    weights * beta * (target - exp(log_decay) * prediction))`` is formed there
    and the ``[E, D]`` deltas are never stored.  Shapes: addresses, weights and
    sort_keys ``[..., H, k]``; prediction/target ``[..., H, D]``;
    beta/log_decay ``[..., H, 1]``; mass ``[...]``.
    """
    base_version: int
    addresses: torch.Tensor   # absolute rows, int64
    weights: torch.Tensor     # route weights, fp32
    prediction: torch.Tensor  # routed read of the write route, fp32
    target: torch.Tensor      # fp32 or bf16
    beta: torch.Tensor        # fp32
    log_decay: torch.Tensor   # fp32
    mass: torch.Tensor        # fp32
    lineage: object
    sort_keys: torch.Tensor | None = None

    @property
    def heads(self):
        return self.addresses.shape[-2]

    @property
    def width(self):
        return self.addresses.shape[-1]


@dataclass(frozen=True)
class LoggedProposal:
    """A deferred write proposal stored in a proposal log (``ProposalLog``):
    rows ``[start, start + rows)`` of the log hold its addresses, collision
    keys and route weights (``width`` per row) and its per-row error and decay
    terms, written when it was made.  ``generation`` is the log's generation
    at that time: the log's rows are reused after each commit, and a proposal
    of an earlier generation no longer has its rows."""
    base_version: int
    lineage: object
    log: object
    generation: int
    start: int
    rows: int

    @property
    def heads(self):
        return self.log.heads

    @property
    def width(self):
        return self.log.width

    @property
    def sort_keys(self):
        return self.log.keys.narrow(0, self.start * self.log.width, self.rows * self.log.width)


@dataclass(frozen=True)
class WriteBuffer:
    base_version: int
    proposals: tuple
    lineage: object


@dataclass
class MemoryCache:
    view: MemoryView
    owner: object
    tokens: int = 0
    pending: tuple = ()
    local: dict = field(default_factory=dict)
    log: object = None      # the stack's ProposalLog for the pending chunk (inference)


class MemoryBank(nn.Module):
    """Learned ``[heads, slots, dim]`` fp32 initializer; snapshots use ``state_dtype``."""

    def __init__(self, heads, slots, dim, state_dtype=torch.float32):
        super().__init__()
        if state_dtype not in STATE_DTYPES:
            raise ValueError("bank state must be float32 or bfloat16")
        self.memory = nn.Parameter(torch.randn(heads, slots, dim) * (heads * dim) ** -0.5)
        self.memory._sdm_memory_bank = True
        self.owner = object()
        self.state_dtype = state_dtype

    def _apply(self, fn, recurse=True):
        # Model casts (e.g. .bfloat16()) leave the learned bank in fp32.
        values = self.memory.detach()
        grad = None if self.memory.grad is None else self.memory.grad.detach()
        super()._apply(fn, recurse)
        self.memory.data = values.to(device=self.memory.device, dtype=torch.float32)
        if grad is not None:
            self.memory.grad.data = grad.to(device=self.memory.device, dtype=torch.float32)
        return self

    def snapshot(self, batch_size):
        # one clone per request; under autograd the reads and commits of the
        # snapshot carry gradients back to the learned bank (S/memory/state.py:61-62)
        base = self.memory.to(self.state_dtype)
        return MemoryView(base.unsqueeze(0).expand(batch_size, -1, -1, -1).clone())

    def new_cache(self, batch_size):
        return MemoryCache(self.snapshot(batch_size), self.owner)

    def validate_cache(self, cache, batch_size):
        expected = (batch_size, *self.memory.shape)
        v = cache.view.values
        if (cache.owner is not self.owner or v.shape != expected or v.device != self.memory.device
                or v.dtype != self.state_dtype):
            raise ValueError("memory cache belongs to another model, batch, device or dtype")
