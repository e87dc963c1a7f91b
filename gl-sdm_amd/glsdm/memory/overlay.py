"""Overlay snapshots: one shared base bank plus each request's touched rows.

The reference snapshots a learned bank by cloning it once per request
(S/memory/state.py:61-62, S/ = projects/gl-sdm/src/gl_sdm/) and commits
functionally into a new full bank (S/memory/transactions.py:96).  An
``OverlayView`` keeps the base ``[H, S, D]`` once, an int32 slot map
``[B, H, S]`` (-1: the base row) and a pool of touched rows; reads resolve a
slot through the map and commits write only touched rows (the plan of
P/OPTIMIZATION_PLAN.md:114-120, P/ = projects/gl-sdm/).  Every result equals
the dense bank's bit for bit (same sort, same per-address summation order,
same bf16 rounding).

Commits update the overlay in place (the stack drops the old view after each
commit, S/layers/stack.py:65); ``copy()`` gives an independent view at the
cost of the map and the used pool rows.  A commit of E entries writes its
newly touched rows into pool rows [next, next + E) (each at its address run's
sorted position: no atomics, deterministic layout), so the host knows the
pool's needs exactly and never synchronises; rows of a run that was already
mapped are left unused (``mapped_rows()`` counts the live ones).
"""
from dataclasses import dataclass, field

import torch

from .. import _native as N
from .backends import hip


@dataclass
class OverlayView:
    base: torch.Tensor        # [H, S, D] fp32 or bf16, shared and never written
    map: torch.Tensor         # [B, H, S] int32, -1 = base row
    pool: torch.Tensor        # [capacity, D], same dtype as base
    version: int = 0
    lineage: object = field(default_factory=object)
    next: int = 0             # first pool row of the next commit

    @classmethod
    def from_base(cls, base, batch_size, capacity=None):
        """Snapshot of ``batch_size`` requests that all start from ``base [H, S, D]``."""
        device = N.require_device(base)
        if base.ndim != 3 or base.dtype not in N.DTYPES:
            raise ValueError("overlay views require a [heads, slots, dim] FP32 or BF16 base")
        H, S, D = base.shape
        if capacity is None:
            capacity = max(1, min(batch_size * H * S, 1 << 16))
        return cls(base, torch.full((batch_size, H, S), -1, dtype=torch.int32, device=device),
                   torch.empty(capacity, D, dtype=base.dtype, device=device))

    @property
    def shape(self):
        B, H, S = self.map.shape
        return B, H, S, self.base.shape[-1]

    def pool_rows(self):
        """Pool rows reserved by the commits so far (host count, no synchronisation)."""
        return self.next

    def mapped_rows(self):
        """Rows of the logical bank that differ from the base's storage (synchronises)."""
        return int((self.map >= 0).sum().item())

    def reserve(self, entries):
        """Grow the pool (doubling) so that the next commit's rows fit."""
        cap = self.pool.shape[0]
        if self.next + entries > cap:
            grown = torch.empty(max(2 * cap, self.next + entries), self.pool.shape[1], dtype=self.pool.dtype,
                                device=self.pool.device)
            grown[:self.next] = self.pool[:self.next]
            self.pool = grown

    def read(self, index, weights, out_dtype=torch.float32):
        """Snapshot read ``sum_j w_j * row_j`` of routes ``index/weights [B, T, H, width]``."""
        N.require_device(index, weights)
        B, H, S, D = self.shape
        if index.ndim != 4 or index.shape[0] != B or index.shape[2] != H or weights.shape != index.shape:
            raise ValueError("overlay read needs [B, T, H, width] int64 index and fp32 weights")
        T, width = index.shape[1], index.shape[3]
        N.check_range(index, S, "overlay read")
        out = torch.empty((B, T, H, D), dtype=out_dtype, device=index.device)
        N.call("glsdm_overlay_read", N.ptr(self.base), N.dtype_code(self.base), N.ptr(self.map), N.ptr(self.pool),
               B, H, S, D, T, width, N.ptr(index), N.ptr(weights), N.ptr(out), N.dtype_code(out),
               N.stream(index.device))
        return out

    def routed_read(self, scores, width, tie="highest", out_dtype=torch.float32):
        """Route fp32 scores ``[B, T, H, 2*half]`` and read: ``(out, index, weights)``."""
        index, weights = hip.route(scores, width, tie)
        return self.read(index, weights, out_dtype), index, weights

    def commit(self, addresses, deltas, keys=None, workspace=None, unique=None):
        """In-place deterministic commit of ``deltas [E, D]`` at absolute rows
        ``(b*H + h)*S + slot``; returns this view with ``version + 1``."""
        N.require_device(addresses, deltas, keys)
        B, H, S, D = self.shape
        E = addresses.numel()
        if addresses.dtype != torch.int64 or deltas.numel() != E * D or (keys is not None and keys.numel() != E):
            raise ValueError("overlay commit needs int64 addresses [E], deltas [E, D] and keys [E]")
        N.check_range(addresses, B * H * S, "overlay commit")
        if E:
            self.reserve(E)
            need = hip.commit_workspace_bytes(E, B * H * S)
            if workspace is None or workspace.numel() < need:
                workspace = torch.empty(need, dtype=torch.uint8, device=deltas.device)
            deltas = deltas.reshape(E, D).contiguous()
            N.call("glsdm_overlay_commit", N.ptr(self.base), N.dtype_code(self.base), B, H, S, D, N.ptr(self.map),
                   N.ptr(self.pool), self.pool.shape[0], self.next, N.ptr(addresses.contiguous()),
                   N.ptr(deltas), N.dtype_code(deltas), N.ptr(None if keys is None else keys.contiguous()), E,
                   N.ptr(workspace), workspace.numel(), N.ptr(unique), N.stream(deltas.device))
            hip.after_commit("overlay commit", workspace, E, B * H * S, deltas.device)
            self.next += E
        self.version += 1
        return self

    def copy(self):
        """An independent view (map and reserved pool rows copied, base shared)."""
        pool = torch.empty_like(self.pool)
        pool[:self.next] = self.pool[:self.next]
        return OverlayView(self.base, self.map.clone(), pool, self.version, object(), self.next)

    def materialise(self):
        """The dense logical bank ``[B, H, S, D]``."""
        B, H, S, D = self.shape
        out = torch.empty((B, H, S, D), dtype=self.base.dtype, device=self.base.device)
        N.call("glsdm_overlay_materialise", N.ptr(self.base), N.dtype_code(self.base), N.ptr(self.map),
               N.ptr(self.pool), B, H, S, D, N.ptr(out), N.stream(self.base.device))
        return out
