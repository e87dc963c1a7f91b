"""Oracle wiring for the layer-stack parity tests (test infrastructure only).

``oracle_memory()`` swaps the stack's three memory steps for the CPU oracle
(the reference's torch equations, ``oracle/torch_oracle.py``) with a host
round trip: the routed read of S/memory/routing.py:10-28, the proposal of
S/layers/global_layer.py:33-54 (gathered rows, ``proposal_delta`` of
S/runtime/dense.py:11-14, keys ``addr*(C*L) + pos*L + layer``) and the commit
of S/memory/transactions.py:69-97.  Everything else (embedding, projections,
attention, MLP, head) runs the same code on the same device, so a comparison
against the native model isolates the memory operator inside the stack.
"""
import contextlib
import sys
from types import SimpleNamespace
from unittest.mock import patch

import torch
import torch.nn.functional as F

from oracle import torch_oracle
from glsdm.layers import global_layer, stack
from glsdm.memory import MemoryView, WriteProposal, routing


_HOST = [None, None]


def _host_copy(values):
    """One host copy per snapshot tensor: the oracle's commits are functional, so
    a snapshot's storage never changes while it is cached (the cache holds the
    tensor itself, so the identity test cannot be fooled by a reused id)."""
    if values.requires_grad:            # training: the differentiable copy, every time
        return values.cpu()
    if _HOST[0] is not values:
        _HOST[:] = [values, values.detach().cpu()]
    return _HOST[1]


def _routed_read(block, memory, scores, width, physical=None, out_dtype=torch.float32):
    del physical
    device = scores.device
    # the reference routes the fp32 widening of the projection (S/layers/global_layer.py:26,42)
    # and reads in fp32; a bf16 out_dtype is its later .to(dtype) of the readings
    out, index, weights = torch_oracle.routed_read(_host_copy(memory), scores.cpu().float(), width, block.attn.tie)
    return out.to(device=device, dtype=out_dtype), index.to(device), weights.to(device)


def _layer_proposal(snapshot, index, weights, prediction, target, beta, log_decay, offset, layer_idx, chunk_size,
                    num_layers, mass=None, deferred=True):
    del deferred
    values = snapshot.values if not snapshot.values.is_cuda else _host_copy(snapshot.values)
    idx = index.cpu()
    B, T = idx.shape[:2]
    rows = torch_oracle.gather_rows(values, idx)
    addresses = torch_oracle.absolute_addresses(values, idx)
    mass = torch.ones(B, T) if mass is None else mass.cpu()
    delta = torch_oracle.proposal_delta(rows, weights.cpu(), prediction.cpu(), target.cpu(), beta.cpu(),
                                        log_decay.cpu(), mass)
    positions = torch.arange(offset, offset + T).view(1, T, 1, 1)
    keys = addresses * (chunk_size * num_layers) + positions * num_layers + layer_idx
    return WriteProposal(snapshot.version, addresses.flatten(), delta.flatten(0, 3), snapshot.lineage, keys.flatten())


def _gates(b_lin, d_lin):
    # the reference's write gates (S/layers/global_layer.py:48-49), on the host
    beta = b_lin.cpu().float().sigmoid().unsqueeze(-1)
    log_decay = -F.softplus(d_lin.cpu().float() - 4).unsqueeze(-1)
    return beta, log_decay


def _log_proposal(log, snapshot, index, weights, prediction, target, b_lin, d_lin, offset, layer_idx, chunk_size,
                  num_layers):
    del log
    beta, log_decay = _gates(b_lin, d_lin)
    return _layer_proposal(snapshot, index, weights, prediction, target, beta, log_decay, offset, layer_idx,
                           chunk_size, num_layers)


def _commit(view, buffer, reference=False, backend="hip", donate=False):
    del reference, backend, donate
    values = view.values
    D = values.shape[-1]
    props = buffer.proposals
    addr = torch.cat([p.addresses.cpu() for p in props])
    delta = torch.cat([p.deltas.cpu() for p in props])
    keys = torch.cat([p.sort_keys.cpu() for p in props])
    flat = _host_copy(values).float().reshape(-1, D)      # differentiable in training, like the reference's
    new = torch_oracle.commit(flat, addr, delta, keys).to(values.dtype)
    return MemoryView(new.reshape(values.shape).to(values.device), view.version + 1, view.lineage)


@contextlib.contextmanager
def oracle_memory():
    _HOST[:] = [None, None]
    with patch.object(routing, "routed_read", _routed_read), \
            patch.object(global_layer, "layer_proposal", _layer_proposal), \
            patch.object(global_layer, "log_proposal", _log_proposal), \
            patch.object(stack, "commit", _commit):
        yield


class Shadow:
    """Runs the oracle beside every memory step of the native stack, on the
    native step's own inputs: each routed read (routes bit for bit, weights and
    readings within fp32 rounding), each proposal (materialised by the oracle
    from the same route, prediction, target and gates) and each commit (the
    oracle's commit of those proposals into a host copy of the snapshot taken
    before the native in-place commit).  Because every comparison starts from
    identical inputs, later layers and chunks are checked as strictly as the
    first, whatever rounding differences accumulate in the stack around them.

    ``bank_tol``: tolerance of the committed bank (the native deltas use the
    device's ``exp(log_decay)``, within an ulp of torch's, and a bf16 bank
    rounds once more)."""

    def __init__(self, read_tol=None, bank_tol=None):
        self.read_tol = read_tol or dict(atol=1e-6, rtol=1e-5)
        self.bank_tol = bank_tol or dict(atol=2e-6, rtol=2e-5)
        self.reads = self.proposals = self.commits = 0
        self._host_of = (None, None)
        self._refs = {}

    def _host(self, values):
        # one host copy per snapshot tensor (the reference keeps it while cached, so
        # the identity test cannot be fooled by a reused object id)
        if self._host_of[0] is not values:
            self._host_of = (values, values.detach().cpu())
        return self._host_of[1]

    def forget(self):
        self._host_of = (None, None)

    @contextlib.contextmanager
    def watch(self):
        native_read, native_propose, native_commit = routing.routed_read, global_layer.layer_proposal, stack.commit
        native_log = global_layer.log_proposal

        def read(block, memory, scores, width, physical=None, out_dtype=torch.float32):
            out, index, weights = native_read(block, memory, scores, width, physical, out_dtype=out_dtype)
            host = self._host(memory)
            r_out, r_idx, r_w = torch_oracle.routed_read(host, scores.cpu().float(), width, block.attn.tie)
            where = f"read {self.reads}"
            assert torch.equal(index.cpu(), r_idx), f"{where}: routes differ from the oracle"
            torch.testing.assert_close(weights.cpu(), r_w, atol=2e-7, rtol=2e-6, msg=lambda m: f"{where}: {m}")
            # readings rounded to bf16 by the read: the oracle's rounded alike, within one bf16 step
            tol = self.read_tol if out.dtype == torch.float32 else dict(atol=self.read_tol["atol"], rtol=2 ** -7)
            torch.testing.assert_close(out.cpu().float(), r_out.to(out.dtype).float(), **tol,
                                       msg=lambda m: f"{where}: {m}")
            self.reads += 1
            return out, index, weights

        def propose(snapshot, index, weights, prediction, target, beta, log_decay, offset, layer_idx, chunk_size,
                    num_layers, mass=None, deferred=True):
            p = native_propose(snapshot, index, weights, prediction, target, beta, log_decay, offset, layer_idx,
                               chunk_size, num_layers, mass=mass, deferred=deferred)
            host = SimpleNamespace(values=self._host(snapshot.values), version=snapshot.version,
                                   lineage=snapshot.lineage)
            self._refs[id(p)] = (p, _layer_proposal(host, index, weights, prediction, target, beta, log_decay,
                                                    offset, layer_idx, chunk_size, num_layers, mass))
            self.proposals += 1
            return p

        def log_propose(log, snapshot, index, weights, prediction, target, b_lin, d_lin, offset, layer_idx,
                        chunk_size, num_layers):
            p = native_log(log, snapshot, index, weights, prediction, target, b_lin, d_lin, offset, layer_idx,
                           chunk_size, num_layers)
            host = SimpleNamespace(values=self._host(snapshot.values), version=snapshot.version,
                                   lineage=snapshot.lineage)
            beta, log_decay = _gates(b_lin, d_lin)
            self._refs[id(p)] = (p, _layer_proposal(host, index, weights, prediction, target, beta, log_decay,
                                                    offset, layer_idx, chunk_size, num_layers))
            self.proposals += 1
            return p

        def commit(view, buffer, reference=False, backend="hip", donate=False):
            refs = [self._refs.pop(id(p))[1] for p in buffer.proposals]
            values = view.values
            D = values.shape[-1]
            before = self._host(values).float().reshape(-1, D)
            addr = torch.cat([p.addresses for p in refs])
            delta = torch.cat([p.deltas for p in refs])
            keys = torch.cat([p.sort_keys for p in refs])
            expect = torch_oracle.commit(before, addr, delta, keys).to(values.dtype)
            new = native_commit(view, buffer, reference=reference, backend=backend, donate=donate)
            self.forget()                       # an in-place commit changed the snapshot's storage
            where = f"commit {self.commits}"
            torch.testing.assert_close(new.values.cpu().reshape(-1, D), expect, **self.bank_tol,
                                       msg=lambda m: f"{where}: {m}")
            self.commits += 1
            return new

        with patch.object(routing, "routed_read", read), patch.object(global_layer, "layer_proposal", propose), \
                patch.object(global_layer, "log_proposal", log_propose), patch.object(stack, "commit", commit):
            yield self


class RouteLog:
    """Records every routed read of a stack run, keyed by (chunk, layer, kind,
    absolute position): kind 0 is a global layer's read route, 1 its write
    route (which sees the layer's output).  In the stack's causal order --
    chunk, then layer, then read before write -- a route depends only on
    routes earlier in that order, so two runs of the same model and tokens
    (native vs oracle memory, decode vs one prefill) must agree bit for bit up
    to their first disagreement, and that first disagreement can only be a
    tie at the rounding level of the path.  Requests never interact, so a
    request whose routes all agree must have the same outputs.

    ``keep_scores``: True, False, or a set of (chunk, layer, kind) groups
    whose factor scores are kept (the tie check needs them)."""

    def __init__(self, chunk, keep_scores=True):
        self.chunk, self.keep_scores = chunk, keep_scores
        self.rows = {}          # key -> (scores [B, H, L] or None, index [B, H, k])
        self._seen = {}

    def _keep(self, group):
        return self.keep_scores is True or (self.keep_scores is not False and group in self.keep_scores)

    @contextlib.contextmanager
    def watch(self, model):
        layer_of = {id(b): i for i, b in enumerate(model.blocks)}
        native = routing.routed_read

        def read(block, memory, scores, width, physical=None, out_dtype=torch.float32):
            out = native(block, memory, scores, width, physical, out_dtype=out_dtype)
            kind = 1 if sys._getframe(1).f_code.co_name == "propose" else 0
            layer = layer_of[id(block)]
            start = self._seen.get((layer, kind), 0)
            T = scores.shape[1]
            self._seen[(layer, kind)] = start + T
            idx = out[1].cpu()
            s = None
            for t in range(T):
                pos = start + t
                group = (pos // self.chunk, layer, kind)
                if self._keep(group) and s is None:
                    s = scores.detach().float().cpu()
                self.rows[group + (pos,)] = (s[:, t] if self._keep(group) else None, idx[:, t])
            return out

        with patch.object(routing, "routed_read", read):
            yield self


def _cell(s, slot, half):
    return (s[..., slot // half] + s[..., half + slot % half]).item()


def compare_routes(a, b):
    """Two RouteLogs in causal order: ``(first disagreeing group or None, its
    disagreeing (key, (request, head)) rows, requests with any disagreement,
    number of keys)``."""
    keys = sorted(a.rows)
    assert keys and keys == sorted(b.rows), "the runs routed different positions"
    first, bad_rows, bad_requests = None, [], set()
    for k in keys:
        diff = (a.rows[k][1] != b.rows[k][1]).any(-1)
        if bool(diff.any()):
            if first is None:
                first = k[:3]
            if k[:3] == first:
                bad_rows += [(k, tuple(r)) for r in diff.nonzero().tolist()]
            bad_requests |= set(diff.any(-1).nonzero().flatten().tolist())
    return first, bad_rows, bad_requests, len(keys)


def check_ties(a, b, bad_rows, tie_rel):
    """Every disagreeing row of the first disagreeing group swaps picks whose
    cells tie within ``tie_rel`` (relative) under both runs' scores, pairing
    the swapped picks by rank."""
    for k, (bb, h) in bad_rows:
        sa, ia = a.rows[k][0][bb, h], a.rows[k][1][bb, h].tolist()
        sb, ib = b.rows[k][0][bb, h], b.rows[k][1][bb, h].tolist()
        half = sa.numel() // 2
        only_a = sorted(set(ia) - set(ib), key=lambda x: -_cell(sa, x, half))
        only_b = sorted(set(ib) - set(ia), key=lambda x: -_cell(sa, x, half))
        for x, y in zip(only_a, only_b):
            for s in (sa, sb):
                cx, cy = _cell(s, x, half), _cell(s, y, half)
                assert abs(cx - cy) <= tie_rel * max(1.0, abs(cx), abs(cy)), (
                    f"first disagreement at {k} row {(bb, h)} is not a tie: slot {x} {cx} vs slot {y} {cy}")
