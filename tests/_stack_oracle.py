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
from unittest.mock import patch

import torch

from oracle import torch_oracle
from glsdm.layers import global_layer, stack
from glsdm.memory import MemoryView, WriteProposal, routing


def _routed_read(block, memory, scores, width, physical=None):
    del physical
    device = scores.device
    # the reference routes the fp32 widening of the projection (S/layers/global_layer.py:26,42)
    out, index, weights = torch_oracle.routed_read(memory.cpu(), scores.cpu().float(), width, block.attn.tie)
    return out.to(device), index.to(device), weights.to(device)


def _layer_proposal(snapshot, index, weights, prediction, target, beta, log_decay, offset, layer_idx, chunk_size,
                    num_layers, mass=None, deferred=True):
    del deferred
    values, idx = snapshot.values.cpu(), index.cpu()
    B, T = idx.shape[:2]
    rows = torch_oracle.gather_rows(values, idx)
    addresses = torch_oracle.absolute_addresses(values, idx)
    mass = torch.ones(B, T) if mass is None else mass.cpu()
    delta = torch_oracle.proposal_delta(rows, weights.cpu(), prediction.cpu(), target.cpu(), beta.cpu(),
                                        log_decay.cpu(), mass)
    positions = torch.arange(offset, offset + T).view(1, T, 1, 1)
    keys = addresses * (chunk_size * num_layers) + positions * num_layers + layer_idx
    return WriteProposal(snapshot.version, addresses.flatten(), delta.flatten(0, 3), snapshot.lineage, keys.flatten())


def _commit(view, buffer, reference=False, backend="hip", donate=False):
    del reference, backend, donate
    values = view.values
    D = values.shape[-1]
    props = buffer.proposals
    addr = torch.cat([p.addresses.cpu() for p in props])
    delta = torch.cat([p.deltas.cpu() for p in props])
    keys = torch.cat([p.sort_keys.cpu() for p in props])
    flat = values.cpu().float().reshape(-1, D)      # differentiable, like the reference's commit
    new = torch_oracle.commit(flat, addr, delta, keys).to(values.dtype)
    return MemoryView(new.reshape(values.shape).to(values.device), view.version + 1, view.lineage)


@contextlib.contextmanager
def oracle_memory():
    with patch.object(routing, "routed_read", _routed_read), \
            patch.object(global_layer, "layer_proposal", _layer_proposal), \
            patch.object(stack, "commit", _commit):
        yield
