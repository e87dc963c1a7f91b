"""Torch-op restatement of the reference GL-SDM memory operator (CPU oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.  The product package
never imports this module.

Every function follows one reference function and uses the same torch op
sequence, because the bit-level result of the reference is defined by those
ops (stable argsort order, fp32 adds, ATen's CPU softmax, segment_reduce):

=====================  ==========================================================
function               reference (``S/`` = ``projects/gl-sdm/src/gl_sdm/``)
=====================  ==========================================================
``route``              ``S/memory/routing.py:10-26`` (tie="highest", chunk path)
                       ``S/layers/router.py:39-61``  (tie="lowest", token path)
``routed_read``        ``S/memory/routing.py:10-28`` and ``:45-66`` (torch branch)
``absolute_addresses`` ``S/memory/routing.py:31-34``
``gather_rows``        ``S/memory/routing.py:37-42``
``commit``             ``S/memory/transactions.py:69-97`` (torch branch)
``commit_dense``       ``S/memory/transactions.py:85-88`` (reference=True branch)
``proposal_delta``     ``S/runtime/dense.py:11-14``
``proposal_error``     ``S/runtime/dense.py:13`` (the error row alone)
``token_addresses``    ``S/memory/transactions.py:13-16``
``token_read``         ``S/memory/transactions.py:19-25,28-35`` (torch branch)
``token_propose``      ``S/memory/transactions.py:38-59`` (torch branch)
``score``              ``S/layers/global_layer.py:26,42`` in its per-head
                       sub-key form (``q @ K^T``, fp32 sequential sums)
=====================  ==========================================================

Pinning (see ``tests/test_oracle.py``): known answers copied as data from the
reference tests, brute force over all ``half**2`` slots on tie-free inputs,
the dense one-hot equations, the C restatement in ``glsdm_oracle.c`` and
invariants (ascending unique indices, weights summing to one, untouched rows
bitwise unchanged, commit independent of arrival order for keyed proposals).
"""
import torch
import torch.nn.functional as F

HIGHEST = "highest"
LOWEST = "lowest"


def route(scores, width, tie=HIGHEST):
    """Product-key route of fp32 factor scores ``[..., 2*half]``.

    Returns ``(index int64 [..., width] ascending, weights fp32 [..., width])``.

    Step order (identical for both tie rules, only the tie direction differs):
      1. per factor, the ``min(width, half)`` best sub-keys by a *stable*
         descending argsort; ``tie="highest"`` runs it on the reversed factor so
         the larger sub-key index wins equal scores (routing.py:15-17),
         ``tie="lowest"`` on the factor as is (router.py:46);
      2. candidate grid: fp32 sums ``s0[i] + s1[j]`` and slot ``i*half + j``;
      3. candidates pre-ordered by slot (descending for "highest", ascending for
         "lowest"), then a stable descending sort by sum keeps ``width``;
      4. chosen slots sorted ascending, softmax over their sums.
    """
    if tie not in (HIGHEST, LOWEST):
        raise ValueError("tie must be 'highest' or 'lowest'")
    lead, L = scores.shape[:-1], scores.shape[-1]
    half = L // 2
    k = min(width, half)
    factors = scores.reshape(*lead, 2, half)
    if tie == HIGHEST:
        pick = half - 1 - factors.flip(-1).argsort(dim=-1, descending=True, stable=True)[..., :k]
    else:
        pick = factors.argsort(dim=-1, descending=True, stable=True)[..., :k]
    best = factors.gather(-1, pick)
    sums = (best[..., 0, :, None] + best[..., 1, None, :]).flatten(-2)
    slots = (pick[..., 0, :, None] * half + pick[..., 1, None, :]).flatten(-2)
    pre = slots.argsort(dim=-1, descending=(tie == HIGHEST), stable=True)
    slots, sums = slots.gather(-1, pre), sums.gather(-1, pre)
    keep = sums.argsort(dim=-1, descending=True, stable=True)[..., :width]
    slots, sums = slots.gather(-1, keep), sums.gather(-1, keep)
    canon = slots.argsort(dim=-1, stable=True)
    return slots.gather(-1, canon), sums.gather(-1, canon).softmax(-1)


def absolute_addresses(memory, index):
    """``(b*H + h)*S + slot`` for ``index [B, T, H, k]`` against ``memory [B, H, S, D]``."""
    B, H, S, _ = memory.shape
    part = torch.arange(B * H, device=memory.device).view(B, 1, H, 1)
    return part * S + index.long()


def gather_rows(memory, index, dense=False):
    """Rows ``[B, T, H, k, D]`` of the flattened bank; ``dense`` uses the one-hot matmul."""
    flat = memory.flatten(0, 2)
    addr = absolute_addresses(memory, index)
    if dense:
        return F.one_hot(addr, flat.shape[0]).to(flat.dtype) @ flat
    return flat[addr]


def read(memory, index, weights, dense=False):
    """Snapshot read ``sum_j w_j * row_j`` in fp32 (routing.py:27-28)."""
    rows = gather_rows(memory, index, dense)
    return (rows * weights[..., None]).sum(-2)


def routed_read(memory, scores, width, tie=HIGHEST, dense=False):
    """Route then read; 5-D scores ``[B, R, T, H, L]`` are flattened like routing.py:60-65."""
    shape = scores.shape
    flat_scores = scores.reshape(shape[0], -1, *shape[-2:])
    index, weights = route(flat_scores, width, tie)
    out = read(memory, index, weights, dense)
    if len(shape) == 5:
        out, index, weights = (t.reshape(*shape[:-1], t.shape[-1]) for t in (out, index, weights))
    return out, index, weights


def commit(flat, addresses, deltas, keys=None):
    """Keyed sequential segmented commit, returns a new ``[rows, D]`` fp32 bank.

    Stable sort by key, group equal consecutive addresses, sum each group in
    sorted order with ``segment_reduce``, then ``old + sum`` into a copy of the
    bank (transactions.py:89-96).
    """
    keys = addresses if keys is None else keys
    order = keys.argsort(stable=True)
    addr, delta = addresses[order], deltas.float()[order]
    unique, lengths = addr.unique_consecutive(return_counts=True)
    sums = torch.segment_reduce(delta, "sum", lengths=lengths)
    return flat.index_copy(0, unique, flat[unique] + sums)


def commit_dense(flat, addresses, deltas):
    """Dense one-hot commit ``flat + one_hot(addr)^T @ delta`` (transactions.py:85-88)."""
    update = F.one_hot(addresses.long(), flat.shape[0]).float().T @ deltas.float()
    return flat + update


def commit_bf16(flat_bf16, addresses, deltas, keys=None):
    """bf16-bank commit semantics of this build: ``bf16_rne(fp32(old) + seq_sum)``.

    The reference keeps the bank fp32; a bf16 bank is an extension whose result
    is the fp32 commit of the widened bank rounded once to bf16.
    """
    return commit(flat_bf16.float(), addresses, deltas, keys).to(torch.bfloat16)


def proposal_error(prediction, target, beta, decay):
    """Error row ``beta * (target - decay * prediction)`` of dense.py:13."""
    return beta * (target.float() - decay * prediction)


def proposal_delta(rows, weights, prediction, target, beta, log_decay, mass, decay=None):
    """Write delta of one proposal, same operation order as dense.py:11-14.

    ``decay`` (``[..., H, 1]``) replaces ``log_decay.exp()`` when given, so a
    test can hold the exponential fixed and compare the rest bitwise.
    """
    g = log_decay.exp() if decay is None else decay
    err = proposal_error(prediction, target, beta, g)
    return mass[..., None, None, None] * ((g[..., None] - 1) * rows + weights[..., None] * err[..., None, :])


def token_addresses(values, requests, indices):
    """Absolute rows ``(request*H + h)*S + index`` of the token-clock API
    (transactions.py:13-16): ``requests [A]`` (any subset, any order),
    ``indices [A, H, K]`` against ``values [B, H, S, D]``."""
    heads, slots = values.shape[1:3]
    part = requests[:, None, None] * heads + torch.arange(heads, device=indices.device)[None, :, None]
    return part * slots + indices


def _token_rows(values, requests, indices, dense):
    flat = values.flatten(0, 2)
    index = token_addresses(values, requests, indices)
    if dense:
        return F.one_hot(index.long(), flat.shape[0]).float() @ flat
    return flat[index]


def token_read(values, requests, indices, weights, dense=False):
    """Token-clock snapshot read ``sum_k w_k * row_k`` -> ``[A, H, D]``
    (transactions.py:28-35, torch branch; ``dense`` is its reference=True branch)."""
    rows = _token_rows(values, requests, indices, dense)
    return (rows * weights.float().unsqueeze(-1)).sum(-2)


def token_propose(values, requests, indices, weights, targets, beta, log_decay, mass, dense=False):
    """Token-clock write proposal (transactions.py:38-59, torch branch).

    Unlike ``proposal_delta`` (dense.py:11-14, the stack's form) the prediction
    is recomputed from the decayed rows, and the delta is formed as
    ``decayed - rows + w * error``.  Returns ``(addresses [A*H*K] int64,
    deltas [A*H*K, D] fp32)``: the fields of the reference's WriteProposal.
    ``beta``/``log_decay`` are ``[A, H, 1]``, ``mass`` is ``[A]``.
    """
    rows = _token_rows(values, requests, indices, dense)
    decay = log_decay.float().exp().unsqueeze(-1)
    decayed = rows * decay
    retrieved = (decayed * weights.float().unsqueeze(-1)).sum(-2)
    error = beta.float() * (targets.float() - retrieved)
    delta = decayed - rows + weights.float().unsqueeze(-1) * error.unsqueeze(-2)
    delta = delta * mass.float()[:, None, None, None]
    return token_addresses(values, requests, indices).flatten(), delta.flatten(0, 2)


def score(queries, subkeys):
    """Factor scores ``[B, T, H, L]`` fp32 of queries ``[B, T, H, dk]`` against
    per-head sub-keys ``[H, L, dk]``: ``sum_e q[e] * k[e]`` with e ascending,
    every product and partial sum rounded to fp32 (the C oracle's loop, as
    a sequence of torch fp32 ops; global_layer.py:26,42 computes these scores
    with the router.q/k Linear)."""
    q = queries.float()
    k = subkeys.float()
    acc = torch.zeros(*q.shape[:-1], k.shape[1], dtype=torch.float32)
    for e in range(q.shape[-1]):
        acc = acc + q[..., e, None] * k[None, None, :, :, e]
    return acc
