"""HIP backend of the GL-SDM memory operator: the native entry points in the
shape of the reference's native backends (S/ = projects/gl-sdm/src/gl_sdm/):

=========================  ===================================================
this module                reference entry point it stands in for
=========================  ===================================================
``routed_snapshot_read``   ``S/memory/backends/urm.py:109-122``
``snapshot_read``          ``S/memory/backends/urm.py:64-82``
``route``                  ``S/memory/backends/token.py:85-114`` (lowest ties)
``commit``                 ``S/memory/backends/commit.py:36-58``
``absolute_addresses``     ``S/memory/routing.py:31-34``
``gather_rows``            ``S/memory/routing.py:37-42``, ``primitives.py:15-20``
``proposal_keys``          ``S/layers/global_layer.py:45,52-53``
``score``                  ``S/layers/global_layer.py:26,42`` (per-head form)
``proposal_delta``         ``S/runtime/dense.py:11-14``
``proposal_error``         ``S/runtime/dense.py:12-13`` (decay and error terms)
``commit_proposals``       ``dense.py:11-14`` + ``global_layer.py:44`` + ``commit``
``require_cuda``           ``S/memory/backends/primitives.py:7-12``
``route_backward``         ``S/memory/backends/token.py:69-82``
``read_backward_*``        autograd of ``S/memory/routing.py:27-28,42``
=========================  ===================================================

All tensors are torch-allocated on the caller's current stream; the library
never allocates device memory and never synchronises.  ``route``,
``snapshot_read``, ``routed_snapshot_read`` and ``commit`` are differentiable
(their backward runs ``glsdm_route_backward``, ``glsdm_read_backward_weights``,
``glsdm_read_backward_rows`` and a row gather); the other entry points are
forward-only and reject inputs that require gradients.
"""
import ctypes

import torch

from ... import _native as N


def require_cuda(*tensors):
    return N.require_device(*tensors)


def after_commit(name, workspace, entries, rows, device):
    """The debug status check of a commit-family call (``_native.set_checks``):
    raise if the commit's sort failed, in which case it wrote no bank row."""
    if not N.checking("status") or entries == 0:
        return
    st = torch.empty(2, dtype=torch.int64, device=device)
    N.call("glsdm_commit_status", N.ptr(workspace), workspace.numel(), entries, rows, N.ptr(st), N.stream(device))
    err = int(st[0])
    if err:
        raise N.NativeError(f"{name}: the commit's sort failed (flags {err}); no bank row was written")


def commit_status(workspace, entries, rows):
    """``(error flags, dropped entries)`` of the last commit-family call made with
    ``workspace`` for ``entries`` entries into ``rows`` rows (synchronises)."""
    device = require_cuda(workspace)
    st = torch.empty(2, dtype=torch.int64, device=device)
    N.call("glsdm_commit_status", N.ptr(workspace), workspace.numel(), entries, rows, N.ptr(st), N.stream(device))
    return tuple(int(x) for x in st.cpu())


def _no_grad(*tensors):
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise NotImplementedError("the HIP memory operator is forward-only; run it under torch.no_grad()")


def _square_root(slots):
    half = int(round(slots ** 0.5))
    while half * half > slots:
        half -= 1
    while (half + 1) * (half + 1) <= slots:
        half += 1
    if half * half != slots:
        raise ValueError("GL-SDM requires square slots and route sizes in [1, slots]")
    return half


def route_workspace(rows, half, width, device):
    """Workspace of the split route path for ``rows`` rows (None when not needed)."""
    size = ctypes.c_size_t(0)
    N.call("glsdm_route_workspace_bytes", rows, half, width, ctypes.byref(size))
    return torch.empty(size.value, dtype=torch.uint8, device=device) if size.value else None


def _route_scores(scores):
    """fp32 or bf16 scores as the kernels take them; bf16 routes exactly as its fp32 widening."""
    if scores.dtype not in N.DTYPES:
        scores = scores.float()
    return scores.contiguous()


def _route(scores, count, tie):
    device = require_cuda(scores)
    half = scores.shape[-1] // 2
    if scores.shape[-1] != 2 * half or not 1 <= count <= half * half:
        raise ValueError("GL-SDM routing needs [..., 2*half] scores and 1 <= count <= half**2")
    index = torch.empty((*scores.shape[:-1], count), dtype=torch.int64, device=device)
    weights = torch.empty((*scores.shape[:-1], count), dtype=torch.float32, device=device)
    rows = scores.numel() // scores.shape[-1]
    # the split-path workspace only within the route's envelope (outside it the route reports the error)
    ws = route_workspace(rows, half, count, device) if half <= 65535 and count <= 64 else None
    N.call("glsdm_route", N.ptr(scores), N.dtype_code(scores), rows, half, count, N.TIES[tie], N.ptr(index),
           N.ptr(weights), N.ptr(ws), 0 if ws is None else ws.numel(), N.stream(device))
    return index, weights


def route_backward(index, weights, grad_weights, half):
    """Factor-score gradient ``[..., 2*half]`` fp32 of a route (token.py:69-82)."""
    device = require_cuda(index, weights, grad_weights)
    width = index.shape[-1]
    out = torch.empty((*index.shape[:-1], 2 * half), dtype=torch.float32, device=device)
    N.call("glsdm_route_backward", N.ptr(index), N.ptr(weights), N.ptr(grad_weights), index.numel() // width,
           half, width, N.ptr(out), N.stream(device))
    return out


class _Route(torch.autograd.Function):
    @staticmethod
    def forward(ctx, scores, count, tie):
        index, weights = _route(scores, count, tie)
        ctx.save_for_backward(index, weights)
        ctx.half = scores.shape[-1] // 2
        ctx.mark_non_differentiable(index)
        return index, weights

    @staticmethod
    def backward(ctx, _, grad_weights):
        index, weights = ctx.saved_tensors
        if grad_weights is None:
            return None, None, None
        return route_backward(index, weights, grad_weights.float().contiguous(), ctx.half), None, None


def route(scores, count, tie="lowest"):
    """Product-key route of fp32 (or bf16) scores ``[..., 2*half]`` -> (index int64, weights fp32)
    ``[..., count]``; bf16 scores route as their fp32 widening.

    Differentiable w.r.t. ``scores`` through the weights (token.py:85-114)."""
    if torch.is_grad_enabled() and scores.requires_grad:
        return _Route.apply(scores.float().contiguous(), count, tie)
    return _route(_route_scores(scores), count, tie)


def _read(values, index, weights, out_dtype, narrow=False):
    """``narrow``: ``glsdm_read_narrow`` (the same bits; fits beside the route kernel)."""
    device = require_cuda(values, index, weights)
    B, H, S, D = values.shape
    if index.ndim != 4 or index.shape[0] != B or index.shape[2] != H or weights.shape != index.shape:
        raise ValueError("snapshot_read needs [B, T, H, width] int64 index and fp32 weights")
    if index.dtype != torch.int64 or weights.dtype != torch.float32:
        raise ValueError("snapshot_read needs int64 index and fp32 weights")
    T, width = index.shape[1], index.shape[3]
    N.check_range(index, S, "snapshot_read")
    out = torch.empty((B, T, H, D), dtype=out_dtype, device=device)
    N.call("glsdm_read_narrow" if narrow else "glsdm_read", N.ptr(values), N.dtype_code(values), B, H, S, D, T,
           width, N.ptr(index), N.ptr(weights), N.ptr(out), N.dtype_code(out), N.stream(device))
    return out


def read_backward_weights(values, index, grad_out):
    """``grad_w[b,t,h,j] = <grad_out[b,t,h], values[b,h,index[b,t,h,j]]>`` (fp32)."""
    device = require_cuda(values, index, grad_out)
    B, H, S, D = values.shape
    T, width = index.shape[1], index.shape[3]
    out = torch.empty(index.shape, dtype=torch.float32, device=device)
    N.call("glsdm_read_backward_weights", N.ptr(values), N.dtype_code(values), B, H, S, D, T, width,
           N.ptr(index), N.ptr(grad_out), N.ptr(out), N.stream(device))
    return out


def read_backward_rows(grad_bank, addresses, weights, grad_out, workspace=None):
    """In place: ``grad_bank.view(-1, D)[addresses[e]] += weights[e] * grad_out[e // width]``,
    each row's terms summed in entry order (fp32 ``grad_bank``)."""
    device = require_cuda(grad_bank, addresses, weights, grad_out)
    if grad_bank.dtype != torch.float32:
        raise ValueError("read_backward_rows accumulates into an fp32 gradient")
    D = grad_bank.shape[-1]
    E, R = addresses.numel(), grad_out.numel() // D
    if E == 0:
        return grad_bank
    if grad_out.shape[-1] != D or R == 0 or E % R != 0 or weights.numel() != E:
        raise ValueError("read_backward_rows needs weights [E], grad_out [R, D] with E a multiple of R")
    width = E // R
    rows = grad_bank.numel() // D
    N.check_range(addresses, rows, "read_backward_rows")
    need = commit_workspace_bytes(E, rows)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    N.call("glsdm_read_backward_rows", N.ptr(grad_bank), rows, D, N.ptr(addresses), E, width, N.ptr(weights),
           N.ptr(grad_out), N.ptr(workspace), workspace.numel(), N.stream(device))
    after_commit("read_backward_rows", workspace, E, rows, device)
    return grad_bank


def _read_grads(ctx_values, index, weights, grad_out, need_values, need_weights):
    grad_out = grad_out.float().contiguous()
    grad_w = read_backward_weights(ctx_values, index, grad_out) if need_weights else None
    grad_v = None
    if need_values:
        grad_v = torch.zeros(ctx_values.shape, dtype=torch.float32, device=ctx_values.device)
        read_backward_rows(grad_v, absolute_addresses(ctx_values, index), weights, grad_out)
        grad_v = grad_v.to(ctx_values.dtype)
    return grad_v, grad_w


class _SnapshotRead(torch.autograd.Function):
    @staticmethod
    def forward(ctx, values, index, weights, out_dtype):
        ctx.save_for_backward(values, index, weights)
        return _read(values, index, weights, out_dtype)

    @staticmethod
    def backward(ctx, grad_out):
        values, index, weights = ctx.saved_tensors
        grad_v, grad_w = _read_grads(values, index, weights, grad_out, ctx.needs_input_grad[0],
                                     ctx.needs_input_grad[2])
        return grad_v, None, grad_w, None


def snapshot_read(values, index, weights, out_dtype=torch.float32):
    """Weighted gather ``sum_j w_j * values[b, h, index_j]`` -> ``[B, T, H, D]``;
    differentiable w.r.t. ``values`` and ``weights``."""
    if torch.is_grad_enabled() and (values.requires_grad or weights.requires_grad):
        return _SnapshotRead.apply(values, index, weights, out_dtype)
    return _read(values, index, weights, out_dtype)


def _routed_read(values, scores, width, tie, out_dtype):
    device = require_cuda(values, scores)
    B, H, S, D = values.shape
    if scores.ndim != 4 or scores.shape[0] != B or scores.shape[2] != H:
        raise ValueError("routed_snapshot_read needs [B, T, H, 2*half] scores matching the bank")
    half = _square_root(S)
    if scores.shape[3] != 2 * half or not 1 <= width <= S:
        raise ValueError("GL-SDM requires square slots and route sizes in [1, slots]")
    T = scores.shape[1]
    out = torch.empty((B, T, H, D), dtype=out_dtype, device=device)
    index = torch.empty((B, T, H, width), dtype=torch.int64, device=device)
    weights = torch.empty((B, T, H, width), dtype=torch.float32, device=device)
    ws = route_workspace(B * T * H, half, width, device) if half <= 65535 and width <= 64 else None
    N.call("glsdm_route_read", N.ptr(values), N.dtype_code(values), B, H, S, D, T, N.ptr(scores),
           N.dtype_code(scores), width, N.TIES[tie], N.ptr(out), N.dtype_code(out), N.ptr(index), N.ptr(weights),
           N.ptr(ws), 0 if ws is None else ws.numel(), N.stream(device))
    return out, index, weights


class _RoutedRead(torch.autograd.Function):
    @staticmethod
    def forward(ctx, values, scores, width, tie, out_dtype):
        out, index, weights = _routed_read(values, scores, width, tie, out_dtype)
        ctx.save_for_backward(values, index, weights)
        ctx.half = scores.shape[-1] // 2
        ctx.mark_non_differentiable(index)
        return out, index, weights

    @staticmethod
    def backward(ctx, grad_out, _, grad_weights):
        values, index, weights = ctx.saved_tensors
        need_v, need_s = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        grad_v, grad_w = None, None
        if grad_out is not None:
            grad_v, grad_w = _read_grads(values, index, weights, grad_out, need_v, need_s)
        grad_s = None
        if need_s:
            total = grad_w if grad_weights is None else (
                grad_weights.float() if grad_w is None else grad_w + grad_weights.float())
            if total is not None:
                grad_s = route_backward(index, weights, total.contiguous(), ctx.half)
        return grad_v, grad_s, None, None, None


def routed_snapshot_read(values, scores, width, allow_large_route=False, tie="highest",
                         out_dtype=torch.float32):
    """Route fp32 (or bf16) scores ``[B, T, H, 2*half]`` and read the bank ``[B, H, half**2, D]``;
    bf16 scores route as their fp32 widening.

    Returns ``(readings [B,T,H,D], index int64 [B,T,H,width] ascending, weights fp32)``;
    differentiable w.r.t. ``values`` and ``scores`` (through readings and weights).
    ``allow_large_route`` is accepted for signature compatibility; every factor
    extent up to 65535 is supported.
    """
    del allow_large_route
    if torch.is_grad_enabled() and (values.requires_grad or scores.requires_grad):
        return _RoutedRead.apply(values, scores.float().contiguous(), width, tie, out_dtype)
    return _routed_read(values, _route_scores(scores), width, tie, out_dtype)


def score(queries, subkeys):
    """Factor scores ``[B, T, H, L]`` fp32 from bf16 queries ``[B, T, H, dk]`` and sub-keys ``[H, L, dk]``."""
    _no_grad(queries, subkeys)
    device = require_cuda(queries, subkeys)
    if queries.dtype != torch.bfloat16 or subkeys.dtype != torch.bfloat16:
        raise ValueError("score needs bf16 queries and sub-keys")
    B, T, H, dk = queries.shape
    if subkeys.ndim != 3 or subkeys.shape[0] != H or subkeys.shape[2] != dk or subkeys.shape[1] % 2:
        raise ValueError("score needs sub-keys [H, 2*half, dk] matching the queries")
    L = subkeys.shape[1]
    out = torch.empty((B, T, H, L), dtype=torch.float32, device=device)
    N.call("glsdm_score", N.ptr(queries), N.ptr(subkeys), B, T, H, dk, L // 2, N.ptr(out), N.stream(device))
    return out


def score_route_workspace_bytes(B, T, H, half, width):
    size = N.ctypes.c_size_t(0)
    N.call("glsdm_score_route_workspace_bytes", B, T, H, half, width, N.ctypes.byref(size))
    return size.value


def score_route(queries, subkeys, width, tie="highest", export_scores=False, split=True, workspace=None):
    """Fused MFMA scoring + route: bf16 queries ``[B,T,H,dk]`` and sub-keys ``[H,L,dk]``
    -> ``(index int64 [B,T,H,width], weights fp32, scores fp32 [B,T,H,L] or None)``.

    ``split`` lets small launches (few tokens, one head) spread each factor's
    sub-key columns over more blocks through a workspace (``workspace``, uint8
    device tensor, allocated here when not given); results are identical either way."""
    _no_grad(queries, subkeys)
    device = require_cuda(queries, subkeys)
    if queries.dtype != torch.bfloat16 or subkeys.dtype != torch.bfloat16:
        raise ValueError("score_route needs bf16 queries and sub-keys")
    B, T, H, dk = queries.shape
    if subkeys.ndim != 3 or subkeys.shape[0] != H or subkeys.shape[2] != dk or subkeys.shape[1] % 2:
        raise ValueError("score_route needs sub-keys [H, 2*half, dk] matching the queries")
    L = subkeys.shape[1]
    half = L // 2
    if not 1 <= width <= half * half:
        raise ValueError("GL-SDM requires square slots and route sizes in [1, slots]")
    index = torch.empty((B, T, H, width), dtype=torch.int64, device=device)
    weights = torch.empty((B, T, H, width), dtype=torch.float32, device=device)
    scores = torch.empty((B, T, H, L), dtype=torch.float32, device=device) if export_scores else None
    need = score_route_workspace_bytes(B, T, H, half, width) if split else 0
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    ws = workspace if need else None
    N.call("glsdm_score_route", N.ptr(queries), N.ptr(subkeys), B, T, H, dk, half, width, N.TIES[tie],
           N.ptr(scores), N.ptr(index), N.ptr(weights), N.ptr(ws), 0 if ws is None else ws.numel(),
           N.stream(device))
    return index, weights, scores


def score_route_keys(queries, subkeys, width, offset, chunk_size, num_layers, layer_idx, tie="highest",
                     split=True, workspace=None):
    """Fused scoring + route + proposal keys: ``(index, weights, addresses, keys)``,
    each ``[B, T, H, width]``; equal to :func:`score_route` followed by
    :func:`proposal_keys` (forward-only)."""
    _no_grad(queries, subkeys)
    device = require_cuda(queries, subkeys)
    if queries.dtype != torch.bfloat16 or subkeys.dtype != torch.bfloat16:
        raise ValueError("score_route_keys needs bf16 queries and sub-keys")
    B, T, H, dk = queries.shape
    L = subkeys.shape[1]
    half = L // 2
    if subkeys.ndim != 3 or subkeys.shape[0] != H or subkeys.shape[2] != dk or L % 2:
        raise ValueError("score_route_keys needs sub-keys [H, 2*half, dk] matching the queries")
    if not 1 <= width <= half * half:
        raise ValueError("GL-SDM requires square slots and route sizes in [1, slots]")
    shape = (B, T, H, width)
    index = torch.empty(shape, dtype=torch.int64, device=device)
    weights = torch.empty(shape, dtype=torch.float32, device=device)
    addresses = torch.empty(shape, dtype=torch.int64, device=device)
    keys = torch.empty(shape, dtype=torch.int64, device=device)
    need = score_route_workspace_bytes(B, T, H, half, width) if split else 0
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    ws = workspace if need else None
    N.call("glsdm_score_route_keys", N.ptr(queries), N.ptr(subkeys), B, T, H, dk, half, width, N.TIES[tie], offset,
           chunk_size, num_layers, layer_idx, N.ptr(index), N.ptr(weights), N.ptr(addresses), N.ptr(keys),
           N.ptr(ws), 0 if ws is None else ws.numel(), N.stream(device))
    return index, weights, addresses, keys


def absolute_addresses(values, index):
    """``(b*H + h)*S + index`` for ``index [B, T, H, width]``."""
    device = require_cuda(values, index)
    B, H, S, _ = values.shape
    if index.ndim != 4 or index.dtype != torch.int64 or index.shape[0] != B or index.shape[2] != H:
        raise ValueError("absolute_addresses needs a [B, T, H, width] int64 index")
    N.check_range(index, S, "absolute_addresses")
    out = torch.empty_like(index)
    N.call("glsdm_absolute_addresses", N.ptr(index), B, index.shape[1], H, index.shape[3], S, N.ptr(out),
           N.stream(device))
    return out


def proposal_keys(values, index, offset, chunk_size, num_layers, layer_idx):
    """Write addresses and collision keys ``addr*(C*L) + (offset + t)*L + layer``."""
    device = require_cuda(values, index)
    B, H, S, _ = values.shape
    if index.ndim != 4 or index.dtype != torch.int64 or index.shape[0] != B or index.shape[2] != H:
        raise ValueError("proposal_keys needs a [B, T, H, width] int64 index")
    N.check_range(index, S, "proposal_keys")
    addresses = torch.empty_like(index)
    keys = torch.empty_like(index)
    N.call("glsdm_proposal_keys", N.ptr(index), B, index.shape[1], H, index.shape[3], S, offset, chunk_size,
           num_layers, layer_idx, N.ptr(addresses), N.ptr(keys), N.stream(device))
    return addresses, keys


def _gather(values, addr, shape):
    D = values.shape[-1]
    N.check_range(addr, values.numel() // D, "gather_rows")
    out = torch.empty((*shape, D), dtype=values.dtype, device=values.device)
    N.call("glsdm_gather_rows", N.ptr(values), N.dtype_code(values), values.numel() // D, D, N.ptr(addr),
           addr.numel(), N.ptr(out), N.stream(values.device))
    return out


class _GatherRows(torch.autograd.Function):
    """The row gather of S/memory/routing.py:31-42; its backward adds each
    gathered row's gradient onto its bank row, a row's terms summed in entry
    order (the accumulating index backward of ``flat[address]``)."""

    @staticmethod
    def forward(ctx, values, index):
        addr = absolute_addresses(values, index)
        ctx.save_for_backward(addr)
        ctx.values_shape, ctx.values_dtype = values.shape, values.dtype
        return _gather(values, addr, index.shape)

    @staticmethod
    def backward(ctx, grad_rows):
        (addr,) = ctx.saved_tensors
        D = ctx.values_shape[-1]
        grad_v = torch.zeros(ctx.values_shape, dtype=torch.float32, device=addr.device)
        ones = torch.ones(addr.numel(), dtype=torch.float32, device=addr.device)
        read_backward_rows(grad_v, addr.reshape(-1), ones, grad_rows.float().reshape(-1, D).contiguous())
        return grad_v.to(ctx.values_dtype), None


def gather_rows(values, index):
    """Rows ``[B, T, H, width, D]`` of the bank at ``index [B, T, H, width]``;
    differentiable w.r.t. ``values``."""
    if torch.is_grad_enabled() and values.requires_grad:
        return _GatherRows.apply(values, index)
    return _gather(values, absolute_addresses(values, index), index.shape)


def gather_flat(values, addresses):
    """Rows ``[*addresses.shape, D]`` of ``values`` viewed as ``[rows, D]`` at absolute ``addresses``."""
    device = require_cuda(values, addresses)
    if addresses.dtype != torch.int64:
        raise ValueError("gather_flat needs int64 addresses")
    D = values.shape[-1]
    N.check_range(addresses, values.numel() // D, "gather_rows")
    out = torch.empty((*addresses.shape, D), dtype=values.dtype, device=device)
    N.call("glsdm_gather_rows", N.ptr(values), N.dtype_code(values), values.numel() // D, D, N.ptr(addresses),
           addresses.numel(), N.ptr(out), N.stream(device))
    return out


def commit_workspace_bytes(entries, rows):
    size = N.ctypes.c_size_t(0)
    N.call("glsdm_commit_workspace_bytes", entries, rows, N.ctypes.byref(size))
    return size.value


def _commit(memory, indices, deltas, keys, donate, workspace, unique):
    device = require_cuda(memory, indices, deltas, keys)
    if indices.dtype != torch.int64 or (keys is not None and keys.dtype != torch.int64):
        raise ValueError("commit needs int64 addresses and keys")
    D = memory.shape[-1]
    E = indices.numel()
    deltas = deltas.reshape(E, D) if deltas.numel() == E * D else None
    if deltas is None or (keys is not None and keys.numel() != E):
        raise ValueError("commit needs deltas [E, D] and keys [E] matching the addresses")
    rows = memory.numel() // D
    N.check_range(indices, rows, "commit")
    out = memory if donate else memory.clone()
    if E == 0:
        return out
    need = commit_workspace_bytes(E, rows)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    N.call("glsdm_commit", N.ptr(out), N.dtype_code(out), rows, D, N.ptr(indices), N.ptr(deltas),
           N.dtype_code(deltas), N.ptr(keys), E, N.ptr(workspace), workspace.numel(), N.ptr(unique),
           N.stream(device))
    after_commit("commit", workspace, E, rows, device)
    return out


class _Commit(torch.autograd.Function):
    """backends/commit.py:36-54: the bank's gradient passes through; each delta's
    gradient is the bank gradient's row at its address (0 for dropped entries)."""

    @staticmethod
    def forward(ctx, memory, indices, deltas, keys):
        ctx.save_for_backward(indices)
        ctx.delta_shape, ctx.delta_dtype = deltas.shape, deltas.dtype
        return _commit(memory, indices, deltas, keys, False, None, None)

    @staticmethod
    def backward(ctx, incoming):
        (indices,) = ctx.saved_tensors
        incoming = incoming.contiguous()
        grad_d = None
        if ctx.needs_input_grad[2]:
            grad_d = gather_flat(incoming.float(), indices.reshape(-1)).reshape(ctx.delta_shape).to(ctx.delta_dtype)
        return incoming, None, grad_d, None


def commit(memory, indices, deltas, keys=None, donate=False, workspace=None, unique=None):
    """Deterministic commit of ``deltas [E, D]`` at absolute rows ``indices [E]``.

    ``memory`` is any contiguous tensor whose last dimension is D (e.g. the
    ``[B, H, S, D]`` bank).  Returns the updated bank: a new tensor, or
    ``memory`` itself updated in place when ``donate=True`` (the caller gives
    up the old contents; no full-bank copy is made).

    ``keys`` (int64 [E], default: arrival order) orders colliding deltas: each
    address's deltas are summed from +0 in ascending (key, entry) order.
    ``workspace`` (uint8 device tensor) and ``unique`` (int64 [1] device
    counter, incremented by the number of touched rows) are optional.
    Differentiable w.r.t. ``memory`` and ``deltas`` (not with ``donate=True``).
    """
    if torch.is_grad_enabled() and (memory.requires_grad or deltas.requires_grad):
        if donate:
            raise ValueError("commit: donate=True cannot be differentiated (the input bank is overwritten)")
        return _Commit.apply(memory, indices, deltas, keys)
    return _commit(memory, indices, deltas, keys, donate, workspace, unique)


def _proposal_rows(prediction, target, beta, log_decay):
    """Shapes of the per-row proposal operands: prediction/target ``[..., H, D]``,
    beta/log_decay ``[..., H, 1]`` -> (R, H, D)."""
    if prediction.ndim < 2 or target.shape != prediction.shape:
        raise ValueError("proposal needs prediction and target of one shape [..., H, D]")
    if prediction.dtype != torch.float32 or target.dtype not in N.DTYPES:
        raise ValueError("proposal needs fp32 prediction and fp32 or bf16 target")
    lead = prediction.shape[:-1]
    for t in (beta, log_decay):
        if t.dtype != torch.float32 or t.shape not in ((*lead, 1), lead):
            raise ValueError("proposal needs fp32 beta and log_decay of shape [..., H, 1]")
    D = prediction.shape[-1]
    return prediction.numel() // D, prediction.shape[-2], D


def proposal_error(prediction, target, beta, log_decay):
    """``(error [..., H, D] fp32, decay [..., H] fp32)``: decay = exp(log_decay),
    error = beta * (target - decay * prediction), the per-row terms of dense.py:12-13."""
    _no_grad(prediction, target, beta, log_decay)
    device = require_cuda(prediction, target, beta, log_decay)
    R, _, D = _proposal_rows(prediction, target, beta, log_decay)
    error = torch.empty(prediction.shape, dtype=torch.float32, device=device)
    decay = torch.empty(prediction.shape[:-1], dtype=torch.float32, device=device)
    N.call("glsdm_proposal_error", R, D, N.ptr(prediction), N.ptr(target), N.dtype_code(target), N.ptr(beta),
           N.ptr(log_decay), N.ptr(error), N.ptr(decay), N.stream(device))
    return error, decay


def proposal_delta(rows, weights, prediction, target, beta, log_decay, mass):
    """Write deltas ``[..., H, k, D]`` fp32 of dense.py:11-14:
    ``mass * ((exp(log_decay) - 1) * rows + weights * beta * (target - exp(log_decay) * prediction))``."""
    _no_grad(rows, weights, prediction, target, beta, log_decay, mass)
    device = require_cuda(rows, weights, prediction, target, beta, log_decay, mass)
    R, H, D = _proposal_rows(prediction, target, beta, log_decay)
    lead = prediction.shape[:-2]
    if rows.ndim != prediction.ndim + 1 or rows.shape[:-2] != prediction.shape[:-1] or rows.shape[-1] != D:
        raise ValueError("proposal_delta needs rows [..., H, k, D] matching the prediction")
    k = rows.shape[-2]
    if weights.shape != rows.shape[:-1] or weights.dtype != torch.float32 or rows.dtype not in N.DTYPES:
        raise ValueError("proposal_delta needs fp32 weights [..., H, k] and fp32 or bf16 rows")
    if mass.shape != lead or mass.dtype != torch.float32:
        raise ValueError("proposal_delta needs fp32 mass of the leading shape [...]")
    out = torch.empty(rows.shape, dtype=torch.float32, device=device)
    N.call("glsdm_proposal_delta", N.ptr(rows), N.dtype_code(rows), R, k, D, N.ptr(weights), N.ptr(prediction),
           N.ptr(target), N.dtype_code(target), N.ptr(beta), N.ptr(log_decay), N.ptr(mass), H, N.ptr(out),
           N.stream(device))
    return out


def commit_proposals(memory, indices, keys, weights, error, decay, mass, donate=False, workspace=None,
                     unique=None):
    """Fused proposal -> commit: commits the deltas
    ``mass[r // H] * ((decay[r] - 1) * memory[indices[e]] + weights[e] * error[r])``, ``r = e // k``,
    evaluated in the commit from each touched row (never stored).

    ``indices``/``keys``/``weights`` ``[..., H, k]`` (absolute rows, collision
    keys or None, route weights), ``error [..., H, D]`` and ``decay [..., H]``
    from :func:`proposal_error`, ``mass`` of the leading shape ``[...]``.  The
    rows must be those the proposal was made against (``memory`` is its
    snapshot).  Bitwise equal to ``commit(memory, indices, proposal_delta(...), keys)``.
    """
    _no_grad(memory, weights, error, decay, mass)
    device = require_cuda(memory, indices, keys, weights, error, decay, mass)
    D = memory.shape[-1]
    if indices.dtype != torch.int64 or (keys is not None and (keys.dtype != torch.int64
                                                               or keys.shape != indices.shape)):
        raise ValueError("commit_proposals needs int64 addresses and keys of one shape")
    if indices.ndim < 2 or weights.shape != indices.shape or weights.dtype != torch.float32:
        raise ValueError("commit_proposals needs fp32 weights [..., H, k] matching the addresses")
    H, k = indices.shape[-2], indices.shape[-1]
    if (error.shape != (*indices.shape[:-1], D) or decay.shape != indices.shape[:-1]
            or mass.shape != indices.shape[:-2]):
        raise ValueError("commit_proposals needs error [..., H, D], decay [..., H] and mass [...] "
                         "matching the addresses [..., H, k]")
    if error.dtype != torch.float32 or decay.dtype != torch.float32 or mass.dtype != torch.float32:
        raise ValueError("commit_proposals needs fp32 error, decay and mass")
    rows = memory.numel() // D
    N.check_range(indices, rows, "commit_proposals")
    out = memory if donate else memory.clone()
    E = indices.numel()
    if E == 0:
        return out
    need = commit_workspace_bytes(E, rows)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    N.call("glsdm_commit_proposals", N.ptr(out), N.dtype_code(out), rows, D, N.ptr(indices), N.ptr(keys), E, k,
           N.ptr(weights), N.ptr(error), N.ptr(decay), N.ptr(mass), H, N.ptr(workspace), workspace.numel(),
           N.ptr(unique), N.stream(device))
    after_commit("commit_proposals", workspace, E, rows, device)
    return out
