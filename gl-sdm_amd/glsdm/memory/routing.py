"""Chunk product-key routing and row selection (HIP backend).

Mirrors S/memory/routing.py:31-66 (S/ = projects/gl-sdm/src/gl_sdm/):
``routed_read`` dispatches on ``block.attn.backend``, takes
[B, T, H, 2*half] or [B, R, T, H, 2*half] fp32 scores and returns
(out fp32 [.., D], index int64 [.., width] ascending, weights fp32).  Equal
scores prefer larger addresses, unless the router carries ``tie = "lowest"``.
"""
import torch

from .backends import hip


def routed_read(block, memory, scores, width, physical=None, out_dtype=torch.float32):
    """Route ``scores`` and read ``memory`` (S/memory/routing.py:10-28); readings in
    ``out_dtype`` (bf16: the fp32 sums rounded once, as a later ``.to(bfloat16)``)."""
    del physical  # the HIP read needs no padded bank copy
    attn = block.attn
    if getattr(attn, "backend", None) != "hip" or getattr(attn, "reference", False):
        raise ValueError("glsdm routed_read serves the hip backend only")
    tie = getattr(attn, "tie", "highest")
    shape = scores.shape
    flat = scores.reshape(shape[0], -1, *shape[-2:])
    out, index, weights = hip.routed_snapshot_read(memory, flat.contiguous(), width, tie=tie, out_dtype=out_dtype)
    if len(shape) == 5:
        out, index, weights = (t.reshape(*shape[:-1], t.shape[-1]) for t in (out, index, weights))
    return out, index, weights


def absolute_addresses(memory, index):
    return hip.absolute_addresses(memory, index.contiguous())


def gather_rows(memory, index):
    return hip.gather_rows(memory, index.contiguous())
