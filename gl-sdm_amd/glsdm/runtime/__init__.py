"""Tensor arithmetic of the write path (mirrors S/runtime of the reference)."""
from .dense import proposal_delta

__all__ = ["proposal_delta"]
