"""Snapshot/proposal/commit API of the GL-SDM memory operator (HIP).

Mirrors S/memory/__init__.py (S/ = projects/gl-sdm/src/gl_sdm/).  The
token-clock ``read``/``propose_write`` of the reference are not on the stack's
path and are not provided.
"""
from .state import MemoryView, WriteProposal, DeferredProposal, LoggedProposal, WriteBuffer, MemoryCache, MemoryBank
from .transactions import merge, commit
from .proposals import layer_proposal, log_proposal, ProposalLog
from .overlay import OverlayView

__all__ = ["MemoryView", "WriteProposal", "DeferredProposal", "LoggedProposal", "WriteBuffer", "MemoryCache",
           "MemoryBank", "merge", "commit", "layer_proposal", "log_proposal", "ProposalLog", "OverlayView"]
