"""Product-key projections of a global layer (S/layers/router.py:13-37,
S/ = projects/gl-sdm/src/gl_sdm/).

``q``/``k`` map the hidden state to per-head factor scores ``[heads, 2*half]``
for the read and the write route; ``v``, ``beta`` and ``decay`` give the write
target and gates; ``proj`` and ``read_norm`` mix the readings back.  The
memory backend is ``"hip"`` (libglsdm.so); the chunk routes break equal scores
towards the larger sub-key and slot index, as S/memory/routing.py:15-17.
"""
import math

from torch import nn

from .common import RMSNorm


class GlobalRouter(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        dim, dk = cfg["hidden_size"], cfg["head_dim"]
        self.heads, self.head_dim = dim // dk, dk
        self.slots = cfg.get("gl_slots", 1024)
        self.half = math.isqrt(self.slots)
        self.num_reads, self.num_writes = cfg.get("gl_reads", 8), cfg.get("gl_writes", 8)
        if (self.half ** 2 != self.slots or min(self.num_reads, self.num_writes) < 1
                or max(self.num_reads, self.num_writes) > self.slots):
            raise ValueError("GL-SDM requires square slots and route sizes in [1, slots]")
        self.q = nn.Linear(dim, self.heads * 2 * self.half)
        self.k = nn.Linear(dim, self.heads * 2 * self.half)
        self.v = nn.Linear(dim, dim)
        self.beta = nn.Linear(dim, self.heads)
        self.decay = nn.Linear(dim, self.heads)
        self.proj = nn.Linear(dim, dim)
        self.read_norm = RMSNorm(dk)
        self.backend = cfg.get("gl_memory_backend", "hip")
        if self.backend != "hip":
            raise ValueError("gl_memory_backend must be hip (libglsdm.so replaces the torch and urm backends)")
        self.tie = "highest"
        self.reference = False
