"""RMSNorm and the gated squared-ReLU MLP of S/layers/common.py:7-27
(S/ = projects/gl-sdm/src/gl_sdm/)."""
import torch
from torch import nn
import torch.nn.functional as F


class RMSNorm(nn.Module):
    """``rms_norm`` over the last dimension, eps 1e-6, weight cast to the input dtype."""

    def __init__(self, dim):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        return F.rms_norm(x, (x.shape[-1],), self.weight.to(x.dtype), eps=1e-6)


class MLP(nn.Module):
    """``proj(gate * relu(u)^2)`` with ``u, gate = fc(x).chunk(2)``; inner width 4*dim by default."""

    def __init__(self, dim, intermediate_size=None):
        super().__init__()
        inner = 4 * dim if intermediate_size is None else intermediate_size
        if inner < 1:
            raise ValueError("intermediate_size must be positive")
        self.fc = nn.Linear(dim, 2 * inner)
        self.proj = nn.Linear(inner, dim)

    def forward(self, x):
        u, gate = self.fc(x).chunk(2, -1)
        return self.proj(gate * u.relu().square())
