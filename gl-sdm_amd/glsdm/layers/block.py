"""Residual block of the stack's local layers: ``x + attn(norm1(x))`` then
``x + mlp(norm2(x))`` (S/baselines/block.py:8-27 with the ``transformer``
mixer, S/ = projects/gl-sdm/src/gl_sdm/)."""
import torch
from torch import nn

from .attention import Transformer
from .common import MLP, RMSNorm


_ZEROS = {}


def zero(x, dtype=None):
    """A 0-d zero of ``dtype`` (default ``x.dtype``) on ``x``'s device, one shared
    tensor per (device, dtype): the regularisers of ``reg_mode == "baseline"`` are
    identically zero, and a fresh fill per layer and chunk is a launch each.
    Read-only; built outside inference mode so autograd may use it."""
    key = (x.device, dtype or x.dtype)
    z = _ZEROS.get(key)
    if z is None:
        with torch.inference_mode(False), torch.no_grad():
            z = torch.zeros((), dtype=key[1], device=key[0])
        _ZEROS[key] = z
    return z


def regulariser(x, reg_mode):
    """The stack's representation regulariser; only ``reg_mode == "baseline"``
    (zero, S/layers/regularization.py:67-68) is part of the operator build."""
    del reg_mode
    return zero(x, torch.float32)


def check_reg_mode(cfg):
    if cfg.get("reg_mode", "baseline") != "baseline":
        raise ValueError("reg_mode must be baseline: the SIGReg sketches are outside the memory-operator build")


class Block(nn.Module):
    def __init__(self, cfg, layer_idx):
        super().__init__()
        if cfg["arch_type"] != "transformer":
            raise ValueError("local layers of the GL-SDM stack use the transformer mixer")
        check_reg_mode(cfg)
        self.arch_type = cfg["arch_type"]
        self.attn = Transformer(cfg, layer_idx)
        self.norm1, self.norm2 = RMSNorm(cfg["hidden_size"]), RMSNorm(cfg["hidden_size"])
        self.mlp = MLP(cfg["hidden_size"], cfg.get("intermediate_size"))
        self.reg_mode = cfg.get("reg_mode", "baseline")

    def forward(self, x, cache=None):
        dtype = self.mlp.fc.weight.dtype
        x = self.attn(self.norm1.cast(x, dtype), cache=cache, residual=x)
        x = self.mlp(self.norm2.cast(x, dtype), residual=x)
        return x, regulariser(x, self.reg_mode), zero(x)
