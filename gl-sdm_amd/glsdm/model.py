"""The GL-SDM layer-stack language model (S/model.py:22-96, S/ =
projects/gl-sdm/src/gl_sdm/), for ``arch_type == "gl_sdm"`` with a
``gl_layer_pattern``: token embedding, the physical stack sharing one memory
bank, final RMSNorm and a soft-capped vocabulary head ``15 * l / sqrt(l^2 + 225)``.

``gl_state_dtype`` (default ``"float32"``, the reference's only choice) selects
the dtype of the request snapshots; ``"bfloat16"`` halves a per-request bank.
"""
import torch
from torch import nn
import torch.nn.functional as F

from .layers.common import RMSNorm, linear
from .layers.stack import forward as stack_forward, make_layers
from .memory import MemoryBank


def soft_cap(logits):
    return 15 * logits * (logits.square() + 15 ** 2).rsqrt()


class Model(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.cfg = dict(cfg)
        if cfg.get("arch_type") != "gl_sdm" or "gl_layer_pattern" not in cfg:
            raise ValueError("glsdm provides the physical GL-SDM layer stack (arch_type gl_sdm with gl_layer_pattern)")
        self.is_layer_stack = True
        dim, layers = cfg["hidden_size"], cfg["num_hidden_layers"]
        if layers < 1 or dim % cfg["head_dim"]:
            raise ValueError("positive layer count and hidden_size divisible by head_dim required")
        self.embed = nn.Embedding(cfg["vocab_size"], dim)
        self.blocks = nn.ModuleList(make_layers(cfg))
        self.bank = MemoryBank(dim // cfg["head_dim"], cfg["gl_slots"], cfg["head_dim"],
                               state_dtype=getattr(torch, cfg.get("gl_state_dtype", "float32")))
        self.norm = RMSNorm(dim)
        self.proj = nn.Linear(dim, cfg["vocab_size"], bias=False)
        self.num_attn_layers = layers
        self.to(dtype=getattr(torch, cfg.get("dtype", "bfloat16")))

    def head(self, x):
        return soft_cap(linear(self.proj, self.norm(x).to(self.proj.weight.dtype)).float())

    def hidden(self, inputs, cache=None):
        x = self.embed(inputs)
        if self.cfg.get("residual_dtype") == "float32":
            x = x.float()
        return stack_forward(self, x, None if cache is None else cache[0])

    def forward(self, inputs, targets):
        x, reg, align = self.hidden(inputs)
        logits = self.head(x)
        return F.cross_entropy(logits.reshape(-1, logits.shape[-1]), targets.reshape(-1), reduction="sum"), reg, align

    def new_cache(self, batch_size):
        return [self.bank.new_cache(batch_size)]

    @torch.inference_mode()
    def prefill(self, inputs, cache=None):
        if self.training:
            raise RuntimeError("call model.eval() before inference")
        cache = self.new_cache(inputs.shape[0]) if cache is None else cache
        x, _, _ = self.hidden(inputs, cache)
        return self.head(x), cache

    @torch.inference_mode()
    def decode(self, inputs, cache):
        if inputs.shape[1] != 1:
            raise ValueError("decode expects one token per request")
        return self.prefill(inputs, cache)


def create_model(cfg):
    return Model(cfg)
