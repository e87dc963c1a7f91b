"""Local causal attention of the stack's local layers.

Mirrors ``Transformer`` of S/layers/attention.py:11-77 (S/ =
projects/gl-sdm/src/gl_sdm/): a query/gate projection ``q: dim -> 2*dim``
(per head ``[query | gate]``), key/value projections, parameter-free RMS
normalisation of queries and keys, rotary positions from absolute token
positions, scaled dot-product attention over a rolling window, and a sigmoid
output gate before ``proj``.  The KV cache keeps the last ``window - 1`` keys
and values and the absolute token count, so chunked prefill and decode see
exactly the keys a full pass sees.
"""
import torch
from torch import nn
import torch.nn.functional as F


class Transformer(nn.Module):
    def __init__(self, cfg, layer_idx):
        super().__init__()
        del layer_idx
        dim, dk = cfg["hidden_size"], cfg["head_dim"]
        self.head_dim, self.num_heads = dk, dim // dk
        self.window = cfg.get("attention_window")
        if self.window is not None and self.window < 1:
            raise ValueError("attention_window must be positive")
        self.num_kv_heads = cfg.get("num_key_value_heads", self.num_heads)
        if self.num_heads % self.num_kv_heads or dk % 4:
            raise ValueError("head_dim must be divisible by 4; KV heads must divide query heads")
        self.q = nn.Linear(dim, 2 * dim)
        self.k = nn.Linear(dim, self.num_kv_heads * dk)
        self.v = nn.Linear(dim, self.num_kv_heads * dk)
        self.proj = nn.Linear(dim, dim)
        # rotary frequencies 1024^-u, u in [0, 1], on the first quarter of each
        # half of a head; the second quarter keeps angle 0
        rising = torch.pow(torch.tensor(1 / 1024), torch.linspace(0, 1, dk // 4))
        self.register_buffer("angular_freq", torch.cat((rising, torch.zeros_like(rising))))
        self.reference = False

    def _apply(self, fn, recurse=True):
        # the rotary frequencies stay fp32 when the projections are cast
        freq = self.angular_freq
        super()._apply(fn, recurse)
        self.angular_freq = freq.to(device=self.angular_freq.device)
        return self

    def rotary(self, x, offset):
        """Rotate ``x [B, T, heads, dk]`` by the angles of absolute positions ``offset + t`` (fp32)."""
        pos = torch.arange(offset, offset + x.shape[1], device=x.device, dtype=torch.float32)
        angle = torch.outer(pos, self.angular_freq.float())[None, :, None]
        cos, sin = angle.cos(), angle.sin()
        a, b = x.float().chunk(2, -1)
        return torch.cat((a * cos + b * sin, -a * sin + b * cos), -1).to(x.dtype)

    def forward(self, x, cache=None):
        B, T, D = x.shape
        dk = self.head_dim
        q, gate = self.q(x).view(B, T, self.num_heads, 2 * dk).chunk(2, -1)
        k = self.k(x).view(B, T, self.num_kv_heads, dk)
        v = self.v(x).view(B, T, self.num_kv_heads, dk).transpose(1, 2)
        previous = cache["k"].shape[2] if cache else 0
        offset = 0 if cache is None else cache.get("tokens", previous)
        q = self.rotary(F.rms_norm(q, (dk,)), offset).transpose(1, 2)
        k = self.rotary(F.rms_norm(k, (dk,)), offset).transpose(1, 2)
        if cache is not None:
            if cache:
                k, v = torch.cat((cache["k"], k), 2), torch.cat((cache["v"], v), 2)
            n = k.shape[2]
            keep = n if self.window is None else min(self.window - 1, n)
            cache.update(k=k[:, :, n - keep:], v=v[:, :, n - keep:], tokens=offset + T)
        groups = self.num_heads // self.num_kv_heads
        if groups != 1:
            k, v = k.repeat_interleave(groups, 1), v.repeat_interleave(groups, 1)
        # keys cover positions [offset - previous, offset + T); a cached prefill
        # needs this offset causal mask (SDPA's own causal mask is upper-left aligned)
        mask = None
        if offset or self.window is not None:
            kpos = torch.arange(offset - previous, offset + T, device=x.device)[None, :]
            qpos = torch.arange(offset, offset + T, device=x.device)[:, None]
            mask = kpos <= qpos
            if self.window is not None:
                mask = mask & (kpos > qpos - self.window)
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=mask is None)
        return self.proj(out.transpose(1, 2).reshape(B, T, D) * gate.reshape(B, T, D).sigmoid())
