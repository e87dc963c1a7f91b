"""Local causal attention of the stack's local layers.

Mirrors ``Transformer`` of S/layers/attention.py:11-77 (S/ =
projects/gl-sdm/src/gl_sdm/): a query/gate projection ``q: dim -> 2*dim``
(per head ``[query | gate]``), key/value projections, parameter-free RMS
normalisation of queries and keys, rotary positions from absolute token
positions, scaled dot-product attention over a rolling window, and a sigmoid
output gate before ``proj``.  The KV cache keeps the last ``window - 1`` keys
and values and the absolute token count, so chunked prefill and decode see
exactly the keys a full pass sees.

On the GPU outside autograd, the QK normalisation and rotary run as one HIP
kernel per projection (``glsdm_qk_norm_rotary``) that also writes the
``[B, heads, T, dk]`` layout; in a decode step one launch
(``glsdm_decode_qkv``) does both projections' and appends the new keys and
values to the KV window buffer.  Under autograd and on the CPU the same
operations run as tensor ops.
"""
import ctypes

import torch
from torch import nn
import torch.nn.functional as F

from .. import _native as N
from .common import linear, linear_group


def qk_norm_rotary(x, freq, offset):
    """``rotary(F.rms_norm(x, (dk,)), offset).transpose(1, 2)`` for ``x [B, T, heads, dk]``
    (fp32 or bf16, rows of dk contiguous elements at a uniform row stride) in one
    HIP launch; returns ``[B, heads, T, dk]`` contiguous."""
    B, T, heads, dk = x.shape
    if not (x.stride(3) == 1 and x.stride(1) == heads * x.stride(2) and x.stride(0) == T * x.stride(1)):
        x = x.contiguous()
    out = torch.empty((B, heads, T, dk), dtype=x.dtype, device=x.device)
    N.call("glsdm_qk_norm_rotary", N.ptr(x), N.dtype_code(x), B, T, heads, dk, x.stride(2), N.ptr(freq), offset,
           N.ptr(out), N.stream(x.device))
    return out


def _token_rows(x):
    """``x [B, T, heads, dk]`` stores row (b*T + t)*heads + h at a uniform row stride
    with contiguous elements (the addressing of the q/k/v kernels)."""
    B, T, H, dk = x.shape
    return (x.stride(3) == 1 and x.stride(2) >= dk and x.stride(1) == H * x.stride(2)
            and x.stride(0) == T * x.stride(1))


def gate_merge(o, gate):
    """``o.transpose(1, 2).reshape(B, T, D) * gate.reshape(B, T, D).sigmoid()`` for
    ``o [B, H, T, dk]`` and ``gate [B, T, H, dk]`` (any strides with contiguous
    rows) in one HIP launch."""
    B, H, T, dk = o.shape
    out = torch.empty((B, T, H * dk), dtype=o.dtype, device=o.device)
    os_, gs = (ctypes.c_int64 * 4)(*o.stride()), (ctypes.c_int64 * 4)(*gate.stride())
    N.call("glsdm_gate_merge", N.ptr(o), os_, N.ptr(gate), gs, N.dtype_code(o), B, T, H, dk, N.ptr(out),
           N.stream(o.device))
    return out


_MASKS = {}
APPEND_MAX_TOKENS = 16    # calls of at most this many tokens (decode) append to the KV window in place


def decode_attention(q, k, v, gate=None):
    """``F.scaled_dot_product_attention(q, k, v)`` for one query row per (request,
    head), ``q [B, H, 1, dk]`` contiguous bf16, ``k``/``v [B, H, L, dk]`` strided
    views with unit last stride, no mask (``glsdm_decode_attention``: fp32 scores,
    softmax and sums, rounded once; within rounding of the library's kernel).
    With ``gate [B, 1, H, dk]`` (unit last stride) the result is
    ``gate_merge(attention, gate)`` as ``[B, 1, H*dk]``, in the same launch."""
    B, H, _, dk = q.shape
    L = k.shape[2]
    if k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("decode_attention needs unit-stride key and value rows")
    ks = (ctypes.c_int64 * 3)(*k.stride()[:3])
    vs = (ctypes.c_int64 * 3)(*v.stride()[:3])
    if gate is None:
        out = torch.empty_like(q)
        N.call("glsdm_decode_attention", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(out), B, H, L, dk, ks, vs,
               ctypes.c_float(dk ** -0.5), N.stream(q.device))
        return out
    if gate.shape != (B, 1, H, dk) or gate.stride(-1) != 1 or gate.dtype != q.dtype:
        raise ValueError("decode_attention needs a gate [B, 1, H, dk] of the query dtype with unit-stride rows")
    out = torch.empty((B, 1, H * dk), dtype=q.dtype, device=q.device)
    gs = (ctypes.c_int64 * 2)(gate.stride(0), gate.stride(2))
    N.call("glsdm_decode_attention_gated", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gate), N.ptr(out), B, H, L, dk, ks,
           vs, gs, ctypes.c_float(dk ** -0.5), N.stream(q.device))
    return out


def _window_mask(previous, T, window, device, dtype):
    """Query i (position offset + i) may see key j (position offset - previous + j)
    when the key is not later and, with a window, less than ``window`` back.  It
    depends on (previous, T, window) only, not on the offset, so one tensor per
    shape is kept (prefill chunks and decode steps reuse it), already in the
    additive form SDPA makes of a boolean mask (0 where allowed, -inf where not,
    in the query dtype), which saves that conversion at every call."""
    key = (previous, T, window, device, dtype)
    mask = _MASKS.get(key)
    if mask is None:
        # an ordinary tensor even when first built under inference mode, so that
        # autograd may save it later
        with torch.inference_mode(False), torch.no_grad():
            kpos = torch.arange(-previous, T, device=device)[None, :]
            qpos = torch.arange(0, T, device=device)[:, None]
            allowed = kpos <= qpos
            if window is not None:
                allowed = allowed & (kpos > qpos - window)
            # rows padded to a multiple of 16 elements: attention kernels want an aligned
            # row stride and would otherwise pad a copy of the mask at every call
            n = allowed.shape[1]
            store = torch.zeros((T, (n + 15) // 16 * 16), dtype=dtype, device=device)
            mask = store[:, :n].masked_fill_(~allowed, float("-inf"))
        if len(_MASKS) >= 64:
            _MASKS.clear()
        _MASKS[key] = mask
    return mask


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
        # decode steps append to a KV window buffer in place (the cache then has one
        # owner); gl_commit_in_place = False keeps the reference's functional cache
        self.append_in_place = bool(cfg.get("gl_commit_in_place", True))
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

    def _append(self, cache, k, v, previous, offset):
        """Inference KV cache for short calls (decode): the window lives in a buffer
        with room to append, so a step writes only its own rows instead of
        re-concatenating the whole window (window - 1 rows per layer and step); when
        the room runs out
        the kept rows move to a fresh buffer.  Returns the visible keys and values
        (the ``previous`` cached rows, then the new ones) as views of the buffer;
        ``cache["k"]``/``cache["v"]`` stay views of the last window - 1 rows.  The
        cache has one owner: two continuations of the same cache would append into
        the same buffer."""
        B, H, T, dk = k.shape
        buf_k, buf_v, end = self._reserve(cache, previous, B, H, T, dk, k.dtype, k.device)
        buf_k[:, :, end:end + T].copy_(k)
        buf_v[:, :, end:end + T].copy_(v)
        return self._finish(cache, buf_k, buf_v, end, previous, T, offset)

    @staticmethod
    def _reserve(cache, previous, B, H, T, dk, dtype, device):
        """The cache's KV window buffers with room for T more rows after its
        ``previous`` rows, which end at the returned position (a fresh buffer, the
        kept rows copied in, when the room has run out)."""
        buf_k, buf_v, end = cache.get("kbuf"), cache.get("vbuf"), cache.get("end", 0)
        tail = cache.get("k")
        in_buffer = (buf_k is not None and tail is not None and tail.shape[2] == previous and previous <= end
                     and (previous == 0 or tail.data_ptr() == buf_k[:, :, end - previous:end].data_ptr()))
        if not in_buffer or end + T > buf_k.shape[2] or buf_k.dtype != dtype or buf_k.device != device:
            room = max(512, T)
            cap = previous + T + room
            buf_k = torch.empty((B, H, cap, dk), dtype=dtype, device=device)
            buf_v = torch.empty((B, H, cap, dk), dtype=dtype, device=device)
            if previous:
                buf_k[:, :, :previous].copy_(cache["k"])
                buf_v[:, :, :previous].copy_(cache["v"])
            end = previous
        return buf_k, buf_v, end

    def _finish(self, cache, buf_k, buf_v, end, previous, T, offset):
        """Record T rows appended at ``end``; the visible keys and values as views."""
        start, end = end - previous, end + T
        n = previous + T
        keep = n if self.window is None else min(self.window - 1, n)
        cache.update(k=buf_k[:, :, end - keep:end], v=buf_v[:, :, end - keep:end], tokens=offset + T, kbuf=buf_k,
                     vbuf=buf_v, end=end)
        return buf_k[:, :, start:end], buf_v[:, :, start:end]

    def forward(self, x, cache=None, residual=None):
        B, T, D = x.shape
        dk = self.head_dim
        q, k, v = linear_group((self.q, self.k, self.v), x)
        q, gate = q.view(B, T, self.num_heads, 2 * dk).chunk(2, -1)
        k = k.view(B, T, self.num_kv_heads, dk)
        v = v.view(B, T, self.num_kv_heads, dk).transpose(1, 2)
        previous = cache["k"].shape[2] if cache and cache.get("k") is not None else 0
        offset = 0 if cache is None else cache.get("tokens", previous)
        fused = (x.is_cuda and dk in (4, 8, 16, 32, 64, 128, 256) and x.dtype in (torch.float32, torch.bfloat16) and offset + T <= 1 << 24
                 and not (torch.is_grad_enabled() and (q.requires_grad or k.requires_grad)))
        appended = False
        if fused:
            freq = self.angular_freq.float().contiguous()
            vt = v.transpose(1, 2)                     # [B, T, kv_heads, dk]
            if (cache is not None and T <= APPEND_MAX_TOKENS and self.append_in_place and q.dtype == k.dtype == v.dtype
                    and _token_rows(q) and _token_rows(k) and _token_rows(vt)):
                # decode: q/k norm and rotary and the KV append in one launch
                buf_k, buf_v, end = self._reserve(cache, previous, B, self.num_kv_heads, T, dk, k.dtype, k.device)
                q_out = torch.empty((B, self.num_heads, T, dk), dtype=q.dtype, device=q.device)
                dst = buf_k[:, :, end:end + T]
                N.call("glsdm_decode_qkv", N.ptr(q), q.stride(2), self.num_heads, N.ptr(k), k.stride(2), N.ptr(vt),
                       vt.stride(2), self.num_kv_heads, N.dtype_code(q), B, T, dk, N.ptr(freq), offset, N.ptr(q_out),
                       N.ptr(dst), N.ptr(buf_v[:, :, end:end + T]), (ctypes.c_int64 * 3)(*dst.stride()[:3]),
                       N.stream(q.device))
                q = q_out
                k, v = self._finish(cache, buf_k, buf_v, end, previous, T, offset)
                appended = True
            else:
                q, k = qk_norm_rotary(q, freq, offset), qk_norm_rotary(k, freq, offset)
        else:
            q = self.rotary(F.rms_norm(q, (dk,)), offset).transpose(1, 2)
            k = self.rotary(F.rms_norm(k, (dk,)), offset).transpose(1, 2)
        if cache is not None and not appended:
            if (T > APPEND_MAX_TOKENS or not self.append_in_place
                    or (torch.is_grad_enabled() and (k.requires_grad or v.requires_grad))):
                # prefill chunks, functional caches and autograd: concatenation (attention
                # reads contiguous windows faster, a functional cache may be continued
                # more than once, and appending in place would modify tensors saved for
                # backward)
                for name in ("kbuf", "vbuf", "end"):
                    cache.pop(name, None)
                if cache.get("k") is not None:
                    k, v = torch.cat((cache["k"], k), 2), torch.cat((cache["v"], v), 2)
                n = k.shape[2]
                keep = n if self.window is None else min(self.window - 1, n)
                cache.update(k=k[:, :, n - keep:], v=v[:, :, n - keep:], tokens=offset + T)
            else:
                k, v = self._append(cache, k, v, previous, offset)
        groups = self.num_heads // self.num_kv_heads
        if groups != 1:
            k, v = k.repeat_interleave(groups, 1), v.repeat_interleave(groups, 1)
        # keys cover positions [offset - previous, offset + T); a cached prefill
        # needs this offset causal mask (SDPA's own causal mask is upper-left aligned)
        if (T == 1 and fused and groups == 1 and q.dtype == torch.bfloat16 and dk in (64, 128) and k.shape[2] <= 1024
                and (self.window is None or previous < self.window) and q.is_contiguous()
                and not (torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad))):
            # one token per request with every cached key inside its window (the mask is
            # all zeros): one HIP launch instead of the library's attention, the output
            # gate applied in it
            if gate.stride(-1) == 1 and gate.dtype == q.dtype:
                return linear(self.proj, decode_attention(q, k, v, gate), residual)
            out = decode_attention(q, k, v)
        else:
            mask = None
            if offset or self.window is not None:
                mask = _window_mask(previous, T, self.window, x.device, q.dtype)
            out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=mask is None)
        if fused and out.stride(-1) == 1 and gate.stride(-1) == 1 and not (
                torch.is_grad_enabled() and (out.requires_grad or gate.requires_grad)):
            return linear(self.proj, gate_merge(out, gate), residual)
        return linear(self.proj, out.transpose(1, 2).reshape(B, T, D) * gate.reshape(B, T, D).sigmoid(), residual)
