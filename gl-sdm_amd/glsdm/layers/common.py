"""RMSNorm and the gated squared-ReLU MLP of S/layers/common.py:7-27
(S/ = projects/gl-sdm/src/gl_sdm/).  On the GPU outside autograd the MLP's
activation ``gate * relu(u)^2`` is one HIP launch (``glsdm_relu2_gate``, the
same roundings as the tensor ops), and the stack's projections of decode-sized
inputs run ``glsdm_linear_small`` (``linear``)."""
import weakref

import torch
from torch import nn
import torch.nn.functional as F

from .. import _native as N

# per-module host-side memos of the decode projections (kept off the modules, so
# copying or pickling a model never meets the ctypes arrays)
_SMALL = weakref.WeakKeyDictionary()
_GROUP = weakref.WeakKeyDictionary()


def linear(layer, x, residual=None):
    """``layer(x)`` for an ``nn.Linear`` (``residual + layer(x)`` with a residual).
    Outside autograd, a bf16 input of at most 64 rows on the device with a bf16
    weight (out features a multiple of 16, in features of 128) runs
    ``glsdm_linear_small``: fp32 accumulation rounded once, as torch's bf16 linear,
    in the kernel's own summation order (results agree to the rounding of the fp32
    sum); an fp32 residual of the output's shape is added in the same launch
    (``glsdm_linear_small_residual``, the bits of torch's add).  A decode step makes
    over a hundred of these calls; the library GEMM's host cost per call (~20 us) is
    what bounds that step."""
    # every eligible shape: alone, the router's 2^15-column score projection takes 41 us here
    # against the library's ~20 us per call, but within a decode step the library's host
    # time costs more (config 5 p50 4.02 ms when such projections go to the library, 3.77 ms)
    if not _small(layer, x):
        return layer(x) if residual is None else residual + layer(x)
    K = x.shape[-1]
    w = layer.weight
    shape = (*x.shape[:-1], w.shape[0])
    if (residual is not None and residual.dtype == torch.float32 and residual.is_contiguous()
            and residual.device == x.device and tuple(residual.shape) == shape):
        out = torch.empty(shape, dtype=torch.float32, device=x.device)
        N.call("glsdm_linear_small_residual", N.ptr(x), N.ptr(w), N.ptr(layer.bias), N.ptr(residual), N.ptr(out),
               x.numel() // K, w.shape[0], K, N.stream(x.device))
        return out
    out = torch.empty(shape, dtype=torch.bfloat16, device=x.device)
    N.call("glsdm_linear_small", N.ptr(x), N.ptr(w), N.ptr(layer.bias), N.ptr(out), x.numel() // K, w.shape[0],
           K, N.stream(x.device))
    return out if residual is None else residual + out


def _small(layer, x):
    """Whether ``glsdm_linear_small`` takes ``layer(x)``: the input checks run per
    call, the weight's (dtype, width, layout, bias dtype) are kept per module with
    the storage, dtype and device they were made for (a decode step asks this over
    a hundred times)."""
    if torch.is_grad_enabled() or x.dtype != torch.bfloat16 or not x.is_cuda:
        return False
    K = x.shape[-1]
    if K % 128 or x.numel() > 64 * K or not x.is_contiguous() or x.data_ptr() % 16:
        return False
    params = layer._parameters
    w, b = params["weight"], params.get("bias")
    key = (w.data_ptr(), w.dtype, w.device, None if b is None else (b.data_ptr(), b.dtype))
    memo = _SMALL.get(layer)
    if memo is None or memo[0] != key:
        ok = (w.dtype == torch.bfloat16 and w.dim() == 2 and w.shape[0] % 16 == 0 and w.is_contiguous()
              and (b is None or b.dtype == torch.bfloat16))
        memo = (key, ok)
        _SMALL[layer] = memo
    return memo[1] and w.shape[1] == K and w.device == x.device


def linear_group(layers, x):
    """``[linear(l, x) for l in layers]``; when every projection is eligible for
    ``glsdm_linear_small``, one launch of ``glsdm_linear_small_group`` computes them
    all (bit-identical to the separate calls: the outputs are contiguous pieces of
    one buffer)."""
    if not 1 < len(layers) <= 8 or not all(_small(l, x) for l in layers):
        return [linear(l, x) for l in layers]
    K, M = x.shape[-1], x.numel() // x.shape[-1]
    # the weight and bias pointer arrays and the widths are kept per first module
    # with the modules and storages they were made for
    key = tuple((id(l), l._parameters["weight"].data_ptr(),
                 0 if l._parameters.get("bias") is None else l._parameters["bias"].data_ptr()) for l in layers)
    memo = _GROUP.get(layers[0])
    count = len(layers)
    P = N.ctypes.c_void_p
    if memo is None or memo[0] != key:
        widths = [l._parameters["weight"].shape[0] for l in layers]
        memo = (key, widths, sum(widths), (P * count)(*(k[1] for k in key)), (P * count)(*(k[2] for k in key)),
                (N.ctypes.c_int64 * count)(*widths))
        _GROUP[layers[0]] = memo
    _, widths, total, weights, biases, width_arr = memo
    flat = torch.empty(M * total, dtype=torch.bfloat16, device=x.device)
    base, lead = flat.data_ptr(), x.shape[:-1]
    outs, ptrs, at = [], [], 0
    for n in widths:
        outs.append(flat[at:at + M * n].view(*lead, n))
        ptrs.append(base + 2 * at)
        at += M * n
    N.call("glsdm_linear_small_group", N.ptr(x), count, weights, biases, (P * count)(*ptrs), width_arr, M, K,
           N.stream(x.device))
    return outs


def relu2_gate(h):
    """``gate * u.relu().square()`` for ``u, gate = h.chunk(2, -1)``, ``h [..., 2*inner]`` contiguous."""
    inner = h.shape[-1] // 2
    out = torch.empty((*h.shape[:-1], inner), dtype=h.dtype, device=h.device)
    N.call("glsdm_relu2_gate", N.ptr(h), N.dtype_code(h), h.numel() // h.shape[-1], inner, N.ptr(out),
           N.stream(h.device))
    return out


class RMSNorm(nn.Module):
    """``rms_norm`` over the last dimension, eps 1e-6, weight cast to the input dtype."""

    def __init__(self, dim):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        return F.rms_norm(x, (x.shape[-1],), self.weight.to(x.dtype), eps=1e-6)

    def cast(self, x, dtype):
        """``self(x).to(dtype)``; on the GPU outside autograd one HIP launch
        (``glsdm_rms_norm_cast``) instead of the norm and the cast."""
        w = self._parameters["weight"]
        codes = N.DTYPES
        xc, oc, wc = codes.get(x.dtype), codes.get(dtype), codes.get(w.dtype)
        if (x.is_cuda and xc is not None and oc is not None and wc is not None and w.is_contiguous()
                and not (torch.is_grad_enabled() and (x.requires_grad or w.requires_grad))):
            if not x.is_contiguous():
                x = x.contiguous()
            out = torch.empty(x.shape, dtype=dtype, device=x.device)
            dim = x.shape[-1]
            N.call("glsdm_rms_norm_cast", x.data_ptr(), xc, w.data_ptr(), wc, x.numel() // dim, dim, 1e-6,
                   out.data_ptr(), oc, N.stream(x.device))
            return out
        return self(x).to(dtype)


class MLP(nn.Module):
    """``proj(gate * relu(u)^2)`` with ``u, gate = fc(x).chunk(2)``; inner width 4*dim by default."""

    def __init__(self, dim, intermediate_size=None):
        super().__init__()
        inner = 4 * dim if intermediate_size is None else intermediate_size
        if inner < 1:
            raise ValueError("intermediate_size must be positive")
        self.fc = nn.Linear(dim, 2 * inner)
        self.proj = nn.Linear(inner, dim)

    def forward(self, x, residual=None):
        """The MLP's output, or ``residual`` plus it.  For a decode step the
        activation and the residual add run inside the down projection's launch
        (``glsdm_linear_small_relu2``)."""
        h = linear(self.fc, x)
        inner = h.shape[-1] // 2
        w = self.proj.weight
        shape = (*h.shape[:-1], w.shape[0])
        if (_small(self.fc, x) and h.dtype == torch.bfloat16 and h.is_contiguous() and inner % 128 == 0
                and h.data_ptr() % 16 == 0 and w.dtype == torch.bfloat16 and w.is_contiguous()
                and w.shape[0] % 16 == 0 and w.shape[1] == inner and w.device == h.device
                and (self.proj.bias is None or self.proj.bias.dtype == torch.bfloat16)
                and (residual is None or (residual.dtype == torch.float32 and residual.is_contiguous()
                                          and residual.device == h.device and tuple(residual.shape) == shape))):
            out = torch.empty(shape, dtype=torch.bfloat16 if residual is None else torch.float32, device=h.device)
            N.call("glsdm_linear_small_relu2", N.ptr(h), N.ptr(w), N.ptr(self.proj.bias), N.ptr(residual),
                   N.ptr(out), h.numel() // h.shape[-1], w.shape[0], inner, N.stream(h.device))
            return out
        if (h.is_cuda and h.dtype in (torch.float32, torch.bfloat16) and h.is_contiguous()
                and inner % (16 // h.element_size()) == 0 and h.data_ptr() % 16 == 0
                and not (torch.is_grad_enabled() and h.requires_grad)):
            return linear(self.proj, relu2_gate(h), residual)
        u, gate = h.chunk(2, -1)
        return linear(self.proj, gate * u.relu().square(), residual)
