"""The fused QK normalisation + rotary kernel vs the local attention's tensor
ops (S/layers/attention.py:38-42,51-52: F.rms_norm, then the rotary in fp32),
run by PyTorch on the same device.

Tolerances: fp32 within a few ulp (the mean's summation order and rsqrt may
differ from PyTorch's kernels).  bf16: a last-bit difference of the fp32
scale can round a normalised value (|y| < 8 here) the other way, which moves
the outputs built from it by up to one bf16 ulp of y (2^-5) -- rare, so the
fraction of differing outputs is bounded as well."""
import pytest
import torch
import torch.nn.functional as F

from glsdm.layers.attention import Transformer, qk_norm_rotary

pytestmark = pytest.mark.gpu


def _reference(x, freq, offset):
    layer = Transformer.__new__(Transformer)
    torch.nn.Module.__init__(layer)
    layer.angular_freq = freq
    return layer.rotary(F.rms_norm(x, (x.shape[-1],)), offset).transpose(1, 2)


def _freq(dk, device):
    rising = torch.pow(torch.tensor(1 / 1024), torch.linspace(0, 1, dk // 4))
    return torch.cat((rising, torch.zeros_like(rising))).to(device)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,heads,dk,offset,strided", [
    (2, 37, 16, 64, 0, True), (1, 5, 4, 16, 3, False), (3, 64, 8, 128, 511, True), (1, 9, 2, 256, 100000, False),
    (4, 512, 16, 64, 7680, True), (1, 1, 1, 4, 0, False), (64, 1, 16, 64, 4095, True),
])
def test_qk_norm_rotary_matches_tensor_ops(device, dtype, B, T, heads, dk, offset, strided):
    g = torch.Generator().manual_seed(B * 1000 + T + dk)
    if strided:   # the query half of a [query | gate] projection, as the layer sees it
        x = (torch.randn(B, T, heads, 2 * dk, generator=g) * 3).to(dtype).to(device).chunk(2, -1)[0]
    else:
        x = (torch.randn(B, T, heads, dk, generator=g) * 3).to(dtype).to(device)
    freq = _freq(dk, device)
    out = qk_norm_rotary(x, freq, offset)
    ref = _reference(x, freq, offset)
    assert out.shape == ref.shape and out.dtype == dtype and out.is_contiguous()
    if dtype == torch.float32:
        torch.testing.assert_close(out, ref, atol=1e-6, rtol=1e-5)
    else:
        torch.testing.assert_close(out.float(), ref.float(), atol=2 ** -5, rtol=2 ** -7)
        assert (out != ref).float().mean().item() < 1e-4


def test_qk_norm_rotary_rejects_bad_shapes(device):
    from glsdm import _native as N
    x = torch.zeros(1, 2, 1, 6, device=device)
    with pytest.raises(ValueError):
        qk_norm_rotary(x, _freq(8, device)[:3], 0)            # dk not a multiple of 4
    with pytest.raises((ValueError, RuntimeError)):
        N.call("glsdm_qk_norm_rotary", N.ptr(x), 0, 1, 2, 1, 512, 512, N.ptr(x), 0, N.ptr(x), N.stream(device))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,T,dk", [(2, 16, 37, 64), (1, 4, 5, 16), (4, 16, 512, 64), (64, 16, 1, 64),
                                      (3, 2, 9, 12)])
def test_gate_merge_matches_tensor_ops(device, dtype, B, H, T, dk):
    """The attention output's gate (S/layers/attention.py:77) bit for bit: the
    same fp32 sigmoid rounded to the dtype, then one rounded product."""
    from glsdm.layers.attention import gate_merge
    g = torch.Generator().manual_seed(B * 100 + T)
    o = (torch.randn(B, T, H, dk, generator=g)).to(dtype).to(device).transpose(1, 2)   # strided, as SDPA may give
    proj = (torch.randn(B, T, H, 2 * dk, generator=g) * 4).to(dtype).to(device)
    gate = proj.chunk(2, -1)[1]
    out = gate_merge(o, gate)
    ref = o.transpose(1, 2).reshape(B, T, H * dk) * gate.reshape(B, T, H * dk).sigmoid()
    assert out.shape == ref.shape and out.dtype == dtype
    torch.testing.assert_close(out, ref, atol=0, rtol=0)
    out2 = gate_merge(o.contiguous(), gate)
    torch.testing.assert_close(out2, ref, atol=0, rtol=0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,inner", [(2048, 4096), (37, 64), (1, 8), (300, 128)])
def test_relu2_gate_matches_tensor_ops(device, dtype, rows, inner):
    """The MLP activation (S/layers/common.py:26-27) bit for bit, NaN and
    signed zeros included."""
    from glsdm.layers.common import relu2_gate
    g = torch.Generator().manual_seed(rows + inner)
    h = (torch.randn(rows, 2 * inner, generator=g) * 2).to(dtype)
    h[0, :4] = torch.tensor([float("nan"), -0.0, 0.0, -3.0]).to(dtype)
    h = h.to(device)
    out = relu2_gate(h)
    u, gate = h.chunk(2, -1)
    ref = gate * u.relu().square()
    torch.testing.assert_close(out, ref, atol=0, rtol=0, equal_nan=True)


@pytest.mark.parametrize("x_dtype,out_dtype", [(torch.float32, torch.bfloat16), (torch.float32, torch.float32),
                                               (torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("w_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,dim", [(2048, 1024), (37, 32), (5, 4096), (64, 100)])
def test_rms_norm_cast_matches_tensor_ops(device, x_dtype, out_dtype, w_dtype, rows, dim):
    """RMSNorm (learned weight, eps 1e-6) then a cast, against the module's
    tensor ops: the mean's summation order differs, so a rare value may round
    the other way once (one ulp of the rounding dtype)."""
    from glsdm.layers.common import RMSNorm
    g = torch.Generator().manual_seed(rows + dim)
    norm = RMSNorm(dim)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(dim, generator=g) + 0.5)
    norm = norm.to(device)
    norm.weight.data = norm.weight.data.to(w_dtype)          # a bf16 model's norm weight
    x = (torch.randn(rows, dim, generator=g) * 3).to(x_dtype).to(device)
    with torch.no_grad():
        out = norm.cast(x, out_dtype)
        ref = norm(x).to(out_dtype)
    assert out.dtype == out_dtype
    coarse = torch.bfloat16 in (x_dtype, out_dtype)
    torch.testing.assert_close(out.float(), ref.float(), atol=1e-6, rtol=2 ** -6 if coarse else 1e-5)
    assert (out != ref).float().mean().item() < (2e-3 if coarse else 1.0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_write_gates_match_tensor_ops(device, dtype):
    """The proposal's write gates (S/layers/global_layer.py:48-49): sigmoid of the
    beta projection and -softplus(decay - 4), over the softplus threshold and
    the sigmoid's saturation too, within a few fp32 ulp of the tensor ops."""
    from glsdm.layers.global_layer import write_gates
    g = torch.Generator().manual_seed(3)
    b = (torch.randn(4, 512, 16, generator=g) * 6).to(dtype)
    d = (torch.randn(4, 512, 16, generator=g) * 12).to(dtype)
    b[0, 0, :4] = torch.tensor([-100.0, 100.0, 0.0, -0.0]).to(dtype)
    d[0, 0, :4] = torch.tensor([24.0, 23.9, 25.0, -80.0]).to(dtype)
    b, d = b.to(device), d.to(device)
    beta, log_decay = write_gates(b, d)
    ref_beta = b.float().sigmoid().unsqueeze(-1)
    ref_ld = -torch.nn.functional.softplus(d.float() - 4).unsqueeze(-1)
    assert beta.shape == ref_beta.shape == log_decay.shape
    torch.testing.assert_close(beta, ref_beta, atol=1e-7, rtol=4e-7)
    torch.testing.assert_close(log_decay, ref_ld, atol=1e-7, rtol=4e-7)


@pytest.mark.parametrize("M,N,K,bias", [
    (64, 3072, 1024, True),        # the config-5 decode projections: 64 streams x one token
    (64, 16, 1024, True),          # a write-gate projection (one column tile)
    (17, 1024, 4096, True),        # ragged rows, a long reduction (the MLP's down projection)
    (1, 32000, 1024, False),       # one row through the vocabulary head (no bias; four column tiles per block)
    (64, 16384, 1024, True),       # a router score projection's width: four column tiles per block
    (40, 48, 128, True),           # the smallest reduction
])
def test_linear_small_matches_float64_and_torch(device, M, N, K, bias):
    """glsdm_linear_small: fp32 accumulation rounded once to bf16, so within a bf16
    rounding of the float64 result and of torch's bf16 linear (the fp32 summation
    orders differ); a dropped bias, a transposed weight or a lost reduction quarter
    would be far outside that."""
    from glsdm import _native as NT
    g = torch.Generator().manual_seed(M * 7 + N + K)
    lin = torch.nn.Linear(K, N, bias=bias).to(device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_((torch.randn(N, K, generator=g) / K ** 0.5).to(device))
        if bias:
            lin.bias.copy_((torch.randn(N, generator=g) * 0.5).to(device))
    x = torch.randn(M, K, generator=g).to(device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        out = torch.empty(M, N, dtype=torch.bfloat16, device=device)
        NT.call("glsdm_linear_small", NT.ptr(x), NT.ptr(lin.weight), NT.ptr(lin.bias), NT.ptr(out), M, N, K,
                NT.stream(device))
        ref_torch = torch.nn.functional.linear(x, lin.weight, lin.bias)
    ref = x.double().cpu() @ lin.weight.double().cpu().T
    if bias:
        ref = ref + lin.bias.double().cpu()
    assert out.dtype == torch.bfloat16 and out.shape == (M, N)
    scale = ref.abs().max().item()
    torch.testing.assert_close(out.double().cpu(), ref, rtol=8e-3, atol=1e-3 * scale)
    torch.testing.assert_close(out.float(), ref_torch.float(), rtol=8e-3, atol=1e-3 * scale)
    # most elements round to the same bf16 as torch's
    assert (out == ref_torch).float().mean().item() > 0.9


def test_linear_routes_decode_projections(device):
    """The stack's ``linear``: decode-sized projections run the kernel (its bits, not
    necessarily torch's); more rows, other widths and autograd go through torch's
    linear unchanged."""
    from glsdm import _native as NT
    from glsdm.layers.common import linear
    g = torch.Generator().manual_seed(5)
    lin = torch.nn.Linear(1024, 3072).to(device=device, dtype=torch.bfloat16)
    x = torch.randn(64, 1024, generator=g).to(device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        direct = torch.empty(64, 3072, dtype=torch.bfloat16, device=device)
        NT.call("glsdm_linear_small", NT.ptr(x), NT.ptr(lin.weight), NT.ptr(lin.bias), NT.ptr(direct), 64, 3072,
                1024, NT.stream(device))
        assert torch.equal(linear(lin, x), direct)
        for shape, n_out, k_in in (((65, 1024), 3072, 1024), ((64, 96), 32, 96), ((64, 1024), 40, 1024)):
            other = torch.nn.Linear(k_in, n_out).to(device=device, dtype=torch.bfloat16)
            y = torch.randn(*shape, generator=g).to(device=device, dtype=torch.bfloat16)
            assert torch.equal(linear(other, y), other(y))
    with torch.enable_grad():
        assert torch.equal(linear(lin, x), lin(x))


@pytest.mark.parametrize("M,N,K", [
    (64, 1024, 1024),              # a local layer's output projection (config 5 decode)
    (64, 1024, 4096),              # the MLP's down projection (sixteen waves over K)
    (5, 16384, 256),               # wide: four column tiles per block
])
def test_linear_small_residual_equals_torch_add(device, M, N, K):
    """glsdm_linear_small_residual: bit-identical to torch's fp32 residual + the
    kernel's bf16 projection, out of place and in place (out = residual)."""
    from glsdm import _native as NT
    from glsdm.layers.common import linear
    g = torch.Generator().manual_seed(M + N + K)
    lin = torch.nn.Linear(K, N).to(device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_((torch.randn(N, K, generator=g) / K ** 0.5).to(device))
        lin.bias.copy_((torch.randn(N, generator=g) * 0.5).to(device))
    x = torch.randn(M, K, generator=g).to(device=device, dtype=torch.bfloat16)
    res = (torch.randn(M, N, generator=g) * 3).to(device)
    with torch.no_grad():
        proj = linear(lin, x)
        want = res + proj
        got = linear(lin, x, res)
        assert got.dtype == torch.float32 and torch.equal(got, want)
        inplace = res.clone()
        NT.call("glsdm_linear_small_residual", NT.ptr(x), NT.ptr(lin.weight), NT.ptr(lin.bias), NT.ptr(inplace),
                NT.ptr(inplace), M, N, K, NT.stream(device))
        assert torch.equal(inplace, want)
        # a bf16 residual (or any other form) takes torch's add of the same projection
        res16 = res.to(torch.bfloat16)
        assert torch.equal(linear(lin, x, res16), res16 + proj)
    # the planted slip of adding the fp32 sum before its bf16 rounding differs from torch's bits
    assert not torch.equal(want, res + (x.float() @ lin.weight.float().T + lin.bias.float()))


@pytest.mark.parametrize("B,H,L,dk", [(64, 16, 512, 64), (2, 4, 77, 128), (3, 2, 1, 64)])
def test_decode_attention_gated_equals_attention_then_gate_merge(device, B, H, L, dk):
    """glsdm_decode_attention_gated: bit-identical to glsdm_decode_attention then
    glsdm_gate_merge, with the gate read from the [query | gate] projection layout."""
    from glsdm.layers.attention import decode_attention, gate_merge
    g = torch.Generator().manual_seed(B + H + L + dk)
    q = torch.randn(B, H, 1, dk, generator=g).to(device=device, dtype=torch.bfloat16)
    k = torch.randn(B, H, L, dk, generator=g).to(device=device, dtype=torch.bfloat16)
    v = torch.randn(B, H, L, dk, generator=g).to(device=device, dtype=torch.bfloat16)
    qg = (torch.randn(B, 1, H, 2 * dk, generator=g) * 3).to(device=device, dtype=torch.bfloat16)
    gate = qg[..., dk:]
    with torch.no_grad():
        want = gate_merge(decode_attention(q, k, v), gate)
        got = decode_attention(q, k, v, gate)
    assert got.shape == (B, 1, H * dk) and torch.equal(got, want)


@pytest.mark.parametrize("B,T,Hq,Hkv,dk,dtype", [
    (64, 1, 16, 16, 64, torch.bfloat16),     # config 5: one token per stream
    (3, 5, 4, 2, 128, torch.bfloat16),      # several tokens, grouped KV heads
    (2, 2, 8, 8, 32, torch.float32),
])
def test_decode_qkv_equals_norm_rotary_and_copies(device, B, T, Hq, Hkv, dk, dtype):
    """glsdm_decode_qkv: q_out and the new buffer rows bit-identical to
    glsdm_qk_norm_rotary of q and k and a copy of v; the buffer rows around the
    new positions untouched."""
    import ctypes
    from glsdm import _native as NT
    from glsdm.layers.attention import qk_norm_rotary
    g = torch.Generator().manual_seed(B * 100 + T + dk)
    qg = torch.randn(B, T, Hq, 2 * dk, generator=g).to(device=device, dtype=dtype)
    q = qg[..., :dk]                                              # the query half of [query | gate]
    k = torch.randn(B, T, Hkv, dk, generator=g).to(device=device, dtype=dtype)
    v = torch.randn(B, T, Hkv, dk, generator=g).to(device=device, dtype=dtype)
    rising = torch.pow(torch.tensor(1 / 1024), torch.linspace(0, 1, dk // 4))
    freq = torch.cat((rising, torch.zeros_like(rising))).to(device)
    offset, end, cap = 700, 9, 9 + T + 6
    buf_k = torch.randn(B, Hkv, cap, dk, generator=g).to(device=device, dtype=dtype)
    buf_v = torch.randn(B, Hkv, cap, dk, generator=g).to(device=device, dtype=dtype)
    want_k, want_v = buf_k.clone(), buf_v.clone()
    with torch.no_grad():
        want_q = qk_norm_rotary(q, freq, offset)
        want_k[:, :, end:end + T] = qk_norm_rotary(k, freq, offset)
        want_v[:, :, end:end + T] = v.transpose(1, 2)
        q_out = torch.empty(B, Hq, T, dk, dtype=dtype, device=device)
        dst = buf_k[:, :, end:end + T]
        NT.call("glsdm_decode_qkv", NT.ptr(q), q.stride(2), Hq, NT.ptr(k), k.stride(2), NT.ptr(v), v.stride(2), Hkv,
                NT.dtype_code(q), B, T, dk, NT.ptr(freq), offset, NT.ptr(q_out), NT.ptr(dst),
                NT.ptr(buf_v[:, :, end:end + T]), (ctypes.c_int64 * 3)(*dst.stride()[:3]), NT.stream(device))
    assert torch.equal(q_out, want_q)
    assert torch.equal(buf_k, want_k)
    assert torch.equal(buf_v, want_v)


@pytest.mark.parametrize("M,N,K,with_residual", [
    (64, 1024, 4096, True),        # config 5: the MLP's down projection with the block's residual
    (64, 1024, 4096, False),
    (17, 1024, 256, True),         # ragged rows, four waves over K
    (3, 16384, 128, False),        # wide: four column tiles per block
])
def test_linear_small_relu2_equals_activation_then_projection(device, M, N, K, with_residual):
    """glsdm_linear_small_relu2: bit-identical to glsdm_relu2_gate followed by
    glsdm_linear_small (or its residual form), with negative, zero and positive
    pre-activations; and the MLP routes a decode step through it."""
    from glsdm import _native as NT
    from glsdm.layers.common import MLP, linear, relu2_gate
    g = torch.Generator().manual_seed(M + N + K + with_residual)
    lin = torch.nn.Linear(K, N).to(device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_((torch.randn(N, K, generator=g) / K ** 0.5).to(device))
        lin.bias.copy_((torch.randn(N, generator=g) * 0.5).to(device))
    h = torch.randn(M, 2 * K, generator=g)
    h[:, :K:7] = 0.0
    h = h.to(device=device, dtype=torch.bfloat16)
    res = (torch.randn(M, N, generator=g) * 3).to(device) if with_residual else None
    with torch.no_grad():
        want = linear(lin, relu2_gate(h), res)
        got = torch.empty(M, N, dtype=want.dtype, device=device)
        NT.call("glsdm_linear_small_relu2", NT.ptr(h), NT.ptr(lin.weight), NT.ptr(lin.bias), NT.ptr(res),
                NT.ptr(got), M, N, K, NT.stream(device))
    assert got.dtype == (torch.float32 if with_residual else torch.bfloat16)
    assert torch.equal(got, want)
    # the activation's intermediate rounding matters: without it the bits differ
    with torch.no_grad():
        u, gate = h.float().chunk(2, -1)
        loose = linear(lin, (gate * u.relu().square()).to(torch.bfloat16), res)
    assert not torch.equal(loose, want)
    if N == 1024 and K == 4096:
        mlp = MLP(N, K).to(device=device, dtype=torch.bfloat16)
        x = torch.randn(M, N, generator=g).to(device=device, dtype=torch.bfloat16)
        with torch.no_grad():
            fc = linear(mlp.fc, x)
            expect = linear(mlp.proj, relu2_gate(fc), res)
            assert torch.equal(mlp(x, residual=res), expect)


@pytest.mark.parametrize("M,widths,K,biases", [
    (64, (2048, 1024, 1024), 1024, (True, True, True)),     # a local layer's q, k, v (config 5 decode)
    (64, (1024, 16, 16), 1024, (True, True, True)),         # a global layer's v, beta, decay
    (17, (48, 1024, 32), 4096, (True, False, True)),        # ragged rows, a long reduction, one bias missing
    (3, (16384, 32768), 256, (False, False)),               # wide projections: four column tiles per block
    (1, tuple(16 * (i + 1) for i in range(8)), 128, (True,) * 8),   # the most projections per launch
])
def test_linear_small_group_equals_separate_calls(device, M, widths, K, biases):
    """glsdm_linear_small_group: each projection's output bit-identical to its own
    glsdm_linear_small call (the same summation order), and within a bf16 rounding
    of the float64 product (a projection reading its neighbour's weights or bias
    would not be)."""
    from glsdm import _native as NT
    from glsdm.layers.common import linear_group
    g = torch.Generator().manual_seed(M + K + len(widths))
    layers = []
    for n, b in zip(widths, biases):
        lin = torch.nn.Linear(K, n, bias=b).to(device=device, dtype=torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_((torch.randn(n, K, generator=g) / K ** 0.5).to(device))
            if b:
                lin.bias.copy_((torch.randn(n, generator=g) * 0.5).to(device))
        layers.append(lin)
    x = torch.randn(M, K, generator=g).to(device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        outs = linear_group(layers, x)
        for lin, out in zip(layers, outs):
            alone = torch.empty(M, lin.out_features, dtype=torch.bfloat16, device=device)
            NT.call("glsdm_linear_small", NT.ptr(x), NT.ptr(lin.weight), NT.ptr(lin.bias), NT.ptr(alone), M,
                    lin.out_features, K, NT.stream(device))
            assert out.shape == (M, lin.out_features) and out.is_contiguous()
            assert torch.equal(out, alone)
            ref = x.double().cpu() @ lin.weight.double().cpu().T
            if lin.bias is not None:
                ref = ref + lin.bias.double().cpu()
            torch.testing.assert_close(out.double().cpu(), ref, rtol=8e-3, atol=1e-3 * ref.abs().max().item())
    # a second call reuses the group's kept pointer arrays; a weight given new storage
    # (new values) is seen
    with torch.no_grad():
        layers[-1].weight.data = layers[-1].weight.data * 2
        again = linear_group(layers, x)
        for lin, out, before in zip(layers, again, outs):
            alone = torch.empty(M, lin.out_features, dtype=torch.bfloat16, device=device)
            NT.call("glsdm_linear_small", NT.ptr(x), NT.ptr(lin.weight), NT.ptr(lin.bias), NT.ptr(alone), M,
                    lin.out_features, K, NT.stream(device))
            assert torch.equal(out, alone)
        assert torch.equal(again[0], outs[0]) and not torch.equal(again[-1], outs[-1])
    # the host-side memos stay off the modules: a used group still copies and pickles,
    # and the copy (its own storages) computes the same
    import copy
    import pickle
    clone = copy.deepcopy(layers)
    pickle.dumps(layers)
    with torch.no_grad():
        assert all(torch.equal(a, b) for a, b in zip(linear_group(clone, x), linear_group(layers, x)))
    # an ineligible member (a width not a multiple of 16) sends every projection to torch
    odd = torch.nn.Linear(K, 24).to(device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        got = linear_group([layers[0], odd], x)
    assert torch.equal(got[1], odd(x).detach())


@pytest.mark.parametrize("B,H,L,dk", [
    (64, 16, 512, 64),             # config 5: a full window of 511 cached keys and the new one
    (3, 2, 1, 64),                 # the first decode step after an empty cache: one key
    (2, 4, 77, 128),               # a ragged key count, wider heads
    (1, 1, 1024, 64),              # the kernel's largest key count
])
def test_decode_attention_matches_sdpa(device, B, H, L, dk):
    """glsdm_decode_attention on strided views of a KV buffer (as the cache holds
    them) against PyTorch's SDPA of the same bf16 operands computed in fp32: within
    bf16 rounding of the output; and against SDPA itself on bf16."""
    from glsdm.layers.attention import decode_attention
    g = torch.Generator().manual_seed(B * 1000 + L + dk)
    q = torch.randn(B, H, 1, dk, generator=g).to(device=device, dtype=torch.bfloat16)
    buf_k = torch.randn(B, H, L + 40, dk, generator=g).to(device=device, dtype=torch.bfloat16)
    buf_v = torch.randn(B, H, L + 40, dk, generator=g).to(device=device, dtype=torch.bfloat16)
    k, v = buf_k[:, :, 7:7 + L], buf_v[:, :, 7:7 + L]      # views inside a larger buffer
    with torch.no_grad():
        out = decode_attention(q, k, v)
        ref32 = F.scaled_dot_product_attention(q.float(), k.float(), v.float())
        ref16 = F.scaled_dot_product_attention(q, k.contiguous(), v.contiguous())
    assert out.shape == q.shape and out.dtype == torch.bfloat16
    torch.testing.assert_close(out.float(), ref32, rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(out.float(), ref16.float(), rtol=2e-2, atol=2e-2)
    # a planted slip -- the value rows read one key late -- is far outside that
    with torch.no_grad():
        slip = decode_attention(q, buf_k[:, :, 7:7 + L], buf_v[:, :, 8:8 + L])
    if L > 1:
        assert (slip.float() - ref32).abs().max() > 5e-2
