"""Host-side checks of the layer stack (no GPU): construction, parameter
layout, validation and the local attention, which is plain PyTorch.

Mirrors P/tests/test_layer_stack.py:14-32,88-90,102-116 (P/ = projects/gl-sdm/).
"""
import pytest
import torch

from glsdm.model import create_model
from glsdm.layers.attention import Transformer
from glsdm.layers.global_layer import GlobalLayer
from glsdm.memory import MemoryBank


def config(**changes):
    base = dict(arch_type="gl_sdm", vocab_size=64, hidden_size=32, head_dim=16, num_hidden_layers=16,
                dtype="float32", gl_layer_pattern=["local", "local", "global", "local"], gl_slots=16, gl_reads=2,
                gl_writes=2, gl_chunk_size=4, gl_local_window=6, gl_memory_backend="hip", seq_len=9)
    return {**base, **changes}


def test_distinct_layers_share_exactly_one_bank():
    model = create_model(config())
    assert len(model.blocks) == 16
    assert [i for i, b in enumerate(model.blocks) if isinstance(b, GlobalLayer)] == [2, 6, 10, 14]
    assert len([b for b in model.modules() if isinstance(b, MemoryBank)]) == 1
    assert len({id(b.mlp.fc.weight) for b in model.blocks}) == 16
    assert model.bank.memory.shape == (2, 16, 16)


def test_parameter_names_follow_the_reference_checkpoint_layout():
    names = dict(create_model(config()).named_parameters())
    for name, shape in [("embed.weight", (64, 32)), ("blocks.0.attn.q.weight", (64, 32)),
                        ("blocks.0.attn.k.weight", (32, 32)), ("blocks.2.attn.q.weight", (2 * 2 * 4, 32)),
                        ("blocks.2.attn.k.bias", (16,)), ("blocks.2.attn.beta.weight", (2, 32)),
                        ("blocks.2.attn.decay.weight", (2, 32)), ("blocks.2.attn.read_norm.weight", (16,)),
                        ("blocks.2.mlp.fc.weight", (256, 32)), ("bank.memory", (2, 16, 16)),
                        ("norm.weight", (32,)), ("proj.weight", (64, 32))]:
        assert names[name].shape == shape, name


def test_casts_keep_the_bank_and_rotary_frequencies_fp32():
    model = create_model(config(dtype="bfloat16"))
    assert model.blocks[2].attn.q.weight.dtype == torch.bfloat16
    assert model.bank.memory.dtype == torch.float32
    assert model.blocks[0].attn.angular_freq.dtype == torch.float32
    assert create_model(config(gl_state_dtype="bfloat16")).bank.state_dtype == torch.bfloat16


@pytest.mark.parametrize("changes,match", [
    (dict(gl_max_steps=4), "no reasoning loops"),
    (dict(gl_layer_pattern=["local"]), "gl_layer_pattern"),
    (dict(num_hidden_layers=6), "gl_layer_pattern"),
    (dict(gl_memory_backend="urm"), "hip"),
    (dict(gl_slots=15), "square slots"),
    (dict(reg_mode="weak"), "baseline"),
    (dict(arch_type="transformer"), "layer stack"),
])
def test_invalid_configs(changes, match):
    with pytest.raises(ValueError, match=match):
        create_model(config(**changes))


def test_no_cpu_fallback():
    model = create_model(config()).eval()
    with pytest.raises(ValueError, match="CUDA"):
        model.prefill(torch.randint(64, (1, 9)))
    with pytest.raises(RuntimeError, match="eval"):
        create_model(config()).prefill(torch.randint(64, (1, 9)))


def test_sliding_window_excludes_old_tokens_and_uses_absolute_rotary_positions():
    torch.manual_seed(3)
    layer = Transformer({**config(), "attention_window": 4}, 0).eval()
    x = torch.randn(1, 13, 32)
    with torch.no_grad():
        full = layer(x)
        changed = x.clone()
        changed[:, 0] += 5
        torch.testing.assert_close(layer(changed)[:, 4:], full[:, 4:], atol=0, rtol=0)
        assert not torch.equal(layer(changed)[:, :4], full[:, :4])
        cache = {}
        parts = [layer(x[:, :6], cache), layer(x[:, 6:11], cache), layer(x[:, 11:12], cache), layer(x[:, 12:], cache)]
    torch.testing.assert_close(torch.cat(parts, 1), full, atol=2e-7, rtol=2e-5)
    assert cache["tokens"] == 13 and cache["k"].shape[2] == 3


def test_attention_matches_dense_softmax_formula():
    """SDPA with the window mask equals the explicit masked-softmax attention in fp32."""
    torch.manual_seed(4)
    layer = Transformer({**config(), "attention_window": 5}, 0).eval()
    x = torch.randn(2, 11, 32)
    with torch.no_grad():
        got = layer(x)
        B, T, D = x.shape
        q, gate = layer.q(x).view(B, T, 2, 32).chunk(2, -1)
        k = layer.k(x).view(B, T, 2, 16)
        v = layer.v(x).view(B, T, 2, 16).transpose(1, 2)
        q = layer.rotary(torch.nn.functional.rms_norm(q, (16,)), 0).transpose(1, 2)
        k = layer.rotary(torch.nn.functional.rms_norm(k, (16,)), 0).transpose(1, 2)
        pos = torch.arange(T)
        allowed = (pos[None, :] <= pos[:, None]) & (pos[None, :] > pos[:, None] - 5)
        att = (q @ k.transpose(-1, -2) / 4.0).masked_fill(~allowed, float("-inf")).softmax(-1) @ v
        ref = layer.proj(att.transpose(1, 2).reshape(B, T, D) * gate.reshape(B, T, D).sigmoid())
    torch.testing.assert_close(got, ref, atol=1e-6, rtol=1e-5)


def test_rotary_is_a_rotation_by_absolute_position():
    """Norm-preserving, identity at position 0, and shifting both query and key
    positions by the same offset keeps their dot product."""
    layer = Transformer(config(), 0)
    g = torch.Generator().manual_seed(5)
    q, k = torch.randn(1, 1, 1, 16, generator=g), torch.randn(1, 1, 1, 16, generator=g)
    torch.testing.assert_close(layer.rotary(q, 0), q)
    torch.testing.assert_close(layer.rotary(q, 37).norm(), q.norm())
    d0 = (layer.rotary(q, 10) * layer.rotary(k, 7)).sum()
    d1 = (layer.rotary(q, 110) * layer.rotary(k, 107)).sum()
    torch.testing.assert_close(d0, d1, atol=1e-5, rtol=1e-5)



def test_kv_cache_decode_equals_full_pass():
    """Hundreds of one-token steps and mixed multi-token calls equal one full
    pass; the cache keeps exactly the last window - 1 keys."""
    torch.manual_seed(6)
    layer = Transformer({**config(), "attention_window": 5}, 0).eval()
    x = torch.randn(2, 700, 32)
    with torch.no_grad():
        full = layer(x)
        cache = {}
        out = torch.cat([layer(x[:, :3], cache)] + [layer(x[:, t:t + 1], cache) for t in range(3, 700)], 1)
        torch.testing.assert_close(out, full, atol=1e-6, rtol=1e-5)
        assert cache["tokens"] == 700 and cache["k"].shape[2] == 4
        torch.testing.assert_close(cache["k"], layer.rotary(torch.nn.functional.rms_norm(
            layer.k(x[:, -4:]).view(2, 4, 2, 16), (16,)), 696).transpose(1, 2))
        cache, parts, t = {}, [], 0
        for n in [1, 7, 300, 2, 1, 1, 388]:
            parts.append(layer(x[:, t:t + n], cache))
            t += n
        torch.testing.assert_close(torch.cat(parts, 1), full, atol=1e-6, rtol=1e-5)


def test_window_mask_cache():
    """The cached additive mask: 0 where query i may see key j (not later, less
    than the window back), -inf elsewhere; built once per shape, and never an
    inference tensor (autograd may save it after a first inference-mode call)."""
    from glsdm.layers.attention import _window_mask
    with torch.inference_mode():
        m = _window_mask(3, 5, 4, torch.device("cpu"), torch.float32)
    assert not m.is_inference() and m.shape == (5, 8)
    kpos = torch.arange(-3, 5)[None, :]
    qpos = torch.arange(5)[:, None]
    allowed = (kpos <= qpos) & (kpos > qpos - 4)
    assert torch.equal(m == 0, allowed) and torch.isinf(m[~allowed]).all()
    assert _window_mask(3, 5, 4, torch.device("cpu"), torch.float32) is m


@pytest.mark.parametrize("in_place", [False, True])
def test_copied_kv_cache_continues_independently_when_functional(in_place):
    """With gl_commit_in_place = False the KV cache is functional, as the
    reference's (S/layers/attention.py:53-58 builds new tensors with torch.cat):
    two continuations of one cache, stepped alternately, each equal a full pass
    over their own tokens.  With the in-place decode append (the default) the
    cache has one owner, so only one continuation is checked."""
    torch.manual_seed(8)
    layer = Transformer({**config(), "attention_window": 5, "gl_commit_in_place": in_place}, 0).eval()
    prompt = torch.randn(1, 6, 32)
    branch = [torch.randn(1, 5, 32), torch.randn(1, 5, 32)]
    with torch.no_grad():
        full = [layer(torch.cat((prompt, b), 1))[:, 6:] for b in branch]
        cache = {}
        layer(prompt, cache)
        caches = [dict(cache), dict(cache)] if not in_place else [cache]
        outs = [[] for _ in caches]
        for t in range(5):
            for c, (cc, out) in enumerate(zip(caches, outs)):
                out.append(layer(branch[c][:, t:t + 1], cc))
        for c, out in enumerate(outs):
            torch.testing.assert_close(torch.cat(out, 1), full[c], atol=1e-6, rtol=1e-5)
