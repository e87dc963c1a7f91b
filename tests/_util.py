"""Shared helpers for the test suite (seeded CPU input generation, fixtures)."""
import json
import os
import re

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def known_answers():
    with open(os.path.join(HERE, "golden", "known_answers.json")) as f:
        return json.load(f)


def gen(seed):
    return torch.Generator("cpu").manual_seed(seed)


def route_scores(kind, shape, seed=0):
    """fp32 factor scores of a given flavour, generated on the CPU."""
    g = gen(seed)
    if kind == "randn":
        return torch.randn(*shape, generator=g)
    if kind == "bf16":      # bf16-rounded scores, as the bf16 router.q Linear produces
        return torch.randn(*shape, generator=g).to(torch.bfloat16).float()
    if kind == "floor":     # massive exact ties (P/tests/test_layer_stack.py:156-161)
        return torch.randn(*shape, generator=g).mul(2).floor()
    if kind == "zeros":
        return torch.zeros(*shape)
    if kind == "signed_zero":
        s = torch.zeros(*shape)
        s[..., ::3] = -0.0
        return s
    if kind == "mixed":     # random rows with some all-zero and floored rows, and infinities
        s = torch.randn(*shape, generator=g)
        flat = s.view(-1, shape[-1])
        flat[::5] = 0.0
        flat[1::7] = flat[1::7].floor()
        flat[2::11, 0] = float("inf")
        flat[3::13, -1] = float("-inf")
        return s
    raise ValueError(kind)


def header_functions():
    """Names of every function declared in include/glsdm.h."""
    with open(os.path.join(ROOT, "include", "glsdm.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(glsdm_\w+)\s*\(", text, re.M)))
