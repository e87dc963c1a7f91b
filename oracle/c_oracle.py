"""ctypes binding of the scalar C oracle ``glsdm_oracle.c``.

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.  Takes and returns
CPU torch tensors; bf16 inputs are widened to fp32 exactly before the call.
"""
import ctypes
import os
import subprocess

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libglsdm_oracle.so")
_lib = None

TIE = {"highest": 0, "lowest": 1}


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_route.argtypes = [p, i64, i32, i32, i32, p, p]
        L.oracle_route.restype = i32
        L.oracle_read.argtypes = [p, i64, i64, i64, i64, i64, i32, p, p, p]
        L.oracle_read.restype = i32
        L.oracle_commit.argtypes = [p, i64, i64, p, p, p, i64]
        L.oracle_commit.restype = i64
        L.oracle_score.argtypes = [p, p, i64, i64, i64, i64, p]
        L.oracle_score.restype = None
        _lib = L
    return _lib


def _cpu(t, dtype):
    return t.detach().to("cpu", dtype).contiguous()


def route(scores, width, tie="highest"):
    """scores ``[..., 2*half]`` -> (index int64, weights fp32) ``[..., width]``."""
    s = _cpu(scores, torch.float32)
    lead, L = s.shape[:-1], s.shape[-1]
    rows = s.numel() // L
    index = torch.empty(*lead, width, dtype=torch.int64)
    weights = torch.empty(*lead, width, dtype=torch.float32)
    rc = lib().oracle_route(s.data_ptr(), rows, L // 2, width, TIE[tie], index.data_ptr(), weights.data_ptr())
    if rc != 0:
        raise ValueError(f"oracle_route failed ({rc})")
    return index, weights


def read(memory, index, weights):
    """memory ``[B,H,S,D]`` (fp32 or bf16), index/weights ``[B,T,H,width]`` -> fp32 ``[B,T,H,D]``."""
    m = _cpu(memory, torch.float32)
    idx = _cpu(index, torch.int64)
    w = _cpu(weights, torch.float32)
    B, H, S, D = m.shape
    T, width = idx.shape[1], idx.shape[-1]
    out = torch.empty(B, T, H, D, dtype=torch.float32)
    rc = lib().oracle_read(m.data_ptr(), B, H, S, D, T, width, idx.data_ptr(), w.data_ptr(), out.data_ptr())
    if rc != 0:
        raise ValueError(f"oracle_read failed ({rc})")
    return out


def commit(flat, addresses, deltas, keys=None):
    """Functional commit: returns (new fp32 bank ``[rows, D]``, unique row count)."""
    bank = _cpu(flat, torch.float32).clone()
    addr = _cpu(addresses, torch.int64)
    d = _cpu(deltas, torch.float32)
    k = None if keys is None else _cpu(keys, torch.int64)
    rows, D = bank.shape
    n = lib().oracle_commit(bank.data_ptr(), rows, D, addr.data_ptr(), d.data_ptr(),
                            None if k is None else k.data_ptr(), addr.numel())
    if n < 0:
        raise ValueError(f"oracle_commit failed ({n})")
    return bank, int(n)


def score(queries, subkeys):
    """queries ``[B,T,H,dk]``, sub-keys ``[H,L,dk]`` -> fp32 scores ``[B,T,H,L]``."""
    q = _cpu(queries, torch.float32)
    k = _cpu(subkeys, torch.float32)
    B, T, H, dk = q.shape
    L = k.shape[1]
    out = torch.empty(B, T, H, L, dtype=torch.float32)
    lib().oracle_score(q.data_ptr(), k.data_ptr(), B * T, H, dk, L, out.data_ptr())
    return out
