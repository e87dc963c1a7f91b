"""ctypes binding of libglsdm.so (declared in include/glsdm.h).

The library is the only compute path of this package: if it is missing, or no
HIP device is present, every native call raises instead of falling back.
"""
import contextlib
import ctypes
import os
import threading

import torch

# the in-tree build; GLSDM_LIB names another build of the same library
LIB_PATH = os.environ.get("GLSDM_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libglsdm.so")

F32, BF16 = 0, 1
TIE_HIGHEST, TIE_LOWEST = 0, 1
TIES = {"highest": TIE_HIGHEST, "lowest": TIE_LOWEST}
DTYPES = {torch.float32: F32, torch.bfloat16: BF16}

OK, ERR_ARG, ERR_UNSUPPORTED, ERR_WORKSPACE, ERR_HIP = 0, -1, -2, -3, -4

_P, _I64, _I32, _SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t
SIGNATURES = {
    "glsdm_version": ([], ctypes.c_char_p),
    "glsdm_last_error": ([], ctypes.c_char_p),
    "glsdm_route": ([_P, _I32, _I64, _I32, _I32, _I32, _P, _P, _P, _SZ, _P], _I32),
    "glsdm_route_workspace_bytes": ([_I64, _I32, _I32, _P], _I32),
    "glsdm_read": ([_P, _I32, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _I32, _P], _I32),
    "glsdm_read_narrow": ([_P, _I32, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _I32, _P], _I32),
    "glsdm_route_read": ([_P, _I32, _I64, _I64, _I64, _I64, _I64, _P, _I32, _I32, _I32, _P, _I32, _P, _P, _P, _SZ,
                          _P], _I32),
    "glsdm_score": ([_P, _P, _I64, _I64, _I64, _I32, _I32, _P, _P], _I32),
    "glsdm_score_route": ([_P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _SZ, _P], _I32),
    "glsdm_score_route_keys": ([_P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _I64, _I64, _I64, _I64, _P, _P,
                                _P, _P, _P, _SZ, _P], _I32),
    "glsdm_score_route_workspace_bytes": ([_I64, _I64, _I64, _I32, _I32, ctypes.POINTER(_SZ)], _I32),
    "glsdm_commit_workspace_bytes": ([_I64, _I64, ctypes.POINTER(_SZ)], _I32),
    "glsdm_commit": ([_P, _I32, _I64, _I64, _P, _P, _I32, _P, _I64, _P, _SZ, _P, _P], _I32),
    "glsdm_commit_prepare": ([_I64, _P, _I64, _P, _SZ, _P], _I32),
    "glsdm_commit_apply": ([_P, _I32, _I64, _I64, _P, _I32, _P, _I64, _P, _SZ, _P, _P], _I32),
    "glsdm_commit_status": ([_P, _SZ, _I64, _I64, _P, _P], _I32),
    "glsdm_commit_noalloc": ([_P, _I32, _I64, _I64, _P, _P, _I32, _P, _I64, _P, _P], _I32),
    "glsdm_debug_force_lookback_timeout": ([_I32], _I32),
    "glsdm_absolute_addresses": ([_P, _I64, _I64, _I64, _I32, _I64, _P, _P], _I32),
    "glsdm_proposal_keys": ([_P, _I64, _I64, _I64, _I32, _I64, _I64, _I64, _I64, _I64, _P, _P, _P], _I32),
    "glsdm_qk_norm_rotary": ([_P, _I32, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _P], _I32),
    "glsdm_decode_qkv": ([_P, _I64, _I64, _P, _I64, _P, _I64, _I64, _I32, _I64, _I64, _I64, _P, _I64, _P, _P, _P,
                          ctypes.POINTER(_I64), _P], _I32),
    "glsdm_gate_merge": ([_P, _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _P, _P], _I32),
    "glsdm_relu2_gate": ([_P, _I32, _I64, _I64, _P, _P], _I32),
    "glsdm_linear_small": ([_P, _P, _P, _P, _I64, _I64, _I64, _P], _I32),
    "glsdm_linear_small_residual": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _P], _I32),
    "glsdm_linear_small_relu2": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _P], _I32),
    "glsdm_linear_small_group": ([_P, _I32, ctypes.POINTER(_P), ctypes.POINTER(_P), ctypes.POINTER(_P),
                                  ctypes.POINTER(_I64), _I64, _I64, _P], _I32),
    "glsdm_decode_attention": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, ctypes.POINTER(_I64), ctypes.POINTER(_I64),
                                ctypes.c_float, _P], _I32),
    "glsdm_decode_attention_gated": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, ctypes.POINTER(_I64),
                                      ctypes.POINTER(_I64), ctypes.POINTER(_I64), ctypes.c_float, _P], _I32),
    "glsdm_rms_norm_cast": ([_P, _I32, _P, _I32, _I64, _I64, ctypes.c_float, _P, _I32, _P], _I32),
    "glsdm_write_gates": ([_P, _P, _I32, _I64, _P, _P, _P], _I32),
    "glsdm_gather_rows": ([_P, _I32, _I64, _I64, _P, _I64, _P, _P], _I32),
    "glsdm_proposal_error": ([_I64, _I64, _P, _P, _I32, _P, _P, _P, _P, _P], _I32),
    "glsdm_proposal_append": ([_P, _P, _P, _P, _I32, _P, _P, _I32, _I64, _I64, _I64, _I32, _I64, _I64, _I64, _I64,
                               _I64, _I64, _P, _P, _P, _P, _P, _P], _I32),
    "glsdm_proposal_delta": ([_P, _I32, _I64, _I32, _I64, _P, _P, _P, _I32, _P, _P, _P, _I64, _P, _P], _I32),
    "glsdm_route_backward": ([_P, _P, _P, _I64, _I32, _I32, _P, _P], _I32),
    "glsdm_read_backward_weights": ([_P, _I32, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _P], _I32),
    "glsdm_read_backward_rows": ([_P, _I64, _I64, _P, _I64, _I32, _P, _P, _P, _SZ, _P], _I32),
    "glsdm_overlay_read": ([_P, _I32, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _I32, _P], _I32),
    "glsdm_overlay_commit": ([_P, _I32, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _P, _I32, _P, _I64, _P,
                              _SZ, _P, _P], _I32),
    "glsdm_overlay_materialise": ([_P, _I32, _P, _P, _I64, _I64, _I64, _I64, _P, _P], _I32),
    "glsdm_commit_proposals": ([_P, _I32, _I64, _I64, _P, _P, _I64, _I32, _P, _P, _P, _P, _I64, _P, _SZ, _P, _P],
                               _I32),
}

_lock = threading.Lock()
_lib = None

# Debug checks, off by default (each costs a host synchronisation per call):
#   status -- after every commit-family call, read the commit's device status
#             words (glsdm_commit_status) and raise NativeError if its sort
#             failed (no bank row was then written);
#   bounds -- before a read, gather or commit, check every slot / address
#             against its range and raise IndexError, as the reference's torch
#             indexing does (flat[index]), instead of the kernels' documented
#             skipping of out-of-range entries.
# GLSDM_CHECKS="status,bounds" in the environment turns them on at import.
_env_checks = {c.strip() for c in os.environ.get("GLSDM_CHECKS", "").split(",") if c.strip()}
_checks = {"status": "status" in _env_checks, "bounds": "bounds" in _env_checks}


def set_checks(status=None, bounds=None):
    """Turn the debug checks on or off; returns the previous settings."""
    prev = dict(_checks)
    if status is not None:
        _checks["status"] = bool(status)
    if bounds is not None:
        _checks["bounds"] = bool(bounds)
    return prev


@contextlib.contextmanager
def checks(status=None, bounds=None):
    prev = set_checks(status, bounds)
    try:
        yield
    finally:
        set_checks(**prev)


def checking(name):
    return _checks[name]


def check_range(index, hi, what):
    """Bounds check (debug): every element of ``index`` in [0, hi), else IndexError."""
    if _checks["bounds"] and index is not None and index.numel():
        bad = (index < 0) | (index >= hi)
        if bool(bad.any()):
            first = int(index[bad].reshape(-1)[0])
            raise IndexError(f"{what}: index {first} is out of bounds for size {hi}")


class NativeError(RuntimeError):
    pass


def lib():
    """Load libglsdm.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise NativeError(f"{LIB_PATH} is missing: build it with `python gl-sdm_amd/build.py` "
                                      "(or __graft_entry__.build()); there is no fallback path")
                L = ctypes.CDLL(LIB_PATH)
                for name, (args, res) in SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.argtypes, fn.restype = args, res
                _lib = L
    return _lib


_fns = {}


def call(name, *args):
    """Invoke an entry point and turn a non-zero status into an exception."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(lib(), name)
    rc = fn(*args)
    if rc != OK:
        msg = lib().glsdm_last_error().decode()
        if rc in (ERR_ARG, ERR_UNSUPPORTED, ERR_WORKSPACE):
            raise ValueError(f"{name}: {msg}")
        raise NativeError(f"{name} failed ({rc}): {msg}")


def ptr(t):
    """A tensor's device address for a ``void *`` argument (None for None): a plain
    int, which ctypes converts for the declared pointer type without building a
    c_void_p object (a decode step passes several hundred of them)."""
    return t.data_ptr() if t is not None else None


def stream(device):
    """The current HIP stream of ``device`` as an address for a ``void *`` argument
    (torch's raw-stream query: a decode step makes over a hundred native calls, and
    the Stream-object path costs several microseconds of host time each)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def dtype_code(t):
    try:
        return DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"GL-SDM native kernels support float32 and bfloat16, not {t.dtype}") from None


def require_device(*tensors):
    """Same contract as the reference's require_cuda (S/memory/backends/primitives.py:7-12):
    contiguous tensors on a HIP device (ROCm torch reports them as CUDA), one device."""
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError("GL-SDM native kernels require contiguous CUDA (HIP) tensors")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError("GL-SDM native operands must share one device")
    return device


def version():
    return lib().glsdm_version().decode()
