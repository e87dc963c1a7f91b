"""The C-ABI library loads and exports every entry point include/glsdm.h declares;
argument validation answers before any device work (no GPU needed)."""
import ctypes

import pytest

from glsdm import _native as N
from _util import header_functions


def test_header_declares_the_expected_surface():
    names = header_functions()
    for required in ("glsdm_route", "glsdm_read", "glsdm_read_narrow", "glsdm_route_read", "glsdm_score", "glsdm_commit",
                     "glsdm_commit_workspace_bytes", "glsdm_absolute_addresses", "glsdm_proposal_keys",
                     "glsdm_gather_rows", "glsdm_version", "glsdm_last_error", "glsdm_proposal_error",
                     "glsdm_proposal_delta", "glsdm_commit_proposals", "glsdm_route_backward",
                     "glsdm_read_backward_weights", "glsdm_read_backward_rows", "glsdm_overlay_read",
                     "glsdm_overlay_commit", "glsdm_overlay_materialise", "glsdm_route_workspace_bytes",
                     "glsdm_score_route", "glsdm_score_route_keys", "glsdm_score_route_workspace_bytes",
                     "glsdm_commit_prepare", "glsdm_commit_apply", "glsdm_qk_norm_rotary", "glsdm_gate_merge", "glsdm_relu2_gate",
                     "glsdm_rms_norm_cast", "glsdm_write_gates"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing
    assert set(header_functions()) == set(N.SIGNATURES)


def test_version():
    assert "gfx950" in N.version()


def _rc(name, *args):
    return getattr(N.lib(), name)(*args)


def _route_rc(scores_dtype, rows, half, width, tie):
    return _rc("glsdm_route", None, scores_dtype, rows, half, width, tie, None, None, None, 0, None)


def test_route_rejects_bad_arguments_before_launch():
    assert _route_rc(0, 4, 8, 0, 0) == N.ERR_UNSUPPORTED
    assert _route_rc(1, 4, 8, 65, 0) == N.ERR_UNSUPPORTED
    assert _route_rc(0, 4, 2, 5, 0) == N.ERR_ARG    # width > slots
    assert _route_rc(0, 4, 8, 4, 7) == N.ERR_ARG    # tie
    assert _route_rc(5, 4, 8, 4, 0) == N.ERR_ARG    # scores dtype
    assert _route_rc(1, 4, 8, 4, 0) == N.ERR_ARG    # null pointers
    assert "null" in N.lib().glsdm_last_error().decode()
    assert _route_rc(0, 0, 8, 4, 0) == N.OK         # empty is a no-op


def test_route_workspace_contract():
    """The split path's workspace: sized for few rows (decode), zero when the
    single-kernel launch already fills the GPU."""
    size = ctypes.c_size_t(7)
    assert _rc("glsdm_route_workspace_bytes", 1024, 1024, 16, ctypes.byref(size)) == N.OK
    assert size.value > 0 and size.value % (1024 * 2 * 16 * 8) == 0
    assert _rc("glsdm_route_workspace_bytes", 1 << 20, 1024, 16, ctypes.byref(size)) == N.OK
    assert size.value == 0
    assert _rc("glsdm_route_workspace_bytes", 1024, 0, 16, ctypes.byref(size)) == N.ERR_ARG


def test_commit_workspace_contract():
    size = ctypes.c_size_t(0)
    assert _rc("glsdm_commit_workspace_bytes", 524288, 1 << 22, ctypes.byref(size)) == N.OK
    assert size.value >= 2 * 8 * 524288
    assert _rc("glsdm_commit_workspace_bytes", 1 << 31, 16, ctypes.byref(size)) == N.ERR_UNSUPPORTED
    assert _rc("glsdm_commit_workspace_bytes", 1 << 29, 1 << 40, ctypes.byref(size)) == N.ERR_UNSUPPORTED
    assert _rc("glsdm_commit", ctypes.c_void_p(1), 0, 16, 4, ctypes.c_void_p(1), ctypes.c_void_p(1), 0,
               None, 8, None, 0, None, None) == N.ERR_WORKSPACE
    assert _rc("glsdm_commit", None, 0, 16, 4, None, None, 0, None, 0, None, 0, None, None) == N.OK


def test_proposal_envelopes():
    one = ctypes.c_void_p(16)
    # D above the supported row width, D not a multiple of 4 above 512
    assert _rc("glsdm_proposal_error", 4, 4096, one, one, 0, one, one, one, one, None) == N.ERR_UNSUPPORTED
    assert _rc("glsdm_proposal_error", 4, 514, one, one, 0, one, one, one, one, None) == N.ERR_UNSUPPORTED
    assert _rc("glsdm_proposal_error", 4, 64, one, one, 3, one, one, one, one, None) == N.ERR_ARG   # dtype
    assert _rc("glsdm_proposal_error", 4, 64, None, one, 0, one, one, one, one, None) == N.ERR_ARG  # null
    assert _rc("glsdm_proposal_error", 0, 64, None, None, 0, None, None, None, None, None) == N.OK
    # R must be whole groups of heads (mass has one value per token)
    assert _rc("glsdm_proposal_delta", one, 0, 6, 2, 64, one, one, one, 0, one, one, one, 4, one,
               None) == N.ERR_ARG
    assert _rc("glsdm_proposal_delta", one, 0, 8, 0, 64, one, one, one, 0, one, one, one, 4, one,
               None) == N.ERR_ARG
    # fused commit: entries must be whole proposal rows, workspace checked before launch
    assert _rc("glsdm_commit_proposals", one, 0, 16, 4, one, None, 10, 4, one, one, one, one, 1, None, 0,
               None, None) == N.ERR_ARG
    assert _rc("glsdm_commit_proposals", one, 0, 16, 4, one, None, 8, 4, one, one, one, one, 1, None, 0,
               None, None) == N.ERR_WORKSPACE
    assert _rc("glsdm_commit_proposals", one, 0, 16, 4, one, None, 8, 4, None, one, one, one, 1, None, 0,
               None, None) == N.ERR_ARG
    assert _rc("glsdm_commit_proposals", None, 0, 16, 4, None, None, 0, 4, None, None, None, None, 1, None, 0,
               None, None) == N.OK


def test_backward_envelopes():
    one = ctypes.c_void_p(16)
    assert _rc("glsdm_route_backward", one, one, one, 4, 8, 65, one, None) == N.ERR_UNSUPPORTED   # width
    assert _rc("glsdm_route_backward", one, one, None, 4, 8, 4, one, None) == N.ERR_ARG           # null
    assert _rc("glsdm_route_backward", None, None, None, 0, 8, 4, None, None) == N.OK            # empty
    assert _rc("glsdm_read_backward_weights", one, 0, 1, 1, 16, 4096, 2, 4, one, one, one, None) == N.ERR_UNSUPPORTED
    assert _rc("glsdm_read_backward_weights", one, 5, 1, 1, 16, 64, 2, 4, one, one, one, None) == N.ERR_ARG
    assert _rc("glsdm_read_backward_rows", one, 16, 4, one, 10, 4, one, one, None, 0, None) == N.ERR_ARG  # 10 % 4
    assert _rc("glsdm_read_backward_rows", one, 16, 4, one, 8, 4, one, one, None, 0, None) == N.ERR_WORKSPACE


def test_overlay_envelopes():
    one = ctypes.c_void_p(16)
    assert _rc("glsdm_overlay_read", one, 0, one, one, 1, 1, 16, 4096, 2, 4, one, one, one, 0, None) == N.ERR_UNSUPPORTED
    assert _rc("glsdm_overlay_read", one, 0, None, one, 1, 1, 16, 64, 2, 4, one, one, one, 0, None) == N.ERR_ARG
    assert _rc("glsdm_overlay_commit", one, 0, 1, 1, 16, 4, one, one, 1 << 31, 0, one, one, 0, None, 8, None, 0,
               None, None) == N.ERR_UNSUPPORTED                                                     # capacity
    assert _rc("glsdm_overlay_commit", one, 0, 1, 1, 16, 4, one, one, 8, 4, one, one, 0, None, 8, None, 0,
               None, None) == N.ERR_ARG                                                             # 4 + 8 > 8
    assert _rc("glsdm_overlay_commit", one, 0, 1, 1, 16, 4, one, one, 8, 0, one, one, 0, None, 8, None, 0,
               None, None) == N.ERR_WORKSPACE
    assert _rc("glsdm_overlay_materialise", one, 3, one, one, 1, 1, 16, 4, one, None) == N.ERR_ARG


def test_read_and_score_envelopes():
    assert _rc("glsdm_read", None, 0, 1, 1, 16, 5000, 1, 4, None, None, None, 0, None) == N.ERR_UNSUPPORTED
    assert _rc("glsdm_score", None, None, 1, 1, 1, 48, 32, None, None) == N.ERR_UNSUPPORTED  # dk % 32
    assert _rc("glsdm_score", None, None, 1, 1, 1, 64, 20, None, None) == N.ERR_UNSUPPORTED  # L % 64
    assert _rc("glsdm_route_read", None, 0, 1, 1, 15, 8, 1, None, 0, 4, 0, None, 0, None, None, None, 0,
               None) == N.ERR_ARG


def test_errors_become_python_exceptions():
    with pytest.raises(ValueError, match="width"):
        N.call("glsdm_route", None, 0, 4, 8, 0, 0, None, None, None, 0, None)


def test_stack_ops_reject_bad_arguments_before_launch():
    """The fused stack entry points check shapes, dtypes, strides and alignment
    on the host and return a status; nothing is launched on these."""
    one = ctypes.c_void_p(16)
    eps = ctypes.c_float(1e-6)
    qk = lambda B, dk, stride, offset: _rc("glsdm_qk_norm_rotary", one, 1, B, 2, 1, dk, stride, one, offset, one, None)
    assert qk(1, 12, 24, 0) == N.ERR_ARG                   # dk not a power of two
    assert qk(1, 512, 512, 0) == N.ERR_ARG                 # dk above 256
    assert qk(1, 64, 32, 0) == N.ERR_ARG                   # row stride below dk
    assert qk(1, 64, 64, 1 << 24) == N.ERR_UNSUPPORTED     # positions not exact in fp32
    assert qk(0, 64, 64, 0) == N.OK                        # empty
    assert _rc("glsdm_relu2_gate", one, 1, 4, 12, one, None) == N.ERR_UNSUPPORTED                # inner % 8
    assert _rc("glsdm_relu2_gate", ctypes.c_void_p(18), 1, 4, 16, one, None) == N.ERR_UNSUPPORTED  # alignment
    assert _rc("glsdm_relu2_gate", one, 3, 4, 16, one, None) == N.ERR_ARG                         # dtype
    strided = (ctypes.c_int64 * 4)(64, 64, 64, 2)
    assert _rc("glsdm_gate_merge", one, strided, one, strided, 1, 1, 1, 1, 64, one, None) == N.ERR_UNSUPPORTED
    assert _rc("glsdm_rms_norm_cast", one, 1, one, 5, 4, 16, eps, one, 1, None) == N.ERR_ARG      # weight dtype
    assert _rc("glsdm_rms_norm_cast", one, 1, one, 0, 4, 0, eps, one, 1, None) == N.ERR_ARG       # dim 0
    assert _rc("glsdm_write_gates", one, one, 1, -1, one, one, None) == N.ERR_ARG
    assert _rc("glsdm_write_gates", None, None, 1, 0, None, None, None) == N.OK                 # empty
    # proposal_append(index, weights, prediction, target, tdtype, beta, decay, gdtype, B, T, H, width, S, D,
    #                 offset, chunk, layers, layer, addresses, keys, weights_out, error, decay_out, stream)
    append = lambda T, D, layer, gdtype: _rc("glsdm_proposal_append", one, one, one, one, 1, one, one, gdtype, 2, T,
                                             4, 8, 64, D, 0, 4, 2, layer, one, one, one, one, one, None)
    assert append(1, 64, 2, 1) == N.ERR_ARG                # layer >= layers
    assert append(1, 4096, 0, 1) == N.ERR_UNSUPPORTED      # D above 2048
    assert append(1, 64, 0, 7) == N.ERR_ARG                # gate dtype
    assert append(0, 64, 0, 1) == N.OK                     # empty


def test_decode_entry_points_reject_bad_arguments_before_launch():
    """The decode-step entry points (projections, q/k/v preparation, attention)
    check counts, shapes and alignment on the host; nothing is launched on these."""
    one, odd = ctypes.c_void_p(16), ctypes.c_void_p(18)
    lin = lambda name, x, M, Nn, K: _rc(name, x, one, None, one, M, Nn, K, None)
    for name in ("glsdm_linear_small",):
        assert lin(name, one, 65, 16, 128) == N.ERR_UNSUPPORTED      # more than 64 rows
        assert lin(name, one, 4, 24, 128) == N.ERR_UNSUPPORTED       # width not a multiple of 16
        assert lin(name, one, 4, 16, 96) == N.ERR_UNSUPPORTED        # depth not a multiple of 128
        assert lin(name, odd, 4, 16, 128) == N.ERR_UNSUPPORTED       # x not 16-byte aligned
        assert lin(name, one, 0, 16, 128) == N.ERR_ARG               # no rows
    res = lambda M, Nn, K, r: _rc("glsdm_linear_small_residual", one, one, None, r, one, M, Nn, K, None)
    assert res(4, 16, 128, None) == N.ERR_ARG                       # residual missing
    assert res(4, 24, 128, one) == N.ERR_UNSUPPORTED
    relu = lambda h, M, Nn, K: _rc("glsdm_linear_small_relu2", h, one, None, None, one, M, Nn, K, None)
    assert relu(one, 4, 16, 100) == N.ERR_UNSUPPORTED               # inner width not a multiple of 128
    assert relu(odd, 4, 16, 128) == N.ERR_UNSUPPORTED
    P = ctypes.c_void_p
    ptrs = (P * 9)(*([16] * 9))
    widths = (ctypes.c_int64 * 9)(*([16] * 9))
    group = lambda count, w: _rc("glsdm_linear_small_group", one, count, ptrs, None, ptrs, w, 4, 128, None)
    assert group(0, widths) == N.ERR_ARG                             # no projection
    assert group(9, widths) == N.ERR_ARG                             # more than 8
    assert group(2, (ctypes.c_int64 * 2)(16, 40)) == N.ERR_UNSUPPORTED   # a width not a multiple of 16
    # decode_qkv(q, q_stride, q_heads, k, k_stride, v, v_stride, kv_heads, dtype, B, T, dk, freq, offset,
    #            q_out, k_dst, v_dst, dst_strides, stream)
    strides = (ctypes.c_int64 * 3)(1024, 64, 64)
    qkv = lambda dk, ks, offset, dtype: _rc("glsdm_decode_qkv", one, 2 * dk, 4, one, ks, one, dk, 4, dtype, 2, 1,
                                            dk, one, offset, one, one, one, strides, None)
    assert qkv(48, 48, 0, 1) == N.ERR_ARG                            # dk not a power of two
    assert qkv(64, 32, 0, 1) == N.ERR_ARG                            # key row stride below dk
    assert qkv(64, 64, 1 << 24, 1) == N.ERR_UNSUPPORTED              # positions not exact in fp32
    assert qkv(64, 64, 0, 4) == N.ERR_ARG                            # dtype
    kv = (ctypes.c_int64 * 3)(64 * 512, 512 * 64, 64)
    gs = (ctypes.c_int64 * 2)(1024, 128)
    att = lambda L, dk, gate: _rc("glsdm_decode_attention_gated", one, one, one, gate, one, 2, 4, L, dk, kv, kv, gs,
                                  ctypes.c_float(0.125), None)
    assert att(1025, 64, one) == N.ERR_UNSUPPORTED                   # more than 1024 keys
    assert att(16, 96, one) == N.ERR_UNSUPPORTED                     # dk other than 64 / 128
    assert att(16, 64, None) == N.ERR_ARG                            # gate missing

