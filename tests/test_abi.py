"""The C ABI library loads and exports every symbol include/fns_hip.h declares; argument validation happens on the
host before any launch (these calls never touch a GPU). Reference error behaviour: unsupported types and shape
preconditions are rejected (reference src/ggml/ggml_mmvq.cu:385, src/kernels.cu:911-918); the C ABI reports them
as status codes, the C++ API aborts."""
from __future__ import annotations

import ctypes

import pytest

from flintnsteel_amd import _lib


def test_exports_every_declared_symbol():
    L = _lib.lib()
    declared = _lib.header_symbols()
    assert len(declared) >= 20
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing, f"declared in include/fns_hip.h but not exported: {missing}"
    untyped = [s for s in declared if s not in _lib.SIGNATURES]
    assert not untyped, f"no ctypes signature for {untyped}"


def test_q8_1_row_bytes_padding():
    L = _lib.lib()
    assert L.fns_hip_q8_1_row_bytes(2048) == 64 * 36
    assert L.fns_hip_q8_1_row_bytes(768) == 32 * 36   # padded to 1024 columns
    assert L.fns_hip_q8_1_row_bytes(1) == 16 * 36


def test_supported_types():
    L = _lib.lib()
    got = {t for t in range(40) if L.fns_hip_mmvq_supports(t)}
    # Q8_0, the K-quants and IQ4_XS always; IQ3_XXS / IQ3_S / IQ2_S once their codebooks are registered
    assert {8, 11, 12, 13, 14, 23} <= got <= {8, 11, 12, 13, 14, 18, 21, 22, 23}


def _buf():
    return ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first


def test_unsupported_type_is_rejected():
    L = _lib.lib()
    rc = L.fns_hip_mmvq(10, _buf(), 2048, 16, _buf(), _buf(), 1, None)  # Q2_K: not accepted
    assert rc == -1
    assert b"not supported" in L.fns_hip_last_error()
    with pytest.raises(_lib.FnsError, match="not supported"):
        _lib.call("fns_hip_mmvq_experts", 99, _buf(), 0, 2048, 16, _buf(), 1, _buf(), 8, _buf(), None)


def test_shape_preconditions():
    L = _lib.lib()
    assert L.fns_hip_mmvq(12, _buf(), 1000, 16, _buf(), _buf(), 1, None) == -2      # ncols % 256
    assert L.fns_hip_mmvq_experts_swiglu(12, _buf(), 0, 0, 2048, 768, _buf(), 3, _buf(), 8, _buf(), None) == -2
    assert L.fns_hip_route_topk(_buf(), _buf(), _buf(), 300, 8, 1, 0, 1, None) == -2  # > 256 experts
    assert L.fns_hip_route_topk(_buf(), _buf(), _buf(), 128, 17, 1, 0, 1, None) == -2  # k > 16
    assert L.fns_hip_gemv_router(0, _buf(), _buf(), _buf(), 2048, 128, 9, None) == -2  # > 8 columns
    assert L.fns_hip_gemv_router(5, _buf(), _buf(), _buf(), 2048, 128, 1, None) == -1  # router dtype


def test_empty_inputs_are_noops():
    L = _lib.lib()
    assert L.fns_hip_mmvq_experts(12, _buf(), 0, 2048, 16, _buf(), 1, _buf(), 0, _buf(), None) == 0
    assert L.fns_hip_quantize_q8_1(_buf(), _buf(), 2048, 0, None) == 0
    assert L.fns_hip_route_topk(_buf(), _buf(), _buf(), 128, 8, 0, 0, 1, None) == 0


def test_mmq_sizes():
    L = _lib.lib()
    # split image: 1056 bytes per 256 columns (q8 * d8 as hi + lo halves, then the 8 sub-block sums as hi + lo)
    assert L.fns_hip_mmq_q8_1_bytes(2048, 1) == 8 * 1056 + 4096
    assert L.fns_hip_mmq_q8_1_bytes(768, 10) == 10 * 3 * 1056 + 4096
    # standalone compaction: bounds [n_expert + 1] and the two group-prefix lists
    assert L.fns_hip_mmq_bounds_bytes(128) == 3 * 129 * 4


def test_mmq_preconditions():
    L = _lib.lib()
    assert L.fns_hip_mmq(10, _buf(), 2048, 64, _buf(), 4, _buf(), _buf(), None) == -1    # Q2_K: not supported
    assert L.fns_hip_mmq(8, _buf(), 1000, 64, _buf(), 4, _buf(), _buf(), None) == -2     # Q8_0 too: ncols % 256
    assert L.fns_hip_mmq(12, _buf(), 1000, 64, _buf(), 4, _buf(), _buf(), None) == -2    # ncols % 256
    assert L.fns_hip_mmq(12, _buf(), 2048, 100, _buf(), 4, _buf(), _buf(), None) == -2   # nrows % 64
    assert L.fns_hip_mmq(12, _buf(), 2048, 64, _buf(), 0, _buf(), _buf(), None) == 0     # no tokens: no-op
    assert L.fns_hip_mmq_compact(_buf(), 4, 8, 300, 1, _buf(), _buf(), _buf(), None) == -2  # > 256 experts
    assert L.fns_hip_mmq_compact(_buf(), 4, 8, 128, 3, _buf(), _buf(), _buf(), None) == -2  # rows per token 1 or k


def test_moe_block_extras_host_checks():
    """The whole-block fields of FnsMoeLayer (RMSNorm, shared expert): the workspace grows with them, and a bad shared
    expert is rejected on the host before any launch."""
    from flintnsteel_amd import ops
    L = _lib.lib()
    buf = ctypes.create_string_buffer(64)
    ptr = ctypes.addressof(buf)
    d = ops.MoeLayerDesc(2048, 512, 256, 6, 1, 1, 1, 30, ptr, 12, 13, ptr, 0, 1024, 2048, None)
    total = ctypes.c_size_t()
    offs = (ctypes.c_size_t * 6)()
    assert L.fns_hip_moe_workspace_layout(ctypes.byref(d), 1, offs, ctypes.byref(total)) == 0
    plain = total.value
    d.shexp_inter, d.shexp_gate, d.shexp_up, d.shexp_down = 1024, ptr, ptr, ptr
    assert L.fns_hip_moe_workspace_layout(ctypes.byref(d), 4, offs, ctypes.byref(total)) == 0
    with_sh4 = total.value
    assert L.fns_hip_moe_workspace_layout(ctypes.byref(d), 1, offs, ctypes.byref(total)) == 0
    assert plain < total.value < with_sh4
    ws = ctypes.create_string_buffer(with_sh4)
    d.shexp_inter = 1000  # not a multiple of 256
    assert L.fns_hip_moe_layer(ctypes.byref(d), ptr, None, ptr, 1, ctypes.addressof(ws), with_sh4, None) == -2
    d.shexp_inter, d.shexp_down = 1024, None  # down missing
    assert L.fns_hip_moe_layer(ctypes.byref(d), ptr, None, ptr, 1, ctypes.addressof(ws), with_sh4, None) == -2
    d.shexp_down, d.shexp_gu_type = ptr, 10  # Q2_K: not accepted
    assert L.fns_hip_moe_layer(ctypes.byref(d), ptr, None, ptr, 1, ctypes.addressof(ws), with_sh4, None) == -1


def test_dense_ffn_host_checks():
    """fns_hip_dense_ffn: workspace sizing and the host-side shape / type / size checks (no launch)."""
    from flintnsteel_amd import ops
    L = _lib.lib()
    buf = ctypes.create_string_buffer(64)
    ptr = ctypes.addressof(buf)
    d = ops.DenseFfnDesc(2048, 6144, 12, 12, 14, ptr, ptr, ptr, None, 1e-6)
    t1, t4 = ctypes.c_size_t(), ctypes.c_size_t()
    assert L.fns_hip_dense_ffn_workspace(ctypes.byref(d), 1, ctypes.byref(t1)) == 0
    assert L.fns_hip_dense_ffn_workspace(ctypes.byref(d), 4, ctypes.byref(t4)) == 0
    assert 0 < t1.value < t4.value and t4.value >= 4 * 4 * (2 * 2048 + 2 * 6144)
    ws = ctypes.create_string_buffer(t1.value)
    assert L.fns_hip_dense_ffn(ctypes.byref(d), ptr, ptr, 1, ctypes.addressof(ws), t1.value - 1, None) == -2
    d.inter = 6000  # not a multiple of 256
    assert L.fns_hip_dense_ffn(ctypes.byref(d), ptr, ptr, 1, ctypes.addressof(ws), t1.value, None) == -2
    d.inter, d.down = 6144, None
    assert L.fns_hip_dense_ffn_prefill(ctypes.byref(d), ptr, ptr, 1, ctypes.addressof(ws), t1.value, None) == -2
    d.down, d.gate_type = ptr, 10  # Q2_K: no GEMV kernel
    assert L.fns_hip_dense_ffn(ctypes.byref(d), ptr, ptr, 1, ctypes.addressof(ws), t1.value, None) == -1
    assert L.fns_hip_dense_ffn(ctypes.byref(d), ptr, ptr, 0, None, 0, None) == 0  # no tokens: no-op
