"""Loader for libfns_hip.so, the HIP (gfx950) implementation of the MoE FFN hot path.

The library is built in-tree by ``__graft_entry__.build()`` (``make -C flintnsteel_amd/csrc``). There is no fallback:
if the library is missing or fails to load, every entry point raises, so a GPU run can never silently take another
path.
"""
from __future__ import annotations

import ctypes
import re
import os
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ["FNS_HIP_LIB"]) if os.environ.get("FNS_HIP_LIB") else PKG_DIR / "libfns_hip.so"
HEADER = PKG_DIR.parent / "include" / "fns_hip.h"


class FnsError(RuntimeError):
    """A libfns_hip entry point returned a non-zero status."""


_P, _I64, _I, _SZ, _F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t, ctypes.c_float

# argtypes of every exported entry point (all return int status unless listed in _RESTYPE).
SIGNATURES: dict[str, list] = {
    "fns_hip_abi_version": [],
    "fns_hip_last_error": [],
    "fns_hip_q8_1_row_bytes": [_I64],
    "fns_hip_quantize_q8_1": [_P, _P, _I64, _I64, _P],
    "fns_hip_mmvq": [_I, _P, _I64, _I64, _P, _P, _I64, _P],
    "fns_hip_mmvq_ids": [_I, _P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _P],
    "fns_hip_mmvq_swiglu": [_I, _P, _P, _I64, _I64, _P, _P, _P],
    "fns_hip_mmvq_ids_swiglu_shared": [_I, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _P, _P, _P],
    "fns_hip_mmvq_experts_swiglu": [_I, _P, _SZ, _SZ, _I64, _I64, _P, _I64, _P, _I64, _P, _P],
    "fns_hip_mmvq_experts": [_I, _P, _SZ, _I64, _I64, _P, _I64, _P, _I64, _P, _P],
    "fns_hip_mmvq_supports": [_I],
    "fns_hip_set_iq_grids": [_P, _P, _P],
    "fns_hip_rms_norm_q8_1": [_P, _P, _P, _P, _I, _F, _I, _P],
    "fns_hip_gemv_router": [_I, _P, _P, _P, _I, _I, _I, _P],
    "fns_hip_gemm_router": [_I, _P, _P, _P, _I, _I, _I, _P],
    "fns_hip_route_topk": [_P, _P, _P, _I, _I, _I, _I, _I, _P],
    "fns_hip_count_routes": [_P, _P, _I, _P],
    "fns_hip_swiglu": [_P, _P, _P, _I, _I, _P],
    "fns_hip_glu_mmvq": [_P, _P, _P, _I, _P],
    "fns_hip_amax_guard": [_P, _P, _I, _I, _P],
    "fns_hip_amax_guard_q8_1": [_P, _P, _P, _I, _I, _P],
    "fns_hip_moe_combine": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "fns_hip_moe_workspace_layout": [_P, _I, _P, _P],
    "fns_hip_moe_layer": [_P, _P, _P, _P, _I, _P, _SZ, _P],
    "fns_hip_moe_layer_profiled": [_P, _P, _P, _P, _I, _P, _SZ, _P, _P],
    "fns_hip_moe_layer_stage": [_P, _I, _P, _P, _P, _I, _P, _SZ, _P],
    "fns_hip_moe_layer_noalloc": [_P, _P, _P, _P, _I, _P],
    "fns_hip_moe_noalloc_max_bytes": [],
    "fns_hip_moe_layer_status": [_P, _I, _P, _I, _P, _P],
    "fns_hip_moe_layer_status_collect": [_P, _I, _P, _P, _P],
    "fns_hip_moe_set_test_hooks": [_I, _I],
    "fns_hip_moe_set_path": [_I],
    "fns_hip_moe_layer_kernels": [_P, _I, _P],
    "fns_hip_mmq_q8_1_bytes": [_I64, _I64],
    "fns_hip_mmq_bounds_bytes": [_I64],
    "fns_hip_mmq": [_I, _P, _I64, _I64, _P, _I64, _P, _P, _P],
    "fns_hip_mmq_experts": [_I, _P, _SZ, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _P, _P, _P, _P, _P],
    "fns_hip_mmq_compact": [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _P],
    "fns_hip_moe_prefill_workspace": [_P, _I64, _P, _P],
    "fns_hip_moe_prefill_section": [_P, _I64, _I, _P, _P],
    "fns_hip_moe_prefill": [_P, _P, _P, _P, _I64, _P, _SZ, _P],
    "fns_hip_moe_prefill_status": [_P, _I64, _P, _I, _P, _P],
    "fns_hip_moe_prefill_status_collect": [_P, _I64, _P, _P, _P],
    "fns_hip_fill_normal": [_P, _I64, ctypes.c_uint64, ctypes.c_uint64, _F, _F, _P],
    "fns_hip_quantize_weights": [_I, _P, _P, _I64, _I64, _P],
    "fns_hip_selftest_lanes": [_P, _P],
    "fns_hip_gguf_open": [ctypes.c_char_p, _P],
    "fns_hip_gguf_close": [_P],
    "fns_hip_gguf_info": [_P, _P, _P, _P, _P],
    "fns_hip_gguf_tensor": [_P, ctypes.c_char_p, _P],
    "fns_hip_gguf_tensor_at": [_P, _I64, _P, _P],
    "fns_hip_gguf_get_u32": [_P, ctypes.c_char_p, _P],
    "fns_hip_gguf_get_f32": [_P, ctypes.c_char_p, _P],
    "fns_hip_gguf_get_bool": [_P, ctypes.c_char_p, _P],
    "fns_hip_gguf_get_str": [_P, ctypes.c_char_p, _P],
    "fns_hip_moe_layer_from_gguf": [_P, _I, _P, _P],
    "fns_hip_moe_resident_free": [_P],
    "fns_hip_add": [_P, _P, _P, _I64, _P],
    "fns_hip_dense_ffn_workspace": [_P, _I64, _P],
    "fns_hip_dense_ffn": [_P, _P, _P, _I64, _P, _SZ, _P],
    "fns_hip_dense_ffn_prefill": [_P, _P, _P, _I64, _P, _SZ, _P],
    "fns_hip_dense_ffn_from_gguf": [_P, _I, _P, _P],
    "fns_hip_dense_resident_free": [_P],
}
_RESTYPE = {
    "fns_hip_last_error": ctypes.c_char_p,
    "fns_hip_q8_1_row_bytes": _SZ,
    "fns_hip_mmq_q8_1_bytes": _SZ,
    "fns_hip_mmq_bounds_bytes": _SZ,
    "fns_hip_moe_noalloc_max_bytes": _SZ,
    "fns_hip_gguf_close": None,
    "fns_hip_moe_resident_free": None,
    "fns_hip_dense_resident_free": None,
}

_lib = None


def header_symbols() -> list[str]:
    """Function names declared in include/fns_hip.h."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(fns_hip_\w+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FnsError(f"{LIB_PATH} is not built: run __graft_entry__.build() (make -C flintnsteel_amd/csrc)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, _I)
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().fns_hip_last_error()
        raise FnsError(f"{what} failed ({rc}): {msg.decode() if msg else ''}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
