"""ctypes binding of the CPU oracle (libfns_oracle.so) - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module. It is the checker: the
product path (flintnsteel_amd, libfns_hip.so) never imports or calls it.

The C sources (fns_oracle.c) restate the reference's MoE FFN path; each function there cites the reference
file:line it follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libfns_oracle.so"

Q8_0, Q8_1, Q3_K, Q4_K, Q5_K, Q6_K = 8, 9, 11, 12, 13, 14
IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS = 18, 21, 22, 23
TYPE_NAMES = {Q8_0: "Q8_0", Q8_1: "Q8_1", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K",
              IQ3_XXS: "IQ3_XXS", IQ3_S: "IQ3_S", IQ2_S: "IQ2_S", IQ4_XS: "IQ4_XS"}
BLOCK_BYTES = {Q8_0: 34, Q8_1: 36, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210,
               IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82, IQ4_XS: 136}
BLOCK_ELEMS = {Q8_0: 32, Q8_1: 32, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256,
               IQ3_XXS: 256, IQ3_S: 256, IQ2_S: 256, IQ4_XS: 256}


def build() -> None:
    """Compile libfns_oracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P, I64, I, SZ, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t, ctypes.c_float
        sigs = {
            "or_f32_to_f16": (ctypes.c_uint16, [F]),
            "or_f16_to_f32": (F, [ctypes.c_uint16]),
            "or_expf": (F, [F]),
            "or_row_bytes": (SZ, [I, I64]),
            "or_quantize": (I, [I, P, P, I64, I64, I]),
            "or_dequantize": (I, [I, P, P, I64, I64]),
            "or_q8_1_row_bytes": (SZ, [I64]),
            "or_quantize_q8_1": (None, [P, P, I64, I64]),
            "or_dequantize_q8_1": (None, [P, P, I64, I64]),
            "or_router_f32": (None, [P, P, P, I64, I64, I64]),
            "or_route_topk": (I, [P, P, P, P, P, I, I, I, I, I]),
            "or_mmvq_experts": (I, [I, P, I64, I64, P, I64, I64, P, I64, P]),
            "or_swiglu": (None, [P, P, P, I64]),
            "or_amax_guard_scale": (F, [P, I64]),
            "or_moe_combine": (None, [P, P, P, P, P, P, I64, I, I64]),
            "or_compact_ids": (I, [P, I64, I, I, I, P, P, P]),
            "or_cpu_moe_layer": (I, [I, I, P, P, SZ, SZ, SZ, P, P, I64, I64, I, I, I]),
            "or_set_iq_grids": (None, [P, P, P]),
            "or_is_iq": (I, [I]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def set_iq_grids(iq3xxs: np.ndarray, iq3s: np.ndarray, iq2s: np.ndarray) -> None:
    """Registers the IQ3_XXS / IQ3_S / IQ2_S codebooks (uint32 [256], uint32 [512], uint64 [1024])."""
    a, b, c = (np.ascontiguousarray(iq3xxs, np.uint32), np.ascontiguousarray(iq3s, np.uint32),
               np.ascontiguousarray(iq2s, np.uint64))
    assert a.shape == (256,) and b.shape == (512,) and c.shape == (1024,)
    lib().or_set_iq_grids(_p(a), _p(b), _p(c))


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def row_bytes(qtype: int, ncols: int) -> int:
    return BLOCK_BYTES[qtype] * ncols // BLOCK_ELEMS[qtype]


def quantize(qtype: int, x: np.ndarray, nthreads: int | None = None) -> np.ndarray:
    """x float32 [..., ncols] -> uint8 [..., row_bytes] in ggml block format (ggml reference quantisers)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    ncols = x.shape[-1]
    nrows = x.size // ncols
    out = np.empty(x.shape[:-1] + (row_bytes(qtype, ncols),), dtype=np.uint8)
    rc = lib().or_quantize(qtype, _p(x), _p(out), nrows, ncols, nthreads or os.cpu_count() or 1)
    if rc:
        raise ValueError(f"or_quantize: bad type/shape {qtype} {x.shape}")
    return out


def dequantize(qtype: int, q: np.ndarray, ncols: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    nrows = q.size // row_bytes(qtype, ncols)
    out = np.empty(q.shape[:-1] + (ncols,), dtype=np.float64)
    if lib().or_dequantize(qtype, _p(q), _p(out), nrows, ncols):
        raise ValueError("or_dequantize: bad type/shape")
    return out


def q8_1_row_bytes(ncols: int) -> int:
    return int(lib().or_q8_1_row_bytes(ncols))


def quantize_q8_1(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    ncols = x.shape[-1]
    nrows = x.size // ncols
    out = np.zeros(x.shape[:-1] + (q8_1_row_bytes(ncols),), dtype=np.uint8)
    lib().or_quantize_q8_1(_p(x), _p(out), ncols, nrows)
    return out


def dequantize_q8_1(xq: np.ndarray, ncols: int) -> np.ndarray:
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    nrows = xq.size // q8_1_row_bytes(ncols)
    out = np.empty(xq.shape[:-1] + (ncols,), dtype=np.float64)
    lib().or_dequantize_q8_1(_p(xq), _p(out), ncols, nrows)
    return out


def router_f32(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, w.shape[1])
    out = np.empty((x.shape[0], w.shape[0]), dtype=np.float32)
    lib().or_router_f32(_p(w), _p(x), _p(out), w.shape[1], w.shape[0], x.shape[0])
    return out


def route_topk(logits: np.ndarray, k: int, gating: int = 0, norm: bool = True):
    """-> ids int32 [T][k], w float32 [T][k], probs float32 [T][NE], logit margin float32 [T]."""
    logits = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1, logits.shape[-1])
    T, NE = logits.shape
    ids = np.empty((T, k), dtype=np.int32)
    w = np.empty((T, k), dtype=np.float32)
    probs = np.empty((T, NE), dtype=np.float32)
    margin = np.empty(T, dtype=np.float32)
    if lib().or_route_topk(_p(logits), _p(ids), _p(w), _p(probs), _p(margin), NE, k, T, gating, int(norm)):
        raise ValueError("or_route_topk: bad shape")
    return ids, w, probs, margin


def mmvq_experts(qtype: int, mats: list[np.ndarray], ncols: int, nrows: int, xq: np.ndarray, n_xq: int, x_div: int,
                 ids: np.ndarray) -> np.ndarray:
    """float64 dst [n_ids][nrows]; mats[e] is expert e's matrix bytes [nrows][row_bytes]."""
    ids = np.ascontiguousarray(ids, dtype=np.int32).ravel()
    mats = [np.ascontiguousarray(m, dtype=np.uint8) for m in mats]
    table = (ctypes.c_void_p * len(mats))(*[m.ctypes.data for m in mats])
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    dst = np.empty((ids.size, nrows), dtype=np.float64)
    if lib().or_mmvq_experts(qtype, ctypes.cast(table, ctypes.c_void_p), ncols, nrows, _p(xq), n_xq, x_div, _p(ids),
                             ids.size, _p(dst)):
        raise ValueError("or_mmvq_experts: bad arguments")
    return dst


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(gate, dtype=np.float64)
    u = np.ascontiguousarray(up, dtype=np.float64)
    out = np.empty_like(g)
    lib().or_swiglu(_p(g), _p(u), _p(out), g.size)
    return out


def amax_guard_scale(row: np.ndarray) -> float:
    r = np.ascontiguousarray(row, dtype=np.float32)
    return float(lib().or_amax_guard_scale(_p(r), r.size))


def moe_combine(dexp: np.ndarray, w: np.ndarray, escale=None, sh=None, x=None) -> np.ndarray:
    """dexp float32 [T][k][n], w [T][k] -> out [T][n] in the reference's slot order."""
    dexp = np.ascontiguousarray(dexp, dtype=np.float32)
    T, k, n = dexp.shape
    w = np.ascontiguousarray(w, dtype=np.float32)
    e = None if escale is None else np.ascontiguousarray(escale, dtype=np.float32)
    s = None if sh is None else np.ascontiguousarray(sh, dtype=np.float32)
    xx = None if x is None else np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty((T, n), dtype=np.float32)
    lib().or_moe_combine(_p(dexp), _p(e), _p(w), _p(s), _p(xx), _p(out), n, k, T)
    return out


def compact_ids(ids: np.ndarray, n_expert: int, x_rows_per_tok: int = 1):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, k = ids.shape
    bounds = np.empty(n_expert + 1, dtype=np.int32)
    src = np.empty(T * k, dtype=np.int32)
    dst = np.empty(T * k, dtype=np.int32)
    n = lib().or_compact_ids(_p(ids), T, k, n_expert, x_rows_per_tok, _p(bounds), _p(src), _p(dst))
    if n < 0:
        raise ValueError("or_compact_ids: expert id out of range")
    return bounds, src, dst, n


def cpu_moe_layer(gu_type: int, down_type: int, router_w: np.ndarray, slots: list[np.ndarray], gate_off: int,
                  up_off: int, down_off: int, x: np.ndarray, hidden: int, inter: int, k: int, nthreads: int) -> np.ndarray:
    """The CPU baseline (not ggml): one batch-1 layer; slots[e] = bytes [gate | up | down] of expert e."""
    router_w = np.ascontiguousarray(router_w, dtype=np.float32)
    table = (ctypes.c_void_p * len(slots))(*[s.ctypes.data for s in slots])
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(hidden, dtype=np.float32)
    rc = lib().or_cpu_moe_layer(gu_type, down_type, _p(router_w), ctypes.cast(table, ctypes.c_void_p), gate_off,
                                up_off, down_off, _p(x), _p(out), hidden, inter, len(slots), k, nthreads)
    if rc:
        raise ValueError("or_cpu_moe_layer: bad arguments")
    return out
