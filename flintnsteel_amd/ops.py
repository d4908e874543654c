"""PyTorch-facing wrappers of libfns_hip.so (device memory and streams come from torch; the compute is the HIP
library's). Names, argument meaning and error behaviour follow the reference's kernel-launch API
(reference include/fns/ggml_kernels.h, src/kernels.cuh): a bad type or shape raises FnsError where the reference
aborts. All tensors are CUDA (HIP) tensors; launches go on torch's current stream.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import call, lib

Q8_1, Q3_K, Q4_K, Q5_K, Q6_K = 9, 11, 12, 13, 14
F32, BF16 = 0, 30
GATING_SOFTMAX, GATING_SIGMOID = 0, 1
BLOCK_BYTES = {Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}
TYPE_NAMES = {Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}


def _p(t: torch.Tensor | None):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    return ctypes.c_void_p(t.data_ptr())


def _s():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def row_bytes(qtype: int, ncols: int) -> int:
    return BLOCK_BYTES[qtype] * (ncols // 256)


def q8_1_row_bytes(ncols: int) -> int:
    return int(lib().fns_hip_q8_1_row_bytes(ncols))


def _empty_f32(*shape, like: torch.Tensor) -> torch.Tensor:
    return torch.empty(*shape, dtype=torch.float32, device=like.device)


def quantize_q8_1(x: torch.Tensor, xq: torch.Tensor | None = None) -> torch.Tensor:
    x = x.contiguous()
    ncols = x.shape[-1]
    nrows = x.numel() // ncols
    if xq is None:
        xq = torch.zeros(nrows, q8_1_row_bytes(ncols), dtype=torch.uint8, device=x.device)
    call("fns_hip_quantize_q8_1", _p(x), _p(xq), ncols, nrows, _s())
    return xq


def mmvq(qtype: int, w: torch.Tensor, ncols: int, nrows: int, xq: torch.Tensor, n_cols: int,
         dst: torch.Tensor | None = None) -> torch.Tensor:
    dst = _empty_f32(n_cols, nrows, like=xq) if dst is None else dst
    call("fns_hip_mmvq", qtype, _p(w), ncols, nrows, _p(xq), _p(dst), n_cols, _s())
    return dst


def mmvq_ids(qtype: int, w: torch.Tensor, ncols: int, nrows: int, n_mats: int, xq: torch.Tensor, n_xq: int,
             ids: torch.Tensor, dst: torch.Tensor | None = None) -> torch.Tensor:
    n_ids = ids.numel()
    dst = _empty_f32(n_ids, nrows, like=xq) if dst is None else dst
    call("fns_hip_mmvq_ids", qtype, _p(w), ncols, nrows, n_mats, _p(xq), n_xq, _p(ids), n_ids, _p(dst), _s())
    return dst


def mmvq_swiglu(qtype: int, w_gate: torch.Tensor, w_up: torch.Tensor, ncols: int, nrows: int, xq: torch.Tensor,
                dst: torch.Tensor | None = None) -> torch.Tensor:
    dst = _empty_f32(nrows, like=xq) if dst is None else dst
    call("fns_hip_mmvq_swiglu", qtype, _p(w_gate), _p(w_up), ncols, nrows, _p(xq), _p(dst), _s())
    return dst


def mmvq_ids_swiglu_shared(qtype: int, w_gate: torch.Tensor, w_up: torch.Tensor, ncols: int, nrows: int, n_mats: int,
                           xq: torch.Tensor, ids: torch.Tensor, sh_gate: torch.Tensor | None = None,
                           sh_up: torch.Tensor | None = None):
    n_ids = ids.numel()
    dst = _empty_f32(n_ids, nrows, like=xq)
    sh_dst = _empty_f32(nrows, like=xq) if sh_gate is not None else None
    call("fns_hip_mmvq_ids_swiglu_shared", qtype, _p(w_gate), _p(w_up), ncols, nrows, n_mats, _p(xq), _p(ids), n_ids,
         _p(dst), _p(sh_gate), _p(sh_up), _p(sh_dst), _s())
    return dst, sh_dst


def mmvq_experts_swiglu(qtype: int, table: torch.Tensor, gate_off: int, up_off: int, ncols: int, nrows: int,
                        xq: torch.Tensor, n_xq: int, ids: torch.Tensor, dst: torch.Tensor | None = None):
    n_ids = ids.numel()
    dst = _empty_f32(n_ids, nrows, like=xq) if dst is None else dst
    call("fns_hip_mmvq_experts_swiglu", qtype, _p(table), gate_off, up_off, ncols, nrows, _p(xq), n_xq, _p(ids),
         n_ids, _p(dst), _s())
    return dst


def mmvq_experts(qtype: int, table: torch.Tensor, off: int, ncols: int, nrows: int, xq: torch.Tensor, n_xq: int,
                 ids: torch.Tensor, dst: torch.Tensor | None = None):
    n_ids = ids.numel()
    dst = _empty_f32(n_ids, nrows, like=xq) if dst is None else dst
    call("fns_hip_mmvq_experts", qtype, _p(table), off, ncols, nrows, _p(xq), n_xq, _p(ids), n_ids, _p(dst), _s())
    return dst


def mmvq_supports(qtype: int) -> bool:
    return bool(lib().fns_hip_mmvq_supports(qtype))


def rms_norm_q8_1(x: torch.Tensor, w: torch.Tensor, eps: float):
    x = x.contiguous()
    n = x.shape[-1]
    rows = x.numel() // n
    out = torch.empty_like(x)
    xq = torch.zeros(rows, q8_1_row_bytes(n), dtype=torch.uint8, device=x.device)
    call("fns_hip_rms_norm_q8_1", _p(x), _p(w), _p(out), _p(xq), n, ctypes.c_float(eps), rows, _s())
    return out, xq


def _dtype_code(w: torch.Tensor) -> int:
    if w.dtype == torch.float32:
        return F32
    if w.dtype == torch.bfloat16:
        return BF16
    raise ValueError(f"router dtype {w.dtype} not supported")


def gemv_router(w: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    nrows, ncols = w.shape
    x = x.contiguous().view(-1, ncols)
    y = _empty_f32(x.shape[0], nrows, like=x)
    call("fns_hip_gemv_router", _dtype_code(w), _p(w), _p(x), _p(y), ncols, nrows, x.shape[0], _s())
    return y


def gemm_router(w: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    nrows, ncols = w.shape
    x = x.contiguous().view(-1, ncols)
    y = _empty_f32(x.shape[0], nrows, like=x)
    call("fns_hip_gemm_router", _dtype_code(w), _p(w), _p(x), _p(y), ncols, nrows, x.shape[0], _s())
    return y


def route_topk(logits: torch.Tensor, k: int, gating: int = GATING_SOFTMAX, norm: bool = True):
    logits = logits.contiguous()
    n_expert = logits.shape[-1]
    n_tok = logits.numel() // n_expert
    ids = torch.empty(n_tok, k, dtype=torch.int32, device=logits.device)
    w = _empty_f32(n_tok, k, like=logits)
    call("fns_hip_route_topk", _p(logits), _p(ids), _p(w), n_expert, k, n_tok, gating, int(norm), _s())
    return ids, w


def count_routes(ids: torch.Tensor, counts: torch.Tensor) -> None:
    call("fns_hip_count_routes", _p(ids), _p(counts), ids.numel(), _s())


def swiglu(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    n = g.shape[-1]
    act = torch.empty_like(g)
    call("fns_hip_swiglu", _p(g.contiguous()), _p(u.contiguous()), _p(act), n, g.numel() // n, _s())
    return act


def glu_mmvq(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    act = torch.empty_like(g)
    call("fns_hip_glu_mmvq", _p(g.contiguous()), _p(u.contiguous()), _p(act), g.numel(), _s())
    return act


def amax_guard(act: torch.Tensor) -> torch.Tensor:
    """In place: act[r] /= e_r; returns escale [rows]."""
    n = act.shape[-1]
    rows = act.numel() // n
    escale = _empty_f32(rows, like=act)
    call("fns_hip_amax_guard", _p(act), _p(escale), n, rows, _s())
    return escale


def amax_guard_q8_1(act: torch.Tensor):
    n = act.shape[-1]
    rows = act.numel() // n
    escale = _empty_f32(rows, like=act)
    xq = torch.zeros(rows, q8_1_row_bytes(n), dtype=torch.uint8, device=act.device)
    call("fns_hip_amax_guard_q8_1", _p(act.contiguous()), _p(escale), _p(xq), n, rows, _s())
    return escale, xq


def moe_combine(dexp: torch.Tensor, w: torch.Tensor, escale=None, sh=None, x=None, out=None) -> torch.Tensor:
    """dexp [T][k][n], w [T][k] -> out [T][n] = (sum_j (dexp_j * e_j) * w_j + sh) + x."""
    T, k, n = dexp.shape
    out = _empty_f32(T, n, like=dexp) if out is None else out
    call("fns_hip_moe_combine", _p(dexp.contiguous()), _p(escale), _p(w.contiguous()), _p(sh), _p(x), _p(out), n, k,
         T, _s())
    return out


class ExpertSlots:
    """Fully resident expert storage: expert e is one slot [gate | up | down] of raw GGUF blocks at
    base + e * slot_bytes (256-byte aligned), plus a device table of slot pointers - the reference engine's
    `exp_table` / `gate_bytes` / `up_bytes` contract (reference include/fns/engine.h:28-32, src/engine.cu:375-471),
    in the trivial case where every expert lives in HBM.
    """

    def __init__(self, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor, pad: int = 4096):
        # gate/up/down: uint8 [n_expert][bytes per expert matrix] (host or device)
        n = gate.shape[0]
        self.n_expert = n
        self.gate_bytes, self.up_bytes, self.down_bytes = gate.shape[1], up.shape[1], down.shape[1]
        raw = self.gate_bytes + self.up_bytes + self.down_bytes
        self.slot_bytes = (raw + 255) // 256 * 256
        self.gate_off, self.up_off, self.down_off = 0, self.gate_bytes, self.gate_bytes + self.up_bytes
        dev = torch.device("cuda")
        self.storage = torch.zeros(n * self.slot_bytes + pad, dtype=torch.uint8, device=dev)
        view = self.storage[: n * self.slot_bytes].view(n, self.slot_bytes)
        view[:, : self.gate_bytes].copy_(gate.to(dev))
        view[:, self.up_off: self.up_off + self.up_bytes].copy_(up.to(dev))
        view[:, self.down_off: self.down_off + self.down_bytes].copy_(down.to(dev))
        base = self.storage.data_ptr()
        self.table = torch.tensor([base + e * self.slot_bytes for e in range(n)], dtype=torch.int64, device=dev)
