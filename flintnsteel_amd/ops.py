"""PyTorch-facing wrappers of libfns_hip.so (device memory and streams come from torch; the compute is the HIP
library's). Names, argument meaning and error behaviour follow the reference's kernel-launch API
(reference include/fns/ggml_kernels.h, src/kernels.cuh): a bad type or shape raises FnsError where the reference
aborts. All tensors are CUDA (HIP) tensors; launches go on torch's current stream.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from ._lib import call, lib

Q8_0, Q8_1, Q3_K, Q4_K, Q5_K, Q6_K = 8, 9, 11, 12, 13, 14
IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS = 18, 21, 22, 23
F32, BF16 = 0, 30
GATING_SOFTMAX, GATING_SIGMOID = 0, 1
STATUS_EXCHANGE_TIMEOUT = 1  # FNS_STATUS_EXCHANGE_TIMEOUT
# bytes per 256 values of a row (a K-quant block; 8 Q8_0 blocks)
BLOCK_BYTES = {Q8_0: 272, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82, IQ4_XS: 136}
TYPE_NAMES = {Q8_0: "Q8_0", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", IQ3_XXS: "IQ3_XXS",
              IQ3_S: "IQ3_S", IQ2_S: "IQ2_S", IQ4_XS: "IQ4_XS"}


def _status_dst(t: torch.Tensor):
    """Pointer of a status collect's destination: a device tensor or pinned host memory of at least 4 bytes."""
    if t.numel() * t.element_size() < 4 or not (t.is_cuda or t.is_pinned()):
        raise ValueError("status destination: a device or pinned host tensor of at least 4 bytes")
    return ctypes.c_void_p(t.data_ptr())


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
                           sh_up: torch.Tensor | None = None, dst: torch.Tensor | None = None,
                           sh_dst: torch.Tensor | None = None):
    n_ids = ids.numel()
    dst = _empty_f32(n_ids, nrows, like=xq) if dst is None else dst
    if sh_gate is not None and sh_dst is None:
        sh_dst = _empty_f32(nrows, like=xq)
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
    in the trivial case where every expert lives in HBM. `pad` bytes of zeros follow the last slot
    (reference src/engine.cu:42-45).
    """

    def __init__(self, n_expert: int, gate_bytes: int, up_bytes: int, down_bytes: int, pad: int = 4096):
        self.n_expert = n_expert
        self.gate_bytes, self.up_bytes, self.down_bytes = gate_bytes, up_bytes, down_bytes
        raw = gate_bytes + up_bytes + down_bytes
        self.slot_bytes = (raw + 255) // 256 * 256
        self.gate_off, self.up_off, self.down_off = 0, gate_bytes, gate_bytes + up_bytes
        self.storage = torch.zeros(n_expert * self.slot_bytes + pad, dtype=torch.uint8, device="cuda")
        base = self.storage.data_ptr()
        self.table = torch.tensor([base + e * self.slot_bytes for e in range(n_expert)], dtype=torch.int64,
                                  device="cuda")

    @classmethod
    def from_tensors(cls, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor, pad: int = 4096):
        """gate/up/down: uint8 [n_expert][bytes of one expert matrix] (host or device)."""
        s = cls(gate.shape[0], gate.shape[1], up.shape[1], down.shape[1], pad)
        for name, t in (("gate", gate), ("up", up), ("down", down)):
            s.view(name).copy_(t.to("cuda"))
        return s

    def view(self, name: str) -> torch.Tensor:
        """[n_expert][bytes] strided view of one matrix kind inside the slots."""
        off = {"gate": self.gate_off, "up": self.up_off, "down": self.down_off}[name]
        size = {"gate": self.gate_bytes, "up": self.up_bytes, "down": self.down_bytes}[name]
        slots = self.storage[: self.n_expert * self.slot_bytes].view(self.n_expert, self.slot_bytes)
        return slots[:, off: off + size]

    def expert_bytes(self, e: int) -> torch.Tensor:
        return self.storage[e * self.slot_bytes: (e + 1) * self.slot_bytes]


class MoeLayerDesc(ctypes.Structure):
    """Mirror of FnsMoeLayer (include/fns_hip.h)."""
    _fields_ = [
        ("hidden", ctypes.c_int), ("inter", ctypes.c_int), ("n_expert", ctypes.c_int), ("k", ctypes.c_int),
        ("gating", ctypes.c_int), ("norm_w", ctypes.c_int), ("guard", ctypes.c_int),
        ("router_dtype", ctypes.c_int), ("router_w", ctypes.c_void_p),
        ("gu_type", ctypes.c_int), ("down_type", ctypes.c_int),
        ("table", ctypes.c_void_p), ("gate_off", ctypes.c_size_t), ("up_off", ctypes.c_size_t),
        ("down_off", ctypes.c_size_t), ("router_bias", ctypes.c_void_p),
        ("ffn_norm", ctypes.c_void_p), ("norm_eps", ctypes.c_float), ("shexp_inter", ctypes.c_int),
        ("shexp_gu_type", ctypes.c_int), ("shexp_down_type", ctypes.c_int),
        ("shexp_gate", ctypes.c_void_p), ("shexp_up", ctypes.c_void_p), ("shexp_down", ctypes.c_void_p),
        ("prefetch", ctypes.c_void_p), ("prefetch_bytes", ctypes.c_size_t),
    ]


WS_SECTIONS = ("logits", "xq", "ids", "w", "act", "escale")

PATH_AUTO, PATH_THREE_KERNELS = 0, 1


class decode_path:
    """Context manager (test hook fns_hip_moe_set_path): restricts the decode path of the calls inside it."""

    def __init__(self, path: int):
        self.path = path

    def __enter__(self):
        call("fns_hip_moe_set_path", self.path)
        return self

    def __exit__(self, *exc):
        call("fns_hip_moe_set_path", PATH_AUTO)
        return False


class MoeLayer:
    """One MoE FFN layer resident in HBM: fp32/bf16 router + expert slots, run by fns_hip_moe_layer."""

    def __init__(self, router_w: torch.Tensor, slots: ExpertSlots, gu_type: int, down_type: int, hidden: int,
                 inter: int, k: int, gating: int = GATING_SOFTMAX, norm: bool = True, guard: bool = False,
                 router_bias: torch.Tensor | None = None, ffn_norm: torch.Tensor | None = None,
                 norm_eps: float = 1e-6, shexp: dict | None = None):
        """shexp: the shared expert, {"gate", "up", "down": uint8 block tensors, "inter": width, "gu_type",
        "down_type"} (the reference's gate_shexp / up_shexp / down_shexp); ffn_norm: f32 [hidden] RMSNorm weights."""
        self.router_w, self.slots, self.router_bias = router_w, slots, router_bias
        self.ffn_norm, self.shexp = ffn_norm, shexp
        sh = shexp or {}
        self.desc = MoeLayerDesc(hidden, inter, slots.n_expert, k, gating, int(norm), int(guard),
                                 _dtype_code(router_w), router_w.data_ptr(), gu_type, down_type,
                                 slots.table.data_ptr(), slots.gate_off, slots.up_off, slots.down_off,
                                 router_bias.data_ptr() if router_bias is not None else None,
                                 ffn_norm.data_ptr() if ffn_norm is not None else None, norm_eps,
                                 sh.get("inter", 0), sh.get("gu_type", 0), sh.get("down_type", 0),
                                 sh["gate"].data_ptr() if sh else None, sh["up"].data_ptr() if sh else None,
                                 sh["down"].data_ptr() if sh else None)

    @classmethod
    def from_gguf(cls, file: "GgufFile", layer: int) -> "MoeLayer":
        """MoE layer `layer` of a GGUF checkpoint made resident in HBM by fns_hip_moe_layer_from_gguf (expert slots,
        table, router, norm and shared expert in library-owned device memory, freed with this object)."""
        obj = cls.__new__(cls)
        obj.desc = MoeLayerDesc()
        obj.router_w = obj.slots = obj.router_bias = obj.ffn_norm = obj.shexp = None
        obj._file = file  # the metadata stays readable while the layer lives
        res = ctypes.c_void_p()
        call("fns_hip_moe_layer_from_gguf", file.handle, layer, ctypes.byref(res), ctypes.byref(obj.desc))
        obj._resident = res
        return obj

    def __del__(self):
        res = getattr(self, "_resident", None)
        if res:
            lib().fns_hip_moe_resident_free(res)
            self._resident = None

    def workspace_layout(self, n_tok: int):
        offs = (ctypes.c_size_t * 6)()
        total = ctypes.c_size_t()
        call("fns_hip_moe_workspace_layout", ctypes.byref(self.desc), n_tok, offs, ctypes.byref(total))
        return list(offs), total.value

    def workspace(self, n_tok: int) -> torch.Tensor:
        _, total = self.workspace_layout(n_tok)
        return torch.zeros(total, dtype=torch.uint8, device="cuda")

    def __call__(self, x: torch.Tensor, out: torch.Tensor | None = None, ws: torch.Tensor | None = None,
                 x_resid: torch.Tensor | None = None) -> torch.Tensor:
        x = x.contiguous()
        n_tok = x.numel() // self.desc.hidden
        out = torch.empty_like(x) if out is None else out
        ws = self.workspace(n_tok) if ws is None else ws
        call("fns_hip_moe_layer", ctypes.byref(self.desc), _p(x), _p(x_resid), _p(out), n_tok, _p(ws), ws.numel(), _s())
        return out

    def status(self, ws: torch.Tensor | None, n_tok: int = 1, clear: bool = False) -> int:
        """The workspace's sticky status word (FNS_STATUS_* bits; 0: every call so far completed its exchange)."""
        st = ctypes.c_uint32()
        call("fns_hip_moe_layer_status", ctypes.byref(self.desc), n_tok, _p(ws), int(clear), ctypes.byref(st), _s())
        return st.value

    def status_collect(self, ws: torch.Tensor | None, dst: torch.Tensor, n_tok: int = 1) -> None:
        """Enqueues the graph-capturable collect (fns_hip_moe_layer_status_collect): a non-zero status word is ORed
        into dst[0] (a uint32-sized tensor, device or pinned host) and cleared."""
        call("fns_hip_moe_layer_status_collect", ctypes.byref(self.desc), n_tok, _p(ws), _status_dst(dst), _s())

    def kernels(self, n_tok: int = 1) -> int:
        """Kernels one call at n_tok tokens launches on the current device: 2 (router + fused layer) or 3 (router,
        gate/up, down)."""
        k = ctypes.c_int()
        call("fns_hip_moe_layer_kernels", ctypes.byref(self.desc), n_tok, ctypes.byref(k))
        return k.value

    def stage(self, stage: int, x: torch.Tensor, out: torch.Tensor, ws: torch.Tensor,
              x_resid: torch.Tensor | None = None) -> None:
        """Launch one of the layer's three kernels (0 router, 1 gate/up, 2 down + combine)."""
        n_tok = x.numel() // self.desc.hidden
        call("fns_hip_moe_layer_stage", ctypes.byref(self.desc), stage, _p(x), _p(x_resid), _p(out), n_tok, _p(ws),
             ws.numel(), _s())

    def profiled(self, x: torch.Tensor, out: torch.Tensor, ws: torch.Tensor, events) -> None:
        """Full layer with torch.cuda.Event markers before each kernel and after the last (4 events, recorded)."""
        n_tok = x.numel() // self.desc.hidden
        arr = (ctypes.c_void_p * 4)(*[e.cuda_event for e in events])
        call("fns_hip_moe_layer_profiled", ctypes.byref(self.desc), _p(x), None, _p(out), n_tok, _p(ws), ws.numel(),
             arr, _s())

    def trace(self, ws: torch.Tensor, n_tok: int) -> dict:
        """Views of the intermediates a call left in its workspace."""
        offs, _ = self.workspace_layout(n_tok)
        d = self.desc
        sizes = {"logits": (torch.float32, (n_tok, d.n_expert)), "xq": (torch.uint8, (n_tok, q8_1_row_bytes(d.hidden))),
                 "ids": (torch.int32, (n_tok, d.k)), "w": (torch.float32, (n_tok, d.k)),
                 "act": (torch.float32, (n_tok * d.k, d.inter)), "escale": (torch.float32, (n_tok * d.k,))}
        out = {}
        for name, off in zip(WS_SECTIONS, offs):
            dt, shape = sizes[name]
            n = int(np.prod(shape)) * torch.tensor([], dtype=dt).element_size()
            out[name] = ws[off:off + n].view(dt).view(*shape)
        return out


PREFILL_SECTIONS = ("logits", "ids", "w", "xpack", "apack", "dexp")


class MoePrefill:
    """Prefill (batched) form of a MoeLayer: fns_hip_moe_prefill over n_tok tokens."""

    def __init__(self, layer: MoeLayer):
        self.layer = layer

    def workspace_layout(self, n_tok: int):
        offs = (ctypes.c_size_t * 6)()
        total = ctypes.c_size_t()
        call("fns_hip_moe_prefill_workspace", ctypes.byref(self.layer.desc), n_tok, offs, ctypes.byref(total))
        return list(offs), total.value

    def workspace(self, n_tok: int) -> torch.Tensor:
        return torch.zeros(self.workspace_layout(n_tok)[1], dtype=torch.uint8, device="cuda")

    def __call__(self, x: torch.Tensor, out: torch.Tensor | None = None, ws: torch.Tensor | None = None,
                 x_resid: torch.Tensor | None = None) -> torch.Tensor:
        x = x.contiguous()
        n_tok = x.numel() // self.layer.desc.hidden
        out = torch.empty_like(x) if out is None else out
        ws = self.workspace(n_tok) if ws is None else ws
        call("fns_hip_moe_prefill", ctypes.byref(self.layer.desc), _p(x), _p(x_resid), _p(out), n_tok, _p(ws),
             ws.numel(), _s())
        return out

    def status(self, ws: torch.Tensor, n_tok: int, clear: bool = False) -> int:
        """The workspace's sticky status word (FNS_STATUS_* bits; 0: every fused gate/up + down wait so far completed)."""
        st = ctypes.c_uint32()
        call("fns_hip_moe_prefill_status", ctypes.byref(self.layer.desc), n_tok, _p(ws), int(clear), ctypes.byref(st),
             _s())
        return st.value

    def status_collect(self, ws: torch.Tensor, dst: torch.Tensor, n_tok: int) -> None:
        """Enqueues the graph-capturable collect (fns_hip_moe_prefill_status_collect) into dst[0]."""
        call("fns_hip_moe_prefill_status_collect", ctypes.byref(self.layer.desc), n_tok, _p(ws), _status_dst(dst),
             _s())

    def section(self, n_tok: int, index: int) -> tuple[int, int]:
        """(byte offset, bytes) of workspace section `index` (fns_hip_moe_prefill_section)."""
        off, size = ctypes.c_size_t(), ctypes.c_size_t()
        call("fns_hip_moe_prefill_section", ctypes.byref(self.layer.desc), n_tok, index, ctypes.byref(off),
             ctypes.byref(size))
        return off.value, size.value

    def trace(self, ws: torch.Tensor, n_tok: int) -> dict:
        """Views of the intermediates a call left in its workspace: logits, ids, w, dexp, the split activation images
        of x ("xpack", [n_tok][image bytes]) and act ("apack", [n_tok * k][image bytes], by (token, slot)), the guard
        scales ("escale") and, with the F16 guard, the f32 act rows after the division ("act")."""
        d = self.layer.desc
        P = n_tok * d.k
        spec = {"logits": (0, torch.float32, (n_tok, d.n_expert)), "ids": (1, torch.int32, (n_tok, d.k)),
                "w": (2, torch.float32, (n_tok, d.k)), "xpack": (3, torch.uint8, (n_tok, -1)),
                "apack": (4, torch.uint8, (P, -1)), "dexp": (5, torch.float32, (n_tok, d.k, d.hidden)),
                "act": (9, torch.float32, (P, d.inter)), "escale": (10, torch.float32, (P,))}
        out = {}
        for name, (idx, dt, shape) in spec.items():
            off, n = self.section(n_tok, idx)
            if n:
                out[name] = ws[off: off + n].view(dt).view(*shape)
        # image rows may be padded to whole cache lines: the views hold each row's image bytes only
        out["xpack"] = out["xpack"][:, : d.hidden // 256 * 1056]
        out["apack"] = out["apack"][:, : d.inter // 256 * 1056]
        return out


def mmq_q8_1_bytes(ncols: int, nrows: int) -> int:
    return int(lib().fns_hip_mmq_q8_1_bytes(ncols, nrows))


def mmq(qtype: int, w: torch.Tensor, ncols: int, nrows: int, x: torch.Tensor, xq: torch.Tensor | None = None,
        out: torch.Tensor | None = None) -> torch.Tensor:
    """dst [n_tok][nrows] = W . q8_1(x); xq: scratch of mmq_q8_1_bytes(ncols, n_tok) bytes (allocated if None)."""
    x = x.contiguous()
    n_tok = x.numel() // ncols
    if xq is None:
        xq = torch.zeros(mmq_q8_1_bytes(ncols, n_tok), dtype=torch.uint8, device=x.device)
    dst = _empty_f32(n_tok, nrows, like=x) if out is None else out
    call("fns_hip_mmq", qtype, _p(w), ncols, nrows, _p(x), n_tok, _p(xq), _p(dst), _s())
    return dst


def mmq_compact(ids: torch.Tensor, n_expert: int, x_rows_per_tok: int = 1):
    """-> (bounds [n_expert + 1], ids_src1, ids_dst) of the stable expert sort."""
    n_tok, k = ids.shape
    src = torch.empty(n_tok * k, dtype=torch.int32, device=ids.device)
    dst = torch.empty_like(src)
    bounds = torch.empty(int(lib().fns_hip_mmq_bounds_bytes(n_expert)) // 4, dtype=torch.int32, device=ids.device)
    call("fns_hip_mmq_compact", _p(ids.contiguous()), n_tok, k, n_expert, x_rows_per_tok, _p(src), _p(dst),
         _p(bounds), _s())
    return bounds[: n_expert + 1], src, dst


def mmq_experts(qtype: int, table: torch.Tensor, off: int, ncols: int, nrows: int, n_expert: int, x: torch.Tensor,
                x_rows_per_tok: int, ids: torch.Tensor) -> torch.Tensor:
    """dst [n_tok][n_used][nrows] = W_e . q8_1(x[t][j % x_rows_per_tok])."""
    n_tok, n_used = ids.shape
    x = x.contiguous()
    src = torch.empty(n_tok * n_used, dtype=torch.int32, device=x.device)
    dst_ids = torch.empty_like(src)
    bounds = torch.empty(n_expert + 1, dtype=torch.int32, device=x.device)   # the reference's MmqIdsScratch sizing
    xq = torch.zeros(mmq_q8_1_bytes(ncols, n_tok * x_rows_per_tok), dtype=torch.uint8, device=x.device)
    dst = _empty_f32(n_tok, n_used, nrows, like=x)
    call("fns_hip_mmq_experts", qtype, _p(table), off, ncols, nrows, n_expert, _p(x), x_rows_per_tok, n_tok,
         _p(ids.contiguous()), n_used, _p(src), _p(dst_ids), _p(bounds), _p(xq), _p(dst), _s())
    return dst


def fill_normal(out: torch.Tensor, seed: int, offset: int = 0, mean: float = 0.0, std: float = 1.0) -> torch.Tensor:
    call("fns_hip_fill_normal", _p(out), out.numel(), seed, offset, ctypes.c_float(mean), ctypes.c_float(std), _s())
    return out


def quantize_weights(qtype: int, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """x f32 [..., ncols] on the device -> uint8 [..., row_bytes] GGUF blocks (ggml reference quantisers)."""
    ncols = x.shape[-1]
    nrows = x.numel() // ncols
    if out is None:
        out = torch.empty(*x.shape[:-1], row_bytes(qtype, ncols), dtype=torch.uint8, device=x.device)
    call("fns_hip_quantize_weights", qtype, _p(x.contiguous()), _p(out), nrows, ncols, _s())
    return out


def selftest_lanes() -> int:
    """Bit mask of failing cross-lane exchange checks on the device (0 = all good)."""
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    call("fns_hip_selftest_lanes", _p(bad), _s())
    return int(bad.item())


def add(x: torch.Tensor, y: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """out = x + y (reference add_inplace, src/kernels.cuh:119); out may be x."""
    out = torch.empty_like(x) if out is None else out
    call("fns_hip_add", _p(x), _p(y), _p(out), x.numel(), _s())
    return out


class DenseFfnDesc(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("inter", ctypes.c_int), ("gate_type", ctypes.c_int),
                ("up_type", ctypes.c_int), ("down_type", ctypes.c_int), ("gate", ctypes.c_void_p),
                ("up", ctypes.c_void_p), ("down", ctypes.c_void_p), ("ffn_norm", ctypes.c_void_p),
                ("norm_eps", ctypes.c_float)]


class DenseFfn:
    """A dense FFN layer (the reference model's leading dense blocks, src/engine.cu:655-667 decode and :331-337
    prefill): out = x + down . q8_1(silu(gate . q8_1(h)) * (up . q8_1(h))), h = RMSNorm(x) * ffn_norm."""

    def __init__(self, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor, gate_type: int, up_type: int,
                 down_type: int, hidden: int, inter: int, ffn_norm: torch.Tensor | None = None,
                 norm_eps: float = 1e-6):
        self.gate, self.up, self.down, self.ffn_norm = gate, up, down, ffn_norm
        self.desc = DenseFfnDesc(hidden, inter, gate_type, up_type, down_type, gate.data_ptr(), up.data_ptr(),
                                 down.data_ptr(), ffn_norm.data_ptr() if ffn_norm is not None else None, norm_eps)

    @classmethod
    def from_gguf(cls, file: "GgufFile", layer: int) -> "DenseFfn":
        """Dense layer `layer` of a GGUF checkpoint made resident by fns_hip_dense_ffn_from_gguf."""
        obj = cls.__new__(cls)
        obj.desc = DenseFfnDesc()
        obj.gate = obj.up = obj.down = obj.ffn_norm = None
        obj._file = file
        res = ctypes.c_void_p()
        call("fns_hip_dense_ffn_from_gguf", file.handle, layer, ctypes.byref(res), ctypes.byref(obj.desc))
        obj._resident = res
        return obj

    def __del__(self):
        res = getattr(self, "_resident", None)
        if res:
            lib().fns_hip_dense_resident_free(res)
            self._resident = None

    def workspace(self, n_tok: int) -> torch.Tensor:
        total = ctypes.c_size_t()
        call("fns_hip_dense_ffn_workspace", ctypes.byref(self.desc), n_tok, ctypes.byref(total))
        return torch.empty(total.value, dtype=torch.uint8, device="cuda")

    def __call__(self, x: torch.Tensor, out: torch.Tensor | None = None, ws: torch.Tensor | None = None,
                 prefill: bool = False) -> torch.Tensor:
        x = x.contiguous()
        n_tok = x.numel() // self.desc.hidden
        out = torch.empty_like(x) if out is None else out
        ws = self.workspace(n_tok) if ws is None else ws
        call("fns_hip_dense_ffn_prefill" if prefill else "fns_hip_dense_ffn", ctypes.byref(self.desc), _p(x),
             _p(out), n_tok, _p(ws), ws.numel(), _s())
        return out


class GgufTensorInfo(ctypes.Structure):
    """Mirror of FnsGgufTensorInfo (include/fns_hip.h)."""
    _fields_ = [("type", ctypes.c_int), ("n_dims", ctypes.c_int), ("ne", ctypes.c_int64 * 4),
                ("nbytes", ctypes.c_size_t), ("offset", ctypes.c_size_t), ("data", ctypes.c_void_p)]


class GgufFile:
    """A GGUF checkpoint mapped by the library's reader (fns_hip_gguf_*; reference src/model.cpp:30-136)."""

    def __init__(self, path: str):
        self.handle = None
        h = ctypes.c_void_p()
        call("fns_hip_gguf_open", str(path).encode(), ctypes.byref(h))
        self.handle = h

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().fns_hip_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def info(self) -> dict:
        v, nt, nk, off = ctypes.c_uint32(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_size_t()
        call("fns_hip_gguf_info", self.handle, ctypes.byref(v), ctypes.byref(nt), ctypes.byref(nk), ctypes.byref(off))
        return {"version": v.value, "n_tensors": nt.value, "n_kv": nk.value, "data_offset": off.value}

    def tensor(self, name: str) -> dict:
        info = GgufTensorInfo()
        call("fns_hip_gguf_tensor", self.handle, name.encode(), ctypes.byref(info))
        return self._as_dict(info)

    def tensors(self) -> list[tuple[str, dict]]:
        out = []
        for i in range(self.info()["n_tensors"]):
            info, name = GgufTensorInfo(), ctypes.c_char_p()
            call("fns_hip_gguf_tensor_at", self.handle, i, ctypes.byref(info), ctypes.byref(name))
            out.append((name.value.decode(), self._as_dict(info)))
        return out

    @staticmethod
    def _as_dict(info: GgufTensorInfo) -> dict:
        raw = (ctypes.c_uint8 * info.nbytes).from_address(info.data) if info.nbytes else b""
        return {"type": info.type, "ne": list(info.ne[: info.n_dims]), "nbytes": info.nbytes, "offset": info.offset,
                "bytes": np.frombuffer(raw, dtype=np.uint8).copy() if info.nbytes else np.zeros(0, np.uint8)}

    def u32(self, key: str) -> int:
        v = ctypes.c_uint32()
        call("fns_hip_gguf_get_u32", self.handle, key.encode(), ctypes.byref(v))
        return v.value

    def f32(self, key: str) -> float:
        v = ctypes.c_float()
        call("fns_hip_gguf_get_f32", self.handle, key.encode(), ctypes.byref(v))
        return v.value

    def bool(self, key: str) -> bool:
        v = ctypes.c_int()
        call("fns_hip_gguf_get_bool", self.handle, key.encode(), ctypes.byref(v))
        return bool(v.value)

    def str(self, key: str) -> str:
        v = ctypes.c_char_p()
        call("fns_hip_gguf_get_str", self.handle, key.encode(), ctypes.byref(v))
        return v.value.decode()
