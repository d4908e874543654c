"""Seeded synthetic MoE layers built on the device (the configs' data: router fp32 ~N(0, 0.02), expert gate/up
[inter x hidden] and down [hidden x inter] ~N(0, 0.02) quantised with ggml's reference quantisers, activations
~N(0, 1)). Everything is generated and quantised by libfns_hip.so on the GPU, so a 48-layer stack of 128 experts
(~18.8 GB of blocks) builds in seconds; nothing here is measured.
"""
from __future__ import annotations

import torch

from . import ops

KIND_ROUTER, KIND_GATE, KIND_UP, KIND_DOWN, KIND_X, KIND_BIAS, KIND_SHEXP, KIND_NORM = range(8)


def tensor_seed(seed: int, layer: int, kind: int) -> int:
    """Independent Philox key per (config seed, layer, tensor kind)."""
    return (seed * 1_000_003 + layer * 1_009 + kind * 7) & 0xFFFFFFFFFFFFFFFF


def quantized_matrices(qtype: int, n_mat: int, nrows: int, ncols: int, seed: int, std: float, out: torch.Tensor,
                       chunk_values: int = 1 << 25) -> None:
    """out[m] <- quantize(N(0, std) [nrows][ncols]) for m < n_mat; fp32 is generated in chunks of whole matrices."""
    per = nrows * ncols
    mats_per_chunk = max(1, chunk_values // per)
    scratch = torch.empty(mats_per_chunk * per, dtype=torch.float32, device="cuda")
    for m0 in range(0, n_mat, mats_per_chunk):
        m = min(mats_per_chunk, n_mat - m0)
        buf = scratch[: m * per]
        ops.fill_normal(buf, seed, offset=m0 * per, std=std)
        q = ops.quantize_weights(qtype, buf.view(m * nrows, ncols))
        out[m0: m0 + m].copy_(q.view(m, -1))


def build_layer(hidden: int, inter: int, n_expert: int, k: int, gu_type: int, down_type: int, seed: int,
                layer: int = 0, gating: int = ops.GATING_SOFTMAX, guard: bool = False,
                router_dtype: torch.dtype = torch.float32, std: float = 0.02) -> ops.MoeLayer:
    router = ops.fill_normal(torch.empty(n_expert, hidden, device="cuda"), tensor_seed(seed, layer, KIND_ROUTER),
                             std=std)
    if router_dtype != torch.float32:
        router = router.to(router_dtype)
    slots = ops.ExpertSlots(n_expert, ops.row_bytes(gu_type, hidden) * inter, ops.row_bytes(gu_type, hidden) * inter,
                            ops.row_bytes(down_type, inter) * hidden)
    quantized_matrices(gu_type, n_expert, inter, hidden, tensor_seed(seed, layer, KIND_GATE), std, slots.view("gate"))
    quantized_matrices(gu_type, n_expert, inter, hidden, tensor_seed(seed, layer, KIND_UP), std, slots.view("up"))
    quantized_matrices(down_type, n_expert, hidden, inter, tensor_seed(seed, layer, KIND_DOWN), std, slots.view("down"))
    return ops.MoeLayer(router, slots, gu_type, down_type, hidden, inter, k, gating=gating, guard=guard)


def build_flint_layer(hidden: int, inter: int, n_expert: int, k: int, shexp_inter: int, gu_type: int, down_type: int,
                      seed: int, layer: int = 0, std: float = 0.02, guard: bool = True) -> ops.MoeLayer:
    """A layer shaped like the reference model's MoE blocks (src/model.cpp:159-164: sigmoid gating, bf16 router,
    normalised top-k weights, a shared expert, RMSNorm before the FFN): build_layer's experts plus the shared
    expert's gate/up [shexp_inter x hidden] and down [hidden x shexp_inter] (same types) and norm weights
    ~N(1, 0.1)."""
    base = build_layer(hidden, inter, n_expert, k, gu_type, down_type, seed, layer=layer,
                       gating=ops.GATING_SIGMOID, guard=guard, router_dtype=torch.bfloat16, std=std)
    sseed = tensor_seed(seed, layer, KIND_SHEXP)
    gate = torch.empty(1, ops.row_bytes(gu_type, hidden) * shexp_inter, dtype=torch.uint8, device="cuda")
    up = torch.empty_like(gate)
    down = torch.empty(1, ops.row_bytes(down_type, shexp_inter) * hidden, dtype=torch.uint8, device="cuda")
    quantized_matrices(gu_type, 1, shexp_inter, hidden, sseed, std, gate)
    quantized_matrices(gu_type, 1, shexp_inter, hidden, sseed + 1, std, up)
    quantized_matrices(down_type, 1, hidden, shexp_inter, sseed + 2, std, down)
    norm = ops.fill_normal(torch.empty(hidden, device="cuda"), tensor_seed(seed, layer, KIND_NORM), mean=1.0, std=0.1)
    shexp = {"gate": gate, "up": up, "down": down, "inter": shexp_inter, "gu_type": gu_type, "down_type": down_type}
    return ops.MoeLayer(base.router_w, base.slots, gu_type, down_type, hidden, inter, k, gating=ops.GATING_SIGMOID,
                        guard=guard, ffn_norm=norm, norm_eps=1e-6, shexp=shexp)


def activations(n_tok: int, hidden: int, seed: int, layer: int = 0, step: int = 0) -> torch.Tensor:
    """x ~ N(0, 1) [n_tok][hidden], fresh per (layer, step)."""
    x = torch.empty(n_tok, hidden, device="cuda")
    return ops.fill_normal(x, tensor_seed(seed, layer, KIND_X), offset=step * n_tok * hidden)


# ---- IQ formats (benchmarks): seeded codebooks and random blocks -------------------------------------------------
# ggml's codebooks are data of the checkpoint's runtime (ggml-common.h), not part of this library: the caller
# registers them (fns_hip_set_iq_grids). For measurement, seeded tables of ggml's shapes whose bytes are drawn from
# the same value sets stand in for them (IQ3_XXS: 4, 12, ..., 52, 62; IQ3_S: the odd values 1..15; IQ2_S: 8, 25, 43);
# the kernels' work per block does not depend on the table's contents.
IQ_BLOCK_BYTES = {18: 98, 21: 110, 22: 82, 23: 136}  # IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS per 256 values
IQ_D_SCALE = {18: 4e-5, 21: 4e-5, 22: 1.2e-4, 23: 1.5e-5}  # f16 d giving weights of the order of N(0, 0.02)


def register_iq_grids(seed: int = 11) -> None:
    import ctypes

    import numpy as np

    from ._lib import call
    rng = np.random.default_rng(seed)
    a = rng.choice(np.array([4, 12, 20, 28, 36, 44, 52, 62], np.uint8), size=(256, 4)).view(np.uint32).reshape(256)
    b = rng.choice(np.arange(1, 16, 2, dtype=np.uint8), size=(512, 4)).view(np.uint32).reshape(512)
    c = rng.choice(np.array([8, 25, 43], np.uint8), size=(1024, 8)).view(np.uint64).reshape(1024)
    a, b, c = (np.ascontiguousarray(g) for g in (a, b, c))
    call("fns_hip_set_iq_grids", a.ctypes.data_as(ctypes.c_void_p), b.ctypes.data_as(ctypes.c_void_p),
         c.ctypes.data_as(ctypes.c_void_p))


def random_iq_blocks(qtype: int, n_blocks: int, seed: int, out: torch.Tensor) -> None:
    """out (uint8, n_blocks * block bytes, on the device) <- random IQ blocks: every index, sign and scale field
    random, f16 d = IQ_D_SCALE * U(0.5, 1.5)."""
    bb = IQ_BLOCK_BYTES[qtype]
    g = torch.Generator(device="cuda")
    g.manual_seed(seed & 0x7FFFFFFFFFFFFFFF)
    blk = out.view(n_blocks, bb)
    blk.copy_(torch.randint(0, 256, (n_blocks, bb), dtype=torch.uint8, device="cuda", generator=g))
    d = (IQ_D_SCALE[qtype] * (0.5 + torch.rand(n_blocks, device="cuda", generator=g))).to(torch.float16)
    blk[:, 0:2].copy_(d.view(torch.uint8).view(n_blocks, 2))


def build_iq_flint_layer(hidden: int, inter: int, n_expert: int, k: int, shexp_inter: int, gu_type: int,
                         down_type: int, seed: int, layer: int = 0) -> ops.MoeLayer:
    """build_flint_layer's shape with IQ experts and shared expert (random blocks; register_iq_grids first)."""
    router = ops.fill_normal(torch.empty(n_expert, hidden, device="cuda"), tensor_seed(seed, layer, KIND_ROUTER),
                             std=0.02).to(torch.bfloat16)
    gb, db = ops.row_bytes(gu_type, hidden) * inter, ops.row_bytes(down_type, inter) * hidden
    slots = ops.ExpertSlots(n_expert, gb, gb, db)
    for name, qt, nbytes, kind in (("gate", gu_type, gb, KIND_GATE), ("up", gu_type, gb, KIND_UP),
                                   ("down", down_type, db, KIND_DOWN)):
        tmp = torch.empty(n_expert * nbytes, dtype=torch.uint8, device="cuda")
        random_iq_blocks(qt, n_expert * nbytes // IQ_BLOCK_BYTES[qt], tensor_seed(seed, layer, kind), tmp)
        slots.view(name).copy_(tmp.view(n_expert, nbytes))
    sseed = tensor_seed(seed, layer, KIND_SHEXP)
    sg = torch.empty(ops.row_bytes(gu_type, hidden) * shexp_inter, dtype=torch.uint8, device="cuda")
    su = torch.empty_like(sg)
    sd = torch.empty(ops.row_bytes(down_type, shexp_inter) * hidden, dtype=torch.uint8, device="cuda")
    for t, qt, s in ((sg, gu_type, sseed), (su, gu_type, sseed + 1), (sd, down_type, sseed + 2)):
        random_iq_blocks(qt, t.numel() // IQ_BLOCK_BYTES[qt], s, t)
    norm = ops.fill_normal(torch.empty(hidden, device="cuda"), tensor_seed(seed, layer, KIND_NORM), mean=1.0, std=0.1)
    shexp = {"gate": sg, "up": su, "down": sd, "inter": shexp_inter, "gu_type": gu_type, "down_type": down_type}
    return ops.MoeLayer(router, slots, gu_type, down_type, hidden, inter, k, gating=ops.GATING_SIGMOID, guard=True,
                        ffn_norm=norm, norm_eps=1e-6, shexp=shexp)
