"""IQ formats on the GPU (IQ4_XS, IQ3_XXS, IQ3_S, IQ2_S; reference src/ggml/ggml_mmvq.cu:101-157,378-385,403-411,
src/ggml/ggml_mmq.cu:59-66): the dense and expert-table GEMVs, the whole decode / verify layer, the prefill GEMM and
the prefill layer against the CPU oracle, which restates the reference's integer sub-block products (GEMV) and the
dequantisers' float sub-block scales (GEMM) with the same codebooks (tests/iq_data.py registers identical seeded
tables in both; ggml's own tables are not in this container, so agreement with them is not pinned).

Bars: GEMV outputs within 1e-5 relative L2 / 1e-4 normalised max of the oracle (fp32 accumulation against float64);
the layer within the north_star's 1e-3 with ids and weights bit-exact; a verify column equal to its batch-1 result.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.helpers import assert_close
from tests.iq_data import random_blocks, register_grids, register_grids_in_library

pytestmark = pytest.mark.gpu

IQ_TYPES = [orc.IQ4_XS, orc.IQ3_XXS, orc.IQ3_S, orc.IQ2_S]


@pytest.fixture(scope="module")
def ops():
    from flintnsteel_amd import ops as o
    grids = register_grids(11)
    register_grids_in_library(grids)
    return o


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def test_supports_after_registration(ops):
    from flintnsteel_amd._lib import lib
    assert [t for t in IQ_TYPES if lib().fns_hip_mmvq_supports(t)] == IQ_TYPES
    bad = np.ones(256, np.uint32)  # a zero byte in the IQ3_XXS codebook (value 1 leaves bytes 1..3 zero)
    from flintnsteel_amd._lib import FnsError, call
    ok = [np.ascontiguousarray(g) for g in register_grids(11)]
    with pytest.raises(FnsError, match="must be 1..127"):
        call("fns_hip_set_iq_grids", bad.ctypes.data_as(ctypes.c_void_p), ok[1].ctypes.data_as(ctypes.c_void_p),
             ok[2].ctypes.data_as(ctypes.c_void_p))


@pytest.mark.parametrize("qtype", IQ_TYPES, ids=lambda t: orc.TYPE_NAMES[t])
@pytest.mark.parametrize("ncols,nrows,ncol_x", [(2048, 96, 1), (512, 64, 3)])
def test_dense_mmvq(ops, qtype, ncols, nrows, ncol_x):
    print(f"IQ dense mmvq {orc.TYPE_NAMES[qtype]} {ncols}x{nrows} cols={ncol_x}", flush=True)
    w = random_blocks(qtype, nrows, ncols, seed=ncols + qtype)
    x = np.random.default_rng(qtype).standard_normal((ncol_x, ncols)).astype(np.float32)
    xq = orc.quantize_q8_1(x)
    w_d, xq_d = torch.from_numpy(w).cuda(), torch.from_numpy(xq).cuda()
    out = torch.empty(ncol_x, nrows, device="cuda")
    from flintnsteel_amd._lib import call
    call("fns_hip_mmvq", qtype, _p(w_d), ncols, nrows, _p(xq_d), _p(out), ncol_x, None)
    got = host(out)
    for c in range(ncol_x):
        ref = orc.mmvq_experts(qtype, [w], ncols, nrows, xq[c:c + 1], 1, 1, np.zeros(1, np.int32))[0]
        assert_close(got[c], ref, f"{orc.TYPE_NAMES[qtype]} column {c}")


@pytest.mark.parametrize("gu,dn", [(orc.IQ3_XXS, orc.IQ4_XS), (orc.IQ2_S, orc.IQ3_S)],
                         ids=["iq3xxs_iq4xs", "iq2s_iq3s"])
def test_expert_table_gemvs(ops, gu, dn):
    """mmvq_experts_swiglu (gate/up over an expert table) and mmvq_experts (down) against the oracle."""
    H, F, NE, C = 1024, 512, 6, 4
    slots = ops.ExpertSlots.from_tensors(torch.from_numpy(random_blocks(gu, NE * F, H, 1).reshape(NE, -1)),
                                         torch.from_numpy(random_blocks(gu, NE * F, H, 2).reshape(NE, -1)),
                                         torch.from_numpy(random_blocks(dn, NE * H, F, 3).reshape(NE, -1)))
    ids = np.array([4, 0, 5, 2], np.int32)
    x = np.random.default_rng(9).standard_normal((1, H)).astype(np.float32)
    xq = orc.quantize_q8_1(x)
    ids_d, xq_d = torch.from_numpy(ids).cuda(), torch.from_numpy(xq).cuda()
    act = torch.empty(C, F, device="cuda")
    from flintnsteel_amd._lib import call
    call("fns_hip_mmvq_experts_swiglu", gu, _p(slots.table), slots.gate_off, slots.up_off, H, F, _p(xq_d), 1,
         _p(ids_d), C, _p(act), None)
    mats = lambda kind, e, n: host(slots.view(kind)[e]).reshape(n, -1)  # noqa: E731
    got = host(act)
    acts = []
    for c, e in enumerate(ids):
        g = orc.mmvq_experts(gu, [mats("gate", e, F)], H, F, xq, 1, 1, np.zeros(1, np.int32))
        u = orc.mmvq_experts(gu, [mats("up", e, F)], H, F, xq, 1, 1, np.zeros(1, np.int32))
        a = orc.swiglu(g, u)[0]
        assert_close(got[c], a, f"act of expert {e}")
        acts.append(got[c])
    aq = orc.quantize_q8_1(np.stack(acts).astype(np.float32))
    aq_d = torch.from_numpy(aq).cuda()
    dexp = torch.empty(C, H, device="cuda")
    call("fns_hip_mmvq_experts", dn, _p(slots.table), slots.down_off, F, H, _p(aq_d), C, _p(ids_d), C, _p(dexp), None)
    got = host(dexp)
    for c, e in enumerate(ids):
        ref = orc.mmvq_experts(dn, [mats("down", e, H)], F, H, aq[c:c + 1], 1, 1, np.zeros(1, np.int32))[0]
        assert_close(got[c], ref, f"down of expert {e}")


LAYER_CASES = {"iq3xxs_iq4xs": (orc.IQ3_XXS, orc.IQ4_XS), "iq3s_iq4xs": (orc.IQ3_S, orc.IQ4_XS),
               "iq2s_iq4xs": (orc.IQ2_S, orc.IQ4_XS), "iq4xs_q4k": (orc.IQ4_XS, orc.Q4_K)}


@pytest.mark.parametrize("case", list(LAYER_CASES))
def test_moe_layer_decode_and_verify(ops, case):
    """The whole layer with IQ experts (the fused decode kernel for the IQ4_XS-down mixes, the three-kernel path
    otherwise): routing bit-exact against the oracle from the layer's logits, output within 1e-3 of the float64
    chain, and the 4-token verify step's columns equal to their batch-1 results bit for bit."""
    gu, dn = LAYER_CASES[case]
    H, F, NE, K = 2048, 512, 32, 4
    print(f"IQ layer {case}", flush=True)
    from flintnsteel_amd import synth
    slots = ops.ExpertSlots.from_tensors(torch.from_numpy(random_blocks(gu, NE * F, H, 11).reshape(NE, -1)),
                                         torch.from_numpy(random_blocks(gu, NE * F, H, 12).reshape(NE, -1)),
                                         torch.from_numpy(random_blocks(dn, NE * H, F, 13).reshape(NE, -1))
                                         if orc.TYPE_NAMES[dn].startswith("IQ") else
                                         torch.from_numpy(orc.quantize(dn, np.random.default_rng(13).normal(
                                             0, 0.02, (NE * H, F)).astype(np.float32)).reshape(NE, -1)))
    router = ops.fill_normal(torch.empty(NE, H, device="cuda"), 77, std=0.02)
    layer = ops.MoeLayer(router, slots, gu, dn, H, F, K)
    x4 = synth.activations(4, H, 5, layer=3)
    outs1 = []
    for t in range(4):
        ws = layer.workspace(1)
        out = host(layer(x4[t:t + 1], ws=ws))
        tr = {k: host(v) for k, v in layer.trace(ws, 1).items()}
        outs1.append(out[0])
        ids, w, _, _ = orc.route_topk(tr["logits"], K, 0)
        assert np.array_equal(ids, tr["ids"]) and np.array_equal(w, tr["w"])
        if t == 0:  # the float64 chain for one token
            xq = orc.quantize_q8_1(host(x4[0:1]))
            mats = lambda kind, e, n: host(slots.view(kind)[e]).reshape(n, -1)  # noqa: E731
            ref = np.zeros(H)
            for j in range(K):
                e = int(ids[0, j])
                g = orc.mmvq_experts(gu, [mats("gate", e, F)], H, F, xq, 1, 1, np.zeros(1, np.int32))
                u = orc.mmvq_experts(gu, [mats("up", e, F)], H, F, xq, 1, 1, np.zeros(1, np.int32))
                act = orc.swiglu(g, u)[0]
                assert_close(tr["act"][j], act, f"act slot {j}")
                aq = orc.quantize_q8_1(tr["act"][j:j + 1])
                ref += orc.mmvq_experts(dn, [mats("down", e, H)], F, H, aq, 1, 1, np.zeros(1, np.int32))[0] * float(w[0, j])
            assert_close(out[0], ref, "layer output")
    out4 = host(layer(x4))
    for t in range(4):
        assert np.array_equal(out4[t], outs1[t]), f"verify column {t} differs from its batch-1 result"


def _dq(qtype, blocks, ncols):
    """float64 [rows][ncols] of IQ blocks (the oracle's dequantiser: the products of ggml's MMQ scales)."""
    return orc.dequantize(qtype, np.ascontiguousarray(blocks), ncols).reshape(blocks.shape[0], ncols)


def _table(slots_dev):
    return torch.tensor([slots_dev.data_ptr() + e * slots_dev.stride(0) for e in range(slots_dev.shape[0])],
                        dtype=torch.int64, device="cuda")


@pytest.mark.parametrize("qtype", IQ_TYPES, ids=lambda t: orc.TYPE_NAMES[t])
def test_mmq_iq_dense_and_experts(ops, qtype):
    """The prefill GEMM (MMQ) on IQ weights (reference src/ggml/ggml_mmq.cu:59-66 accepts all four): the dense form
    and the expert form over every group shape, against the float64 dot of the oracle's dequantised weights with the
    Q8_1 activations (ggml's MMQ applies each sub-block's scale as the dequantiser's float product, which the f16 split
    GEMM reproduces exactly before its fp32 accumulation)."""
    print(f"IQ mmq {orc.TYPE_NAMES[qtype]}", flush=True)
    rng = np.random.default_rng(qtype)
    T, ncols, nrows = 77, 768, 192
    w = random_blocks(qtype, nrows, ncols, seed=300 + qtype)
    x = rng.standard_normal((T, ncols)).astype(np.float32)
    got = host(ops.mmq(qtype, torch.from_numpy(w).cuda(), ncols, nrows, torch.from_numpy(x).cuda()))
    xdq = orc.dequantize_q8_1(orc.quantize_q8_1(x), ncols).reshape(T, ncols)
    assert_close(got, xdq @ _dq(qtype, w, ncols).T, f"mmq dense {orc.TYPE_NAMES[qtype]}")
    loads = [0, 1, 16, 17, 32, 33, 63, 64, 65, 129]
    NE, ncols, nrows = len(loads), 512, 128
    pairs = np.concatenate([np.full(n, e, np.int32) for e, n in enumerate(loads)])
    ids = pairs[rng.permutation(len(pairs))].reshape(-1, 1)
    mats = np.stack([random_blocks(qtype, nrows, ncols, seed=400 + 10 * qtype + e) for e in range(NE)])
    md = torch.from_numpy(mats.reshape(NE, -1)).cuda()
    x = rng.standard_normal((len(ids), ncols)).astype(np.float32)
    got = host(ops.mmq_experts(qtype, _table(md), 0, ncols, nrows, NE, torch.from_numpy(x).cuda(), 1,
                               torch.from_numpy(ids).cuda())).reshape(len(ids), nrows)
    xdq = orc.dequantize_q8_1(orc.quantize_q8_1(x), ncols).reshape(len(ids), ncols)
    ref = np.stack([xdq[i] @ _dq(qtype, mats[ids[i, 0]], ncols).T for i in range(len(ids))])
    assert_close(got, ref, f"mmq_experts group shapes {orc.TYPE_NAMES[qtype]}")


@pytest.mark.parametrize("gu,dn", [(orc.IQ3_XXS, orc.IQ4_XS), (orc.IQ2_S, orc.IQ3_S)], ids=["iq3xxs_iq4xs", "iq2s_iq3s"])
def test_moe_prefill_iq(ops, gu, dn):
    """The prefill layer with IQ experts (two-launch MMQ path): routing bit-exact against the oracle from the layer's
    logits; the act image within half a Q8_1 step of the float64 SwiGLU of the dequantised gate / up products; the
    output against the float64 chain fed with the GPU's act codes (tight bounds)."""
    from tests.helpers import image_to_q8_1
    from flintnsteel_amd import synth
    H, F, NE, K, T = 512, 256, 8, 2, 77
    print(f"IQ prefill {orc.TYPE_NAMES[gu]}/{orc.TYPE_NAMES[dn]}", flush=True)
    g_, u_, d_ = (random_blocks(gu, NE * F, H, 21), random_blocks(gu, NE * F, H, 22), random_blocks(dn, NE * H, F, 23))
    slots = ops.ExpertSlots.from_tensors(*(torch.from_numpy(a.reshape(NE, -1)) for a in (g_, u_, d_)))
    layer = ops.MoeLayer(ops.fill_normal(torch.empty(NE, H, device="cuda"), 5, std=0.05), slots, gu, dn, H, F, K)
    pre = ops.MoePrefill(layer)
    x = synth.activations(T, H, 7, layer=2)
    ws = pre.workspace(T)
    out = host(pre(x, ws=ws))
    tr = {k: host(v) for k, v in pre.trace(ws, T).items()}
    ids, w, _, _ = orc.route_topk(tr["logits"], K, 0)
    assert np.array_equal(ids, tr["ids"]) and np.array_equal(w, tr["w"])
    xdq = orc.dequantize_q8_1(orc.quantize_q8_1(host(x)), H).reshape(T, H)
    G, U, D = (_dq(gu, g_, H).reshape(NE, F, H), _dq(gu, u_, H).reshape(NE, F, H), _dq(dn, d_, F).reshape(NE, H, F))
    aq = image_to_q8_1(tr["apack"], F)
    adq = orc.dequantize_q8_1(aq, F).reshape(T, K, F)
    ref = np.zeros((T, H))
    for t in range(T):
        for j in range(K):
            e = int(ids[t, j])
            act = orc.swiglu((G[e] @ xdq[t])[None], (U[e] @ xdq[t])[None])[0]
            step = np.repeat(np.abs(adq[t, j]).reshape(-1, 32).max(axis=1) / 127.0, 32)
            assert (np.abs(adq[t, j] - act) <= 0.5 * step + 1e-3 * np.abs(act).max()).all(), f"act image t={t} j={j}"
            ref[t] += (D[e] @ adq[t, j]) * float(w[t, j])
    assert_close(out, ref, f"IQ prefill {orc.TYPE_NAMES[gu]}/{orc.TYPE_NAMES[dn]} (GPU act codes)")
