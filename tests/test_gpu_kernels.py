"""Parity of the HIP kernels (called through the C ABI of libfns_hip.so) against the CPU oracle.

Shapes follow the configs (hidden 2048, expert inter 768) at reduced expert counts so the oracle finishes in
seconds; the expert ids reuse the reference's fixed recipe {0, 255, 17, 128, 3, 200, 64, 9} reduced mod the
expert count (reference tests/expert_parity.cu:86).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.helpers import assert_close, gaussian, make_expert_mats

pytestmark = pytest.mark.gpu

H, F = 2048, 768
NE = 16
REF_IDS = [0, 255, 17, 128, 3, 200, 64, 9]
TYPES = [orc.Q8_0, orc.Q3_K, orc.Q4_K, orc.Q5_K, orc.Q6_K]


@pytest.fixture(scope="module")
def ops():
    from flintnsteel_amd import ops as o
    return o


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def ids_for(n_expert: int) -> np.ndarray:
    return np.array([i % n_expert for i in REF_IDS], dtype=np.int32)


def test_lane_exchange_selftest(ops):
    """The DPP / permlane-swap xor exchanges equal the LDS-crossbar shuffles (all offsets, butterfly sums)."""
    assert ops.selftest_lanes() == 0


# ---- Q8_1 ----------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("nrows,ncols", [(1, 2048), (8, 768), (3, 100), (2, 512), (1, 32)])
def test_quantize_q8_1_bit_exact(ops, nrows, ncols):
    rng = np.random.default_rng(20261022 + ncols)
    x = gaussian(rng, (nrows, ncols))
    x[0, :min(32, ncols)] = 0.0                       # all-zero block: d = 0, q = 0
    if ncols >= 64:
        x[0, 40] = 1e4                                # one dominant value
        x[-1, 32:64] = np.arange(32, dtype=np.float32) - 15.5  # halfway cases of roundf
    got = host(ops.quantize_q8_1(dev(x)))
    ref = orc.quantize_q8_1(x)
    assert got.shape == ref.shape
    assert np.array_equal(got, ref), f"first diff at byte {np.argmax(got.ravel() != ref.ravel())}"


def test_rms_norm_q8_1(ops):
    rng = np.random.default_rng(7)
    x = gaussian(rng, (3, H))
    w = gaussian(rng, (H,), 1.0)
    out, xq = ops.rms_norm_q8_1(dev(x), dev(w), 1e-6)
    out_h = host(out)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * w
    assert_close(out_h, ref, "rms_norm", 1e-5, 1e-6)
    assert np.array_equal(host(xq), orc.quantize_q8_1(out_h))


# ---- expert GEMVs -----------------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def gate_up_mats():
    return {t: (make_expert_mats(t, NE, F, H, 100 + t), make_expert_mats(t, NE, F, H, 200 + t)) for t in TYPES}


@pytest.fixture(scope="module")
def down_mats():
    return {t: make_expert_mats(t, NE, H, F, 300 + t) for t in TYPES}


def table_of(mats_dev: torch.Tensor, order=None) -> torch.Tensor:
    n = mats_dev.shape[0]
    base, stride = mats_dev.data_ptr(), mats_dev.stride(0)
    return torch.tensor([base + e * stride for e in (order if order is not None else range(n))],
                        dtype=torch.int64, device="cuda")


@pytest.mark.parametrize("qtype", TYPES)
def test_mmvq_experts_swiglu_vs_oracle(ops, gate_up_mats, qtype):
    g, u = gate_up_mats[qtype]
    rng = np.random.default_rng(20261022)
    x = gaussian(rng, (1, H))
    xq = orc.quantize_q8_1(x)
    ids = ids_for(NE)
    # expert slot = [gate | up]
    slots = np.concatenate([g, u], axis=1)
    slots_d = dev(slots)
    got = host(ops.mmvq_experts_swiglu(qtype, table_of(slots_d), 0, g.shape[1], H, F, dev(xq), 1, dev(ids)))
    mats_g = [m.reshape(F, -1) for m in g]
    mats_u = [m.reshape(F, -1) for m in u]
    gr = orc.mmvq_experts(qtype, mats_g, H, F, xq, 1, len(ids), ids)
    ur = orc.mmvq_experts(qtype, mats_u, H, F, xq, 1, len(ids), ids)
    ref = orc.swiglu(gr, ur)
    assert_close(got, ref, f"gate/up {orc.TYPE_NAMES[qtype]}")


@pytest.mark.parametrize("qtype", TYPES)
def test_mmvq_experts_down_vs_oracle(ops, down_mats, qtype):
    d = down_mats[qtype]
    rng = np.random.default_rng(5)
    act = gaussian(rng, (8, F), 0.3)
    xq = orc.quantize_q8_1(act)
    ids = ids_for(NE)
    d_dev = dev(d)
    got = host(ops.mmvq_experts(qtype, table_of(d_dev), 0, F, H, dev(xq), 8, dev(ids)))
    ref = orc.mmvq_experts(qtype, [m.reshape(H, -1) for m in d], F, H, xq, 8, 1, ids)
    assert_close(got, ref, f"down {orc.TYPE_NAMES[qtype]}")


@pytest.mark.parametrize("qtype", TYPES)
def test_table_equals_contiguous_bitwise(ops, down_mats, gate_up_mats, qtype):
    """Pointer-table kernels == contiguous MUL_MAT_ID kernels, bit for bit (reference tests/expert_parity.cu:1-8)."""
    g, u = gate_up_mats[qtype]
    rng = np.random.default_rng(11)
    x = gaussian(rng, (1, H))
    xq = dev(orc.quantize_q8_1(x))
    ids = dev(ids_for(NE))
    g_d, u_d = dev(g), dev(u)
    a, _ = ops.mmvq_ids_swiglu_shared(qtype, g_d, u_d, H, F, NE, xq, ids)
    # table over a permuted copy of the slots: slot positions differ, contents are the same
    perm = np.random.default_rng(3).permutation(NE)
    slots = np.concatenate([g, u], axis=1)[perm]
    slots_d = dev(slots)
    inv = np.argsort(perm)
    base = slots_d.data_ptr()
    table = torch.tensor([base + int(inv[e]) * slots.shape[1] for e in range(NE)], dtype=torch.int64, device="cuda")
    b = ops.mmvq_experts_swiglu(qtype, table, 0, g.shape[1], H, F, xq, 1, ids)
    assert np.array_equal(host(a), host(b))
    dn = down_mats[qtype]
    act = gaussian(rng, (8, F), 0.3)
    aq = dev(orc.quantize_q8_1(act))
    dn_d = dev(dn)
    a = ops.mmvq_ids(qtype, dn_d, F, H, NE, aq, 8, ids)
    b = ops.mmvq_experts(qtype, table_of(dn_d), 0, F, H, aq, 8, ids)
    assert np.array_equal(host(a), host(b))


@pytest.mark.parametrize("qtype", [orc.Q4_K, orc.Q6_K, orc.Q8_0])
def test_mmvq_columns_bit_identical(ops, down_mats, qtype):
    """Column c of a 4-column launch == the single-column launch (reference src/ggml/ggml_mmvq.cu:25-27)."""
    w = down_mats[qtype][1].reshape(H, -1)
    rng = np.random.default_rng(13)
    x = gaussian(rng, (6, F))
    xq = orc.quantize_q8_1(x)
    w_d, xq_d = dev(w), dev(xq)
    many = host(ops.mmvq(qtype, w_d, F, H, xq_d, 6))
    for c in range(6):
        one = host(ops.mmvq(qtype, w_d, F, H, xq_d[c:c + 1].contiguous(), 1))
        assert np.array_equal(many[c], one[0]), f"column {c}"
    ref = orc.mmvq_experts(qtype, [w], F, H, xq, 6, 1, np.zeros(6, np.int32))
    assert_close(many, ref, "mmvq 6 cols")


def test_mmvq_ids_swiglu_shared_expert(ops, gate_up_mats):
    qtype = orc.Q4_K
    g, u = gate_up_mats[qtype]
    rng = np.random.default_rng(17)
    x = gaussian(rng, (1, H))
    xq = orc.quantize_q8_1(x)
    ids = ids_for(NE)[:6]
    dst, sh = ops.mmvq_ids_swiglu_shared(qtype, dev(g), dev(u), H, F, NE, dev(xq), dev(ids), dev(g[5]), dev(u[7]))
    ref_sh = orc.swiglu(orc.mmvq_experts(qtype, [g[5].reshape(F, -1)], H, F, xq, 1, 1, np.zeros(1, np.int32)),
                        orc.mmvq_experts(qtype, [u[7].reshape(F, -1)], H, F, xq, 1, 1, np.zeros(1, np.int32)))
    assert_close(host(sh), ref_sh[0], "shared expert")
    ref = orc.swiglu(orc.mmvq_experts(qtype, [m.reshape(F, -1) for m in g], H, F, xq, 1, 6, ids),
                     orc.mmvq_experts(qtype, [m.reshape(F, -1) for m in u], H, F, xq, 1, 6, ids))
    assert_close(host(dst), ref, "routed experts with shared")
    # dense GLU == one-channel routed result
    one = host(ops.mmvq_swiglu(qtype, dev(g[ids[2]]), dev(u[ids[2]]), H, F, dev(xq)))
    assert np.array_equal(one, host(dst)[2])


def test_mmvq_vs_exact_input(ops, gate_up_mats):
    """Against the unquantised input the only error is Q8_1's: rel L2 < 2e-2 (reference tests/kernel_parity.py:86-88)."""
    qtype = orc.Q4_K
    g, _ = gate_up_mats[qtype]
    rng = np.random.default_rng(20261022)
    x = (rng.standard_normal(H) * 0.5).astype(np.float32)[None]
    got = host(ops.mmvq(qtype, dev(g[3].reshape(F, -1)), H, F, dev(orc.quantize_q8_1(x)), 1))[0]
    w = orc.dequantize(qtype, g[3].reshape(F, -1), H)
    ref = w @ x[0].astype(np.float64)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 2e-2


# ---- routing, combine, guard -------------------------------------------------------------------------------------

@pytest.mark.parametrize("n_expert,k,gating", [(128, 8, 0), (256, 6, 1), (100, 8, 0), (256, 8, 0), (64, 1, 1),
                                               (128, 16, 0), (200, 8, 1), (256, 1, 0), (256, 12, 1), (129, 6, 0)])
@pytest.mark.parametrize("n_tok", [5, 70])
def test_route_topk_bit_exact(ops, n_expert, k, gating, n_tok):
    """Both launch forms (1024 threads per token up to 64 tokens, 256 beyond) against the oracle, with ties."""
    rng = np.random.default_rng(n_expert * 31 + k + n_tok)
    logits = gaussian(rng, (n_tok, n_expert), 2.0)
    logits[1, 10:20] = 1.5        # exact ties: the lower index wins
    logits[2] = 0.0               # all equal
    ids, w = ops.route_topk(dev(logits), k, gating)
    rid, rw, _, _ = orc.route_topk(logits, k, gating)
    assert np.array_equal(host(ids), rid)
    assert np.array_equal(host(w).view(np.uint32), rw.view(np.uint32))


def test_gemv_router_f32_and_bf16(ops):
    rng = np.random.default_rng(9)
    w = gaussian(rng, (128, H), 0.02)
    x = gaussian(rng, (4, H))
    got = host(ops.gemv_router(dev(w), dev(x)))
    assert_close(got, orc.router_f32(w, x), "router f32", 1e-5, 1e-6)
    wb = torch.from_numpy(w).to(torch.bfloat16)
    got = host(ops.gemv_router(wb.cuda(), dev(x)))
    ref = wb.float().numpy().astype(np.float64) @ x.T.astype(np.float64)
    assert_close(got, ref.T, "router bf16", 1e-5, 1e-6)
    got = host(ops.gemm_router(dev(w), dev(np.tile(x, (20, 1)))))
    assert_close(got, np.tile(orc.router_f32(w, x), (20, 1)), "router gemm f32", 1e-5, 1e-6)


@pytest.mark.parametrize("ncols", [200, 1000])
def test_gemm_router_ragged_width(ops, ncols):
    """Widths that are not a multiple of 64 take the guarded loads of the router GEMM (f32 and bf16 weights)."""
    rng = np.random.default_rng(ncols)
    w = gaussian(rng, (40, ncols), 0.02)
    x = gaussian(rng, (19, ncols))
    got = host(ops.gemm_router(dev(w), dev(x)))
    assert_close(got, orc.router_f32(w, x), "router gemm f32 ragged", 1e-5, 1e-6)
    wb = torch.from_numpy(w).to(torch.bfloat16)
    xb = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = host(ops.gemm_router(wb.cuda(), dev(x)))
    ref = xb.astype(np.float64) @ wb.float().numpy().astype(np.float64).T
    assert_close(got, ref, "router gemm bf16 ragged", 1e-5, 1e-6)


@pytest.mark.parametrize("k,n", [(8, H), (6, H), (1, 256), (3, 2050), (12, H)])
def test_moe_combine_bit_exact(ops, k, n):
    """k <= 8 with n % 4 == 0 takes the four-column kernel; the others the per-column one: same bits either way."""
    rng = np.random.default_rng(4 + k)
    dexp = gaussian(rng, (3, k, n))
    w = np.abs(gaussian(rng, (3, k)))
    e = np.exp2(rng.integers(0, 3, (3, k))).astype(np.float32)
    sh = gaussian(rng, (3, n))
    x = gaussian(rng, (3, n))
    got = host(ops.moe_combine(dev(dexp), dev(w), dev(e), dev(sh), dev(x)))
    ref = orc.moe_combine(dexp, w, e, sh, x)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("n", [96, 512, F, 2048, 2560])
def test_amax_guard_q8_1(ops, n):
    """Rows of every width class of the kernel (register-held rows up to 2048 padded columns, the looping form
    beyond): the guard scales and the Q8_1 bytes bit-exact."""
    rng = np.random.default_rng(12 + n)
    act = gaussian(rng, (4, n), 0.5)
    act[1] *= 5000.0  # amax > 1024: e = 2^k
    escale, xq = ops.amax_guard_q8_1(dev(act))
    e = host(escale)
    ref_e = np.array([orc.amax_guard_scale(r) for r in act], dtype=np.float32)
    assert np.array_equal(e, ref_e)
    assert e[0] == 1.0 and e[1] > 1.0
    assert np.array_equal(host(xq), orc.quantize_q8_1((act / e[:, None]).astype(np.float32)))
    a2 = dev(act)
    e2 = host(ops.amax_guard(a2))
    assert np.array_equal(e2, ref_e)
    assert np.array_equal(host(a2), (act / ref_e[:, None]).astype(np.float32))


def test_swiglu_epilogues(ops):
    rng = np.random.default_rng(2)
    g = gaussian(rng, (4, F), 3.0)
    u = gaussian(rng, (4, F))
    ref = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
    assert_close(host(ops.swiglu(dev(g), dev(u))), ref, "swiglu", 1e-6, 1e-6)
    assert_close(host(ops.glu_mmvq(dev(g), dev(u))), ref, "glu_mmvq", 1e-6, 1e-6)


def test_count_routes(ops):
    counts = torch.zeros(128, dtype=torch.uint32, device="cuda")
    ids = dev(np.array([3, 5, 3, 127, 0, 9], dtype=np.int32))
    ops.count_routes(ids, counts)
    ops.count_routes(ids, counts)
    c = host(counts.to(torch.int64))
    assert c[3] == 4 and c[5] == 2 and c[127] == 2 and c[0] == 2 and c.sum() == 12


@pytest.mark.parametrize("n,off", [(4096, 0), (1027, 0), (1027, 1), (5, 3)])
def test_add(ops, n, off):
    """out = x + y (the reference's add_inplace, out-of-place), float4 form and the element form for arrays that
    are not 16-byte aligned; in place too."""
    rng = np.random.default_rng(n + off)
    x, y = gaussian(rng, (n + off,)), gaussian(rng, (n + off,))
    xd, yd = dev(x), dev(y)
    got = host(ops.add(xd[off:], yd[off:]))
    assert np.array_equal(got, (x[off:] + y[off:]).astype(np.float32))
    ops.add(xd[off:], yd[off:], out=xd[off:])
    assert np.array_equal(host(xd)[off:], got)
