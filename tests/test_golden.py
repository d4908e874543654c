"""Committed golden vectors (tests/golden/golden.npz, written by tests/golden/make_golden.py from the CPU oracle on
the reference's input recipes). CPU: the oracle still reproduces every vector. GPU: the HIP kernels, called through
the C ABI, reproduce them - bit-exact for Q8_1 bytes, expert ids, routing weights, the combine and the compaction;
within the fp32 tolerance of tests/helpers.py for the K-quant GEMVs (float64 oracle)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import assert_close

G = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz")
KQ = [orc.Q3_K, orc.Q4_K, orc.Q5_K, orc.Q6_K]


def test_oracle_reproduces_q8_1():
    assert np.array_equal(orc.quantize_q8_1(G["q8_x"]), G["q8_xq"])


def test_oracle_reproduces_routing():
    ids, w, _, _ = orc.route_topk(G["rt_logits_sm"], 8, 0, True)
    assert np.array_equal(ids, G["rt_ids_sm"]) and np.array_equal(w, G["rt_w_sm"])
    ids, w, _, _ = orc.route_topk(G["rt_logits_sg"], 6, 1, True)
    assert np.array_equal(ids, G["rt_ids_sg"]) and np.array_equal(w, G["rt_w_sg"])
    # tie in row 3 (experts 5 and 9 share the top logit): the lower index comes first
    assert list(G["rt_ids_sm"][3, :2]) == [5, 9]


@pytest.mark.parametrize("qtype", KQ)
def test_oracle_reproduces_mmvq(qtype):
    w = G[f"mv_w_{qtype}"]
    got = orc.mmvq_experts(qtype, list(w), 512, 16, G["mv_xq"], 2, 1, G["mv_ids"])
    assert np.array_equal(got, G[f"mv_dst_{qtype}"])


def test_oracle_reproduces_combine_and_compaction():
    out = orc.moe_combine(G["cb_dexp"], G["cb_w"], G["cb_e"], None, G["cb_x"])
    assert np.array_equal(out, G["cb_out"])
    b, s, d, _ = orc.compact_ids(G["cp_ids"], 16, 1)
    assert np.array_equal(b, G["cp_bounds"]) and np.array_equal(s, G["cp_src"]) and np.array_equal(d, G["cp_dst"])


# ---- the HIP path against the same vectors ----------------------------------------------------------------------

@pytest.fixture(scope="module")
def ops():
    from flintnsteel_amd import ops as o
    return o


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.gpu
def test_hip_q8_1_golden(ops):
    assert np.array_equal(_host(ops.quantize_q8_1(_dev(G["q8_x"]))), G["q8_xq"])


@pytest.mark.gpu
def test_hip_routing_golden(ops):
    ids, w = ops.route_topk(_dev(G["rt_logits_sm"]), 8, 0, True)
    assert np.array_equal(_host(ids), G["rt_ids_sm"]) and np.array_equal(_host(w), G["rt_w_sm"])
    ids, w = ops.route_topk(_dev(G["rt_logits_sg"]), 6, 1, True)
    assert np.array_equal(_host(ids), G["rt_ids_sg"]) and np.array_equal(_host(w), G["rt_w_sg"])


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", KQ)
def test_hip_mmvq_golden(ops, qtype):
    import torch
    w = _dev(G[f"mv_w_{qtype}"])
    table = torch.tensor([w.data_ptr() + e * w.stride(0) for e in range(w.shape[0])], dtype=torch.int64,
                         device="cuda")
    got = _host(ops.mmvq_experts(qtype, table, 0, 512, 16, _dev(G["mv_xq"]), 2, _dev(G["mv_ids"])))
    assert_close(got, G[f"mv_dst_{qtype}"], f"mmvq {orc.TYPE_NAMES[qtype]} golden")


@pytest.mark.gpu
def test_hip_combine_golden(ops):
    out = _host(ops.moe_combine(_dev(G["cb_dexp"]), _dev(G["cb_w"]), escale=_dev(G["cb_e"]), x=_dev(G["cb_x"])))
    assert np.array_equal(out, G["cb_out"])
