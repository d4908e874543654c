"""Writes tests/golden/golden.npz: small input/output vectors of the MoE FFN path, produced by the CPU oracle.

The reference commits no golden vectors for this path (its parity programs need a GPU and real GGUF checkpoints:
reference tests/expert_parity.cu, tests/kernel_parity.py, tests/mmq_parity.cu). These fixtures freeze the oracle's
outputs on the reference's own input recipes so that (1) a later change of the oracle is caught by the CPU suite and
(2) the HIP kernels are checked against fixed vectors without the oracle in the loop:
  - the LCG input of reference tests/expert_parity.cu:43-47 (s = s * 1664525 + 1013904223),
  - the fixed expert ids {0, 255, 17, 128, 3, 200, 64, 9} of reference tests/expert_parity.cu:86 (mod n_expert),
  - numpy default_rng(20261022) inputs scaled by 0.5 as reference tests/kernel_parity.py:58-59.

    python tests/golden/make_golden.py        (from the repo root; needs oracle/libfns_oracle.so)
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as orc  # noqa: E402

REF_IDS = [0, 255, 17, 128, 3, 200, 64, 9]


def lcg_floats(n: int, seed: int = 12345) -> np.ndarray:
    """reference tests/expert_parity.cu:43-47: s = s*1664525 + 1013904223 (mod 2^32), x = (s >> 8) / 2^24 - 0.5."""
    out = np.empty(n, dtype=np.float32)
    s = seed & 0xFFFFFFFF
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32((s >> 8) / 16777216.0 - 0.5)
    return out


def make() -> dict:
    g = {}
    rng = np.random.default_rng(20261022)
    # Q8_1: LCG rows, a ragged width (1000 -> padded to 1024), an all-zero block and round-half cases
    x = (lcg_floats(3 * 1000) * 4.0).reshape(3, 1000)
    x[0, :32] = 0.0
    x[1, 32:64] = np.arange(32, dtype=np.float32) - 15.5
    x[2, 64] = 1e4
    g["q8_x"] = x
    g["q8_xq"] = orc.quantize_q8_1(x)
    # routing: softmax top-8 of 128 and sigmoid top-6 of 256 (the reference's own Flint gating), plus an exact tie
    lg = (rng.standard_normal((4, 128)) * 0.5).astype(np.float32)
    lg[3, 5] = lg[3, 9] = np.float32(3.0)  # tie -> lower index first
    g["rt_logits_sm"] = lg
    g["rt_ids_sm"], g["rt_w_sm"], _, _ = orc.route_topk(lg, 8, 0, True)
    ls = (rng.standard_normal((2, 256)) * 0.5).astype(np.float32)
    g["rt_logits_sg"] = ls
    g["rt_ids_sg"], g["rt_w_sg"], _, _ = orc.route_topk(ls, 6, 1, True)
    # expert GEMVs per K-quant type: 4 experts [16 rows][512 cols], Q8_1 x (kernel_parity recipe: N(0,1) * 0.5)
    ncols, nrows, ne = 512, 16, 4
    xv = (rng.standard_normal((2, ncols)) * 0.5).astype(np.float32)
    xq = orc.quantize_q8_1(xv)
    g["mv_xq"] = xq
    ids = np.array([REF_IDS[i] % ne for i in range(4)], dtype=np.int32)  # [0, 3, 1, 0]
    g["mv_ids"] = ids
    for t in (orc.Q3_K, orc.Q4_K, orc.Q5_K, orc.Q6_K):
        w = (rng.standard_normal((ne, nrows, ncols)) * 0.02).astype(np.float32)
        q = orc.quantize(t, w).reshape(ne, nrows, -1)
        g[f"mv_w_{t}"] = q
        # channel c reads x row c % 2 (mmvq_experts semantics with n_xq = 2)
        g[f"mv_dst_{t}"] = orc.mmvq_experts(t, list(q), ncols, nrows, xq, 2, 1, ids)
    # combine in slot order with guard scales and residual
    dexp = (rng.standard_normal((2, 8, 64))).astype(np.float32)
    wv = np.abs(rng.standard_normal((2, 8))).astype(np.float32)
    es = np.array([[1, 2, 1, 1, 4, 1, 1, 1], [1] * 8], dtype=np.float32)
    xr = rng.standard_normal((2, 64)).astype(np.float32)
    g["cb_dexp"], g["cb_w"], g["cb_e"], g["cb_x"] = dexp, wv, es, xr
    g["cb_out"] = orc.moe_combine(dexp, wv, es, None, xr)
    # expert-id compaction of 5 tokens x top-8 of 16 experts (the prefill sort)
    cid = np.stack([rng.permutation(16)[:8] for _ in range(5)]).astype(np.int32)
    g["cp_ids"] = cid
    g["cp_bounds"], g["cp_src"], g["cp_dst"], _ = orc.compact_ids(cid, 16, 1)
    return g


if __name__ == "__main__":
    out = Path(__file__).resolve().parent / "golden.npz"
    np.savez_compressed(out, **make())
    print(f"wrote {out} ({out.stat().st_size} bytes)")
