"""Shared test helpers: seeded synthetic inputs quantised by the CPU oracle, and error metrics.

Tolerance policy (written here once, used by every parity test):
  - integer / byte / index results (Q8_1 blocks, expert ids, compaction) must be bit-exact;
  - fp32 outputs against the float64 oracle on identical quantised blocks and identical Q8_1 activations:
    normalised max error max|y - ref| / max|ref| <= 1e-4 and relative L2 <= 1e-5. The north_star bound is 1e-3 max
    relative error; the reference's own threshold is relative L2 < 1e-4 against the Q8_1-quantised input
    (reference tests/kernel_parity.py:13,86-88). Both are looser than what fp32 accumulation of exact integer
    sub-block dots gives, so the tighter bound is used and a real indexing mistake still shows as an O(1) error.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as orc

MAX_TOL = 1e-4
L2_TOL = 1e-5


def norm_max_err(y: np.ndarray, ref: np.ndarray) -> float:
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def rel_l2(y: np.ndarray, ref: np.ndarray) -> float:
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30))


def assert_close(y, ref, what: str, max_tol: float = MAX_TOL, l2_tol: float = L2_TOL) -> None:
    m, l2 = norm_max_err(y, ref), rel_l2(y, ref)
    assert m <= max_tol and l2 <= l2_tol, f"{what}: normalised max err {m:.3e} (tol {max_tol}), rel L2 {l2:.3e} (tol {l2_tol})"


def gaussian(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    return (rng.standard_normal(shape) * std).astype(np.float32)


def make_expert_mats(qtype: int, n_expert: int, nrows: int, ncols: int, seed: int, std: float = 0.02) -> np.ndarray:
    """uint8 [n_expert][nrows * row_bytes]: N(0, std) fp32 quantised with the oracle's ggml reference quantiser."""
    rng = np.random.default_rng(seed)
    w = gaussian(rng, (n_expert, nrows, ncols), std)
    q = orc.quantize(qtype, w)
    return q.reshape(n_expert, -1)


def expert_rows(mats: np.ndarray, e: int, nrows: int) -> np.ndarray:
    return mats[e].reshape(nrows, -1)
