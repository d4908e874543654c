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


REL_TOL = 1e-3      # the north_star's element-wise max relative error
REL_FLOOR = 1e-2    # ... with |ref| floored at 1% of max|ref| (elements near zero carry only absolute error)


def max_rel_err(y: np.ndarray, ref: np.ndarray, floor: float = REL_FLOOR) -> float:
    """Element-wise max |y - ref| / max(|ref|, floor * max|ref|)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.maximum(np.abs(ref), floor * max(np.abs(ref).max(), 1e-30))
    return float((np.abs(y - ref) / den).max())


def assert_close(y, ref, what: str, max_tol: float = MAX_TOL, l2_tol: float = L2_TOL, rel_tol: float = REL_TOL) -> None:
    m, l2, r = norm_max_err(y, ref), rel_l2(y, ref), max_rel_err(y, ref)
    assert m <= max_tol and l2 <= l2_tol and r <= rel_tol, (
        f"{what}: normalised max err {m:.3e} (tol {max_tol}), rel L2 {l2:.3e} (tol {l2_tol}), "
        f"max rel err {r:.3e} (tol {rel_tol}, floor {REL_FLOOR} max|ref|)")


# An oracle chain that computes its own fp32 act (instead of taking the GPU's) can round a Q8_1 code of act one step
# the other way where the two fp32 sums differ in their last bits (different summation orders). One such step moves
# an output element by d_act * |W_down| - about 4e-4 of max|out| here, a few percent of an element near 1% of
# max|out|. Such chains are held to the north_star's 1e-3 normalised bound, rel L2 5e-4 (the reference holds its MMQ
# against its MMVQ to per-row rel L2 < 2e-2, tests/mmq_parity.cu:107) and this element-wise bound; the chains fed with
# the GPU's own act are held to the tight bounds above.
CHAIN_MAX_TOL, CHAIN_L2_TOL, CHAIN_REL_TOL = 1e-3, 5e-4, 5e-2


def assert_close_chain(y, ref, what: str) -> None:
    assert_close(y, ref, what + " (independent chain)", CHAIN_MAX_TOL, CHAIN_L2_TOL, CHAIN_REL_TOL)


def image_to_q8_1(img: np.ndarray, ncols: int) -> np.ndarray:
    """Inverse of split_image for the values: Q8_1 blocks ([rows][q8_1 row bytes]: f16 d, sum field 0, int8 q) whose
    q * d are the image's hi + lo (d = max|q d| / 127, exact: the block maximum has |q| = 127)."""
    rows = img.shape[0]
    nb = ncols // 256
    main = img[:, : nb * 1024].view(np.float16).astype(np.float32).reshape(rows, nb, 2, 2, 16, 8)
    perm = np.array([0, 2, 1, 3, 4, 6, 5, 7])
    v = (main[:, :, :, 0] + main[:, :, :, 1])[..., perm].reshape(rows, ncols // 32, 32).astype(np.float64)
    d = np.abs(v).max(axis=2) / 127.0
    q = np.where(d[..., None] > 0, np.rint(v / np.where(d > 0, d, 1.0)[..., None]), 0.0)
    assert np.array_equal(q * d[..., None], v), "image values are not q * d"
    out = np.zeros((rows, orc.q8_1_row_bytes(ncols)), np.uint8)
    blk = out[:, : (ncols // 32) * 36].reshape(rows, ncols // 32, 36)
    blk[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(rows, ncols // 32, 2)
    blk[:, :, 4:36] = q.astype(np.int8).view(np.uint8)
    return out


def split_image(xq: np.ndarray, ncols: int) -> np.ndarray:
    """The prefill GEMM's split activation image rows (uint8 [rows][ncols / 256 * 1056]) that Q8_1 blocks `xq`
    ([rows][q8_1 row bytes], the oracle's quantize_q8_1) must produce, byte for byte: per 256-column superblock kb, at
    kb * 1024 two 128-column halves [hi 128 f16][lo 128 f16] of q * d (d the block's f16 scale; hi = f16(q d),
    lo = f16(q d - hi)); then at nb * 1024 + 32 kb the sums S_s = d_s * sum(q of block s) as [hi 8 f16][lo 8 f16].
    Within every 8 columns and every 8 sums the order is 0 2 1 3 4 6 5 7."""
    rows = xq.shape[0]
    nblk = ncols // 32
    blk = xq[:, : nblk * 36].reshape(rows, nblk, 36)
    d = blk[:, :, 0:2].copy().view(np.float16)[:, :, 0].astype(np.float32)           # [rows][nblk]
    q = blk[:, :, 4:36].view(np.int8).astype(np.float32)                              # [rows][nblk][32]
    x = (q * d[:, :, None]).reshape(rows, ncols)                                       # exact in f32
    hi = x.astype(np.float16)
    lo = (x - hi.astype(np.float32)).astype(np.float16)
    perm = np.array([0, 2, 1, 3, 4, 6, 5, 7])
    nb = ncols // 256
    main = np.empty((rows, nb, 2, 2, 16, 8), np.float16)  # [sb][half][hi/lo][group of 8][8]
    for part, arr in ((0, hi), (1, lo)):
        a = arr.reshape(rows, nb, 2, 16, 8)
        main[:, :, :, part] = a[..., perm]
    sums = (q.sum(axis=2) * d).astype(np.float32).reshape(rows, nb, 8)               # exact (|sum q| < 2^12)
    shi = sums.astype(np.float16)
    slo = (sums - shi.astype(np.float32)).astype(np.float16)
    mins = np.stack([shi[..., perm], slo[..., perm]], axis=2)                           # [rows][nb][2][8]
    return np.concatenate([main.reshape(rows, -1).view(np.uint8), mins.reshape(rows, -1).view(np.uint8)], axis=1)


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
