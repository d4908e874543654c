"""Test data for the IQ formats: seeded codebooks of ggml's shapes and value sets, and random IQ blocks.

ggml's own codebooks (iq3xxs_grid, iq3s_grid, iq2s_grid of ggml-common.h, llama.cpp 19ab5a5e) are not in this
container. The tests register tables of the same sizes whose bytes are drawn from the same value sets (IQ3_XXS: the
8 levels 4, 12, ..., 52, 62; IQ3_S: the odd values 1..15; IQ2_S: 8, 25, 43), in both the oracle and the library, so
kernel parity is pinned for any codebook; agreement with ggml's particular tables is not.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as orc

IQ3XXS_LEVELS = np.array([4, 12, 20, 28, 36, 44, 52, 62], np.uint8)
IQ3S_LEVELS = np.arange(1, 16, 2, dtype=np.uint8)
IQ2S_LEVELS = np.array([8, 25, 43], np.uint8)


def synthetic_grids(seed: int = 11):
    rng = np.random.default_rng(seed)
    a = rng.choice(IQ3XXS_LEVELS, size=(256, 4)).view(np.uint32).reshape(256)
    b = rng.choice(IQ3S_LEVELS, size=(512, 4)).view(np.uint32).reshape(512)
    c = rng.choice(IQ2S_LEVELS, size=(1024, 8)).view(np.uint64).reshape(1024)
    return a, b, c


def register_grids(seed: int = 11):
    """Registers the same codebooks in the oracle and (when loaded) the HIP library; returns them."""
    grids = synthetic_grids(seed)
    orc.set_iq_grids(*grids)
    return grids


def register_grids_in_library(grids) -> None:
    import ctypes
    from flintnsteel_amd._lib import call
    a, b, c = (np.ascontiguousarray(g) for g in grids)
    call("fns_hip_set_iq_grids", a.ctypes.data_as(ctypes.c_void_p), b.ctypes.data_as(ctypes.c_void_p),
         c.ctypes.data_as(ctypes.c_void_p))


# f16 d of each format chosen so the decoded weights are of the order of N(0, 0.02)
D_SCALE = {orc.IQ4_XS: 1.5e-5, orc.IQ3_XXS: 4e-5, orc.IQ3_S: 4e-5, orc.IQ2_S: 1.2e-4}


def random_blocks(qtype: int, nrows: int, ncols: int, seed: int) -> np.ndarray:
    """uint8 [nrows][row_bytes]: random IQ blocks (every index, sign and scale field random) with d > 0."""
    rng = np.random.default_rng(seed)
    nb = nrows * ncols // 256
    bb = orc.BLOCK_BYTES[qtype]
    blk = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    d = (D_SCALE[qtype] * rng.uniform(0.5, 1.5, nb)).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    return blk.reshape(nrows, ncols // 256 * bb)
