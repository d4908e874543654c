"""Device-side synthetic data: the GPU K-quant quantisers must produce the same bytes as the CPU oracle's
restatement of ggml's reference quantisers; the Philox normal generator must be seeded, reproducible, chunkable
and N(0, 1)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.helpers import gaussian

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from flintnsteel_amd import ops as o
    return o


@pytest.mark.parametrize("qtype", [orc.Q3_K, orc.Q4_K, orc.Q5_K, orc.Q6_K])
def test_gpu_quantizer_equals_oracle(ops, qtype):
    rng = np.random.default_rng(qtype + 100)
    w = gaussian(rng, (96, 1024), 0.02)
    w[0] = 0.0                                  # zero blocks
    w[1] = 0.013                                # constant blocks
    w[2, 5] = 3.0                               # an outlier
    w[3] = gaussian(rng, (1024,), 1e-20)        # below GROUP_MAX_EPS-scale magnitudes
    w[4, :256] = np.linspace(-1, 1, 256)
    got = ops.quantize_weights(qtype, torch.from_numpy(w).cuda()).cpu().numpy()
    ref = orc.quantize(qtype, w)
    assert got.shape == ref.shape
    bad = np.nonzero((got != ref).any(1))[0]
    assert bad.size == 0, f"rows differing from the oracle quantiser: {bad[:10]}"


def test_fill_normal(ops):
    n = 1 << 22
    a = ops.fill_normal(torch.empty(n, device="cuda"), seed=20261022)
    b = ops.fill_normal(torch.empty(n, device="cuda"), seed=20261022)
    c = ops.fill_normal(torch.empty(n, device="cuda"), seed=20261023)
    assert torch.equal(a, b) and not torch.equal(a, c)
    # chunked generation (offset) equals one-shot generation
    part = ops.fill_normal(torch.empty(1000, device="cuda"), seed=20261022, offset=4096)
    assert torch.equal(part, a[4096:5096])
    m, s = a.double().mean().item(), a.double().std().item()
    assert abs(m) < 3e-3 and abs(s - 1) < 3e-3
    # fourth moment of a normal is 3
    k4 = (a.double() ** 4).mean().item()
    assert abs(k4 - 3.0) < 0.03
    scaled = ops.fill_normal(torch.empty(n, device="cuda"), seed=1, mean=0.5, std=0.02)
    assert abs(scaled.double().mean().item() - 0.5) < 1e-4 and abs(scaled.double().std().item() - 0.02) < 1e-4
