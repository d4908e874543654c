"""fns_hip_moe_layer_noalloc (the layer with its workspace in a device array inside the library, for callers that
cannot allocate) against fns_hip_moe_layer with a caller workspace, through the C ABI: bit for bit on two calls in a
row, the second smaller (4-token verify, then batch-1 decode of another layer), and the size limit."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from flintnsteel_amd import _lib

pytestmark = pytest.mark.gpu

H, F, NE, K = 2048, 768, 128, 8
SEED = 20261022


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def noalloc(layer, x: torch.Tensor, resid: torch.Tensor | None = None) -> torch.Tensor:
    out = torch.full_like(x, float("nan"))
    n_tok = x.numel() // layer.desc.hidden
    rc = _lib.lib().fns_hip_moe_layer_noalloc(ctypes.byref(layer.desc), ctypes.c_void_p(x.data_ptr()),
                                              ctypes.c_void_p(resid.data_ptr()) if resid is not None else None,
                                              ctypes.c_void_p(out.data_ptr()), n_tok, _stream())
    _lib.check(rc, "fns_hip_moe_layer_noalloc")
    return out


def test_noalloc_matches_workspace_entry_point():
    from flintnsteel_amd import synth
    big = synth.build_layer(H, F, NE, K, 12, 14, SEED, layer=31)
    small = synth.build_layer(1024, 512, 64, 6, 13, 12, SEED, layer=32, gating=1)
    x4 = synth.activations(4, H, SEED, layer=33)
    x1 = synth.activations(1, 1024, SEED, layer=34)
    r1 = synth.activations(1, 1024, SEED, layer=35)
    got4 = noalloc(big, x4)          # first call: 4 tokens (verify path)
    got1 = noalloc(small, x1, r1)    # second call: smaller (1 token of a smaller layer, residual add)
    got1b = noalloc(small, x1, r1)   # and again: the scratch keeps the previous call's contents
    ref4 = big(x4, ws=big.workspace(4))
    ref1 = small(x1, ws=small.workspace(1), x_resid=r1)
    torch.cuda.synchronize()
    assert np.array_equal(got4.cpu().numpy(), ref4.cpu().numpy())
    assert np.array_equal(got1.cpu().numpy(), ref1.cpu().numpy())
    assert np.array_equal(got1b.cpu().numpy(), ref1.cpu().numpy())


def test_noalloc_rejects_layers_beyond_the_scratch():
    from flintnsteel_amd import ops
    L = _lib.lib()
    limit = L.fns_hip_moe_noalloc_max_bytes()
    assert limit == 4 << 20
    d = ops.MoeLayerDesc(2048, 16384, 128, 16, 0, 1, 0, 0, ctypes.c_void_p(0x1000), 12, 12,
                         ctypes.c_void_p(0x1000), 0, 0, 0)
    x = torch.zeros(4, 2048, device="cuda")
    rc = L.fns_hip_moe_layer_noalloc(ctypes.byref(d), ctypes.c_void_p(x.data_ptr()), None,
                                     ctypes.c_void_p(x.data_ptr()), 4, _stream())
    assert rc == -4 and b"device scratch" in L.fns_hip_last_error()
