"""The decode layer's two paths through the C ABI, bit for bit: the two-kernel path (router kernel + fused layer
kernel, which the library takes for one token when all its workgroups can be resident) and the three-kernel path
(router, gate/up, down), on every type mix the fused kernel holds. Both restate the same per-(row, slot) arithmetic;
tests/test_gpu_moe_layer.py holds them against the CPU oracle. Also: a HIP graph of several layers replayed with eager
work between the replays, and the workspace's fixed header (the status word sits at the same place for every layer
shape, so a workspace or the no-allocation scratch shared by shapes keeps it).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

H, F, NE, K = 2048, 768, 128, 8
SEED = 20261022
TRACE = ("logits", "xq", "ids", "w", "act", "escale")


@pytest.fixture(scope="module")
def ops():
    from flintnsteel_amd import ops as o
    return o


@pytest.fixture(scope="module")
def synth():
    from flintnsteel_amd import synth as s
    return s


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def run(layer, x, path, ops, x_resid=None, ws=None):
    ws = layer.workspace(1) if ws is None else ws
    with ops.decode_path(path):
        out = host(layer(x, ws=ws, x_resid=x_resid))
    return out, {k: host(v) for k, v in layer.trace(ws, 1).items()}


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


CASES = {
    "cfg0_q4k": (12, 12),
    "cfg1_q3k_q5k": (11, 13),
    "cfg3_q4k_q6k": (12, 14),
    "q6k_q3k": (14, 11),
    "q5k_q4k": (13, 12),
    "q8_0": (8, 8),
}


def test_kernel_count(ops, synth):
    layer = synth.build_layer(H, F, NE, K, 12, 12, SEED, layer=41)
    assert layer.kernels(1) == 2, "config 0 at one token should take the fused kernel on an MI355X"
    assert layer.kernels(4) == 3
    with ops.decode_path(ops.PATH_THREE_KERNELS):
        assert layer.kernels(1) == 3


@pytest.mark.parametrize("case", list(CASES))
def test_fused_equals_three_kernel(ops, synth, case):
    gu, dn = CASES[case]
    layer = synth.build_layer(H, F, NE, K, gu, dn, SEED, layer=40 + gu + dn)
    x = synth.activations(1, H, SEED, layer=43)
    resid = synth.activations(1, H, SEED, layer=44)
    out2, tr2 = run(layer, x, ops.PATH_AUTO, ops, x_resid=resid)
    out3, tr3 = run(layer, x, ops.PATH_THREE_KERNELS, ops, x_resid=resid)
    assert np.isfinite(out2).all()
    for name in TRACE:
        assert same_bits(tr2[name], tr3[name]), f"{case}: {name} differs between the paths"
    assert same_bits(out2, out3), f"{case}: output differs between the paths"


def test_graph_replays_match_eager(ops, synth):
    """Four layers captured in a HIP graph (one workspace each) and replayed 5 times with eager work and
    synchronisations between the replays: every replay equals the eager result bit for bit, the status words stay 0."""
    layers = [synth.build_layer(H, F, NE, K, 12, 12, SEED, layer=60 + l) for l in range(4)]
    xs = [synth.activations(1, H, SEED, layer=70 + l) for l in range(4)]
    wss = [layer.workspace(1) for layer in layers]
    outs = [torch.empty(1, H, device="cuda") for _ in layers]
    eager = [host(layer(x, ws=layer.workspace(1))) for layer, x in zip(layers, xs)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for layer, x, o, w in zip(layers, xs, outs, wss):
            layer(x, out=o, ws=w)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for layer, x, o, w in zip(layers, xs, outs, wss):
            layer(x, out=o, ws=w)
    for rep in range(5):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for l in range(4):
            assert same_bits(host(outs[l]), eager[l]), f"replay {rep} layer {l}"
        _ = layers[0](xs[1], ws=layers[0].workspace(1))  # eager work between replays
        torch.cuda.synchronize()
    for w, layer in zip(wss, layers):
        assert layer.status(w) == 0


def _noalloc(layer, x: torch.Tensor) -> torch.Tensor:
    from flintnsteel_amd import _lib
    out = torch.full_like(x, float("nan"))
    n_tok = x.numel() // layer.desc.hidden
    rc = _lib.lib().fns_hip_moe_layer_noalloc(ctypes.byref(layer.desc), ctypes.c_void_p(x.data_ptr()), None,
                                              ctypes.c_void_p(out.data_ptr()), n_tok,
                                              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "fns_hip_moe_layer_noalloc")
    return out


def test_status_word_shared_by_shapes(ops, synth):
    """Calls of layers of different shapes and token counts alternate on the no-allocation scratch (and on one caller
    workspace): the status word stays 0 through all of them, every result equals the layer's own workspace result,
    and after a forced timeout (test hooks) the word is set and stays set through later calls of other shapes, until
    cleared."""
    from flintnsteel_amd._lib import call
    big = synth.build_layer(H, F, NE, K, 12, 14, SEED, layer=90)
    small = synth.build_layer(1024, 512, 64, 6, 13, 12, SEED, layer=91, gating=1)
    xb1 = synth.activations(1, H, SEED, layer=92)
    xb4 = synth.activations(4, H, SEED, layer=93)
    xs1 = synth.activations(1, 1024, SEED, layer=94)
    refs = {"b1": host(big(xb1, ws=big.workspace(1))), "b4": host(big(xb4, ws=big.workspace(4))),
            "s1": host(small(xs1, ws=small.workspace(1)))}
    calls = [("b1", big, xb1), ("s1", small, xs1), ("b4", big, xb4), ("s1", small, xs1), ("b1", big, xb1)]
    # one caller workspace big enough for every call
    ws = torch.zeros(max(big.workspace_layout(4)[1], small.workspace_layout(1)[1]), dtype=torch.uint8, device="cuda")
    for name, layer, x in calls:
        assert same_bits(host(layer(x, ws=ws)), refs[name]), f"shared workspace: {name}"
        assert big.status(ws, 1) == 0 and small.status(ws, 1) == 0 and big.status(ws, 4) == 0
    big.status(None, 1, clear=True)
    for name, layer, x in calls:
        assert same_bits(host(_noalloc(layer, x)), refs[name]), f"no-allocation scratch: {name}"
        assert big.status(None, 1) == 0 and small.status(None, 1) == 0 and big.status(None, 4) == 0
    try:
        call("fns_hip_moe_set_test_hooks", 64, 1)
        bad = host(_noalloc(big, xb1))
    finally:
        call("fns_hip_moe_set_test_hooks", 0, 0)
    assert np.isnan(bad).all()
    assert big.status(None, 1) == ops.STATUS_EXCHANGE_TIMEOUT
    for name, layer, x in calls:  # other shapes do not erase it
        assert same_bits(host(_noalloc(layer, x)), refs[name])
        assert small.status(None, 1) == ops.STATUS_EXCHANGE_TIMEOUT and big.status(None, 4) == ops.STATUS_EXCHANGE_TIMEOUT
    assert small.status(None, 1, clear=True) == ops.STATUS_EXCHANGE_TIMEOUT
    assert big.status(None, 1) == 0


def test_status_collect_in_graph(ops, synth):
    """fns_hip_moe_layer_status_collect captured in a HIP graph after the layer, into pinned host memory: clean
    replays leave it 0; after an eager call that times out (test hooks), a replay of a graph holding only the collect
    ORs the bit in and clears the word, and the next replays stay clean and equal the first."""
    from flintnsteel_amd._lib import call
    layer = synth.build_layer(H, F, NE, K, 12, 12, SEED, layer=950)
    x = synth.activations(1, H, SEED, layer=951)
    ws = layer.workspace(1)
    out = torch.empty(1, H, device="cuda")
    dst = torch.zeros(1, dtype=torch.int32).pin_memory()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer(x, out=out, ws=ws)
        layer.status_collect(ws, dst)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    ref = host(out)
    g, gc = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer(x, out=out, ws=ws)
        layer.status_collect(ws, dst)
    with torch.cuda.graph(gc):
        layer.status_collect(ws, dst)
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert int(dst[0]) == 0 and same_bits(host(out), ref), f"clean replay {rep}"
    print("forced exchange timeout (withheld arrivals, poll limit 64)", flush=True)
    call("fns_hip_moe_set_test_hooks", 64, 1)
    try:
        bad = host(layer(x, ws=ws))
    finally:
        call("fns_hip_moe_set_test_hooks", 0, 0)
    assert np.isnan(bad).all()
    gc.replay()
    torch.cuda.synchronize()
    assert int(dst[0]) == ops.STATUS_EXCHANGE_TIMEOUT and layer.status(ws, 1) == 0
    dst.zero_()
    for rep in range(2):
        g.replay()
        torch.cuda.synchronize()
        assert int(dst[0]) == 0 and same_bits(host(out), ref), f"replay {rep} after the timeout"


@pytest.mark.parametrize("n_tok", [1, 4])
def test_prefetch_hint_changes_nothing(ops, synth, n_tok):
    """The read-ahead hint (FnsMoeLayer.prefetch: the next layer's router) leaves every output and intermediate
    bit-identical, for sizes below, at and above the router kernel's two loads per thread and not a multiple of 16."""
    print(f"prefetch hint n_tok={n_tok}", flush=True)
    a = synth.build_layer(H, F, NE, K, 12, 12, SEED, layer=901)
    b = synth.build_layer(H, F, NE, K, 12, 12, SEED, layer=902)
    x = synth.activations(n_tok, H, SEED, layer=903)
    ws = a.workspace(n_tok)
    ref = host(a(x, ws=ws))
    ref_tr = {k: host(v).copy() for k, v in a.trace(ws, n_tok).items()}
    big = torch.zeros(5 << 20, dtype=torch.uint8, device="cuda")
    for ptr, nbytes in ((b.router_w.data_ptr(), b.router_w.numel() * 4), (b.router_w.data_ptr(), 1000),
                        (big.data_ptr(), big.numel() - 7), (b.router_w.data_ptr(), 0)):
        a.desc.prefetch, a.desc.prefetch_bytes = ptr, nbytes
        ws.zero_()
        out = host(a(x, ws=ws))
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), f"prefetch {nbytes} B: output differs"
        for k, v in a.trace(ws, n_tok).items():
            assert np.array_equal(host(v), ref_tr[k]), f"prefetch {nbytes} B: {k} differs"
    a.desc.prefetch, a.desc.prefetch_bytes = None, 0
