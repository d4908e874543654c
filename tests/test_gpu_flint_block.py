"""The reference model's whole MoE block as one call (Engine::ffn_block, src/engine.cu:655-696; the prefill form
src/engine.cu:331-357): RMSNorm of the residual stream, bf16 router with sigmoid gating over 256 experts, top-6
normalised, expert width 512 (src/model.cpp:159-164), F16 guard, and the shared expert (width 1024) whose output
joins the combine as out = (moe + sh) + x. Decode (fused kernel), the 4-token verify step and prefill (MMQ) against
the float64 oracle chain.

Bars: the RMSNorm output and its Q8_1 equal the standalone rms_norm_q8_1 kernel's (pinned against float64 in
test_gpu_kernels); routing bit-exact given the layer's logits; the block output within the north_star's 1e-3 of the
float64 chain (its shared expert re-quantises its own act, so a Q8_1 code can differ by one step).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.helpers import assert_close, assert_close_chain

pytestmark = pytest.mark.gpu

H, F, NE, K, FS = 2048, 512, 256, 6, 1024
SEED = 20261022
GU, DN = orc.Q4_K, orc.Q5_K


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.fixture(scope="module")
def ops():
    from flintnsteel_amd import ops as o
    return o


@pytest.fixture(scope="module")
def layer():
    from flintnsteel_amd import synth
    return synth.build_flint_layer(H, F, NE, K, FS, GU, DN, SEED, layer=21)


@pytest.fixture(scope="module")
def mats(layer):
    slots = {k: layer.slots.view(k).cpu().numpy() for k in ("gate", "up", "down")}
    sh = {k: host(layer.shexp[k]).reshape(H if k == "down" else FS, -1) for k in ("gate", "up", "down")}
    return slots, sh


def mv(qtype, m, ncols, nrows, xq_row):
    return orc.mmvq_experts(qtype, [m], ncols, nrows, xq_row[None], 1, 1, np.zeros(1, np.int32))[0]


def block_ref(mats, h: np.ndarray, ids: np.ndarray, w: np.ndarray, resid: np.ndarray, sgu: int = GU,
              sdn: int = DN) -> np.ndarray:
    """float64 chain of the whole block for given h and routing (each act re-quantised from its own fp32 value)."""
    slots, sh = mats
    xq = orc.quantize_q8_1(h)
    out = np.zeros((h.shape[0], H))
    for t in range(h.shape[0]):
        for j in range(K):
            e = int(ids[t, j])
            g = mv(GU, slots["gate"][e].reshape(F, -1), H, F, xq[t])
            u = mv(GU, slots["up"][e].reshape(F, -1), H, F, xq[t])
            act = orc.swiglu(g, u).astype(np.float32)
            esc = orc.amax_guard_scale(act)
            aq = orc.quantize_q8_1((act / np.float32(esc)).astype(np.float32)[None])[0]
            out[t] += mv(DN, slots["down"][e].reshape(H, -1), F, H, aq) * esc * float(w[t, j])
        act_sh = orc.swiglu(mv(sgu, sh["gate"], H, FS, xq[t]), mv(sgu, sh["up"], H, FS, xq[t])).astype(np.float32)
        out[t] += mv(sdn, sh["down"], FS, H, orc.quantize_q8_1(act_sh[None])[0])
    return out + resid


def check_front(ops, layer, x: torch.Tensor, logits: np.ndarray, xq_layer: np.ndarray | None, bf16_x: bool):
    """RMSNorm output via the standalone kernel; Q8_1 of h equal to the layer's; logits; routing from the logits."""
    h_d, xq_d = ops.rms_norm_q8_1(x, layer.ffn_norm, 1e-6)
    h = host(h_d)
    if xq_layer is not None:
        assert np.array_equal(xq_layer, host(xq_d)), "Q8_1 of h differs from rms_norm_q8_1's"
    w32 = layer.router_w.float().cpu().numpy()
    hr = torch.from_numpy(h).to(torch.bfloat16).float().numpy() if bf16_x else h
    ref = orc.router_f32(w32, hr)
    assert np.abs(logits - ref).max() <= 1e-4 * np.abs(ref).max()
    ids, w, _, _ = orc.route_topk(logits, K, 1, True)
    return h, ids, w


def test_flint_block_decode(ops, layer, mats):
    from flintnsteel_amd import synth
    x = synth.activations(1, H, SEED, layer=31)
    ws = layer.workspace(1)
    out = host(layer(x, ws=ws, x_resid=x))
    tr = {k: host(v) for k, v in layer.trace(ws, 1).items()}
    h, ids, w = check_front(ops, layer, x, tr["logits"], tr["xq"], bf16_x=False)
    assert np.array_equal(ids, tr["ids"]) and np.array_equal(w.view(np.uint32), tr["w"].view(np.uint32))
    ref = block_ref(mats, h, ids, w, host(x))
    assert_close_chain(out, ref, "flint block decode")


def test_flint_block_in_place(ops, layer):
    """out aliasing x (the reference's x_ += ...): same result as a separate output buffer."""
    from flintnsteel_amd import synth
    x = synth.activations(1, H, SEED, layer=32)
    ws = layer.workspace(1)
    sep = host(layer(x, ws=ws, x_resid=x))
    xi = x.clone()
    layer(xi, out=xi, ws=ws, x_resid=xi)
    assert np.array_equal(host(xi), sep)


def test_flint_block_verify_columns(ops, layer, mats):
    """4-token verify step: each column bit-identical to its batch-1 run (routed and shared experts)."""
    from flintnsteel_amd import synth
    x4 = synth.activations(4, H, SEED, layer=33)
    ws4 = layer.workspace(4)
    out4 = host(layer(x4, ws=ws4, x_resid=x4))
    tr4 = {k: host(v) for k, v in layer.trace(ws4, 4).items()}
    for t in range(4):
        xt = x4[t:t + 1].contiguous()
        ws1 = layer.workspace(1)
        out1 = host(layer(xt, ws=ws1, x_resid=xt))
        assert np.array_equal(out4[t], out1[0]), f"column {t}"
    h, ids, w = check_front(ops, layer, x4, tr4["logits"], tr4["xq"], bf16_x=False)
    assert np.array_equal(ids, tr4["ids"])
    assert_close_chain(out4, block_ref(mats, h, ids, w, host(x4)), "flint block verify")


def test_flint_block_prefill(ops, layer, mats):
    from flintnsteel_amd import synth
    T = 70
    pre = ops.MoePrefill(layer)
    x = synth.activations(T, H, SEED, layer=34)
    ws = pre.workspace(T)
    out = host(pre(x, ws=ws, x_resid=x))
    tr = {k: host(v) for k, v in pre.trace(ws, T).items()}
    h, ids, w = check_front(ops, layer, x, tr["logits"], None, bf16_x=True)
    assert np.array_equal(ids, tr["ids"]) and np.array_equal(w, tr["w"])
    toks = [0, 1, 33, 64, 69]
    ref = block_ref(mats, h[toks], ids[toks], w[toks], host(x)[toks])
    assert_close_chain(out[toks], ref, "flint block prefill")


def test_flint_block_shared_types_differ(ops, layer, mats):
    """A shared expert whose types differ from the routed ones (Q6_K gate/up, Q4_K down) is not fused into the decode
    kernel: the dense-mode gate/up and down kernels compute it, at one token and at four."""
    from flintnsteel_amd import synth
    sgu, sdn = orc.Q6_K, orc.Q4_K
    seed = synth.tensor_seed(SEED, 22, synth.KIND_SHEXP)
    g = torch.empty(1, ops.row_bytes(sgu, H) * FS, dtype=torch.uint8, device="cuda")
    u = torch.empty_like(g)
    d = torch.empty(1, ops.row_bytes(sdn, FS) * H, dtype=torch.uint8, device="cuda")
    synth.quantized_matrices(sgu, 1, FS, H, seed, 0.02, g)
    synth.quantized_matrices(sgu, 1, FS, H, seed + 1, 0.02, u)
    synth.quantized_matrices(sdn, 1, H, FS, seed + 2, 0.02, d)
    shexp = {"gate": g, "up": u, "down": d, "inter": FS, "gu_type": sgu, "down_type": sdn}
    lay2 = ops.MoeLayer(layer.router_w, layer.slots, GU, DN, H, F, K, gating=ops.GATING_SIGMOID, guard=True,
                        ffn_norm=layer.ffn_norm, norm_eps=1e-6, shexp=shexp)
    sh_np = {"gate": host(g).reshape(FS, -1), "up": host(u).reshape(FS, -1), "down": host(d).reshape(H, -1)}
    x4 = synth.activations(4, H, SEED, layer=35)
    out4 = host(lay2(x4, ws=lay2.workspace(4), x_resid=x4))
    for t in range(4):
        xt = x4[t:t + 1].contiguous()
        ws1 = lay2.workspace(1)
        out1 = host(lay2(xt, ws=ws1, x_resid=xt))
        assert np.array_equal(out4[t], out1[0]), f"column {t}"
        tr = {k: host(v) for k, v in lay2.trace(ws1, 1).items()}
        h, ids, w = check_front(ops, lay2, xt, tr["logits"], tr["xq"], bf16_x=False)
        ref = block_ref((mats[0], sh_np), h, ids, w, host(xt), sgu, sdn)
        assert_close_chain(out1, ref, f"flint block, shared {orc.TYPE_NAMES[sgu]}/{orc.TYPE_NAMES[sdn]}")
