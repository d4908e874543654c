"""Pins the CPU oracle (oracle/fns_oracle.c) before it is trusted as the checker.

The reference holds no golden vectors for this path (its parity programs need a GPU and the real GGUF files),
so each oracle function is pinned here by what fixes it independently:
  - half precision: exhaustively against numpy's IEEE float16;
  - exp: against float64 math.exp (<= 2 ulp);
  - block dequantisation: hand-built blocks with hand-computed values (the scale/min bit packing, nibble and
    high-bit positions of each K-quant layout);
  - weight quantisers: round-trip error bounds typical of each format and the zero block;
  - Q8_1: literal rounding cases (half away from zero, as the reference's roundf), invariants, exact sums;
  - gating/top-k: float64 softmax/sigmoid, brute-force stable sort, the renormalisation clamp;
  - compaction: brute-force stable grouping; combine and F16 guard: literal cases;
  - GEMV: a hand-built row whose dot product is known in closed form.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import gaussian


def f16(v: float) -> int:
    return int(np.float16(v).view(np.uint16))


# ---- half precision and exp ----------------------------------------------------------------------------------

def test_f16_to_f32_exhaustive():
    L = orc.lib()
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32).view(np.uint32)
    got = np.array([L.or_f16_to_f32(int(v)) for v in h], dtype=np.float32).view(np.uint32)
    nan = np.isnan(h.view(np.float16))
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.isnan(got.view(np.float32)[nan]).all()


def test_f32_to_f16_round_to_nearest_even():
    L = orc.lib()
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(50000) * rng.choice([1e-7, 1e-5, 1e-2, 1, 1e2, 6e4, 7e4], 50000)).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08,
                      1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, np.inf, -np.inf], dtype=np.float32)
    x = np.concatenate([x, edges])
    got = np.array([L.or_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_expf_within_2ulp():
    L = orc.lib()
    xs = np.concatenate([np.linspace(-103.9, 88.7, 20011), np.linspace(-1, 1, 2001)]).astype(np.float32)
    worst = 0.0
    for x in xs:
        got = np.float32(L.or_expf(float(x)))
        ref = math.exp(float(x))
        if ref < 1.2e-38:  # subnormal range: absolute error
            assert abs(float(got) - ref) <= 2 * 1.4e-45
            continue
        ulp = float(np.spacing(np.float32(ref)))
        worst = max(worst, abs(float(got) - ref) / ulp)
    assert worst <= 2.0, worst
    assert L.or_expf(0.0) == 1.0
    assert L.or_expf(-200.0) == 0.0


# ---- hand-built blocks ----------------------------------------------------------------------------------------

K4_SCALES = [0x41, 0x02, 0x03, 0x04, 0x05, 0x06, 0x87, 0x08, 0x19, 0x2A, 0x3B, 0x4C]
# unpacked by hand from K4_SCALES with the 6-bit layout (bytes 0-3: sc 0-3 + high bits of sc 4-7, bytes 4-7: m 0-3 +
# high bits of m 4-7, bytes 8-11: low nibbles of sc 4-7 | m 4-7)
K4_SC = [1, 2, 3, 4, 25, 10, 11, 12]
K4_M = [5, 6, 7, 8, 1, 2, 35, 4]


def q4k_block() -> np.ndarray:
    b = bytearray()
    b += f16(0.5).to_bytes(2, "little") + f16(0.25).to_bytes(2, "little")
    b += bytes(K4_SCALES)
    b += bytes(((l % 16) | ((15 - l % 16) << 4)) for l in range(128))
    return np.frombuffer(bytes(b), dtype=np.uint8)


def test_dequant_q4_K_hand_block():
    y = orc.dequantize(orc.Q4_K, q4k_block(), 256)
    expect = {0: -1.25, 40: 5.5, 150: 74.75, 200: 35.25, 255: -1.0, 100: 20.0, 180: 54.5}
    for i, v in expect.items():
        assert y[i] == v, (i, y[i], v)
    # every value: d * sc[s] * nibble - dmin * m[s], positions: low nibbles of qs[32g..] = values 64g.., high = 64g+32..
    for g in range(4):
        for p in range(32):
            q = (32 * g + p) % 16
            assert y[64 * g + p] == 0.5 * K4_SC[2 * g] * q - 0.25 * K4_M[2 * g]
            assert y[64 * g + 32 + p] == 0.5 * K4_SC[2 * g + 1] * (15 - q) - 0.25 * K4_M[2 * g + 1]


def test_dequant_q5_K_hand_block():
    b = bytearray()
    b += f16(0.5).to_bytes(2, "little") + f16(0.25).to_bytes(2, "little")
    b += bytes(K4_SCALES)
    b += bytes([0xA5] * 32)  # bits 0, 2, 5, 7 set
    b += bytes(((l % 16) | ((15 - l % 16) << 4)) for l in range(128))
    y = orc.dequantize(orc.Q5_K, np.frombuffer(bytes(b), dtype=np.uint8), 256)
    expect = {0: 6.75, 40: 5.5, 150: 74.75, 180: 134.5, 100: 20.0, 70: 31.25}
    for i, v in expect.items():
        assert y[i] == v, (i, y[i], v)


def test_dequant_q6_K_hand_block():
    ql = bytes(((i % 16) | ((i % 7) << 4)) for i in range(128))
    qh = bytes(range(64))
    sc = np.array([1, -2, 3, -4, 5, -6, 7, -8, 9, -10, 11, -12, 13, -14, 15, -16], dtype=np.int8).tobytes()
    b = ql + qh + sc + f16(0.125).to_bytes(2, "little")
    y = orc.dequantize(orc.Q6_K, np.frombuffer(b, dtype=np.uint8), 256)
    expect = {0: -4.0, 37: -4.125, 70: -16.25, 255: 62.0, 150: -7.5}
    for i, v in expect.items():
        assert y[i] == v, (i, y[i], v)


def test_dequant_q3_K_hand_block():
    hmask = bytes(((i * 53) & 0xFF) for i in range(32))
    qs = bytes(((i * 37) & 0xFF) for i in range(64))
    scales = bytes([0x21, 0x43, 0x65, 0x87, 0xA9, 0xCB, 0xED, 0x0F, 0xE4, 0x1B, 0x00, 0xFF])
    b = hmask + qs + scales + f16(0.5).to_bytes(2, "little")
    y = orc.dequantize(orc.Q3_K, np.frombuffer(b, dtype=np.uint8), 256)
    expect = {0: 62.0, 17: 9.5, 83: 16.5, 200: -52.0, 255: -32.0}
    for i, v in expect.items():
        assert y[i] == v, (i, y[i], v)


# ---- quantisers ----------------------------------------------------------------------------------------------

@pytest.mark.parametrize("qtype,bound", [(orc.Q3_K, 0.17), (orc.Q4_K, 0.08), (orc.Q5_K, 0.04), (orc.Q6_K, 0.02),
                                         (orc.Q8_0, 0.006)])
def test_quantizer_roundtrip_error(qtype, bound):
    rng = np.random.default_rng(qtype)
    w = gaussian(rng, (32, 2048), 0.02)
    q = orc.quantize(qtype, w)
    assert q.shape == (32, orc.row_bytes(qtype, 2048))
    d = orc.dequantize(qtype, q, 2048)
    err = np.sqrt(((d - w) ** 2).mean()) / np.sqrt((w ** 2).mean())
    assert err < bound, err
    # the quantiser must use the whole grid: not a degenerate (all-zero) encoding
    assert np.abs(d).max() > 0.5 * np.abs(w).max()


@pytest.mark.parametrize("qtype", [orc.Q3_K, orc.Q4_K, orc.Q5_K, orc.Q6_K])
def test_quantizer_zero_block(qtype):
    q = orc.quantize(qtype, np.zeros((1, 256), np.float32))
    assert np.all(orc.dequantize(qtype, q, 256) == 0.0)


def test_quantizer_q8_0_half_step():
    rng = np.random.default_rng(1)
    w = gaussian(rng, (4, 256))
    q = orc.quantize(orc.Q8_0, w)
    d = orc.dequantize(orc.Q8_0, q, 256)
    step = np.abs(w.reshape(-1, 32)).max(1) / np.float32(127)
    # rounding to the grid of the fp32 step, plus the f16 rounding of the stored scale times |q| <= 127
    stored = step.astype(np.float16).astype(np.float64)
    bound = step * 0.5 + 127 * np.abs(stored - step) + 1e-7
    assert np.all(np.abs(d - w).reshape(-1, 32) <= bound[:, None])


def test_quantizer_is_deterministic_and_thread_independent():
    rng = np.random.default_rng(2)
    w = gaussian(rng, (64, 1024), 0.02)
    for t in (orc.Q3_K, orc.Q4_K, orc.Q5_K, orc.Q6_K):
        assert np.array_equal(orc.quantize(t, w, nthreads=1), orc.quantize(t, w, nthreads=7))


# ---- Q8_1 ----------------------------------------------------------------------------------------------------

def q8_1_fields(xq: np.ndarray):
    b = xq.reshape(-1, 36)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    s = b[:, 2:4].copy().view(np.float16).astype(np.float32).ravel()
    q = b[:, 4:].view(np.int8)
    return d, s, q


def test_q8_1_rounding_half_away_from_zero():
    x = np.zeros((1, 32), np.float32)
    x[0, :8] = [127, 2.5, -2.5, 0.5, -0.5, 1.5, -126.5, 0.49999997]
    d, s, q = q8_1_fields(orc.quantize_q8_1(x))
    assert d[0] == 1.0
    assert list(q[0, :8]) == [127, 3, -3, 1, -1, 2, -127, 0]
    assert s[0] == np.float16(127 + 2.5 - 2.5 + 0.5 - 0.5 + 1.5 - 126.5 + 0.49999997)


def test_q8_1_invariants_and_padding():
    rng = np.random.default_rng(3)
    x = gaussian(rng, (5, 700), 3.0)
    x[2, 64:96] = 0.0
    xq = orc.quantize_q8_1(x)
    assert xq.shape == (5, orc.q8_1_row_bytes(700)) == (5, 32 * 36)  # padded to 1024 columns
    d, s, q = q8_1_fields(xq)
    q = q.reshape(5, 32, 32)
    d = d.reshape(5, 32)
    assert np.abs(q.astype(int)).max() <= 127
    xp = np.zeros((5, 1024), np.float32)
    xp[:, :700] = x
    blocks = xp.reshape(5, 32, 32)
    amax = np.abs(blocks).max(2)
    nz = amax > 0
    assert np.all(d[nz] == (amax[nz] / np.float32(127)).astype(np.float16).astype(np.float32))
    am = np.abs(blocks).argmax(2)
    picked = np.take_along_axis(np.abs(q.astype(int)), am[..., None], 2)[..., 0]
    assert np.all(picked[nz] == 127)
    assert np.all(q[~nz] == 0) and np.all(d[~nz] == 0)          # zero block and padding
    # q = round-half-away(x / d) with the fp32 quotient
    with np.errstate(invalid="ignore", divide="ignore"):
        quot = (blocks / (amax / np.float32(127))[..., None]).astype(np.float32).astype(np.float64)
    expect = np.where(nz[..., None], np.sign(quot) * np.floor(np.abs(quot) + 0.5), 0)
    assert np.array_equal(q, expect.astype(np.int8))


def test_q8_1_sum_exact_for_integers():
    rng = np.random.default_rng(4)
    x = rng.integers(-50, 50, (3, 512)).astype(np.float32)
    _, s, _ = q8_1_fields(orc.quantize_q8_1(x))
    assert np.array_equal(s, x.reshape(-1, 32).sum(1).astype(np.float16).astype(np.float32))


# ---- router and gating ---------------------------------------------------------------------------------------

def test_router_f32_matches_float64():
    rng = np.random.default_rng(5)
    w = gaussian(rng, (64, 512), 0.02)
    x = gaussian(rng, (3, 512))
    ref = (x.astype(np.float64) @ w.T.astype(np.float64)).astype(np.float32)
    assert np.array_equal(orc.router_f32(w, x), ref)


@pytest.mark.parametrize("gating", [0, 1])
def test_route_topk_against_float64_and_sort(gating):
    rng = np.random.default_rng(6 + gating)
    logits = gaussian(rng, (40, 128), 1.5)
    k = 8
    ids, w, probs, margin = orc.route_topk(logits, k, gating)
    l64 = logits.astype(np.float64)
    if gating == 0:
        p64 = np.exp(l64 - l64.max(1, keepdims=True))
        p64 /= p64.sum(1, keepdims=True)
    else:
        p64 = 1 / (1 + np.exp(-l64))
    assert np.abs(probs - p64).max() / p64.max() < 1e-6
    for t in range(40):
        order = sorted(range(128), key=lambda e: (-l64[t, e], e))[:k]
        assert list(ids[t]) == order
        sel = p64[t, order]
        np.testing.assert_allclose(w[t], sel / sel.sum(), rtol=2e-6)
        srt = np.sort(logits[t])[::-1]
        assert margin[t] == srt[k - 1] - srt[k]


def test_route_topk_ties_and_clamp():
    logits = np.array([[1.0, 3.0, 3.0, 2.0]], np.float32)
    ids, w, _, _ = orc.route_topk(logits, 2, 0)
    assert list(ids[0]) == [1, 2]
    np.testing.assert_allclose(w[0], [0.5, 0.5], rtol=1e-6)
    # sigmoid of very negative logits: sum below the clamp 6.103515625e-5, weights are p / clamp (not normalised)
    logits = np.full((1, 8), -30.0, np.float32)
    logits[0, 3] = -29.0
    ids, w, probs, _ = orc.route_topk(logits, 2, 1)
    assert list(ids[0]) == [3, 0]
    np.testing.assert_allclose(w[0], probs[0, [3, 0]] / 6.103515625e-5, rtol=1e-6)
    ids, w, _, _ = orc.route_topk(logits, 2, 1, norm=False)
    np.testing.assert_allclose(w[0], 1 / (1 + np.exp(-np.array([-29.0, -30.0]))), rtol=1e-5)


# ---- GEMV, compaction, combine, guard ------------------------------------------------------------------------

def test_mmvq_oracle_closed_form():
    # row: one Q4_K block with every value = 0.5 * 1 * 1 - 0 (sc = 1, m = 0, nibbles 1)
    b = bytearray(f16(0.5).to_bytes(2, "little") + f16(0.0).to_bytes(2, "little"))
    b += bytes([1, 1, 1, 1, 0, 0, 0, 0, 0x01, 0x01, 0x01, 0x01])
    b += bytes([0x11] * 128)
    row = np.frombuffer(bytes(b), dtype=np.uint8).reshape(1, 144)
    assert np.all(orc.dequantize(orc.Q4_K, row, 256) == 0.5)
    x = np.arange(256, dtype=np.float32)[None] / 256.0
    xq = orc.quantize_q8_1(x)
    xd = orc.dequantize_q8_1(xq, 256)
    y = orc.mmvq_experts(orc.Q4_K, [row], 256, 1, xq, 1, 1, np.zeros(1, np.int32))
    assert y[0, 0] == 0.5 * xd.sum()


def test_compact_ids_brute_force():
    rng = np.random.default_rng(8)
    ids = np.stack([rng.permutation(32)[:6] for _ in range(77)]).astype(np.int32)
    for xr in (1, 6):
        bounds, src, dst, n = orc.compact_ids(ids, 32, xr)
        pairs = sorted((int(ids[t, j]), t, j) for t in range(77) for j in range(6))
        assert n == len({p[0] for p in pairs})
        assert bounds[0] == 0 and bounds[-1] == 77 * 6 and np.all(np.diff(bounds) >= 0)
        for p, (e, t, j) in enumerate(pairs):
            assert bounds[e] <= p < bounds[e + 1]
            assert dst[p] == t * 6 + j
            assert src[p] == (t if xr == 1 else t * 6 + j)


def test_moe_combine_literal():
    dexp = np.array([[[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]]], np.float32)
    w = np.array([[0.5, 0.25, 0.125]], np.float32)
    e = np.array([[1.0, 2.0, 4.0]], np.float32)
    sh = np.array([[10.0, 20.0]], np.float32)
    x = np.array([[100.0, 200.0]], np.float32)
    out = orc.moe_combine(dexp, w, e, sh, x)
    assert list(out[0]) == [0.5 + 1.5 + 2.5 + 10 + 100, 1.0 + 2.0 + 3.0 + 20 + 200]


def test_amax_guard_scale_literal():
    assert orc.amax_guard_scale(np.array([3.0, -1000.0], np.float32)) == 1.0
    assert orc.amax_guard_scale(np.array([3000.0], np.float32)) == 4.0        # ceil(log2(3000/1024)) = 2
    assert orc.amax_guard_scale(np.array([-5000.0], np.float32)) == 8.0


def test_cpu_layer_matches_float64_chain():
    """The CPU baseline (integer sub-block dots) agrees with the float64 oracle chain."""
    rng = np.random.default_rng(10)
    H_, F_, NE_, K_ = 512, 256, 8, 2
    g = orc.quantize(orc.Q4_K, gaussian(rng, (NE_, F_, H_), 0.02)).reshape(NE_, -1)
    u = orc.quantize(orc.Q4_K, gaussian(rng, (NE_, F_, H_), 0.02)).reshape(NE_, -1)
    dn = orc.quantize(orc.Q6_K, gaussian(rng, (NE_, H_, F_), 0.02)).reshape(NE_, -1)
    slots = [np.ascontiguousarray(np.concatenate([g[e], u[e], dn[e]])) for e in range(NE_)]
    wr = gaussian(rng, (NE_, H_), 0.02)
    x = gaussian(rng, (H_,))
    out = orc.cpu_moe_layer(orc.Q4_K, orc.Q6_K, wr, slots, 0, g.shape[1], 2 * g.shape[1], x, H_, F_, K_, 2)
    logits = orc.router_f32(wr, x)
    ids, w, _, _ = orc.route_topk(logits, K_, 0)
    xq = orc.quantize_q8_1(x[None])
    act = orc.swiglu(orc.mmvq_experts(orc.Q4_K, [m.reshape(F_, -1) for m in g], H_, F_, xq, 1, K_, ids[0]),
                     orc.mmvq_experts(orc.Q4_K, [m.reshape(F_, -1) for m in u], H_, F_, xq, 1, K_, ids[0]))
    aq = orc.quantize_q8_1(act.astype(np.float32))
    dexp = orc.mmvq_experts(orc.Q6_K, [m.reshape(H_, -1) for m in dn], F_, H_, aq, K_, 1, ids[0])
    ref = (dexp * w[0][:, None]).sum(0)
    assert np.abs(out - ref).max() / np.abs(ref).max() < 1e-3


def test_split_image_helper_decodes_to_q8_1():
    """The test helper that spells out the prefill GEMM's split activation image: hi + lo of every column is the
    oracle's dequantised Q8_1 value (q * f16 d) exactly, and the sums are d * sum(q) per 32-column block."""
    from tests.helpers import split_image
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((3, 512)) * 3).astype(np.float32)
    x[1] = 0.0
    xq = orc.quantize_q8_1(x)
    img = split_image(xq, 512)
    assert img.shape == (3, 2 * 1056)
    deq = orc.dequantize_q8_1(xq, 512)
    perm = np.array([0, 2, 1, 3, 4, 6, 5, 7])
    for kb in range(2):
        main = img[:, kb * 1024:(kb + 1) * 1024].view(np.float16).astype(np.float32).reshape(3, 2, 2, 16, 8)
        val = (main[:, :, 0] + main[:, :, 1])[..., perm].reshape(3, 256)  # stored order is an involution
        assert np.array_equal(val, deq[:, kb * 256:(kb + 1) * 256])
        s = img[:, 2048 + 32 * kb: 2048 + 32 * (kb + 1)].view(np.float16).astype(np.float32).reshape(3, 2, 8)
        sums = (s[:, 0] + s[:, 1])[:, perm]
        assert np.array_equal(sums, deq[:, kb * 256:(kb + 1) * 256].reshape(3, 8, 32).sum(axis=2))
    assert not img[1].any()


def test_image_to_q8_1_inverts_split_image():
    from tests.helpers import image_to_q8_1, split_image
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((4, 768)) * 2).astype(np.float32)
    x[2, 64:96] = 0.0
    xq = orc.quantize_q8_1(x)
    back = image_to_q8_1(split_image(xq, 768), 768)
    a = xq[:, : 24 * 36].reshape(4, 24, 36)
    b = back[:, : 24 * 36].reshape(4, 24, 36)
    assert np.array_equal(a[:, :, 0:2], b[:, :, 0:2]) and np.array_equal(a[:, :, 4:], b[:, :, 4:])


# ---- IQ formats (restated from ggml-common.h / ggml-quants.c at the pinned commit; codebooks registered) ----------

def _f16(x: float) -> bytes:
    return np.array([x], np.float16).tobytes()


def test_iq4_xs_layout_closed_form():
    """d = 1, every sub-block scale 33 (dl = 1): the values are the IQ4_NL table read through the nibble order (low
    nibbles = values 0..15 of a sub-block, high = 16..31) and the 6-bit scale split (scales_l nibbles, scales_h
    2-bit fields)."""
    kv = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    qs = bytes(((j & 15) | ((15 - j) << 4)) for _ in range(8) for j in range(16))
    blk = _f16(1.0) + (0xAAAA).to_bytes(2, "little") + bytes([0x11] * 4) + qs
    y = orc.dequantize(orc.IQ4_XS, np.frombuffer(blk, np.uint8)[None], 256)[0]
    for ib in range(8):
        assert list(y[32 * ib:32 * ib + 16]) == kv
        assert list(y[32 * ib + 16:32 * ib + 32]) == kv[::-1]
    # scale field of sub-block 5 = 40 (low nibble 8, high bits 2): dl = 8 for that sub-block only
    sl = bytearray([0x11] * 4)
    sl[2] = 0x81
    y2 = orc.dequantize(orc.IQ4_XS, np.frombuffer(_f16(1.0) + (0xAAAA).to_bytes(2, "little") + bytes(sl) + qs,
                                                  np.uint8)[None], 256)[0]
    assert np.array_equal(y2[160:192], 8 * y[160:192]) and np.array_equal(y2[:160], y[:160])


def test_iq_codebook_formats_closed_form():
    """One block of each codebook format with hand-chosen indices, signs and scales: values = scale * codebook byte *
    sign, with the sign rules of each format (IQ3_XXS: 7 stored bits + even parity)."""
    from tests.iq_data import register_grids
    g3x, g3s, g2s = register_grids(5)
    byte = lambda g, i, j: int((int(g[i]) >> (8 * j)) & 0xFF)  # noqa: E731
    # IQ3_XXS: sub-block 0: indices 0..7, sign field 0b0000011 for pair 0 (bits 0,1 negative), scale 1 -> db = 0.75
    qs = bytearray(96)
    qs[0:8] = bytes(range(8))
    aux = 0b0000011 | (1 << 28)
    qs[64:68] = aux.to_bytes(4, "little")
    y = orc.dequantize(orc.IQ3_XXS, np.frombuffer(_f16(1.0) + bytes(qs), np.uint8)[None], 256)[0]
    exp = [0.75 * byte(g3x, l // 4, l % 4) * (-1 if l < 2 else 1) for l in range(32)]
    assert np.allclose(y[:32], exp, rtol=0, atol=0)
    # parity: a single stored negative sign turns on the eighth sign (bit 7 -> value 7 of the group)
    qs[64:68] = (0b0000001 | (1 << 28)).to_bytes(4, "little")
    y = orc.dequantize(orc.IQ3_XXS, np.frombuffer(_f16(1.0) + bytes(qs), np.uint8)[None], 256)[0]
    assert y[0] < 0 and y[7] < 0 and all(v > 0 for v in y[1:7])
    # IQ3_S: sub-block 1, index 3 with its 9th bit set (entry 256 + 3), sign nibble 0b0101, scale 2 -> db = 5
    qs = bytearray(64)
    qs[8 + 3] = 3
    qh = bytearray(8)
    qh[1] = 1 << 3
    signs = bytearray(32)
    signs[4 + 1] = 0b0101 << 4   # byte l/2 = 1, nibble l%2 = 1
    scales = bytearray(4)
    scales[0] = 2 << 4           # sub-block 1: high nibble of byte 0
    blk = _f16(1.0) + bytes(qs) + bytes(qh) + bytes(signs) + bytes(scales)
    y = orc.dequantize(orc.IQ3_S, np.frombuffer(blk, np.uint8)[None], 256)[0]
    got = y[32 + 12:32 + 16]
    want = [5 * byte(g3s, 259, j) * (-1 if (0b0101 >> j) & 1 else 1) for j in range(4)]
    assert np.array_equal(got, want)
    # IQ2_S: sub-block 2, group 3: index 7 + high bits 2 (entry 519), sign byte 0x81, scales low 1 / high 3
    qs = bytearray(64)
    qs[4 * 2 + 3] = 7
    qs[32 + 4 * 2 + 3] = 0x81
    qh = bytearray(8)
    qh[2] = 2 << 6
    sc = bytearray(8)
    sc[2] = 1 | (3 << 4)
    y = orc.dequantize(orc.IQ2_S, np.frombuffer(_f16(1.0) + bytes(qs) + bytes(qh) + bytes(sc), np.uint8)[None], 256)[0]
    dl = (0.5 + 3) * 0.25  # group 3 uses the high nibble
    want = [dl * byte(g2s, 519, j) * (-1 if j in (0, 7) else 1) for j in range(8)]
    assert np.array_equal(y[64 + 24:64 + 32], want)


@pytest.mark.parametrize("qtype", [23, 18, 21, 22])
def test_iq_integer_products_match_dequantised_dot(qtype):
    """The oracle's GEMV for IQ types restates the reference's integer sub-block products (scale applied in integers,
    C division truncating); it must equal the independent float64 dequant . dequant dot up to that truncation:
    exact for IQ4_XS and IQ3_S, at most one unit of d_w * d8 per sub-block for IQ3_XXS and IQ2_S."""
    from tests.iq_data import random_blocks, register_grids
    register_grids(5)
    ncols, nrows = 1024, 16
    w = random_blocks(qtype, nrows, ncols, seed=qtype)
    x = np.random.default_rng(qtype).standard_normal((1, ncols)).astype(np.float32)
    xq = orc.quantize_q8_1(x)
    got = orc.mmvq_experts(qtype, [w], ncols, nrows, xq, 1, 1, np.zeros(1, np.int32))[0]
    ref = orc.dequantize(qtype, w, ncols) @ orc.dequantize_q8_1(xq, ncols)[0]
    d_w = w.reshape(nrows, -1, orc.BLOCK_BYTES[qtype])[:, :, :2].copy().view(np.float16).astype(np.float64)[..., 0]
    d8 = xq[0].reshape(-1, 36)[:, :2].copy().view(np.float16).astype(np.float64)[:ncols // 32, 0]
    bound = np.abs(d_w).repeat(8, axis=1) @ np.abs(d8)  # one unit per sub-block
    if qtype in (orc.IQ4_XS, orc.IQ3_S):
        assert np.allclose(got, ref, rtol=1e-12, atol=1e-15)
    else:
        assert np.all(np.abs(got - ref) <= bound * (1.0 + 1e-9)) and not np.array_equal(got, ref)
