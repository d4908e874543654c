"""Parity of the prefill / batched expert path (MMQ: compaction, f16-MFMA split-operand grouped GEMM, prefill layer) with the CPU
oracle, called through the C ABI of libfns_hip.so.

Reference tests this follows: tests/mmq_parity.cu (T = 77 tokens, not a tile multiple, synthetic distinct-per-token
routing; MMQ against per-token MMVQ, per-row rel-L2 p99 < 2e-2) - held here to the float64 oracle on the same Q8_1
activations at the tolerance of tests/helpers.py, which is tighter. The compaction is checked bit for bit against
the oracle's stable sort (ggml mm_ids_helper semantics).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.helpers import assert_close, assert_close_chain, gaussian, image_to_q8_1, make_expert_mats, split_image

pytestmark = pytest.mark.gpu

TYPES = [orc.Q3_K, orc.Q4_K, orc.Q5_K, orc.Q6_K]


@pytest.fixture(scope="module")
def ops():
    from flintnsteel_amd import ops as o
    return o


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def distinct_ids(rng, n_tok, k, n_expert):
    if n_tok == 0:
        return np.zeros((0, k), np.int32)
    return np.stack([rng.permutation(n_expert)[:k] for _ in range(n_tok)]).astype(np.int32)


def table_of(mats_dev):
    return torch.tensor([mats_dev.data_ptr() + e * mats_dev.stride(0) for e in range(mats_dev.shape[0])],
                        dtype=torch.int64, device="cuda")


@pytest.mark.parametrize("n_tok,k,n_expert,xr", [(0, 8, 16, 1), (77, 8, 16, 1), (77, 8, 16, 8), (1, 1, 1, 1), (600, 8, 128, 1),
                                                 (5, 6, 256, 6), (1100, 4, 8, 1), (4096, 8, 128, 1),
                                                 (1024, 8, 128, 1), (1023, 8, 64, 8)])
def test_compaction_bit_exact(ops, n_tok, k, n_expert, xr):
    rng = np.random.default_rng(n_tok * 31 + k)
    ids = distinct_ids(rng, n_tok, k, n_expert)
    bounds, src, dst = ops.mmq_compact(dev(ids), n_expert, xr)
    rb, rs, rd, _ = orc.compact_ids(ids, n_expert, xr)
    assert np.array_equal(host(bounds), rb)
    assert np.array_equal(host(src), rs)
    assert np.array_equal(host(dst), rd)


def _group_prefix(counts: np.ndarray) -> np.ndarray:
    """The GEMM's group lists from the per-expert counts: 64-row groups (n_e // 64 full ones and the remainder if
    it is > 32 rows), then the <= 32-row remainders, each as an exclusive prefix with its total."""
    r = counts % 64
    g = counts // 64 + (r > 32)
    g2 = ((r > 0) & (r <= 32)).astype(np.int64)
    pre = lambda v: np.concatenate([[0], np.cumsum(v)]).astype(np.int32)  # noqa: E731
    return np.concatenate([pre(g), pre(g2)])


@pytest.mark.parametrize("n_tok,k,n_expert,gating", [(1, 8, 128, 0), (3, 6, 256, 1), (77, 8, 128, 0), (512, 8, 128, 0),
                                                     (700, 6, 256, 1), (50, 4, 16, 0), (4096, 8, 128, 1),
                                                     (8192, 8, 128, 0)])
def test_prefill_routing_and_compaction_sections(ops, n_tok, k, n_expert, gating):
    """The prefill layer's routing and compaction launches: ids and weights bit-exact against the oracle's routing of
    the layer's own logits, and the sorted lists, expert bounds and group prefixes against the oracle's compaction
    (ggml mm_ids_helper order) - with the workspace full of junk before the first call (the GEMM's arrival counters
    are reset by the compaction launch), then a second call on the same workspace with fewer tokens."""
    from flintnsteel_amd import synth
    print(f"prefill routing + compaction n_tok={n_tok} k={k} ne={n_expert}", flush=True)
    H = 256
    layer = synth.build_layer(H, 256, n_expert, k, orc.Q4_K, orc.Q4_K, seed=n_tok + k, layer=3, gating=gating,
                              std=0.3)
    pre = ops.MoePrefill(layer)
    ws = pre.workspace(n_tok)
    ws.fill_(0x4F)
    for T in (n_tok, max(1, n_tok // 3)):
        x = synth.activations(T, H, seed=T, layer=5)
        pre(x, ws=ws)
        tr = {kk: host(v) for kk, v in pre.trace(ws, T).items()}
        ids_r, w_r, _, _ = orc.route_topk(tr["logits"], k, gating, True)
        assert np.array_equal(tr["ids"], ids_r), f"T={T}: ids differ given the same logits"
        assert np.array_equal(tr["w"].view(np.uint32), w_r.view(np.uint32)), f"T={T}: weights differ"
        P = T * k
        rb, rs, rd, _ = orc.compact_ids(tr["ids"], n_expert, 1)
        off6, _ = pre.section(T, 6)
        off7, _ = pre.section(T, 7)
        off8, _ = pre.section(T, 8)
        src = host(ws[off6: off6 + 4 * P].view(torch.int32))
        dst = host(ws[off7: off7 + 4 * P].view(torch.int32))
        sec8 = host(ws[off8: off8 + 4 * 3 * (n_expert + 1)].view(torch.int32))
        assert np.array_equal(sec8[: n_expert + 1], rb), f"T={T}: bounds"
        assert np.array_equal(src, rs) and np.array_equal(dst, rd), f"T={T}: sorted lists"
        counts = np.diff(rb)
        assert np.array_equal(sec8[n_expert + 1:], _group_prefix(counts)), f"T={T}: group prefixes"


@pytest.mark.parametrize("n_tok,ncols", [(77, 2048), (512, 2048), (33, 768), (1, 256)])
def test_mmq_activation_image_bit_exact(ops, n_tok, ncols):
    """The MMQ activation quantiser (the split image fns_hip_mmq writes into its xq scratch) holds exactly the
    reference's Q8_1 codes and f16 scales of x (oracle quantize_q8_1), byte for byte; zero rows and values at a
    rounding half included."""
    from flintnsteel_amd._lib import call
    rng = np.random.default_rng(n_tok + ncols)
    x = gaussian(rng, (n_tok, ncols))
    if n_tok > 2:
        x[1] = 0.0                                   # amax = 0: q = 0, d = 0
        x[2, :32] = np.arange(32, dtype=np.float32) - 15.5   # halfway quotients round away from zero
    w = make_expert_mats(orc.Q4_K, 1, 128, ncols, 3)[0]
    xq = torch.full((ops.mmq_q8_1_bytes(ncols, n_tok),), 0xA5, dtype=torch.uint8, device="cuda")
    dst = torch.empty(n_tok, 128, dtype=torch.float32, device="cuda")
    call("fns_hip_mmq", orc.Q4_K, dev(w).data_ptr(), ncols, 128, dev(x).data_ptr(), n_tok, xq.data_ptr(),
         dst.data_ptr(), torch.cuda.current_stream().cuda_stream)
    img = host(xq)
    want = split_image(orc.quantize_q8_1(x), ncols)
    got = img[: want.size].reshape(want.shape)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} image bytes differ, first at (row, byte) {tuple(bad[0])}"


def check_routing(tr_logits, ref_logits, gpu_ids, k, gating, min_clear=1.0):
    """The GPU's expert ids against the oracle's routing of its own logits (float64-accumulated router). With b twice
    the measured GPU-oracle logit difference: every token's selection is a valid top-k of the oracle's gate values
    within b (no selected expert below, no unselected one above, the oracle's k-th value by more than b); tokens whose
    oracle margin (k-th minus (k+1)-th logit) exceeds b have exactly the oracle's ids, in order, and they are at least
    `min_clear` of all tokens."""
    ids_o, _, probs, margin = orc.route_topk(ref_logits, k, gating, True)
    bound = 2.0 * float(np.abs(tr_logits - ref_logits).max()) + 1e-7
    clear = margin > bound
    assert clear.mean() >= min_clear, f"{(~clear).sum()} of {len(clear)} tokens are near-ties"
    assert np.array_equal(ids_o[clear], gpu_ids[clear]), "ids differ from the oracle's routing of its own logits"
    kth = np.sort(probs, axis=1)[:, -k][:, None]
    sel = np.zeros(probs.shape, bool)
    np.put_along_axis(sel, gpu_ids.astype(np.int64), True, axis=1)
    assert (probs[sel].reshape(-1, k) >= kth - bound).all() and (np.where(sel, -np.inf, probs) <= kth + bound).all(), \
        "a selection is not a top-k of the oracle's gate values"


@pytest.mark.parametrize("qtype", TYPES)
def test_mmq_experts_gate_like(ops, qtype):
    """x_rows_per_tok = 1: one activation row per token shared by its k experts (the gate/up call)."""
    T, K, NE, ncols, nrows = 77, 4, 16, 512, 256
    rng = np.random.default_rng(100 + qtype)
    mats = make_expert_mats(qtype, NE, nrows, ncols, 500 + qtype)
    x = gaussian(rng, (T, ncols))
    ids = distinct_ids(rng, T, K, NE)
    md = dev(mats)
    got = host(ops.mmq_experts(qtype, table_of(md), 0, ncols, nrows, NE, dev(x), 1, dev(ids)))
    xq = orc.quantize_q8_1(x)
    ref = orc.mmvq_experts(qtype, [m.reshape(nrows, -1) for m in mats], ncols, nrows, xq, T, K, ids.ravel())
    assert_close(got.reshape(T * K, nrows), ref, f"mmq_experts gate-like {orc.TYPE_NAMES[qtype]}")


@pytest.mark.parametrize("qtype", TYPES)
def test_mmq_experts_down_like(ops, qtype):
    """x_rows_per_tok = k: one activation row per (token, slot) (the down call); includes an expert with > 128 rows."""
    T, K, NE, ncols, nrows = 150, 2, 4, 256, 128
    rng = np.random.default_rng(200 + qtype)
    mats = make_expert_mats(qtype, NE, nrows, ncols, 600 + qtype)
    x = gaussian(rng, (T, K, ncols), 0.3)
    ids = distinct_ids(rng, T, K, NE)
    md = dev(mats)
    got = host(ops.mmq_experts(qtype, table_of(md), 0, ncols, nrows, NE, dev(x), K, dev(ids)))
    xq = orc.quantize_q8_1(x.reshape(T * K, ncols))
    ref = orc.mmvq_experts(qtype, [m.reshape(nrows, -1) for m in mats], ncols, nrows, xq, T * K, 1, ids.ravel())
    assert_close(got.reshape(T * K, nrows), ref, f"mmq_experts down-like {orc.TYPE_NAMES[qtype]}")


def test_mmq_experts_reference_scratch_sizes(ops):
    """The scratch sizes the reference engine allocates (src/engine.cu:228-231: ids n_tok*k + 128, expert_bounds
    n_expert + 1, xq mmq_q8_1_bytes(max(E, F), n_tok*k)) are enough: nothing is written past any of them."""
    from flintnsteel_amd._lib import call
    T, K, NE, ncols, nrows, xr = 90, 4, 64, 512, 128, 4
    rng = np.random.default_rng(9)
    mats = make_expert_mats(orc.Q4_K, NE, nrows, ncols, 901)
    x = gaussian(rng, (T, xr, ncols), 0.5)
    ids = distinct_ids(rng, T, K, NE)
    canary = 1 << 12
    src = torch.full((T * K + 128 + canary,), -7, dtype=torch.int32, device="cuda")
    dsti = torch.full_like(src, -7)
    bounds = torch.full((NE + 1 + canary,), -7, dtype=torch.int32, device="cuda")
    xq_bytes = ops.mmq_q8_1_bytes(ncols, T * K)
    xq = torch.full((xq_bytes + 4 * canary,), 0x5A, dtype=torch.uint8, device="cuda")
    dst = torch.empty(T, K, nrows, dtype=torch.float32, device="cuda")
    md = dev(mats)
    xd = dev(x)
    idd = dev(ids)
    call("fns_hip_mmq_experts", orc.Q4_K, table_of(md).data_ptr(), 0, ncols, nrows, NE, xd.data_ptr(), xr, T,
         idd.data_ptr(), K, src.data_ptr(), dsti.data_ptr(), bounds.data_ptr(), xq.data_ptr(), dst.data_ptr(),
         torch.cuda.current_stream().cuda_stream)
    got = host(dst)
    assert (host(src[T * K + 128:]) == -7).all() and (host(dsti[T * K + 128:]) == -7).all()
    assert (host(bounds[NE + 1:]) == -7).all()
    assert (host(xq[xq_bytes:]) == 0x5A).all()
    rb, _, _, _ = orc.compact_ids(ids, NE, xr)
    assert np.array_equal(host(bounds[:NE + 1]), rb)
    xq8 = orc.quantize_q8_1(x.reshape(T * xr, ncols))
    ref = orc.mmvq_experts(orc.Q4_K, [m.reshape(nrows, -1) for m in mats], ncols, nrows, xq8, T * K, 1,
                           ids.ravel())
    assert_close(got.reshape(T * K, nrows), ref, "mmq_experts with reference scratch sizes")


@pytest.mark.parametrize("qtype", TYPES)
def test_mmq_experts_group_shapes(ops, qtype):
    """Expert loads chosen to hit every group shape of the two launches: empty experts, remainders of 1, 16, 17, 32
    rows (2-tile list) and 33, 63 rows (4-tile list), whole 64-row groups, 64 + remainder, 128 + 1."""
    loads = [0, 1, 16, 17, 32, 33, 63, 64, 65, 96, 129, 0]
    NE, ncols, nrows = len(loads), 512, 128
    pairs = np.concatenate([np.full(n, e, np.int32) for e, n in enumerate(loads)])
    rng = np.random.default_rng(11)
    pairs = pairs[rng.permutation(len(pairs))]
    K = 1
    T = len(pairs)
    ids = pairs.reshape(T, K)
    mats = make_expert_mats(qtype, NE, nrows, ncols, 700 + qtype)
    x = gaussian(rng, (T, ncols))
    md = dev(mats)  # the table points into it: keep it alive
    got = host(ops.mmq_experts(qtype, table_of(md), 0, ncols, nrows, NE, dev(x), 1, dev(ids)))
    xq = orc.quantize_q8_1(x)
    ref = orc.mmvq_experts(qtype, [m.reshape(nrows, -1) for m in mats], ncols, nrows, xq, T, K, ids.ravel())
    assert_close(got.reshape(T * K, nrows), ref, f"mmq_experts group shapes {orc.TYPE_NAMES[qtype]}")


@pytest.mark.parametrize("nrows", [96, 128, 320])
def test_mmq_q8_0_dense_and_experts(ops, nrows):
    """Q8_0 (the reference's dense and output-head type, src/ggml/ggml_mmq.cu:59) through fns_hip_mmq and
    fns_hip_mmq_experts against the float64 oracle - the tiled MFMA GEMM when nrows is a multiple of 64, the GEMV
    kernels over the token columns otherwise; gate-like and down-like activation rows."""
    print(f"mmq Q8_0 nrows={nrows}", flush=True)
    rng = np.random.default_rng(8 + nrows)
    T, ncols = 37, 512
    w = orc.quantize(orc.Q8_0, rng.normal(0, 0.02, (nrows, ncols)).astype(np.float32))
    x = gaussian(rng, (T, ncols))
    got = host(ops.mmq(orc.Q8_0, dev(w), ncols, nrows, dev(x)))
    xq = orc.quantize_q8_1(x)
    assert_close(got, orc.mmvq_experts(orc.Q8_0, [w], ncols, nrows, xq, T, 1, np.zeros(T, np.int32)), "mmq dense Q8_0")
    K, NE = 3, 5
    mats = np.stack([orc.quantize(orc.Q8_0, rng.normal(0, 0.02, (nrows, ncols)).astype(np.float32)) for _ in range(NE)])
    ids = distinct_ids(rng, T, K, NE)
    md = dev(mats.reshape(NE, -1))
    for xr in (1, K):
        xx = gaussian(rng, (T, xr, ncols))
        got = host(ops.mmq_experts(orc.Q8_0, table_of(md), 0, ncols, nrows, NE, dev(xx), xr, dev(ids)))
        xq = orc.quantize_q8_1(xx.reshape(T * xr, ncols))
        ref = orc.mmvq_experts(orc.Q8_0, list(mats), ncols, nrows, xq, T * xr if xr > 1 else T, 1 if xr > 1 else K,
                               ids.ravel())
        assert_close(got.reshape(T * K, nrows), ref, f"mmq_experts Q8_0 x_rows_per_tok={xr}")


def test_mmq_q8_0_dense_ffn_shape(ops):
    """The tiled Q8_0 GEMM at the reference model's dense FFN shape (2048 -> 6144 and 6144 -> 2048, 512 tokens):
    a sample of tokens against the float64 oracle, and weight blocks with d = 0, tiny d (the lo operand subnormal)
    and the largest codes."""
    print("mmq Q8_0 dense FFN shape", flush=True)
    rng = np.random.default_rng(81)
    T = 512
    toks = [0, 1, 63, 64, 200, 511]
    for ncols, nrows in ((2048, 6144), (6144, 2048)):
        wf = rng.normal(0, 0.02, (nrows, ncols)).astype(np.float32)
        wf[:3, :64] = 0.0                      # d = 0 blocks
        wf[3, :32] = 1e-4 * rng.standard_normal(32)  # tiny d: products below 2^-3, lo subnormal
        wf[4, 32:64] = 1.0                      # |code| = 127
        w = orc.quantize(orc.Q8_0, wf)
        x = gaussian(rng, (T, ncols))
        got = host(ops.mmq(orc.Q8_0, dev(w), ncols, nrows, dev(x)))
        xq = orc.quantize_q8_1(x[toks])
        ref = orc.mmvq_experts(orc.Q8_0, [w], ncols, nrows, xq, len(toks), 1, np.zeros(len(toks), np.int32))
        assert_close(got[toks], ref, f"mmq Q8_0 {ncols}->{nrows}")


def test_mmq_dense(ops):
    T, ncols, nrows = 130, 768, 192
    rng = np.random.default_rng(3)
    w = make_expert_mats(orc.Q4_K, 1, nrows, ncols, 77)
    x = gaussian(rng, (T, ncols))
    got = host(ops.mmq(orc.Q4_K, dev(w[0]), ncols, nrows, dev(x)))
    xq = orc.quantize_q8_1(x)
    ref = orc.mmvq_experts(orc.Q4_K, [w[0].reshape(nrows, -1)], ncols, nrows, xq, T, 1, np.zeros(T, np.int32))
    assert_close(got, ref, "mmq dense Q4_K")


@pytest.mark.parametrize("qtype", [orc.Q4_K, orc.Q6_K])
def test_mmq_repeatable(ops, qtype):
    """Repeated launches give bit-identical outputs (a missing wait between the LDS-DMA staging, the workgroup barriers
    and the LDS reads shows up as run-to-run differences); odd superblock count, ragged groups, two row blocks."""
    T, ncols, nrows = 130, 768, 192
    rng = np.random.default_rng(5)
    w = dev(make_expert_mats(qtype, 1, nrows, ncols, 78)[0])
    x = dev(gaussian(rng, (T, ncols)))
    first = host(ops.mmq(qtype, w, ncols, nrows, x))
    for _ in range(8):
        assert np.array_equal(host(ops.mmq(qtype, w, ncols, nrows, x)), first)


def _oracle_layer_tokens(layer, slots_np, x, toks, ids, w, gu, dn, H, F, aq_gpu=None, esc=None):
    """float64 chain per token: act = swiglu(gate . q8(x), up . q8(x)); out = sum_j w_j e_j down . q8(act_j / e_j).
    aq_gpu [n_tok * k] Q8_1 rows: take the GPU's act codes (decoded from its act image) for the down products instead
    of the oracle's own; esc [n_tok * k]: guard scales (default 1). Returns (out [len(toks)][H], act [len(toks)][k][F])."""
    xq = orc.quantize_q8_1(x[toks])
    K = ids.shape[1]
    out = np.zeros((len(toks), H))
    acts = np.zeros((len(toks), K, F), np.float32)
    z = np.zeros(1, np.int32)
    for n, t in enumerate(toks):
        for j in range(K):
            e, p = int(ids[t, j]), t * K + j
            g = orc.mmvq_experts(gu, [slots_np["gate"][e].reshape(F, -1)], H, F, xq[n:n + 1], 1, 1, z)
            u = orc.mmvq_experts(gu, [slots_np["up"][e].reshape(F, -1)], H, F, xq[n:n + 1], 1, 1, z)
            acts[n, j] = orc.swiglu(g, u).astype(np.float32)[0]
            s = 1.0 if esc is None else float(esc[p])
            aq = aq_gpu[p:p + 1] if aq_gpu is not None else orc.quantize_q8_1((acts[n, j] / np.float32(s))[None])
            d = orc.mmvq_experts(dn, [slots_np["down"][e].reshape(H, -1)], F, H, aq, 1, 1, z)[0]
            out[n] += d * s * float(w[t, j])
    return out, acts


def check_prefill_chains(tr, layer, slots_np, xh, toks, ids, gu, dn, H, F, what, resid=None):
    """The prefill output against two float64 chains: (a) fed with the GPU's act codes (decoded from its act image),
    held to the tight bounds; (b) fully independent, held to the chain bounds. The GPU's act image itself lies within
    half a quantisation step (plus the GEMM tolerance) of the oracle's act / e."""
    K = ids.shape[1]
    esc = tr["escale"] if layer.desc.guard else np.ones(tr["apack"].shape[0], np.float32)  # written with the guard only
    aq = image_to_q8_1(tr["apack"], F)
    out = tr["out"][toks] - (0.0 if resid is None else resid[toks])
    ref_g, act_ref = _oracle_layer_tokens(layer, slots_np, xh, toks, ids, tr["w"], gu, dn, H, F, aq, esc)
    assert_close(out, ref_g, what + " (GPU act codes)")
    ref_i, _ = _oracle_layer_tokens(layer, slots_np, xh, toks, ids, tr["w"], gu, dn, H, F, None, esc)
    assert_close_chain(out, ref_i, what)
    rows = np.array([t * K + j for t in toks for j in range(K)])
    esc_ref = np.array([orc.amax_guard_scale(a) for a in act_ref.reshape(-1, F)], np.float32)
    assert (esc[rows] == 1.0).all() or np.array_equal(esc[rows], esc_ref), f"{what}: guard scales differ"
    vals = orc.dequantize_q8_1(aq[rows], F).reshape(len(toks), K, F)
    dstep = np.repeat(np.abs(vals).reshape(len(toks), K, F // 32, 32).max(axis=3) / 127.0, 32, axis=2)
    want = act_ref / esc[rows].reshape(len(toks), K, 1)
    # half a step of the image's own scale plus the fp32 difference of the two act computations (1e-3 of the row's
    # max: act = up * silu(gate) carries the GEMV errors of both factors; still a fraction of one step, max / 127)
    slack = 0.5 * dstep + 1e-3 * np.abs(want).max(axis=2, keepdims=True)
    excess = np.abs(vals - want) / slack
    worst = np.unravel_index(int(np.argmax(excess)), excess.shape)
    assert excess.max() <= 1.0 + 1e-6, (f"{what}: act image beyond half a step of the oracle's act at {worst}: "
                                        f"{vals[worst]} vs {want[worst]}, step {dstep[worst]}")


@pytest.mark.parametrize("gu,dn,guard", [(orc.Q4_K, orc.Q4_K, False), (orc.Q3_K, orc.Q5_K, False),
                                         (orc.Q4_K, orc.Q6_K, True)])
def test_moe_prefill_vs_oracle(ops, gu, dn, guard):
    """77 tokens: router logits against the float64 oracle; ids from the oracle's own logits (every token's top-k
    margin clear of the logit difference); the x and act activation images byte-exact against the oracle's Q8_1 of
    x and of the GPU's act (guard on: f32 act rows exposed, no row scaled, so every act image is the GEMM epilogue's);
    the layer against the float64 chain."""
    from flintnsteel_amd import synth
    H, F, NE, K, T = 512, 256, 16, 4, 77
    layer0 = synth.build_layer(H, F, NE, K, gu, dn, seed=11, layer=gu * 10 + dn)
    layer = ops.MoeLayer(layer0.router_w, layer0.slots, gu, dn, H, F, K, guard=guard) if guard else layer0
    pre = ops.MoePrefill(layer)
    x = synth.activations(T, H, seed=11, layer=3)
    ws = pre.workspace(T)
    out = host(pre(x, ws=ws))
    tr = {k: host(v) for k, v in pre.trace(ws, T).items()}
    xh = host(x)
    ref_logits = orc.router_f32(host(layer.router_w), xh)
    assert_close(tr["logits"], ref_logits, "prefill logits", 1e-5, 1e-6)
    check_routing(tr["logits"], ref_logits, tr["ids"], K, 0)
    ids = tr["ids"]
    ids_g, w_g, _, _ = orc.route_topk(tr["logits"], K, 0, True)
    assert np.array_equal(ids_g, ids), "ids differ given the same logits"
    assert np.array_equal(w_g.view(np.uint32), tr["w"].view(np.uint32)), "weights differ given the same logits"
    assert np.array_equal(tr["xpack"], split_image(orc.quantize_q8_1(xh), H)), "x image differs from the oracle's Q8_1"
    if guard:
        assert (tr["escale"] == 1.0).all()
        act = tr["act"]
        want = split_image(orc.quantize_q8_1(act), F)
        assert np.array_equal(tr["apack"], want), "act image differs from the oracle's Q8_1 of act"
    slots_np = {k: layer.slots.view(k).cpu().numpy() for k in ("gate", "up", "down")}
    tr["out"] = out
    check_prefill_chains(tr, layer, slots_np, xh, list(range(T)), ids, gu, dn, H, F,
                         f"prefill layer {orc.TYPE_NAMES[gu]}/{orc.TYPE_NAMES[dn]}")


def test_moe_prefill_config4_sample(ops):
    """Config 4 shapes (512 tokens, hidden 2048, 128 experts top-8, inter 768, Q4_K) with a Dirichlet-skewed router
    bias: logits against the oracle, ids against the oracle's routing of its own logits (tokens with a clear margin),
    the x image of all 512 tokens and the fused launch's act image of all 4096 rows byte-exact, 64 tokens (among them every token of the largest expert group up to 40)
    against the float64 chain, residual added; then all 512 tokens against the batch-1 decode path."""
    from flintnsteel_amd import synth
    H, F, NE, K, T = 2048, 768, 128, 8, 512
    layer = synth.build_layer(H, F, NE, K, orc.Q4_K, orc.Q4_K, seed=20261022, layer=400)
    rng = np.random.default_rng(20261022)
    bias = np.log(rng.dirichlet(np.full(NE, 0.3)) + 1e-6).astype(np.float32) * 0.5
    layer_b = ops.MoeLayer(layer.router_w, layer.slots, orc.Q4_K, orc.Q4_K, H, F, K, router_bias=dev(bias))
    pre = ops.MoePrefill(layer_b)
    x = synth.activations(T, H, seed=20261022, layer=401)
    resid = synth.activations(T, H, seed=20261022, layer=402)
    ws = pre.workspace(T)
    out = host(pre(x, ws=ws, x_resid=resid))
    tr = {k: host(v) for k, v in pre.trace(ws, T).items()}
    xh = host(x)
    logits_ref = orc.router_f32(layer.router_w.cpu().numpy(), xh) + bias
    assert_close(tr["logits"], logits_ref, "config-4 logits", 1e-5, 1e-6)
    check_routing(tr["logits"], logits_ref, tr["ids"], K, 0, min_clear=0.98)
    ids, w, _, _ = orc.route_topk(tr["logits"], K, 0, True)
    assert np.array_equal(ids, tr["ids"]) and np.array_equal(w, tr["w"])
    assert np.array_equal(tr["xpack"], split_image(orc.quantize_q8_1(xh), H)), "x image differs from the oracle"
    # the fused launch's act image (the gate/up epilogue's Q8_1 of act, no f32 act kept) against the oracle's Q8_1 of
    # the GPU's f32 act: the same layer with the F16 guard on runs gate/up as its own launch and keeps the f32 rows;
    # with every guard scale 1 its image is that epilogue's too, and the fused image must equal it byte for byte
    layer_g = ops.MoeLayer(layer.router_w, layer.slots, orc.Q4_K, orc.Q4_K, H, F, K, router_bias=dev(bias), guard=True)
    pre_g = ops.MoePrefill(layer_g)
    ws_g = pre_g.workspace(T)
    pre_g(x, ws=ws_g, x_resid=resid)
    tr_g = {k: host(v) for k, v in pre_g.trace(ws_g, T).items()}
    assert np.array_equal(tr_g["ids"], tr["ids"]) and (tr_g["escale"] == 1.0).all()
    assert np.array_equal(tr_g["apack"], split_image(orc.quantize_q8_1(tr_g["act"]), F)), \
        "act image (two launches) differs from the oracle's Q8_1 of act"
    assert np.array_equal(tr["apack"], tr_g["apack"]), "fused launch's act image differs"
    counts = np.bincount(ids.ravel(), minlength=NE)
    assert counts.max() > 128, "the skewed bias should give at least one expert more than one tile group"
    big = np.flatnonzero((ids == counts.argmax()).any(axis=1))
    rest = rng.choice(np.setdiff1d(np.arange(T), big), 64 - min(40, len(big)) - 3, replace=False)
    toks = sorted(set([0, 77, 511] + list(big[:40]) + list(rest)))
    slots_np = {k: layer.slots.view(k).cpu().numpy() for k in ("gate", "up", "down")}
    tr["out"] = out
    check_prefill_chains(tr, layer, slots_np, xh, toks, ids, orc.Q4_K, orc.Q4_K, H, F, "config-4 prefill sample",
                         resid=host(resid))
    # all 512 tokens against the batch-1 decode path of the same layer (parity-checked against the oracle on its own):
    # the tokens both paths route alike agree within the chain bounds (the two paths round act to Q8_1 from different
    # fp32 sums, so a code can differ by one step)
    ws1 = layer_b.workspace(1)
    dec = np.zeros_like(out)
    same = np.zeros(T, bool)
    for t in range(T):
        dec[t] = host(layer_b(x[t:t + 1].contiguous(), ws=ws1, x_resid=resid[t:t + 1].contiguous()))[0]
        same[t] = np.array_equal(host(layer_b.trace(ws1, 1)["ids"])[0], ids[t])
    assert same.mean() >= 0.98, f"decode and prefill routing agree on {same.sum()} of {T} tokens"
    assert_close_chain(out[same] - host(resid)[same], dec[same] - host(resid)[same], "config-4 prefill vs decode, all tokens")


def test_moe_prefill_guard_bf16_sigmoid_residual(ops):
    """The Flint-style prefill: bf16 router, sigmoid gating, F16 guard active (act amax > 1024: the act rows are
    divided by e = 2^ceil(log2(amax / 1024)) before Q8_1 and the combine multiplies back; reference
    src/kernels.cu:534-577, src/engine.cu:349-357), residual added; 33 tokens against the float64 chain."""
    from flintnsteel_amd import synth
    H, F, NE, K, T = 512, 256, 32, 6, 33
    base = synth.build_layer(H, F, NE, K, orc.Q4_K, orc.Q6_K, seed=5, layer=77, std=0.5)
    router_bf16 = base.router_w.to(torch.bfloat16)
    layer = ops.MoeLayer(router_bf16, base.slots, orc.Q4_K, orc.Q6_K, H, F, K, gating=ops.GATING_SIGMOID, guard=True)
    pre = ops.MoePrefill(layer)
    x = synth.activations(T, H, seed=5, layer=78) * 40.0
    resid = synth.activations(T, H, seed=5, layer=79)
    ws = pre.workspace(T)
    out = host(pre(x, ws=ws, x_resid=resid))
    tr = {k: host(v) for k, v in pre.trace(ws, T).items()}
    xh = host(x)
    # router: bf16 weights, x rounded to bf16 (the reference's cuBLAS BF16 path), fp32 accumulation
    w32 = router_bf16.float().cpu().numpy()
    xb = torch.from_numpy(xh).to(torch.bfloat16).float().numpy()
    logits_ref = orc.router_f32(w32, xb)
    assert np.abs(tr["logits"] - logits_ref).max() <= 1e-4 * np.abs(logits_ref).max()
    ids, w, _, _ = orc.route_topk(tr["logits"], K, 1, True)
    assert np.array_equal(ids, tr["ids"]) and np.array_equal(w, tr["w"])
    # (x is scaled by 40, so many sigmoid gates saturate and tie: a valid top-k check for every token)
    check_routing(tr["logits"], logits_ref, tr["ids"], K, 1, min_clear=0.0)
    # act images: every row here is guarded, so re-quantised from act / e (the GEMM epilogue's own images are checked
    # in test_moe_prefill_vs_oracle), byte-exact
    assert (tr["escale"] > 1.0).any()
    want = split_image(orc.quantize_q8_1(tr["act"]), F)
    assert np.array_equal(tr["apack"], want), "act image differs from the oracle's Q8_1 of act"
    slots = {k: base.slots.view(k).cpu().numpy() for k in ("gate", "up", "down")}
    tr["out"] = out
    check_prefill_chains(tr, layer, slots, xh, list(range(T)), ids, orc.Q4_K, orc.Q6_K, H, F,
                         "guarded bf16 sigmoid prefill", resid=host(resid))


def test_moe_prefill_unaligned_inputs_take_the_two_launch_router(ops):
    """x 4 bytes off a 16-byte boundary: the prefill takes the separate router GEMM (guarded loads) and activation
    quantiser instead of the one-launch router + image kernel. Same chunk order, products and Q8_1 arithmetic, so the
    logits, the x image and the output equal the aligned call's bit for bit."""
    from flintnsteel_amd import synth
    H, F, NE, K, T = 512, 256, 16, 4, 45
    layer = synth.build_layer(H, F, NE, K, orc.Q4_K, orc.Q4_K, seed=3, layer=31)
    pre = ops.MoePrefill(layer)
    x = synth.activations(T, H, seed=3, layer=32)
    xu = torch.empty(T * H + 1, device="cuda")[1:].view(T, H)
    xu.copy_(x)
    assert xu.data_ptr() % 16 == 4
    wa, wu = pre.workspace(T), pre.workspace(T)
    a, b = host(pre(x, ws=wa)), host(pre(xu, ws=wu))
    ta, tb = pre.trace(wa, T), pre.trace(wu, T)
    for name in ("logits", "xpack", "ids", "w"):
        assert np.array_equal(host(ta[name]), host(tb[name])), f"{name} differs on the unaligned path"
    assert np.array_equal(a, b), "output differs on the unaligned path"


def _skewed_q4k_layer(ops, guard):
    from flintnsteel_amd import synth
    H, F, NE, K = 2048, 768, 128, 8
    base = synth.build_layer(H, F, NE, K, orc.Q4_K, orc.Q4_K, seed=20261022, layer=400)
    rng = np.random.default_rng(20261022)
    bias = dev(np.log(rng.dirichlet(np.full(NE, 0.3)) + 1e-6).astype(np.float32) * 0.5)
    return ops.MoeLayer(base.router_w, base.slots, orc.Q4_K, orc.Q4_K, H, F, K, router_bias=bias, guard=guard)


def test_moe_prefill_fused_launch_equals_two_launches(ops):
    """Without the F16 guard, gate/up and down run as one launch (down workgroups wait for their row group's gate/up
    workgroups); with the guard on and no row scaled, as two launches with the guard pass between them. Every per-item
    computation is the same, so the outputs agree bit for bit - over three calls in a row (the arrival counters are
    re-armed by each call's compaction) and a smaller batch on the same workspace."""
    from flintnsteel_amd import synth
    fused, two = ops.MoePrefill(_skewed_q4k_layer(ops, False)), ops.MoePrefill(_skewed_q4k_layer(ops, True))
    ws_f = fused.workspace(512)
    for T in (512, 512, 77):
        print(f"fused vs two launches, T={T}", flush=True)
        x = synth.activations(T, 2048, seed=20261022, layer=401 + T)
        ws_t = two.workspace(T)
        if T != 512:  # the status word sits elsewhere in another batch size's layout: clear it there first
            fused.status(ws_f, T, clear=True)
        a = host(fused(x, ws=ws_f))
        b = host(two(x, ws=ws_t))
        assert (host(two.trace(ws_t, T)["escale"]) == 1.0).all()
        st = fused.status(ws_f, T)
        rows = np.flatnonzero((a != b).any(axis=1))
        assert np.isfinite(a).all() and rows.size == 0, (f"T={T}: fused launch differs from two launches: status {st}, "
                                                         f"{int(np.isnan(a).sum())} NaN, rows {rows[:16].tolist()} "
                                                         f"of {rows.size}")
        assert st == 0


def test_moe_prefill_fused_wait_timeout_is_reported(ops):
    """Host-forced failure of the fused launch's wait (test hooks: one arrival withheld per group, a short poll
    limit): every down workgroup gives up, writes NaN rows and sets the sticky status bit; every kernel exits. After
    the hooks are reset and the word cleared, the same call is clean and matches its earlier result."""
    from flintnsteel_amd import synth
    from flintnsteel_amd._lib import call
    pre = ops.MoePrefill(_skewed_q4k_layer(ops, False))
    T = 96
    x = synth.activations(T, 2048, seed=3, layer=5)
    ws = pre.workspace(T)
    good = host(pre(x, ws=ws))
    assert pre.status(ws, T) == 0
    print("forced wait timeout (withheld arrivals, poll limit 200)", flush=True)
    call("fns_hip_moe_set_test_hooks", 200, 1)
    try:
        bad = host(pre(x, ws=ws))
    finally:
        call("fns_hip_moe_set_test_hooks", 0, 0)
    assert pre.status(ws, T, clear=True) == ops.STATUS_EXCHANGE_TIMEOUT
    assert np.isnan(bad).any()
    assert pre.status(ws, T) == 0
    again = host(pre(x, ws=ws))
    assert np.array_equal(again, good) and pre.status(ws, T) == 0
    # the graph-capturable collect: nothing to report leaves the destination alone; after a forced timeout it ORs the
    # bit into the destination and clears the word
    dst = torch.full((1,), 4, dtype=torch.int32, device="cuda")
    pre.status_collect(ws, dst, T)
    assert int(host(dst)[0]) == 4
    call("fns_hip_moe_set_test_hooks", 200, 1)
    try:
        pre(x, ws=ws)
    finally:
        call("fns_hip_moe_set_test_hooks", 0, 0)
    pre.status_collect(ws, dst, T)
    assert int(host(dst)[0]) == 4 | ops.STATUS_EXCHANGE_TIMEOUT and pre.status(ws, T) == 0


def test_moe_prefill_fused_launch_with_shared_expert_in_place(ops):
    """The fused gate/up + down launch with everything the layer adds around it: the shared expert, RMSNorm,
    sigmoid gating over 256 experts, and the residual in place (out = x_resid) - bit for bit against the same layer
    with the F16 guard on (two GEMM launches; no row scaled)."""
    from flintnsteel_amd import synth
    H, F, NE, K, FS, T = 2048, 512, 256, 6, 1024, 200
    print("fused launch with shared expert, in place", flush=True)
    lay = synth.build_flint_layer(H, F, NE, K, FS, orc.Q4_K, orc.Q4_K, 20261022, layer=55, guard=False)
    twin = ops.MoeLayer(lay.router_w, lay.slots, orc.Q4_K, orc.Q4_K, H, F, K, gating=ops.GATING_SIGMOID, guard=True,
                        ffn_norm=lay.ffn_norm, norm_eps=1e-6, shexp=lay.shexp)
    fused, two = ops.MoePrefill(lay), ops.MoePrefill(twin)
    x = synth.activations(T, H, seed=20261022, layer=56)
    r1, r2 = synth.activations(T, H, seed=20261022, layer=57), synth.activations(T, H, seed=20261022, layer=57)
    ws_f, ws_t = fused.workspace(T), two.workspace(T)
    fused(x, out=r1, ws=ws_f, x_resid=r1)
    two(x, out=r2, ws=ws_t, x_resid=r2)
    a, b = host(r1), host(r2)
    assert (host(two.trace(ws_t, T)["escale"]) == 1.0).all()
    assert fused.status(ws_f, T) == 0
    rows = np.flatnonzero((a != b).any(axis=1))
    assert np.isfinite(a).all() and rows.size == 0, f"rows {rows[:16].tolist()} of {rows.size} differ"
