"""GGUF checkpoints: the library's reader (fns_hip_gguf_*, include/fns/gguf.h) against files written by
tests/gguf_writer.py, and MoE layers made resident from them (fns_hip_moe_layer_from_gguf).

Reference: src/model.cpp:30-136 (gguf header and tensor table, tensors viewed in the mapped file),
src/engine.cu:375-471 (expert slots [gate | up | down], the device table). The reader tests run on the CPU (no HIP
call); the resident-layer tests run the GGUF-loaded layer and the same layer built directly from the generated
arrays through the decode and prefill paths and require identical outputs, bit for bit: the loader must place every
byte where the slot contract says (the directly built layers are pinned against the float64 oracle elsewhere)."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from oracle import oracle as orc
from tests.gguf_writer import (BF16, F32, GGUF_ARRAY, GGUF_BOOL, GGUF_F32, GGUF_I8, GGUF_STRING, GGUF_U32, bf16_bits,
                               write_gguf)

H, F, NE, K, FS = 512, 256, 16, 4, 512


def _moe_file(path, arch="flint", gating=None, gu=orc.Q4_K, dn=orc.Q6_K, router_dtype=BF16, with_shexp=True,
              with_bias=True, layer=1, seed=3, alignment=32, extra_kv=()):
    """A checkpoint with one MoE block at blk.<layer> (Flint tensor names and metadata) and the arrays it holds."""
    rng = np.random.default_rng(seed)
    w = lambda *s: rng.normal(0, 0.02, s).astype(np.float32)  # noqa: E731
    gate, up, down = orc.quantize(gu, w(NE, F, H)), orc.quantize(gu, w(NE, F, H)), orc.quantize(dn, w(NE, H, F))
    router = w(NE, H) * 50
    router_bits = bf16_bits(router) if router_dtype == BF16 else router
    norm = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(NE)).astype(np.float32)
    p = f"blk.{layer}."
    tensors = [(p + "ffn_norm.weight", F32, [H], norm),
               (p + "ffn_gate_inp.weight", router_dtype, [H, NE], router_bits),
               (p + "ffn_gate_exps.weight", gu, [H, F, NE], gate),
               (p + "ffn_up_exps.weight", gu, [H, F, NE], up),
               (p + "ffn_down_exps.weight", dn, [F, H, NE], down)]
    arrays = {"gate": gate, "up": up, "down": down, "router": router_bits, "norm": norm}
    if with_bias:
        tensors.append((p + "exp_probs_b.bias", F32, [NE], bias))
        arrays["bias"] = bias
    if with_shexp:
        sg, su, sd = orc.quantize(gu, w(FS, H)), orc.quantize(gu, w(FS, H)), orc.quantize(dn, w(H, FS))
        tensors += [(p + "ffn_gate_shexp.weight", gu, [H, FS], sg), (p + "ffn_up_shexp.weight", gu, [H, FS], su),
                    (p + "ffn_down_shexp.weight", dn, [FS, H], sd)]
        arrays.update(sg=sg, su=su, sd=sd)
    kv = [("general.architecture", GGUF_STRING, arch), (f"{arch}.block_count", GGUF_U32, layer + 1),
          (f"{arch}.expert_count", GGUF_U32, NE), (f"{arch}.expert_used_count", GGUF_U32, K),
          (f"{arch}.expert_weights_norm", GGUF_BOOL, 1),
          (f"{arch}.attention.layer_norm_rms_epsilon", GGUF_F32, 1e-6),
          (f"{arch}.attention.sliding_window_pattern", GGUF_ARRAY, (GGUF_I8, [1, 0])),
          ("tokenizer.ggml.tokens", GGUF_ARRAY, (GGUF_STRING, ["<s>", "a", "b"]))]
    if gating is not None:
        kv.append((f"{arch}.expert_gating_func", GGUF_U32, gating))
    kv += list(extra_kv)
    # a tensor of another kind first, so the MoE tensors sit at non-zero offsets
    tensors.insert(0, ("token_embd.weight", 8, [H, 3], np.zeros(3 * H // 32 * 34, np.uint8) + 7))  # Q8_0
    write_gguf(path, kv, tensors, alignment=alignment)
    return arrays


def test_reader_header_metadata_and_tensors(tmp_path):
    from flintnsteel_amd import ops
    path = tmp_path / "m.gguf"
    arrays = _moe_file(path, alignment=64)
    f = ops.GgufFile(path)
    info = f.info()
    assert info["version"] == 3 and info["n_tensors"] == 10 and info["n_kv"] == 9 and info["data_offset"] % 64 == 0
    assert f.str("general.architecture") == "flint"
    assert f.u32("flint.expert_used_count") == K and f.u32("flint.expert_count") == NE
    assert f.bool("flint.expert_weights_norm") is True
    assert abs(f.f32("flint.attention.layer_norm_rms_epsilon") - 1e-6) < 1e-12
    t = f.tensor("blk.1.ffn_gate_exps.weight")
    assert t["type"] == orc.Q4_K and t["ne"] == [H, F, NE] and t["offset"] % 64 == 0
    assert np.array_equal(t["bytes"], arrays["gate"].reshape(-1))
    assert np.array_equal(f.tensor("blk.1.ffn_down_exps.weight")["bytes"], arrays["down"].reshape(-1))
    r = f.tensor("blk.1.ffn_gate_inp.weight")
    assert r["type"] == BF16 and r["ne"] == [H, NE] and np.array_equal(r["bytes"].view(np.uint16), arrays["router"].reshape(-1))
    names = [n for n, _ in f.tensors()]
    assert names[0] == "token_embd.weight" and "blk.1.ffn_down_shexp.weight" in names
    from flintnsteel_amd._lib import FnsError
    with pytest.raises(FnsError, match="no tensor"):
        f.tensor("blk.1.nope")
    with pytest.raises(FnsError, match="missing"):
        f.u32("flint.nope")
    with pytest.raises(FnsError, match="not a u32"):
        f.u32("general.architecture")


def test_reader_rejects_malformed_files(tmp_path):
    from flintnsteel_amd import ops
    from flintnsteel_amd._lib import FnsError
    good = tmp_path / "good.gguf"
    _moe_file(good, with_shexp=False)
    data = good.read_bytes()
    cases = {"bad magic": b"GGUX" + data[4:], "truncated file|larger than the file": data[:600],
             "truncated file|implausible": data[:300],
             "unsupported version": data[:4] + struct.pack("<I", 9) + data[8:],
             "tensor outside the file": data[:-4096]}
    for what, blob in cases.items():
        p = tmp_path / "bad.gguf"
        p.write_bytes(blob)
        with pytest.raises(FnsError, match=what):
            ops.GgufFile(p)
    with pytest.raises(FnsError, match="cannot open"):
        ops.GgufFile(tmp_path / "missing.gguf")


def test_reader_rejects_sizes_that_would_wrap(tmp_path):
    """A tensor whose dimensions multiply past 2^128 bytes (each one allowed, 2^40: 2^42-byte f32 rows x 2^120 = 2^162,
    which a 128-bit product wraps to 0) is rejected as larger than the file instead of wrapping to a small byte count
    (the product is checked one factor at a time); so is one past 2^64."""
    from flintnsteel_amd import ops
    from flintnsteel_amd._lib import FnsError
    p = tmp_path / "huge.gguf"
    big = 1 << 40
    write_gguf(p, [("general.architecture", GGUF_STRING, "flint")],
               [("blk.0.huge.weight", F32, [big, big, big, big], np.zeros(64, np.float32))])
    with pytest.raises(FnsError, match="larger than the file"):
        ops.GgufFile(p)
    p2 = tmp_path / "wrap.gguf"  # 2^40 x 2^24 f32 = 2^66 bytes: a plain 64-bit product would wrap to 0
    write_gguf(p2, [("general.architecture", GGUF_STRING, "flint")],
               [("blk.0.wrap.weight", F32, [big, 1 << 24], np.zeros(64, np.float32))])
    with pytest.raises(FnsError, match="larger than the file"):
        ops.GgufFile(p2)


def test_layer_build_rejects_expert_weights_scale(tmp_path):
    """The reference requires <arch>.expert_weights_scale == 1 (src/model.cpp:83,167); the combine applies no scale,
    so a checkpoint with another value is rejected (CPU: the check runs before any device allocation)."""
    from flintnsteel_amd import ops
    from flintnsteel_amd._lib import FnsError
    p = tmp_path / "scaled.gguf"
    _moe_file(p, with_shexp=False, extra_kv=[("flint.expert_weights_scale", GGUF_F32, 2.5)])
    f = ops.GgufFile(p)
    with pytest.raises(FnsError, match="expert_weights_scale"):
        ops.MoeLayer.from_gguf(f, 1)


def test_layer_build_rejects_unsupported_checkpoints(tmp_path):
    """Shape and type checks run before any device allocation (CPU): unsupported expert type, missing tensors."""
    from flintnsteel_amd import ops
    from flintnsteel_amd._lib import FnsError
    p = tmp_path / "q2k.gguf"
    rng = np.random.default_rng(0)
    q2k = rng.integers(0, 255, NE * F * (H // 256) * 84, dtype=np.uint8)
    write_gguf(p, [("general.architecture", GGUF_STRING, "flint"), ("flint.expert_used_count", GGUF_U32, K)],
               [("blk.0.ffn_gate_exps.weight", 10, [H, F, NE], q2k), ("blk.0.ffn_up_exps.weight", 10, [H, F, NE], q2k),
                ("blk.0.ffn_down_exps.weight", 10, [F, H, NE], q2k),
                ("blk.0.ffn_gate_inp.weight", F32, [H, NE], np.zeros(H * NE, np.float32))])
    f = ops.GgufFile(p)
    with pytest.raises(FnsError, match="not supported by the GEMV kernels"):
        ops.MoeLayer.from_gguf(f, 0)
    with pytest.raises(FnsError, match="missing tensor"):
        ops.MoeLayer.from_gguf(f, 3)


def _direct_layer(ops, torch, arrays, gu, dn, router_dtype, gating, guard, with_shexp, with_bias):
    """The same layer built from the arrays through ops.MoeLayer (ExpertSlots)."""
    slots = ops.ExpertSlots.from_tensors(torch.from_numpy(arrays["gate"].reshape(NE, -1)),
                                         torch.from_numpy(arrays["up"].reshape(NE, -1)),
                                         torch.from_numpy(arrays["down"].reshape(NE, -1)))
    if router_dtype == BF16:
        router = torch.from_numpy(arrays["router"].astype(np.int16)).view(torch.bfloat16).cuda()
    else:
        router = torch.from_numpy(arrays["router"]).cuda()
    shexp = None
    if with_shexp:
        shexp = {"gate": torch.from_numpy(arrays["sg"]).cuda(), "up": torch.from_numpy(arrays["su"]).cuda(),
                 "down": torch.from_numpy(arrays["sd"]).cuda(), "inter": FS, "gu_type": gu, "down_type": dn}
    return ops.MoeLayer(router, slots, gu, dn, H, F, K, gating=gating, guard=guard,
                        router_bias=torch.from_numpy(arrays["bias"]).cuda() if with_bias else None,
                        ffn_norm=torch.from_numpy(arrays["norm"]).cuda(), norm_eps=1e-6, shexp=shexp)


@pytest.mark.gpu
@pytest.mark.parametrize("variant", ["flint", "softmax_f32"])
def test_gguf_layer_equals_directly_built_layer(tmp_path, variant):
    import torch
    from flintnsteel_amd import ops, synth
    flint = variant == "flint"
    kw = dict(arch="flint" if flint else "testmoe", gating=None if flint else 1,
              router_dtype=BF16 if flint else F32, with_shexp=flint, with_bias=flint)
    print(f"gguf layer variant {variant}", flush=True)
    path = tmp_path / "m.gguf"
    arrays = _moe_file(path, **kw)
    f = ops.GgufFile(path)
    g = ops.MoeLayer.from_gguf(f, 1)
    d = g.desc
    assert (d.hidden, d.inter, d.n_expert, d.k) == (H, F, NE, K)
    assert d.gating == (ops.GATING_SIGMOID if flint else ops.GATING_SOFTMAX) and d.norm_w == 1
    assert d.guard == int(flint) and d.shexp_inter == (FS if flint else 0)
    ref = _direct_layer(ops, torch, arrays, orc.Q4_K, orc.Q6_K, kw["router_dtype"], d.gating, bool(d.guard),
                        kw["with_shexp"], kw["with_bias"])
    for n_tok in (1, 4):
        x = synth.activations(n_tok, H, 5, layer=n_tok)
        a, b = g(x, x_resid=x), ref(x, x_resid=x)
        torch.cuda.synchronize()
        assert np.array_equal(a.cpu().numpy(), b.cpu().numpy()), f"decode/verify n_tok={n_tok} differs"
    x = synth.activations(37, H, 5, layer=9)
    a, b = ops.MoePrefill(g)(x, x_resid=x), ops.MoePrefill(ref)(x, x_resid=x)
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy(), b.cpu().numpy()), "prefill differs"
    del g
    f.close()


DF = 768  # dense FFN width of the small files


def _dense_file(path, gt=orc.Q4_K, ut=orc.Q4_K, dt=orc.Q6_K, layer=0, seed=11, h=H, f=DF, down_shape=None):
    """A checkpoint with one dense FFN block at blk.<layer> (reference names, src/model.cpp:120-125)."""
    rng = np.random.default_rng(seed)
    w = lambda *s: rng.normal(0, 0.02, s).astype(np.float32)  # noqa: E731
    gate, up, down = orc.quantize(gt, w(f, h)), orc.quantize(ut, w(f, h)), orc.quantize(dt, w(h, f))
    norm = (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32)
    p = f"blk.{layer}."
    tensors = [(p + "ffn_norm.weight", F32, [h], norm), (p + "ffn_gate.weight", gt, [h, f], gate),
               (p + "ffn_up.weight", ut, [h, f], up), (p + "ffn_down.weight", dt, down_shape or [f, h], down)]
    kv = [("general.architecture", GGUF_STRING, "flint"), ("flint.block_count", GGUF_U32, layer + 1),
          ("flint.attention.layer_norm_rms_epsilon", GGUF_F32, 1e-5)]
    tensors.insert(0, ("token_embd.weight", 8, [h, 3], np.zeros(3 * h // 32 * 34, np.uint8) + 7))
    write_gguf(path, kv, tensors)
    return {"gate": gate, "up": up, "down": down, "norm": norm}


def test_dense_build_rejects_unsupported_checkpoints(tmp_path):
    """The dense loader's checks run before any device allocation (CPU): a type without a GEMV kernel, a down matrix
    whose shape does not match gate / up, a missing tensor."""
    from flintnsteel_amd import ops
    from flintnsteel_amd._lib import FnsError
    p = tmp_path / "d.gguf"
    _dense_file(p)
    f = ops.GgufFile(p)
    with pytest.raises(FnsError, match="missing tensor"):
        ops.DenseFfn.from_gguf(f, 1)
    f.close()
    p2 = tmp_path / "d2.gguf"
    rng = np.random.default_rng(1)
    q2k = rng.integers(0, 255, DF * (H // 256) * 84, dtype=np.uint8)
    q4k = orc.quantize(orc.Q4_K, np.zeros((DF, H), np.float32))
    write_gguf(p2, [("general.architecture", GGUF_STRING, "flint")],
               [("blk.0.ffn_gate.weight", 10, [H, DF], q2k), ("blk.0.ffn_up.weight", 10, [H, DF], q2k),
                ("blk.0.ffn_down.weight", orc.Q4_K, [DF, H], orc.quantize(orc.Q4_K, np.zeros((H, DF), np.float32))),
                ("blk.1.ffn_gate.weight", orc.Q4_K, [H, DF], q4k), ("blk.1.ffn_up.weight", orc.Q4_K, [H, DF], q4k),
                ("blk.1.ffn_down.weight", orc.Q4_K, [DF, H // 2],
                 orc.quantize(orc.Q4_K, np.zeros((H // 2, DF), np.float32)))])
    f2 = ops.GgufFile(p2)
    with pytest.raises(FnsError, match="not supported by the GEMV kernels"):
        ops.DenseFfn.from_gguf(f2, 0)
    with pytest.raises(FnsError, match="dense FFN layer 1: unexpected shape of blk.1.ffn_down.weight"):
        ops.DenseFfn.from_gguf(f2, 1)
    f2.close()


def _dense_ref(arrays, gt, ut, dt, h_dim, f_dim, x: np.ndarray, eps: float) -> np.ndarray:
    """float64 chain of the dense block: RMSNorm, Q8_1, gate / up GEMVs, SwiGLU, Q8_1 of act, down, + x."""
    x64 = x.astype(np.float64)
    hn = (x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + eps) * arrays["norm"]).astype(np.float32)
    xq = orc.quantize_q8_1(hn)
    n = x.shape[0]
    mv = lambda t, m, nc, nr, q: orc.mmvq_experts(t, [m], nc, nr, q, q.shape[0], 1, np.zeros(q.shape[0], np.int32))  # noqa: E731
    g = mv(gt, arrays["gate"].reshape(f_dim, -1), h_dim, f_dim, xq)
    u = mv(ut, arrays["up"].reshape(f_dim, -1), h_dim, f_dim, xq)
    act = orc.swiglu(g, u).astype(np.float32)
    y = mv(dt, arrays["down"].reshape(h_dim, -1), f_dim, h_dim, orc.quantize_q8_1(act))
    assert y.shape == (n, h_dim)
    return y + x64


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["small", "small_same", "flint", "flint_k"])
def test_gguf_dense_ffn(tmp_path, shape):
    """A dense FFN block loaded from GGUF (fns_hip_dense_ffn_from_gguf) equals the same block built from the arrays,
    bit for bit, in the decode (1 and 4 tokens) and prefill forms, and both forms match the float64 chain. "flint" is
    the reference model's dense shape (hidden 2048, FFN 6144, src/model.cpp:163) with Q8_0 gate / up."""
    import torch
    from flintnsteel_amd import ops, synth
    from tests.helpers import assert_close_chain
    # small: gate / up of different types (three mmq calls); small_same, flint, flint_k: one GLU launch for gate and
    # up and the down GEMM with its K range split (K-quant min terms in flint_k)
    h_dim, f_dim = (H, DF) if shape.startswith("small") else (2048, 6144)
    gt, ut, dt = {"small": (orc.Q4_K, orc.Q5_K, orc.Q6_K), "small_same": (orc.Q4_K, orc.Q4_K, orc.Q6_K),
                  "flint": (orc.Q8_0, orc.Q8_0, orc.Q6_K), "flint_k": (orc.Q5_K, orc.Q5_K, orc.Q4_K)}[shape]
    print(f"dense ffn {shape} {h_dim}x{f_dim}", flush=True)
    path = tmp_path / "d.gguf"
    arrays = _dense_file(path, gt, ut, dt, layer=1, h=h_dim, f=f_dim)
    f = ops.GgufFile(path)
    g = ops.DenseFfn.from_gguf(f, 1)
    d = g.desc
    assert (d.hidden, d.inter, d.gate_type, d.up_type, d.down_type) == (h_dim, f_dim, gt, ut, dt)
    assert abs(d.norm_eps - 1e-5) < 1e-12
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    ref = ops.DenseFfn(cu(arrays["gate"]), cu(arrays["up"]), cu(arrays["down"]), gt, ut, dt, h_dim, f_dim,
                       ffn_norm=cu(arrays["norm"]), norm_eps=1e-5)
    for n_tok, prefill in ((1, False), (4, False), (37, True)):
        x = synth.activations(n_tok, h_dim, 5, layer=n_tok)
        a, b = g(x, prefill=prefill), ref(x, prefill=prefill)
        torch.cuda.synchronize()
        a, b = a.cpu().numpy(), b.cpu().numpy()
        assert np.array_equal(a, b), f"n_tok={n_tok} prefill={prefill}: GGUF-built layer differs"
        toks = [0, n_tok - 1] if n_tok > 1 else [0]
        xs = x.cpu().numpy()
        assert_close_chain(a[toks], _dense_ref(arrays, gt, ut, dt, h_dim, f_dim, xs[toks], 1e-5),
                           f"dense ffn {shape} n_tok={n_tok} prefill={prefill}")
        if n_tok == 4:  # verify columns equal the single-token decode, column by column
            for t in range(4):
                one = ref(x[t:t + 1].contiguous())
                torch.cuda.synchronize()
                assert np.array_equal(one.cpu().numpy()[0], a[t]), f"verify column {t}"
    # in place (out = x), as the reference's add_inplace on the residual stream
    x = synth.activations(1, h_dim, 6, layer=0)
    want = ref(x)
    ref(x, out=x)
    torch.cuda.synchronize()
    assert np.array_equal(x.cpu().numpy(), want.cpu().numpy()), "in-place call differs"
    del g
    f.close()


@pytest.mark.gpu
def test_mmvq_bench_tool_on_a_file(tmp_path):
    """The GEMV timing tool (flintnsteel_amd/mmvq_bench.py, the reference's fns-mmvq-bench) runs on a GGUF file:
    gate + up, down, the dense GEMV over the shared expert's gate, and the whole layer."""
    import argparse
    from flintnsteel_amd import mmvq_bench
    print("mmvq_bench on a file", flush=True)
    path = tmp_path / "m.gguf"
    _moe_file(path)
    lines = mmvq_bench.run(argparse.Namespace(model=str(path), synthetic=False, layer=1, reps=3, gu=None, down=None))
    assert len(lines) == 4 and "gate+up Q4_K" in lines[0] and "down    Q6_K" in lines[1], lines
    assert "ffn_gate_shexp.weight" in lines[2] and "whole MoE layer" in lines[3], lines
