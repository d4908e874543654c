"""Timing of the expert GEMVs on GGUF blocks, in isolation (diagnostic; the reference's fns-mmvq-bench,
tests/mmvq_bench.cu:1-91).

    python -m flintnsteel_amd.mmvq_bench --model F.gguf [--layer 3] [--reps 200]
    python -m flintnsteel_amd.mmvq_bench --synthetic [--gu IQ3_XXS] [--down IQ4_XS] [--reps 200]

For one MoE layer: gate + up + SwiGLU of 6 experts (mmvq_ids_swiglu_shared, one input), down (mmvq_ids, 6 inputs),
a dense GEMV over the layer's attn_q (or, when the file has none, its shared expert's gate), and the whole decode
layer (fns_hip_moe_layer). Median of `reps` timings (HIP events) and the effective GB/s of the bytes each call
must read. --synthetic builds the reference model's MoE block shape (hidden 2048, 256 experts of width 512, top-6,
shared expert 1024) from random blocks of the given types and seeded IQ codebooks (ggml's own tables are data of
the caller, registered with fns_hip_set_iq_grids; see the library's documentation) instead of reading a file.
"""
from __future__ import annotations

import argparse
import sys

import torch

from . import ops, synth

TYPES = {"Q4_K": ops.Q4_K, "Q5_K": ops.Q5_K, "Q6_K": ops.Q6_K, "Q3_K": ops.Q3_K, "Q8_0": ops.Q8_0,
         "IQ3_XXS": ops.IQ3_XXS, "IQ3_S": ops.IQ3_S, "IQ2_S": ops.IQ2_S, "IQ4_XS": ops.IQ4_XS}
IDS = [3, 77, 140, 201, 9, 250]  # the reference tool's expert ids


def median_us(reps: int, fn) -> float:
    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t = []
    for _ in range(reps):
        a.record()
        fn()
        b.record()
        b.synchronize()
        t.append(a.elapsed_time(b) * 1e3)
    t.sort()
    return t[len(t) // 2]


def _dev(info: dict) -> torch.Tensor:
    """A tensor's blocks on the device, with 4096 zero bytes after them (the reference tool's upload)."""
    out = torch.zeros(info["nbytes"] + 4096, dtype=torch.uint8, device="cuda")
    out[: info["nbytes"]].copy_(torch.from_numpy(info["bytes"].reshape(-1)))
    return out


def run(args) -> list[str]:
    reps = args.reps
    if args.model:
        f = ops.GgufFile(args.model)
        p = f"blk.{args.layer}."
        gi, ui, di = (f.tensor(p + n) for n in ("ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight"))
        H, F, NE = gi["ne"][0], gi["ne"][1], gi["ne"][2]
        gu_t, dn_t = gi["type"], di["type"]
        g, u, dn = _dev(gi), _dev(ui), _dev(di)
        dense = None
        for name in ("attn_q.weight", "ffn_gate_shexp.weight"):
            try:
                t = f.tensor(p + name)
            except Exception:  # noqa: BLE001 - the tensor is optional
                continue
            dense = (name, t["type"], _dev(t), t["ne"][0], t["ne"][1], t["nbytes"])
            break
        layer = ops.MoeLayer.from_gguf(f, args.layer)
    else:
        gu_t, dn_t = TYPES[args.gu], TYPES[args.down]
        H, F, NE = 2048, 512, 256
        if gu_t in synth.IQ_BLOCK_BYTES or dn_t in synth.IQ_BLOCK_BYTES:
            synth.register_iq_grids()
            layer = synth.build_iq_flint_layer(H, F, NE, 6, 1024, gu_t, dn_t, 20261022, layer=3)
        else:
            layer = synth.build_flint_layer(H, F, NE, 6, 1024, gu_t, dn_t, 20261022, layer=3)
        s = layer.slots
        g, u, dn = (torch.cat([s.view(n).reshape(-1), torch.zeros(4096, dtype=torch.uint8, device="cuda")])
                    for n in ("gate", "up", "down"))
        sh = layer.shexp
        dense = ("ffn_gate_shexp (synthetic)", gu_t, sh["gate"], H, sh["inter"], sh["gate"].numel())
    K = len(IDS)
    ids = torch.tensor(IDS, dtype=torch.int32, device="cuda") % NE
    x = torch.full((K, max(H, F)), 0.25, device="cuda")
    xq = ops.quantize_q8_1(x[:1, :H].contiguous())
    y = torch.empty(K, max(H, F), device="cuda")
    gu_bytes = 2.0 * K * ops.row_bytes(gu_t, H) * F
    dn_bytes = 1.0 * K * ops.row_bytes(dn_t, F) * H
    t_gu = median_us(reps, lambda: ops.mmvq_ids_swiglu_shared(gu_t, g, u, H, F, NE, xq, ids, dst=y[:, :F]))
    xq6 = ops.quantize_q8_1(x[:, :F].contiguous())
    t_dn = median_us(reps, lambda: ops.mmvq_ids(dn_t, dn, F, H, NE, xq6, K, ids, dst=y[:, :H]))
    lines = [f"layer {args.layer}  gate+up {ops.TYPE_NAMES[gu_t]:7s} {t_gu:7.1f} us  {gu_bytes / t_gu / 1e3:6.0f} GB/s",
             f"layer {args.layer}  down    {ops.TYPE_NAMES[dn_t]:7s} {t_dn:7.1f} us  {dn_bytes / t_dn / 1e3:6.0f} GB/s"]
    if dense:
        name, dt, w, nc, nr, nb = dense
        if ops.mmvq_supports(dt):
            dy = torch.empty(nr, device="cuda")
            t_q = median_us(reps, lambda: ops.mmvq(dt, w, nc, nr, xq, 1, dst=dy))
            lines.append(f"layer {args.layer}  {name} {ops.TYPE_NAMES.get(dt, dt)}  {t_q:7.1f} us  {nb / t_q / 1e3:6.0f} GB/s")
    xl = torch.randn(1, H, device="cuda")
    out = torch.empty_like(xl)
    ws = layer.workspace(1)
    t_l = median_us(reps, lambda: layer(xl, out=out, ws=ws, x_resid=xl))
    lines.append(f"layer {args.layer}  whole MoE layer (decode) {t_l:7.1f} us")
    return lines


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--model")
    ap.add_argument("--synthetic", action="store_true")
    ap.add_argument("--layer", type=int, default=3)
    ap.add_argument("--reps", type=int, default=200)
    ap.add_argument("--gu", default="IQ3_XXS", choices=sorted(TYPES))
    ap.add_argument("--down", default="IQ4_XS", choices=sorted(TYPES))
    args = ap.parse_args(argv)
    if not args.model and not args.synthetic:
        print("usage: python -m flintnsteel_amd.mmvq_bench --model F.gguf [--layer N] [--reps N] | --synthetic",
              file=sys.stderr)
        return 2
    for line in run(args):
        print(line, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
