"""HBM bandwidth of the standalone codec / GLU kernels at the C2 and C3 shapes.

    python -m compact_amd.bench_codec [--iters 20] [--json out.json]

These kernels are HBM-bound; each line gives the algorithmic bytes of one
launch (every input read once, every output written once), the mean time
over `--iters` launches (HIP events on the current stream, after 3 warmup
launches) and the achieved GB/s as a fraction of MI355X's 8 TB/s and of a
1 GiB device-to-device copy measured in the same run.

Shapes: C2 is 8192 tokens x d_ff 11008 with the int8 g128 cache; C3 is the
same with the int4 g64 cache and the top-1% (110) outlier channels kept in
bf16.  The kernels are the standalone K1 / K2 (the reference's
`triton_silu_mul_quant` / `triton_dequant_swiglu_backward`,
src/flashffn.py:1314-1373), the plain codec (`v3_quantize_group_absmax` /
`v3_dequantize_group_absmax`, :1055-1110), the GLU kernels (:205-293) and
the outlier variants of C3.
"""

from __future__ import annotations

import argparse
import json

import torch

from . import kernels as K

PEAK_GBS = 8000.0


def _time(fn, iters):
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def _payload(n, d, bits):
    return n * d // 2 if bits == 4 else n * d


def cases(n, d, dev):
    """(name, fn, algorithmic bytes) for every standalone kernel at (n, d)."""
    g = torch.Generator(device=dev).manual_seed(0)
    hg = (torch.randn(n, d, device=dev, generator=g) * 3).bfloat16()
    hu = (torch.randn(n, d, device=dev, generator=g) * 2).bfloat16()
    dh = torch.randn(n, d, device=dev, generator=g).bfloat16()
    e = n * d * 2                      # one bf16 [n, d] tensor
    out = []
    for tag, bits, gs in (("c2 int8 g128", 8, 128), ("c3 int4 g64", 4, 64)):
        pay, sc = _payload(n, d, bits), n * (d // gs) * 2
        _, qg, sg, qu, su = K.silu_mul_quant(hg, hu, bits, gs)
        out += [
            (f"K1 silu_mul_quant {tag}", lambda b=bits, s=gs: K.silu_mul_quant(hg, hu, b, s),
             2 * e + e + 2 * pay + 2 * sc),
            (f"K2 dequant_swiglu_backward {tag} (+h_mid^)",
             lambda b=bits, s=gs, q=(qg, sg, qu, su): K.dequant_swiglu_backward(
                 dh, *q, b, s, want_h_mid=True),
             e + 2 * pay + 2 * sc + 3 * e),
            (f"quantize {tag}", lambda b=bits, s=gs: K.v3_quantize_group_absmax(hg, b, s),
             e + pay + sc),
            (f"dequantize {tag}",
             lambda b=bits, s=gs, q=(qg, sg): K.v3_dequantize_group_absmax(q[0], q[1], b, s),
             pay + sc + e),
        ]
    # C3 outlier channels: 1% of d (floor), HyC-LoRA's int(N * ratio)
    k = int(d * 0.01)
    slot_g, _ = K.outlier_select(hg, k)
    slot_u, _ = K.outlier_select(hu, k)
    pay, sc, ob = _payload(n, d, 4), n * (d // 64) * 2, n * k * 2
    r = K.silu_mul_quant_outlier(hg, hu, 4, 64, slot_g, slot_u, k)
    out += [
        ("K1 silu_mul_quant c3 int4 g64 + 1% outliers",
         lambda: K.silu_mul_quant_outlier(hg, hu, 4, 64, slot_g, slot_u, k),
         2 * e + e + 2 * pay + 2 * sc + 2 * ob),
        ("K2 dequant_swiglu_backward c3 int4 g64 + 1% outliers (+h_mid^)",
         lambda: K.dequant_swiglu_backward_outlier(dh, r[1], r[2], r[3], slot_g, r[4], r[5],
                                                   r[6], slot_u, 4, 64, want_h_mid=True),
         e + 2 * pay + 2 * sc + 2 * ob + 3 * e),
        ("outlier_select c3 (column norms + radix select)", lambda: K.outlier_select(hg, k), e),
        ("silu_mul (GLU fwd)", lambda: K.silu_mul(hg, hu), 3 * e),
        ("swiglu_backward_glu (GLU bwd + h_mid)",
         lambda: K.swiglu_backward_glu(dh, hg, hu, True), 6 * e),
    ]
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=8192)
    ap.add_argument("--inter", type=int, default=11008)
    ap.add_argument("--json", default=None)
    args = ap.parse_args()
    dev = "cuda"
    src = torch.empty(1 << 29, dtype=torch.bfloat16, device=dev)   # 1 GiB
    dst = torch.empty_like(src)
    copy_ms = _time(lambda: dst.copy_(src), args.iters)
    copy_gbs = 2 * src.numel() * 2 / copy_ms / 1e6
    del src, dst
    print(f"{'1 GiB device copy':62s} {copy_ms:8.3f} ms {copy_gbs:8.0f} GB/s "
          f"{copy_gbs / PEAK_GBS:5.2f} of 8 TB/s", flush=True)
    res = {"copy_gbs": copy_gbs, "kernels": {}}
    for name, fn, nbytes in cases(args.tokens, args.inter, dev):
        ms = _time(fn, args.iters)
        gbs = nbytes / ms / 1e6
        res["kernels"][name] = {"ms": ms, "bytes": nbytes, "gbs": gbs,
                                "frac_peak": gbs / PEAK_GBS, "frac_copy": gbs / copy_gbs}
        print(f"{name:62s} {ms:8.3f} ms {gbs:8.0f} GB/s {gbs / PEAK_GBS:5.2f} of 8 TB/s "
              f"{gbs / copy_gbs:5.2f} of copy  ({nbytes / 1e6:.1f} MB)", flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump(res, f, indent=1)


if __name__ == "__main__":
    main()
