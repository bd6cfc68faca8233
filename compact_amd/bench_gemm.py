"""Per-GEMM comparison on the C2 FFN shapes: this build's dispatch (the
16x16x32 loop at these shapes, with its fused FlashFFN kernels), the 32x32x16
engine where a plain product can be forced onto it, and the library GEMM torch
calls (hipBLASLt) with the standalone codec kernels.

    python -m compact_amd.bench_gemm [--iters 20] [--json out.json]

Prints one line per GEMM of a C2 fwd+bwd step (8192 tokens, d_model 4096,
d_ff 11008, bf16), timed with HIP events on the current stream.
"""

from __future__ import annotations

import argparse
import json

import torch

from . import gemm as G
from . import kernels as K


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--json", default=None)
    args = ap.parse_args()
    n, h, d, gs = 8192, 4096, 11008, 128
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(n, h, device=dev, generator=g).bfloat16()
    gy = torch.randn(n, h, device=dev, generator=g).bfloat16()
    wg = (torch.randn(d, h, device=dev, generator=g) * .02).bfloat16()
    wu = (torch.randn(d, h, device=dev, generator=g) * .02).bfloat16()
    wd = (torch.randn(h, d, device=dev, generator=g) * .02).bfloat16()
    hm = torch.randn(n, d, device=dev, generator=g).bfloat16()
    _, qg, sg, qu, su = K.silu_mul_quant(hm, hm, 8, gs)
    fl = 2 * n * h * d

    def lib_gate_up():
        a, b = x @ wg.t(), x @ wu.t()
        return K.silu_mul_quant(a, b, 8, gs)

    def lib_dgrad():
        return K.dequant_swiglu_backward(gy @ wd, qg, sg, qu, su, 8, gs, want_h_mid=True)

    # arms: this build's dispatch (the 16x16x32 loop at these shapes), the
    # 32x32x16 engine where one plain product can be forced onto it
    # (gemm.mm_engine), and hipBLASLt (+ the standalone codec kernels)
    cases = [
        ("fwd gate/up + GLU + int8 codec", lambda: G.ffn_gate_up(x, wg, wu, 8, gs), None, lib_gate_up, 2 * fl),
        ("fwd down  h_mid @ Wd^T", lambda: G.linear(hm, wd), lambda: G.mm_engine(hm, wd.t()),
         lambda: hm @ wd.t(), fl),
        ("bwd gy @ Wd + dequant + SwiGLU bwd", lambda: G.ffn_down_dgrad(gy, wd, 8, gs, qg, sg, qu, su, True),
         None, lib_dgrad, fl),
        ("bwd gy @ Wd", lambda: G.mm(gy, wd), lambda: G.mm_engine(gy, wd), lambda: gy @ wd, fl),
        ("bwd dWd = gy^T @ h_mid", lambda: G.mm(gy.t(), hm), lambda: G.mm_engine(gy.t(), hm),
         lambda: gy.t() @ hm, fl),
        ("bwd dx = dg @ Wg + du @ Wu", lambda: G.mm2(hm, wg, hm, wu), None, lambda: hm @ wg + hm @ wu, 2 * fl),
        ("bwd dWg = dg^T @ x", lambda: G.mm(hm.t(), x), lambda: G.mm_engine(hm.t(), x), lambda: hm.t() @ x, fl),
    ]
    out = {}
    for name, mine, eng, lib, flops in cases:
        a, b = _time(mine, args.iters), _time(lib, args.iters)
        e = _time(eng, args.iters) if eng is not None else None
        out[name] = {"build_ms": a, "engine_ms": e, "library_ms": b, "build_tflops": flops / a / 1e9,
                     "engine_tflops": flops / e / 1e9 if e else None,
                     "library_tflops": flops / b / 1e9}
        es = f"engine {e:7.3f} ms {flops / e / 1e9:7.1f} TF/s" if e else f"{'engine -':30s}"
        print(f"{name:38s} build {a:7.3f} ms {flops / a / 1e9:7.1f} TF/s | {es} | "
              f"library {b:7.3f} ms {flops / b / 1e9:7.1f} TF/s", flush=True)
    # The down projection's weight gradient, both routes of this build: K2
    # writing h_mid^ and the plain TN GEMM, against K2 without h_mid^ and the
    # GEMM that rebuilds h^ from the int8 cache in its operand staging.
    def k2_then_tn():
        _, _, hmh = K.dequant_swiglu_backward(hm, qg, sg, qu, su, 8, gs, want_h_mid=True)
        return G.mm(gy.t(), hmh)

    def k2_then_glu():
        K.dequant_swiglu_backward(hm, qg, sg, qu, su, 8, gs, want_h_mid=False)
        return G.wgrad_glu(gy, 8, gs, qg, sg, qu, su)

    a, b = _time(k2_then_tn, args.iters), _time(k2_then_glu, args.iters)
    c = _time(lambda: G.wgrad_glu(gy, 8, gs, qg, sg, qu, su), args.iters)
    out["dWd route"] = {"k2_h_mid_then_tn_ms": a, "k2_then_wgrad_glu_ms": b,
                        "wgrad_glu_alone_ms": c, "wgrad_glu_tflops": fl / c / 1e9}
    print(f"{'bwd dWd: K2 + h_mid^ + TN GEMM':38s} {a:7.3f} ms | K2 + GEMM with the GLU in its "
          f"operand staging {b:7.3f} ms (that GEMM alone {c:7.3f} ms, {fl / c / 1e9:7.1f} TF/s)",
          flush=True)
    if args.json:
        json.dump(out, open(args.json, "w"), indent=1)


if __name__ == "__main__":
    main()
