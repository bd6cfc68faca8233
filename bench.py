"""Benchmark: FlashFFN v3 SwiGLU FFN fwd+bwd tokens/s + saved-activation MB on
one MI355X (BASELINE.json metric), workload C2: Llama-7B FFN dims
d_model=4096, d_ff=11008, 8x1024 tokens, bf16, int8 per-group(128) GLU cache,
full fine-tune (dense weight grads), synthetic seeded inputs.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Prints ONE JSON line.  A step is one forward + backward of the FFN block on
the same resident inputs.  `roofline` is for the dominant HIP kernel of this
build, timed live with HIP events on its launch stream inside the timed steps;
`kernels` lists every timed kernel.  `cpu_baseline` times the CPU oracle (the
restatement of the reference's FlashFFNv3Function; the reference itself
cannot run on a CPU) on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# workload C2; C3 with --workload c3
N_TOK, HID, INTER, GROUP, BITS = 8 * 1024, 4096, 11008, 128, 8
MODE = "int8"
WORKLOADS = {
    "c2": dict(group=128, bits=8, mode="int8", lora_rank=0, outlier_ratio=0.0,
               desc="C2: SwiGLU FFN fwd+bwd, d_model=4096, d_ff=11008, 8x1024 tokens, bf16, "
                    "int8 per-group(128) cache, full-FT"),
    "c2f": dict(group=128, bits=8, mode="int8", lora_rank=0, outlier_ratio=0.0, frozen=True,
                desc="C2 frozen: C2 with the weights frozen and no adapter (grad_x only), the "
                     "frozen-weight variant of C2"),
    "c3": dict(group=64, bits=4, mode="int4", lora_rank=16, outlier_ratio=0.01,
               desc="C3: C2 + LoRA r16 (alpha 32) on gate/up/down, frozen base, int4 "
                    "per-group(64) cache with top-1% outlier channels in bf16"),
}

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, published
PROBE_COPY_BYTES = 1 << 30      # calibration copy of the --probe mode
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16, published


def codec_bytes(n, d, bits, group, want_h_mid=True):
    """Algorithmic HBM bytes of the standalone codec kernels (per launch).
    K1: read g,u bf16; write h_mid bf16, 2 payloads, 2 fp16 scale arrays.
    K2: read dh bf16, 2 payloads, 2 scale arrays; write dg, du (+ h_mid^) bf16."""
    payload = n * d // 2 if bits == 4 else n * d
    scales = n * (d // group) * 2
    k1 = 2 * n * d * 2 + n * d * 2 + 2 * payload + 2 * scales
    k2 = n * d * 2 + 2 * payload + 2 * scales + 2 * n * d * 2 + (n * d * 2 if want_h_mid else 0)
    return k1, k2


def algorithmic_work(n, h, d):
    """Per-launch algorithmic work of every timed kernel: (amount, bound),
    FLOPs for the MFMA-bound GEMMs (2*M*N*K per product), bytes for the
    HBM-bound standalone codec kernels."""
    k1_bytes, k2_bytes = codec_bytes(n, d, BITS, GROUP)
    gemm = 2 * n * h * d
    return {
        "ffn_gate_up": (2 * gemm, "mfma"),          # x @ [Wg; Wu]^T (+ GLU + codec)
        "gemm_fwd_down": (gemm, "mfma"),            # h_mid @ Wd^T
        "ffn_down_dgrad": (gemm, "mfma"),           # gy @ Wd (+ dequant + SwiGLU bwd)
        "gemm_dgrad_down": (gemm, "mfma"),          # gy @ Wd (K2 runs after it)
        "gemm_wgrad_down": (gemm, "mfma"),          # gy^T @ h_mid^
        "gemm_dgrad_x": (2 * gemm, "mfma"),         # dg @ Wg + du @ Wu
        "gemm_wgrad_gate": (gemm, "mfma"),          # dg^T @ x
        "gemm_wgrad_up": (gemm, "mfma"),            # du^T @ x
        "silu_mul_quant": (k1_bytes, "hbm"),
        "dequant_swiglu_backward": (k2_bytes, "hbm"),
    }


def gemm_flops_fwd_bwd(n, h, d, full_ft=True):
    """3 GEMMs forward, 6 backward (full-FT) of 2*N*H*D FLOPs each."""
    return (18 if full_ft else 12) * n * h * d


def saved_bytes(fn, exclude_ptrs):
    """Saved-for-backward bytes, deduplicated by storage, parameters and x
    excluded (the reference's accounting, src/verify_flashffn_v3.py:523-543)."""
    import torch
    seen, total = set(), 0

    def pack(t):
        nonlocal total
        key = (t.data_ptr(), t.nbytes)
        if t.data_ptr() not in exclude_ptrs and key not in seen:
            seen.add(key)
            total += t.nbytes
        return t

    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        y = fn()
    del y
    return total


def cpu_baseline(budget_tokens=512):
    """Times the CPU oracle's FlashFFNv3Function (fp32, int8 g128, full-FT)
    on `budget_tokens` tokens of the C2 shape: 1 warmup + 3 reps, median."""
    import torch
    from oracle import flashffn_ref as R
    torch.set_num_threads(os.cpu_count() or 1)
    ps = R.synthetic_param_set("fullft", HID, INTER, 0, 0.0, seed=0, dtype=torch.float32)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(budget_tokens, HID, generator=g)
    gy = torch.randn(budget_tokens, HID, generator=g)
    times = []
    for rep in range(4):
        t0 = time.perf_counter()
        R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, x, gy, MODE, GROUP)
        dt = time.perf_counter() - t0
        if rep:
            times.append(dt)
    times.sort()
    med = times[len(times) // 2]
    return {"value": budget_tokens / med, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{budget_tokens} tokens of C2 (H={HID}, D={INTER}), fp32, int8 g{GROUP}, "
                      f"full-FT fwd+bwd; oracle FlashFFNv3Function on CPU, median of 3",
            "median_s": med}


def library_arm(x, gy, wg, wu, wd, steps, warmup, frozen=False):
    """The same C2 step in the reference's structure (src/flashffn.py:1409-1587)
    with every GEMM through torch.matmul (hipBLASLt on ROCm) and the codec as the
    standalone K1 / K2 kernels of this build: what the reference's composition
    of library GEMMs and separate codec kernels gives on this GPU.  `frozen`
    drops the weight gradients and K2's h_mid^ (only grad_x is needed).
    Returns ms per step (HIP events around `steps` steps, mean)."""
    import torch
    from compact_amd import kernels as K

    def lib_step():
        hg = x @ wg.t()
        hu = x @ wu.t()
        h_mid, cg, sg, cu, su = K.silu_mul_quant(hg, hu, BITS, GROUP)
        del hg, hu
        y = h_mid @ wd.t()
        del h_mid, y
        ghm = gy @ wd
        dg, du, hmh = K.dequant_swiglu_backward(ghm, cg, sg, cu, su, BITS, GROUP,
                                                want_h_mid=not frozen)
        del ghm
        gx = dg @ wg
        gx = gx + du @ wu
        if frozen:
            return (gx,)
        gwd = gy.t() @ hmh
        gwg = dg.t() @ x
        gwu = du.t() @ x
        return gx, gwg, gwu, gwd

    with torch.no_grad():
        for _ in range(warmup):
            lib_step()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            lib_step()
        e1.record(stream)
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` at `workload`, measured with
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE over `bench.py --probe` and
    calibrated by the probe's copy kernel.  Read from the committed profile
    summaries (a line `traffic_bytes_per_launch <kernel> <workload> <bytes>`);
    None if no summary covers the pair."""
    pdir = os.path.join(ROOT, "profiles")
    if not os.path.isdir(pdir):
        return None
    for fn in sorted(os.listdir(pdir)):
        if not fn.endswith(".md"):
            continue
        for line in open(os.path.join(pdir, fn)):
            parts = line.strip().strip("`").split()
            if len(parts) == 4 and parts[0] == "traffic_bytes_per_launch" \
                    and parts[1] == kernel and parts[2] == workload:
                return float(parts[3])
    return None


def model_step_bench(args):
    """Whole-model training step (BASELINE configs C4 / C5): tokens/s of the
    step (forward, backward, AdamW) with every MLP on FlashFFN v3, the per-step
    saved-for-backward bytes of the MLPs, and the dominant FFN kernel's
    roofline.  Random-initialised weights, uniform-random token IDs."""
    import torch
    import compact_amd as cpt
    from compact_amd import e2e
    from compact_amd.kernels import KernelTimer

    cfg = e2e.CONFIGS[args.workload]
    dev = torch.device("cuda:0")
    model, opt = e2e.prepare(cfg, dev, flash=True)
    ids = e2e.random_batch(cfg, dev)
    n_tok = cfg["batch"] * cfg["seq"]

    # saved-for-backward bytes of the MLPs only: count while inside an MLP forward
    mlps = [layer.mlp for layer in model.model.layers]
    inside = [False]
    seen, total = set(), [0]
    exclude = {p.data_ptr() for p in model.parameters()}

    def pack(t):
        if inside[0]:
            key = (t.data_ptr(), t.nbytes)
            if t.data_ptr() not in exclude and key not in seen:
                seen.add(key)
                total[0] += t.nbytes
        return t
    hooks = []
    for m in mlps:
        hooks.append(m.register_forward_pre_hook(lambda mod, a: inside.__setitem__(0, True)))
        hooks.append(m.register_forward_hook(lambda mod, a, o: inside.__setitem__(0, False)))
    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t), e2e.fused_attention_only():
        loss = model(input_ids=ids, labels=ids).loss
    del loss
    for h in hooks:
        h.remove()
    ffn_saved = total[0]

    for _ in range(args.warmup):
        e2e.train_step(model, opt, ids)
    torch.cuda.synchronize()
    cpt.v3_reset_counters()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with KernelTimer() as kt:
        e0.record(stream)
        for _ in range(args.steps):
            loss = e2e.train_step(model, opt, ids)
        e1.record(stream)
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    assert cpt._V3_COUNTERS["forward"] == args.steps * cfg["layers"], cpt._V3_COUNTERS
    kern = kt.avg_ms()
    h, d = cfg["hidden"], cfg["inter"]
    global GROUP, BITS
    GROUP, BITS = cfg["group"], 4 if cfg["cache_mode"] == "int4" else 8
    work = algorithmic_work(n_tok, h, d)
    work["gemm_fwd_gate"] = work["gemm_fwd_up"] = work["gemm_dgrad_down"] = \
        (2 * n_tok * h * d, "mfma")
    dom_name = max((k for k in kern if k in work), key=lambda k: kern[k]["total_ms"])
    amount, bound = work[dom_name]
    rate = amount / (kern[dom_name]["avg_ms"] * 1e-3)
    roofline = {"kernel": dom_name, "bound": "mfma", "achieved": rate / 1e12,
                "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": rate / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                "traffic": measured_traffic(dom_name, args.workload),
                "algorithmic_flops": amount}
    if bound == "hbm":
        roofline.update(bound="hbm", achieved=rate / 1e9, peak=HBM_PEAK_GBS, unit="GB/s",
                        frac=rate / 1e9 / HBM_PEAK_GBS)
    out = {
        "metric": "whole-model training step tokens/sec (every MLP on FlashFFN v3), 1 MI355X",
        "value": n_tok / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights, uniform-random token IDs, seed 0)",
        "config": {"workload": cfg["desc"], "tokens": n_tok, "layers": cfg["layers"],
                   "d_model": h, "d_ff": d, "cache_mode": cfg["cache_mode"],
                   "group_size": cfg["group"], "outlier_ratio": cfg["outlier_ratio"],
                   "parallelism": "none (1 GPU)"},
        "loss": float(loss),
        "ffn_saved_activation_mb": ffn_saved / 1e6,
        "ffn_saved_activation_mb_per_layer": ffn_saved / 1e6 / cfg["layers"],
        "roofline": roofline,
        "kernels": kern,
    }
    print(json.dumps(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=N_TOK)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=512)
    ap.add_argument("--no-library-arm", action="store_true",
                    help="skip timing the hipBLASLt composition of the same step")
    ap.add_argument("--workload", choices=sorted(WORKLOADS) + ["c4", "c5"], default="c2",
                    help="c2 (default) / c3: the FFN block; c4 / c5: a whole-model training "
                         "step (TinyLlama full-FT / Llama-7B LoRA) with every MLP on FlashFFN v3")
    ap.add_argument("--probe", action="store_true",
                    help="HBM-counter probe (run under rocprofv3 --pmc): a 1 GiB calibration "
                         "copy, then --steps untimed steps; prints one status line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not a code path)"}))
        sys.exit(2)
    if args.workload in ("c4", "c5"):
        model_step_bench(args)
        return
    wl = WORKLOADS[args.workload]
    global GROUP, BITS, MODE
    GROUP, BITS, MODE = wl["group"], wl["bits"], wl["mode"]

    import torch
    import compact_amd as cpt
    from compact_amd.kernels import KernelTimer

    dev = torch.device("cuda:0")
    n, h, d = args.tokens, HID, INTER
    batch = 8 if n % 8 == 0 else 1          # 8 sequences of 1024 tokens at the default size
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(n, h, device=dev, generator=g).to(torch.bfloat16)
    gy = torch.randn(n, h, device=dev, generator=g).to(torch.bfloat16)
    frozen = wl.get("frozen", False)
    full_ft = wl["lora_rank"] == 0 and not frozen
    wg = (torch.randn(d, h, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(d, h, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(h, d, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    x.requires_grad_()
    lora = {}
    scale = 0.0
    if full_ft:
        params = tuple(w.requires_grad_() for w in (wg, wu, wd))
    elif frozen:
        params = ()
    else:
        # LoRA r16, alpha 32: A ~ kaiming-uniform(a=sqrt(5)) (bound 1/sqrt(in)), B ~ N(0, 0.01)
        r = wl["lora_rank"]
        scale = 32.0 / r
        for key, d_in, d_out in (("gate", h, d), ("up", h, d), ("down", d, h)):
            bound = 1.0 / d_in ** 0.5
            lora["a_" + key] = ((torch.rand(r, d_in, device=dev, generator=g) * 2 - 1) * bound
                                ).to(torch.bfloat16).requires_grad_()
            lora["b_" + key] = (torch.randn(d_out, r, device=dev, generator=g) * 0.01
                                ).to(torch.bfloat16).requires_grad_()
        params = tuple(lora.values())

    def fwd():
        # [batch, seq, H] as a LlamaMLP receives it: the first sequence ranks
        # the C3 outlier channels (HyC-LoRA's x_[0] statistics)
        return cpt.FlashFFNv3Function.apply(
            x.view(batch, n // batch, h), wg, lora.get("a_gate"), lora.get("b_gate"),
            wu, lora.get("a_up"), lora.get("b_up"), wd, lora.get("a_down"), lora.get("b_down"),
            scale, scale, scale, MODE, GROUP, True, wl["outlier_ratio"])

    def step():
        for p in params + (x,):
            p.grad = None
        y = fwd()
        y.backward(gy.view_as(y))

    if args.probe:
        # calibration: torch's copy kernel reads and writes exactly PROBE_COPY_BYTES
        src = torch.ones(PROBE_COPY_BYTES // 2, device=dev, dtype=torch.bfloat16)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        del src, dst
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        print(json.dumps({"probe": args.workload, "steps": args.steps,
                          "copy_bytes": PROBE_COPY_BYTES}))
        return

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    cpt.v3_reset_counters()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with KernelTimer() as kt:
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(args.steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
    total_ms = e0.elapsed_time(e1)
    ms = total_ms / args.steps
    assert cpt._V3_COUNTERS["triton_quant_fwd"] == args.steps, "fused codec (K1) did not run"
    assert cpt._V3_COUNTERS["triton_dequant_bwd"] == args.steps, "fused dequant (K2) did not run"
    kern = kt.avg_ms()

    # parameters (trainable or frozen) and x are excluded, x counted once
    # (src/verify_flashffn_v3.py:523-543,594-597)
    all_params = set(params) | {wg, wu, wd}
    sb = saved_bytes(fwd, {p.data_ptr() for p in all_params} | {x.data_ptr()}) + x.nbytes

    algo = algorithmic_work(n, h, d)
    algo["gemm_fwd_gate"] = algo["gemm_fwd_up"] = algo["gemm_dgrad_down"] = (2 * n * h * d, "mfma")
    kernels = {}
    for name, st in kern.items():
        entry = dict(st)
        if name in algo:
            amount, bound = algo[name]
            rate = amount / (st["avg_ms"] * 1e-3)
            if bound == "hbm":
                entry["gbs"] = rate / 1e9
                entry["frac_hbm"] = entry["gbs"] / HBM_PEAK_GBS
            else:
                entry["tflops"] = rate / 1e12
                entry["frac_mfma_bf16"] = entry["tflops"] / MFMA_BF16_PEAK_TFLOPS
        kernels[name] = entry
    # dominant HIP kernel of this build by total time in the timed steps
    dom = max((k for k in kern if k in algo), key=lambda k: kern[k]["total_ms"])
    amount, bound = algo[dom]
    rate = amount / (kern[dom]["avg_ms"] * 1e-3)
    if bound == "hbm":
        roofline = {"kernel": dom, "bound": "hbm", "achieved": rate / 1e9, "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": rate / 1e9 / HBM_PEAK_GBS,
                    "traffic": measured_traffic(dom, args.workload),
                    "algorithmic_bytes": amount}
    else:
        roofline = {"kernel": dom, "bound": "mfma", "achieved": rate / 1e12,
                    "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": rate / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                    "traffic": measured_traffic(dom, args.workload),
                    "algorithmic_flops": amount}
    flops = gemm_flops_fwd_bwd(n, h, d, full_ft)
    if wl["lora_rank"]:   # thin adapter GEMMs: 18 * N * r * (H + D)
        flops += 18 * n * wl["lora_rank"] * (h + d)
    out = {
        "metric": "FFN fwd+bwd tokens/sec + saved-activation MB, Llama-7B FFN shape, 1 MI355X",
        "value": n / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seed 0, X~N(0,1), W~N(0,0.02))",
        "config": {"workload": wl["desc"], "tokens": n, "batch": batch, "seq_len": n // batch,
                   "d_model": h, "d_ff": d,
                   "cache_mode": MODE, "group_size": GROUP, "lora_rank": wl["lora_rank"],
                   "outlier_ratio": wl["outlier_ratio"], "frozen_base": not full_ft,
                   "parallelism": "none (1 GPU)"},
        "saved_activation_mb": sb / 1e6,
        "step_tflops": flops / (ms * 1e-3) / 1e12,
        "step_frac_mfma_bf16": flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "roofline": roofline,
        "kernels": kernels,
    }
    if (full_ft or frozen) and not args.no_library_arm:
        lib_ms = library_arm(x.detach(), gy, wg.detach(), wu.detach(), wd.detach(),
                             args.steps, args.warmup, frozen)
        out["library_arm"] = {
            "ms_per_step": lib_ms, "tokens_per_s": n / (lib_ms * 1e-3),
            "speedup_of_this_build": lib_ms / ms,
            "what": "same step in the reference's structure: GEMMs through torch.matmul "
                    "(hipBLASLt), K1/K2 codec as standalone kernels, same inputs and box"}
    if not args.no_cpu_baseline and args.workload == "c2":
        out["cpu_baseline"] = cpu_baseline(args.cpu_tokens)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
