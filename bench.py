"""Benchmark: FlashFFN v3 SwiGLU FFN fwd+bwd tokens/s + saved-activation MB on
one MI355X (BASELINE.json metric), workload C2: Llama-7B FFN dims
d_model=4096, d_ff=11008, 8x1024 tokens, bf16, int8 per-group(128) GLU cache,
full fine-tune (dense weight grads), synthetic seeded inputs.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Prints ONE JSON line.  A step is one forward + backward of the FFN block on
the same resident inputs.  The headline (`value`, `ms_per_step` = the mean
over the K timed steps, plus their median / p10 / p90 from one HIP event
pair per step) is timed with no per-kernel events.  A second pass over K
more steps records HIP events around every kernel on its launch stream:
`kernels` lists them and `roofline` is the dominant HIP kernel's rate from
that pass, with `frac` against the 2.5 PF/s spec peak and
`frac_of_achievable` against `achievable_peak`, the register-only MFMA rate
(cpt_probe_mfma_rate) timed in the same run.  The same line carries C3 (LoRA r16, int4 g64 + 1% outlier
channels) under "c3", timed the same way, and the whole-model training
steps C4 (TinyLlama-1.1B full fine-tune) and C5 (Llama-7B LoRA) under "c4"
and "c5" (HIP events around each step, no per-kernel events; --no-e2e skips
them).  `cpu_baseline` times the CPU
oracle (the restatement of the reference's FlashFFNv3Function; the reference
itself cannot run on a CPU) on a bounded sample of C2, and config C1 (the
reference's own CPU case) at full size under "c1_full".
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HID, INTER, N_TOK = 4096, 11008, 8 * 1024
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


def algorithmic_work(n, h, d, bits, group):
    """Per-launch algorithmic work of every timed kernel: (amount, bound),
    FLOPs for the MFMA-bound GEMMs (2*M*N*K per product), bytes for the
    HBM-bound standalone codec kernels."""
    k1_bytes, k2_bytes = codec_bytes(n, d, bits, group)
    gemm = 2 * n * h * d
    return {
        "ffn_gate_up": (2 * gemm, "mfma"),          # x @ [Wg; Wu]^T (+ GLU + codec)
        "gemm_fwd_down": (gemm, "mfma"),            # h_mid @ Wd^T
        "gemm_fwd_gate": (gemm, "mfma"),
        "gemm_fwd_up": (gemm, "mfma"),
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


def cpu_model() -> str:
    """The host CPU's model name as lscpu prints it ('Model name'), with the
    family / model / stepping numbers from /proc/cpuinfo, which identify the
    part where a virtualised host shortens the name."""
    name = ""
    try:
        r = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10)
        for line in r.stdout.splitlines():
            if line.strip().lower().startswith("model name"):
                name = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" in line:
                    k, v = (t.strip() for t in line.split(":", 1))
                    info.setdefault(k.lower(), v)
                elif info:
                    break
    except OSError:
        pass
    name = name or info.get("model name", "unknown")
    ids = [f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info]
    return f"{name} ({', '.join(ids)})" if ids else name


def usable_cores() -> tuple:
    """(cores to use, os.cpu_count(), how it was bounded): os.cpu_count()
    bounded by this process's CPU affinity and its cgroup CPU quota, so the
    baseline's threads are the host cores it may actually run on."""
    n = os.cpu_count() or 1
    use, why = n, "os.cpu_count()"
    try:
        aff = len(os.sched_getaffinity(0))
        if aff < use:
            use, why = aff, "CPU affinity"
    except (AttributeError, OSError):
        pass
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            q = max(1, int(int(quota) // int(period)))
            if q < use:
                use, why = q, "cgroup CPU quota"
    except (OSError, ValueError):
        pass
    return use, n, why


def _oracle_median(ps, x, gy, mode, group, reps=3):
    """1 warmup + `reps` timed fwd+bwd of the CPU oracle Function: median s."""
    from oracle import flashffn_ref as R
    times = []
    for rep in range(reps + 1):
        t0 = time.perf_counter()
        R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, x, gy, mode, group)
        if rep:
            times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def cpu_baseline(c2_tokens=2048):
    """The CPU oracle's FlashFFNv3Function (the reference's algorithm restated;
    the reference itself cannot run on a CPU) on every host core this process
    may run on: torch.set_num_threads(os.cpu_count()), bounded by the CPU
    affinity and cgroup quota (usable_cores):
      value   C2's shape (H 4096, D 11008, int8 g128, full-FT) on a bounded
              sample of `c2_tokens` tokens, in fp32 (CPU bf16 GEMM support
              varies by host);
      c1_full config C1 exactly: fp32, 4 x 512 tokens, H 2048, D 5632, int8
              g128, full-FT, seed 0.
    1 warmup + 3 timed reps each, median; tokens/s = tokens / median."""
    import torch
    from oracle import flashffn_ref as R
    cores, n_cpu, bound = usable_cores()
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(cores)
    out = {}
    for key, (n, h, d) in (("c2", (c2_tokens, HID, INTER)), ("c1", (2048, 2048, 5632))):
        ps = R.synthetic_param_set("fullft", h, d, 0, 0.0, seed=0, dtype=torch.float32)
        g = torch.Generator().manual_seed(0)
        x = torch.randn(n, h, generator=g)
        gy = torch.randn(n, h, generator=g)
        out[key] = (n, _oracle_median(ps, x, gy, "int8", 128))
    (n2, t2), (n1, t1) = out["c2"], out["c1"]
    torch.set_num_threads(prev_threads)
    return {"value": n2 / t2, "unit": "tokens/s", "cores": cores, "os_cpu_count": n_cpu,
            "cores_bounded_by": bound, "kind": "port", "cpu": cpu_model(),
            "sample": f"{n2} tokens of C2 (H={HID}, D={INTER}), fp32, int8 g128, full-FT "
                      "fwd+bwd; oracle FlashFFNv3Function on CPU, median of 3",
            "median_s": t2,
            "c1_full": {"value": n1 / t1, "unit": "tokens/s", "median_s": t1,
                        "sample": "config C1 at full size: fp32, 4x512 tokens, d_model 2048, "
                                  "d_ff 5632, int8 g128, full-FT fwd+bwd, seed 0"}}


def library_arm(x, gy, wg, wu, wd, steps, warmup, bits, group, frozen=False):
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
        h_mid, cg, sg, cu, su = K.silu_mul_quant(hg, hu, bits, group)
        del hg, hu
        y = h_mid @ wd.t()
        del h_mid, y
        ghm = gy @ wd
        dg, du, hmh = K.dequant_swiglu_backward(ghm, cg, sg, cu, su, bits, group,
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


def timed_steps(step, steps):
    """`steps` calls of step() bracketed by synchronize, one HIP event pair
    per step on the current stream.  Returns (total_ms, sorted per-step ms)."""
    import torch
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for a, b in ev:
        a.record(stream)
        step()
        b.record(stream)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1), sorted(a.elapsed_time(b) for a, b in ev)


def _pct(sorted_ms, q):
    return sorted_ms[min(len(sorted_ms) - 1, int(q * (len(sorted_ms) - 1) + 0.5))]


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


def model_step_summary(workload: str, steps: int, warmup: int) -> dict:
    """Tokens/s of a whole-model training step (C4 / C5), timed with HIP
    events around `steps` steps after `warmup` untimed ones, no per-kernel
    events inside: ms per step (mean of the timed region and median of the
    per-step events), the last loss.  For the default line's extra keys."""
    import gc
    import torch
    import compact_amd as cpt
    from compact_amd import e2e

    cfg = e2e.CONFIGS[workload]
    dev = torch.device("cuda:0")
    model, opt = e2e.prepare(cfg, dev, flash=True)
    ids = e2e.random_batch(cfg, dev)
    n_tok = cfg["batch"] * cfg["seq"]
    for _ in range(warmup):
        e2e.train_step(model, opt, ids)
    torch.cuda.synchronize()
    cpt.v3_reset_counters()
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record(stream)
    for i in range(steps):
        loss = e2e.train_step(model, opt, ids)
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    per = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
    ms = ev[0].elapsed_time(ev[steps]) / steps
    assert cpt._V3_COUNTERS["forward"] == steps * cfg["layers"], cpt._V3_COUNTERS
    out = {"workload": cfg["desc"], "tokens_per_s": n_tok / (ms * 1e-3), "ms_per_step": ms,
           "ms_per_step_median": per[len(per) // 2], "steps": steps, "warmup": warmup,
           "tokens": n_tok, "layers": cfg["layers"], "loss": float(loss)}
    del model, opt, ids, loss
    gc.collect()
    torch.cuda.empty_cache()
    return out


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
    work = algorithmic_work(n_tok, h, d, 4 if cfg["cache_mode"] == "int4" else 8, cfg["group"])
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


def ffn_case(name, n, dev):
    """Seeded C2 / C3 inputs on the device and the Function step over them."""
    import torch
    import compact_amd as cpt
    wl = WORKLOADS[name]
    h, d = HID, INTER
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
            scale, scale, scale, wl["mode"], wl["group"], True, wl["outlier_ratio"])

    def step():
        for p in params + (x,):
            p.grad = None
        y = fwd()
        y.backward(gy.view_as(y))

    return dict(wl=wl, n=n, batch=batch, x=x, gy=gy, wg=wg, wu=wu, wd=wd, params=params,
                fwd=fwd, step=step, full_ft=full_ft, frozen=frozen)


_ACHIEVABLE = {}


def achievable_mfma_peak(launches: int = 200) -> dict:
    """The bf16 MFMA rate this part sustains with nothing else running, for
    the instruction the FFN's GEMMs issue: cpt_probe_mfma_rate with
    v_mfma_f32_16x16x32_bf16 back to back on register operands (no memory
    traffic), timed over `launches` back-to-back launches of about 1 ms.
    Measured once per process; the spec peak (2.5 PF/s) assumes a clock this
    part does not hold under MFMA load."""
    if "v" in _ACHIEVABLE:
        return _ACHIEVABLE["v"]
    import torch
    from compact_amd import _lib
    from compact_amd._lib import check
    # shape 1: 16x16x32, 768 blocks (three per CU) x 2730 iterations x 64 MFMAs
    shape, blocks, iters, per = 1, 768, 2730, 16384
    out = torch.empty(blocks * 4, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    lib = _lib.lib()

    def launch():
        check(lib.cpt_probe_mfma_rate(shape, blocks, iters, 0.5, out.data_ptr(), stream.cuda_stream),
              "probe_mfma_rate")
    for _ in range(20):
        launch()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(launches):
        launch()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / launches
    flops = blocks * iters * 64 * per
    _ACHIEVABLE["v"] = {"value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s",
                        "source": "cpt_probe_mfma_rate: v_mfma_f32_16x16x32_bf16 (the instruction "
                                  "the FFN's GEMMs issue) back to back on register operands, no "
                                  "memory traffic, timed in this run"}
    return _ACHIEVABLE["v"]


def run_ffn(name, n, steps, warmup, dev, library=True):
    """Headline, per-kernel pass and saved bytes of one FFN workload."""
    import torch
    import compact_amd as cpt
    from compact_amd.kernels import KernelTimer
    c = ffn_case(name, n, dev)
    wl, h, d = c["wl"], HID, INTER
    for _ in range(warmup):
        c["step"]()
    torch.cuda.synchronize()
    cpt.v3_reset_counters()
    total_ms, per_step = timed_steps(c["step"], steps)
    ms = total_ms / steps
    assert cpt._V3_COUNTERS["triton_quant_fwd"] == steps, "the fused codec (K1) did not run"
    assert cpt._V3_COUNTERS["triton_dequant_bwd"] == steps, "the fused dequant (K2) did not run"

    # per-kernel pass: HIP events on each kernel's launch stream, separate steps
    with KernelTimer() as kt:
        timed_steps(c["step"], steps)
    kern = kt.avg_ms()

    # parameters (trainable or frozen) and x are excluded, x counted once
    # (src/verify_flashffn_v3.py:523-543,594-597)
    x = c["x"]
    all_params = set(c["params"]) | {c["wg"], c["wu"], c["wd"]}
    sb = saved_bytes(c["fwd"], {p.data_ptr() for p in all_params} | {x.data_ptr()}) + x.nbytes

    algo = algorithmic_work(n, h, d, wl["bits"], wl["group"])
    kernels = {}
    for kname, st in kern.items():
        entry = dict(st)
        if kname in algo:
            amount, bound = algo[kname]
            rate = amount / (st["avg_ms"] * 1e-3)
            if bound == "hbm":
                entry["gbs"] = rate / 1e9
                entry["frac_hbm"] = entry["gbs"] / HBM_PEAK_GBS
            else:
                entry["tflops"] = rate / 1e12
                entry["frac_mfma_bf16"] = entry["tflops"] / MFMA_BF16_PEAK_TFLOPS
        kernels[kname] = entry
    # dominant HIP kernel of this build by total time in the per-kernel pass
    dom = max((k for k in kern if k in algo), key=lambda k: kern[k]["total_ms"])
    amount, bound = algo[dom]
    rate = amount / (kern[dom]["avg_ms"] * 1e-3)
    traffic = measured_traffic(dom, name)
    if bound == "hbm":
        roofline = {"kernel": dom, "bound": "hbm", "achieved": rate / 1e9, "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": rate / 1e9 / HBM_PEAK_GBS, "traffic": traffic,
                    "algorithmic_bytes": amount}
    else:
        roofline = {"kernel": dom, "bound": "mfma", "achieved": rate / 1e12,
                    "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": rate / 1e12 / MFMA_BF16_PEAK_TFLOPS, "traffic": traffic,
                    "algorithmic_flops": amount}
    roofline["timing"] = "mean of the per-kernel pass's HIP events on the launch stream"
    roofline["traffic_source"] = ("profiles/ rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE summary of "
                                  "bench.py --probe" if traffic is not None else None)
    if bound != "hbm":
        ach = achievable_mfma_peak()
        roofline["achievable_peak"] = ach
        roofline["frac_of_achievable"] = rate / 1e12 / ach["value"]
    flops = gemm_flops_fwd_bwd(n, h, d, c["full_ft"])
    if wl["lora_rank"]:   # thin adapter GEMMs: 18 * N * r * (H + D)
        flops += 18 * n * wl["lora_rank"] * (h + d)
    res = {
        "value": n / (ms * 1e-3), "ms_per_step": ms,
        "ms_per_step_median": _pct(per_step, 0.5), "ms_per_step_p10": _pct(per_step, 0.1),
        "ms_per_step_p90": _pct(per_step, 0.9),
        "config": {"workload": wl["desc"], "tokens": n, "batch": c["batch"],
                   "seq_len": n // c["batch"], "d_model": h, "d_ff": d,
                   "cache_mode": wl["mode"], "group_size": wl["group"],
                   "lora_rank": wl["lora_rank"], "outlier_ratio": wl["outlier_ratio"],
                   "frozen_base": not c["full_ft"], "parallelism": "none (1 GPU)"},
        "saved_activation_mb": sb / 1e6,
        "step_tflops": flops / (ms * 1e-3) / 1e12,
        "step_frac_mfma_bf16": flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "roofline": roofline,
        "kernels": kernels,
    }
    if library and (c["full_ft"] or c["frozen"]):
        lib_ms = library_arm(x.detach(), c["gy"], c["wg"].detach(), c["wu"].detach(),
                             c["wd"].detach(), steps, warmup, wl["bits"], wl["group"],
                             c["frozen"])
        res["library_arm"] = {
            "ms_per_step": lib_ms, "tokens_per_s": n / (lib_ms * 1e-3),
            "speedup_of_this_build": lib_ms / ms,
            "what": "same step in the reference's structure: GEMMs through torch.matmul "
                    "(hipBLASLt), K1/K2 codec as standalone kernels, same inputs and box"}
    return res, c


def probe(name, n, steps, dev):
    """HBM-counter probe (run under rocprofv3 --pmc): a 1 GiB calibration copy,
    then `steps` untimed steps; prints one status line."""
    import torch
    c = ffn_case(name, n, dev)
    # calibration: torch's copy kernel reads and writes exactly PROBE_COPY_BYTES
    src = torch.ones(PROBE_COPY_BYTES // 2, device=dev, dtype=torch.bfloat16)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    del src, dst
    for _ in range(steps):
        c["step"]()
    torch.cuda.synchronize()
    print(json.dumps({"probe": name, "steps": steps, "copy_bytes": PROBE_COPY_BYTES}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=N_TOK)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=2048)
    ap.add_argument("--no-library-arm", action="store_true",
                    help="skip timing the hipBLASLt composition of the same step")
    ap.add_argument("--no-c3", action="store_true",
                    help="skip the C3 workload that the default C2 line carries under 'c3'")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the C4 and C5 whole-model steps that the default C2 line "
                         "carries under 'c4' and 'c5'")
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

    import torch
    dev = torch.device("cuda:0")
    if args.probe:
        probe(args.workload, args.tokens, args.steps, dev)
        return
    res, case = run_ffn(args.workload, args.tokens, args.steps, args.warmup, dev,
                        library=not args.no_library_arm)
    del case
    out = {
        "metric": "FFN fwd+bwd tokens/sec + saved-activation MB, Llama-7B FFN shape, 1 MI355X",
        "value": res.pop("value"), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": res.pop("ms_per_step"), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seed 0, X~N(0,1), W~N(0,0.02))",
    }
    out.update(res)
    if args.workload == "c2" and not args.no_c3:
        torch.cuda.empty_cache()
        c3, case = run_ffn("c3", args.tokens, args.steps, args.warmup, dev, library=False)
        del case
        c3.pop("kernels")
        out["c3"] = {"tokens_per_s": c3.pop("value"), **c3}
    if args.workload == "c2" and not args.no_e2e:
        # whole-model steps, fewer steps than the FFN (each is 0.1-0.4 s); a
        # failure here is recorded and does not cost the headline line
        for wl, (w, k) in (("c4", (3, 10)), ("c5", (2, 5))):
            print(f"bench: {wl} whole-model step", file=sys.stderr, flush=True)
            try:
                out[wl] = model_step_summary(wl, k, w)
            except Exception as e:  # noqa: BLE001 - reported in the line itself
                out[wl] = {"error": f"{type(e).__name__}: {e}"}
                torch.cuda.empty_cache()
    if not args.no_cpu_baseline and args.workload == "c2":
        out["cpu_baseline"] = cpu_baseline(args.cpu_tokens)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
