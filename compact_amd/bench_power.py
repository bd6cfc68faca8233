"""Board power and shader clock while each C2 GEMM runs back to back.

    python -m compact_amd.bench_power [--secs 3]

Runs every GEMM of a C2 fwd+bwd step (8192 tokens, d_model 4096, d_ff 11008,
bf16) on this build's dispatch (the 16x16x32 loop at these shapes), on the
32x32x16 engine where one plain product can be forced onto it, and through
torch's `@` (hipBLASLt), each in a loop for --secs seconds, while a thread reads the GPU's metrics table through
amdsmi (read-only queries: socket power, current gfx clock) every 10 ms.
The first two lines are the register-only MFMA probe (v_mfma_f32_32x32x16_bf16,
then v_mfma_f32_16x16x32_bf16, on every SIMD, no memory traffic): the MFMA
rate the power cap allows when nothing else draws power.  Prints, per product: time per launch, TFLOP/s, mean power (W) and clock (MHz)
over the loop (the first 0.8 s dropped), TFLOP/s per GHz (work per clock) and
energy per FLOP (pJ).  The board's power cap is printed first.
"""

from __future__ import annotations

import argparse
import threading
import time

import torch

from . import _lib
from . import gemm as G
from ._lib import check


class PowerSampler:
    """Samples (time, socket power W, gfx clock MHz) in a background thread."""

    def __init__(self, period: float = 0.01):
        import amdsmi  # the ROCm SMI library's Python binding; queries only
        self._smi = amdsmi
        amdsmi.amdsmi_init()
        self._h = amdsmi.amdsmi_get_processor_handles()[0]
        self.period = period
        self.samples: list[tuple[float, float, float]] = []
        self._stop = False
        self._th = threading.Thread(target=self._run, daemon=True)

    def power_cap_w(self) -> float:
        return self._smi.amdsmi_get_power_cap_info(self._h)["power_cap"] / 1e6

    def _run(self):
        while not self._stop:
            m = self._smi.amdsmi_get_gpu_metrics_info(self._h)
            p, c = m.get("current_socket_power"), m.get("current_gfxclk")
            if isinstance(p, (int, float)) and isinstance(c, (int, float)):
                self.samples.append((time.time(), float(p), float(c)))
            time.sleep(self.period)

    def start(self):
        self._th.start()
        return self

    def stop(self):
        self._stop = True
        self._th.join()

    def mean(self, t0: float, t1: float) -> tuple[float, float]:
        s = [(p, c) for (t, p, c) in self.samples if t0 <= t <= t1]
        if not s:
            return float("nan"), float("nan")
        return sum(p for p, _ in s) / len(s), sum(c for _, c in s) / len(s)


def sustained(fn, secs: float, sampler: PowerSampler | None):
    """ms per call over a back-to-back loop of about `secs`, and the mean
    power / clock over it (ramp-up second dropped)."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.time()
    n = 0
    e0.record()
    while time.time() - t0 < secs:
        for _ in range(5):
            fn()
        n += 5
        torch.cuda.synchronize()
    e1.record()
    torch.cuda.synchronize()
    t1 = time.time()
    ms = e0.elapsed_time(e1) / n
    pw, ck = sampler.mean(t0 + 0.8, t1) if sampler else (float("nan"), float("nan"))
    return ms, pw, ck


def mfma_probe(shape: int):
    """One launch of the register-only MFMA probe (no memory traffic) with
    shape 0 (32x32x16: 512 registers a lane, one block of 4 waves per CU,
    256 blocks) or 1 (16x16x32: 132 registers, three blocks per CU, 768
    blocks); about 1 ms each.  Returns (callable, FLOPs per launch)."""
    blocks, iters, per = (256, 4096, 32768) if shape == 0 else (768, 2730, 16384)
    out = torch.empty(blocks * 4, dtype=torch.float32, device="cuda")
    lib = _lib.lib()

    def run():
        check(lib.cpt_probe_mfma_rate(shape, blocks, iters, 0.5, out.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream), "probe_mfma_rate")
    return run, blocks * iters * 64 * per


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--secs", type=float, default=3.0)
    args = ap.parse_args()
    n, h, d = 8192, 4096, 11008
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(n, h, device=dev, generator=g).bfloat16()
    gy = torch.randn(n, h, device=dev, generator=g).bfloat16()
    wg = (torch.randn(d, h, device=dev, generator=g) * .02).bfloat16()
    wu = (torch.randn(d, h, device=dev, generator=g) * .02).bfloat16()
    wd = (torch.randn(h, d, device=dev, generator=g) * .02).bfloat16()
    hm = torch.randn(n, d, device=dev, generator=g).bfloat16()
    fl = 2 * n * h * d
    try:
        sampler = PowerSampler().start()
        print(f"power cap {sampler.power_cap_w():.0f} W", flush=True)
    except Exception as e:   # no amdsmi on this machine: times only
        sampler = None
        print(f"no power readings ({e})", flush=True)
    idle0 = time.time()
    time.sleep(2.0)
    if sampler:
        pw, ck = sampler.mean(idle0 + 0.5, time.time())
        print(f"{'idle':40s} {'':>9s} {'':>12s} {pw:7.0f} W {ck:6.0f} MHz", flush=True)
    p32, p32_fl = mfma_probe(0)
    p16, p16_fl = mfma_probe(1)
    # arms: this build's dispatch (the 16x16x32 loop at these shapes), the
    # 32x32x16 engine for the single-pair products (gemm.mm_engine), hipBLASLt
    cases = [
        ("MFMA 32x32x16 only, registers", p32, None, None, p32_fl),
        ("MFMA 16x16x32 only, registers", p16, None, None, p16_fl),
        ("NT x.Wg^T, K 4096", lambda: G.linear(x, wg), lambda: G.mm_engine(x, wg.t()),
         lambda: x @ wg.t(), fl),
        ("NT h_mid.Wd^T, K 11008", lambda: G.linear(hm, wd), lambda: G.mm_engine(hm, wd.t()),
         lambda: hm @ wd.t(), fl),
        ("NN gy.Wd, K 4096", lambda: G.mm(gy, wd), lambda: G.mm_engine(gy, wd), lambda: gy @ wd, fl),
        ("NN dg.Wg + du.Wu, K 2 x 11008", lambda: G.mm2(hm, wg, hm, wu), None,
         lambda: hm @ wg + hm @ wu, 2 * fl),
        ("TN gy^T.h_mid, K 8192", lambda: G.mm(gy.t(), hm), lambda: G.mm_engine(gy.t(), hm),
         lambda: gy.t() @ hm, fl),
        ("F1 gate/up + GLU + int8 codec", lambda: G.ffn_gate_up(x, wg, wu, 8, 128), None, None, 2 * fl),
    ]
    for name, mine, eng, lib, flops in cases:
        for arm, fn in (("build", mine), ("engine", eng), ("hipBLASLt", lib)):
            if fn is None:
                continue
            ms, pw, ck = sustained(fn, args.secs, sampler)
            tf = flops / ms / 1e9
            print(f"{name:30s} {arm:9s} {ms:7.3f} ms {tf:7.1f} TF/s {pw:7.0f} W {ck:6.0f} MHz "
                  f"{tf / ck:6.3f} TF/GHz {pw / tf:6.3f} pJ/FLOP", flush=True)
    if sampler:
        sampler.stop()


if __name__ == "__main__":
    main()
