"""The reference's V5 end-to-end gate on MI355X, on synthetic text
(src/verify_flashffn_v3.py:780-882).

    python -m compact_amd.bench_v5 [--steps 30] [--json out.json]

The gate: TinyLlama-1.1B with PEFT LoRA r8 / alpha 16 on gate/up/down (B
zero-initialised, adapters in bf16), batch 8 x 512 tokens, AdamW lr 5e-4,
30 steps; arms baseline / v3_int4 / v3_recompute, each from the same seed
(:786-812).  It passes when each v3 arm's 30-step loss sum is within 2% of
the baseline's and its peak memory is lower (:855-866).

Here the model is random-initialised from TinyLlama's config (no checkpoint
on the box) and the text is synthetic (no wikitext): sequences from a seeded
sparse bigram chain, each token followed by one of 4 successors, so the loss
has 1.39 nats of entropy to fall towards from ln(32000) and the arms'
trajectories can be compared.  The MLPs are patched with `make_v3_forward`
through `apply_flash_ffn_v3`, as the gate patches every LlamaMLP (:803-810).
"""

from __future__ import annotations

import argparse
import gc
import json
import statistics
import time

import numpy as np
import torch

from . import e2e
from .kernels import _V3_COUNTERS, v3_reset_counters
from .model_patch import apply_flash_ffn_v3, inject_lora

CFG = dict(layers=22, hidden=2048, inter=5632, heads=32, kv_heads=4, vocab=32000, batch=8,
           seq=512)
RANK, ALPHA, LR = 8, 16.0, 5e-4


def bigram_batches(n_steps: int, batch: int, seq: int, vocab: int, succ: int = 4,
                   seed: int = 0):
    """n_steps batches [batch, seq] of a sparse bigram chain: token t is
    followed by one of `succ` fixed random successors, uniformly."""
    rng = np.random.default_rng(seed)
    table = rng.integers(0, vocab, size=(vocab, succ))
    out = []
    for _ in range(n_steps):
        ids = np.empty((batch, seq), np.int64)
        ids[:, 0] = rng.integers(0, vocab, size=batch)
        pick = rng.integers(0, succ, size=(batch, seq))
        for p in range(1, seq):
            ids[:, p] = table[ids[:, p - 1], pick[:, p]]
        out.append(torch.from_numpy(ids))
    return out


def run_arm(arm: str, batches, device, seed: int = 0, lr: float = LR):
    torch.manual_seed(seed)
    model = e2e.build_llama(CFG, device, seed=seed)
    model.config.use_cache = False
    inject_lora(model, ("gate_proj", "up_proj", "down_proj"), RANK, ALPHA)   # B = 0 (PEFT)
    n_patched = 0
    if arm != "baseline":
        n_patched = apply_flash_ffn_v3(model, "int4" if arm == "v3_int4" else "recompute", 64)
        assert n_patched == CFG["layers"], n_patched
    model.train()
    opt = torch.optim.AdamW([p for p in model.parameters() if p.requires_grad], lr=lr,
                            foreach=True)
    v3_reset_counters()
    gc.collect()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    losses, times = [], []
    for ids in batches:
        ids = ids.to(device)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        loss = e2e.train_step(model, opt, ids)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        losses.append(float(loss))
    peak = torch.cuda.max_memory_allocated()
    counters = dict(_V3_COUNTERS)
    if arm == "baseline":
        assert counters["forward"] == 0, "v3 ran in the baseline arm"
    else:
        want = n_patched * len(batches)
        assert counters["forward"] == want and counters["backward"] == want, counters
    del model, opt
    gc.collect()
    torch.cuda.empty_cache()
    return {"losses": losses, "loss_sum": sum(losses), "peak_mem_mib": peak / 2 ** 20,
            "median_step_s": statistics.median(times), "n_patched": n_patched}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--lr", type=float, default=LR,
                    help="the gate's 5e-4 barely moves a random-initialised model in 30 steps; "
                         "a larger rate gives the arms a trajectory to agree on")
    ap.add_argument("--json", default=None)
    args = ap.parse_args()
    device = torch.device("cuda:0")
    batches = bigram_batches(args.steps, CFG["batch"], CFG["seq"], CFG["vocab"], seed=args.seed)
    res = {}
    for arm in ("baseline", "v3_int4", "v3_recompute"):
        r = res[arm] = run_arm(arm, batches, device, args.seed, args.lr)
        print(f"{arm:13s} loss first/last {r['losses'][0]:.4f} / {r['losses'][-1]:.4f}, "
              f"sum {r['loss_sum']:.4f} | peak {r['peak_mem_mib']:.0f} MiB | "
              f"{r['median_step_s'] * 1e3:.1f} ms/step", flush=True)
    base = res["baseline"]
    checks = {}
    for arm in ("v3_int4", "v3_recompute"):
        r = res[arm]
        rel = abs(r["loss_sum"] - base["loss_sum"]) / base["loss_sum"]
        ok = rel < 0.02 and r["peak_mem_mib"] < base["peak_mem_mib"]
        checks[arm] = {"loss_sum_rel_diff": rel,
                       "peak_mem_savings": 1 - r["peak_mem_mib"] / base["peak_mem_mib"],
                       "pass": ok}
        print(f"{arm}: loss-sum difference {rel * 100:.3f}% (< 2%), peak memory saving "
              f"{checks[arm]['peak_mem_savings'] * 100:.1f}% -> {'PASS' if ok else 'FAIL'}",
              flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump({"config": dict(CFG, lora_r=RANK, lora_alpha=ALPHA, lr=args.lr,
                                      steps=args.steps),
                       "arms": res, "checks": checks}, f, indent=1)


if __name__ == "__main__":
    main()
