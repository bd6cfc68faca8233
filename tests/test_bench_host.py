"""Host-side checks of bench.py: the algorithmic work it divides by and the
one-GPU contract.  No GPU is touched.

The expected figures are the closed forms of the hot path's work at the
BASELINE configurations (reference shapes: Llama-7B FFN, d_model 4096,
d_ff 11008, 8192 tokens; codec traffic per src/flashffn.py:1314-1373).
"""

import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

N, H, D = 8192, 4096, 11008


def test_codec_bytes_c2():
    # K1: read g, u (2 x 180.4 MB); write h_mid (180.4 MB), 2 int8 payloads
    # (2 x 90.2 MB), 2 fp16 scale arrays (2 x 1.41 MB) = 724.24 MB.
    # K2: read dh, 2 payloads, 2 scale arrays; write dg, du, h_mid^ = 904.59 MB.
    k1, k2 = bench.codec_bytes(N, D, 8, 128)
    assert k1 == 724_238_336
    assert k2 == 904_593_408
    # term by term: 5 bf16 [N, D] tensors cross HBM in K1, 4 in K2
    e = N * D * 2
    assert k1 == 3 * e + 2 * N * D + 2 * N * (D // 128) * 2
    assert k2 == 4 * e + 2 * N * D + 2 * N * (D // 128) * 2


def test_codec_bytes_c3_int4():
    # int4 g64: payload N x D/2 bytes per tensor, scales N x D/64 fp16
    k1, k2 = bench.codec_bytes(N, D, 4, 64)
    assert k1 == 636_878_848
    assert k2 == 817_233_920
    k1n, k2n = bench.codec_bytes(N, D, 4, 64, want_h_mid=False)
    assert k1n == k1 and k2 - k2n == N * D * 2


def test_gemm_flops():
    # full fine-tune: 3 forward + 6 backward products of 2 N H D each
    assert bench.gemm_flops_fwd_bwd(N, H, D) == 18 * N * H * D == 6_648_609_374_208
    # frozen weights: the 3 weight gradients drop out
    assert bench.gemm_flops_fwd_bwd(N, H, D, full_ft=False) == 4_432_406_249_472


def test_algorithmic_work_bounds():
    w = bench.algorithmic_work(N, H, D, 8, 128)
    gemm = 2 * N * H * D
    assert w["ffn_gate_up"] == (2 * gemm, "mfma")
    assert w["gemm_dgrad_x"] == (2 * gemm, "mfma")
    for k in ("gemm_fwd_down", "gemm_dgrad_down", "gemm_wgrad_down", "gemm_wgrad_gate",
              "gemm_wgrad_up", "ffn_down_dgrad"):
        assert w[k] == (gemm, "mfma")
    assert w["silu_mul_quant"][1] == "hbm" and w["dequant_swiglu_backward"][1] == "hbm"


def test_workloads_table():
    wl = bench.WORKLOADS
    assert set(wl) >= {"c2", "c2f", "c3"}
    assert (wl["c2"]["bits"], wl["c2"]["group"], wl["c2"]["lora_rank"]) == (8, 128, 0)
    assert wl["c2f"].get("frozen") and wl["c2f"]["lora_rank"] == 0
    assert (wl["c3"]["bits"], wl["c3"]["group"], wl["c3"]["lora_rank"]) == (4, 64, 16)
    assert wl["c3"]["outlier_ratio"] == 0.01


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 2
    msg = json.loads(p.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_measured_traffic_reads_profiles():
    # the committed HBM-traffic summary carries the figure bench.py reports;
    # a pair no summary covers gives None
    import re
    text = open(os.path.join(ROOT, "profiles", "ffn_c2_c3_hbm_traffic.md")).read()
    for wl in ("c2", "c3"):
        m = re.search(rf"traffic_bytes_per_launch ffn_gate_up {wl} (\d+)", text)
        assert m, f"no traffic line for {wl}"
        assert bench.measured_traffic("ffn_gate_up", wl) == float(m.group(1))
        # F1 moves at least its algorithmic bytes (x, W_gate, W_up, codes, h_mid)
        assert bench.measured_traffic("ffn_gate_up", wl) > 6e8
    assert bench.measured_traffic("ffn_gate_up", "no_such_workload") is None


def test_v4_harness_model():
    """The V4 speed-gate harness builds the reference gate's MLP: TinyLlama
    dims, LoRA r8 / alpha 16 on gate, up and down with only the adapters
    trainable, and the v2 arm's merged weight W + s B A."""
    import torch
    from compact_amd import bench_v4
    mlp = bench_v4.build_mlp("cpu")
    assert mlp.gate_proj.in_features == 2048 and mlp.gate_proj.out_features == 5632
    trainable = [n for n, p in mlp.named_parameters() if p.requires_grad]
    assert len(trainable) == 6 and all("lora_" in n for n in trainable)
    p = mlp.up_proj
    a, b = p.lora_A["default"].weight.detach(), p.lora_B["default"].weight.detach()
    assert a.shape == (8, 2048) and b.shape == (5632, 8) and p.scaling["default"] == 2.0
    assert float(b.float().std()) > 0.01            # re-drawn N(0, 0.02), not PEFT's zeros
    w = p.get_base_layer().weight
    want = (w.float() + 2.0 * (b.float() @ a.float())).to(torch.bfloat16)
    got = bench_v4.lora_eff_weight(p).detach()
    assert got.dtype == torch.bfloat16
    assert (got.float() - want.float()).abs().max() <= 2 ** -7 * want.float().abs().max()


def test_v5_bigram_batches():
    """The V5 harness's synthetic text: each token is followed by one of 4
    fixed successors, so every observed transition comes from the table."""
    from compact_amd import bench_v5
    bs = bench_v5.bigram_batches(3, 4, 64, 1000, succ=4, seed=1)
    assert len(bs) == 3 and tuple(bs[0].shape) == (4, 64)
    succ = {}
    for b in bs:
        for row in b.tolist():
            for t0, t1 in zip(row, row[1:]):
                succ.setdefault(t0, set()).add(t1)
    assert max(len(v) for v in succ.values()) <= 4
    again = bench_v5.bigram_batches(3, 4, 64, 1000, succ=4, seed=1)
    assert all((x == y).all() for x, y in zip(bs, again))


def test_step_percentiles_and_cpu_model():
    assert bench._pct([1.0, 2.0, 3.0, 4.0, 5.0], 0.5) == 3.0
    assert bench._pct([1.0, 2.0, 3.0, 4.0, 5.0], 0.1) == 1.0
    assert bench._pct([7.0], 0.9) == 7.0
    assert isinstance(bench.cpu_model(), str) and bench.cpu_model()


def test_cpu_baseline_shapes_are_the_configs():
    """The CPU baseline's C1 leg is config C1 exactly (BASELINE.json
    configs[0]): 4 x 512 tokens, d_model 2048, d_ff 5632, int8 g128."""
    import inspect
    src = inspect.getsource(bench.cpu_baseline)
    assert '("c1", (2048, 2048, 5632))' in src and '"int8", 128' in src
