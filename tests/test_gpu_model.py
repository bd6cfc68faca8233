"""Model-level GPU checks (BASELINE configs C4/C5 shape, scaled down): a
random-initialised LLaMA whose MLPs run FlashFFN v3 against the same model
unpatched, on the same weights and tokens.

  * full fine-tune, int8 g128 cache: loss within 1e-2 relative, every
    parameter gradient at cosine >= 0.99 of the unpatched model's (bf16 GEMMs
    and the quantised GLU cache both perturb the gradient);
  * LoRA on q/v/gate/up/down, int4 g64 + 1% outliers: same gates on the LoRA
    gradients (cosine >= 0.98, the reference's int4 adapter gate);
  * a training step runs end to end (AdamW) and the patched MLPs are the ones
    that ran (v3 counters).
"""

import pytest

from compact_amd import e2e
from compact_amd.kernels import _V3_COUNTERS, v3_reset_counters
from oracle import flashffn_ref as R

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, hidden=256, inter=768, heads=4, kv_heads=2, vocab=512, batch=2, seq=128)


def _grads(cfg, device, flash):
    model, _ = e2e.prepare(cfg, device, flash=flash, seed=3)
    ids = e2e.random_batch(cfg, device, seed=4)
    with e2e.fused_attention_only():
        out = model(input_ids=ids, labels=ids)
        out.loss.backward()
    grads = {k: p.grad.detach().float().cpu() for k, p in model.named_parameters()
             if p.requires_grad}
    return out.loss.detach().float().item(), grads


@pytest.mark.parametrize("lora", [False, True])
def test_patched_model_matches_unpatched(device, lora):
    cfg = dict(SMALL)
    if lora:
        cfg.update(lora=("q_proj", "v_proj", "gate_proj", "up_proj", "down_proj"), lora_r=16,
                   lora_alpha=32.0, cache_mode="int4", group=64, outlier_ratio=0.01)
    else:
        cfg.update(lora=None, cache_mode="int8", group=128, outlier_ratio=0.0)
    v3_reset_counters()
    loss_f, g_f = _grads(cfg, device, flash=True)
    assert _V3_COUNTERS["forward"] == cfg["layers"] and _V3_COUNTERS["backward"] == cfg["layers"]
    loss_r, g_r = _grads(cfg, device, flash=False)
    assert abs(loss_f - loss_r) / abs(loss_r) < 1e-2
    assert set(g_f) == set(g_r) and g_f
    floor = 0.98 if lora else 0.99
    for k in g_r:
        if g_r[k].norm() == 0:
            continue
        c = R.tensor_cos(g_f[k], g_r[k])
        assert c >= floor, (k, c)


def test_training_step_runs(device):
    cfg = dict(SMALL, lora=None, cache_mode="int8", group=128, outlier_ratio=0.0)
    model, opt = e2e.prepare(cfg, device, flash=True)
    ids = e2e.random_batch(cfg, device)
    losses = [float(e2e.train_step(model, opt, ids)) for _ in range(3)]
    assert all(l == l and l > 0 for l in losses)
    assert losses[-1] < losses[0]          # same batch: AdamW must make progress
