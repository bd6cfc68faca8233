"""End-to-end training steps with every MLP on FlashFFN v3 (BASELINE configs
C4 and C5): a random-initialised LLaMA built from its config (no checkpoint),
the MLPs patched by `apply_flash_ffn_v3`, uniform-random token IDs as input
and labels, causal-LM loss, AdamW.  Everything outside the MLPs (embedding,
RMSNorm, attention, LM head, optimizer) is stock PyTorch / transformers.

Attention is pinned to SDPA's fused flash / memory-efficient kernels: its
math fallback would issue batched bf16 products with transposed operands.
"""

from __future__ import annotations

import contextlib

import torch

from .model_patch import apply_flash_ffn_v3, inject_lora

# BASELINE.json configs[3] and configs[4]
CONFIGS = {
    "c4": dict(layers=22, hidden=2048, inter=5632, heads=32, kv_heads=4, vocab=32000,
               batch=8, seq=1024, lora=None, cache_mode="int8", group=128, outlier_ratio=0.0,
               desc="C4: TinyLlama-1.1B full fine-tune step (22 layers, d_model 2048, d_ff 5632, "
                    "32/4 heads, vocab 32000), 8x1024 tokens, AdamW, every MLP FlashFFN int8 g128"),
    "c5": dict(layers=32, hidden=4096, inter=11008, heads=32, kv_heads=32, vocab=32000,
               batch=4, seq=2048, lora=("q_proj", "v_proj", "gate_proj", "up_proj", "down_proj"),
               lora_r=16, lora_alpha=32.0, cache_mode="int4", group=64, outlier_ratio=0.01,
               desc="C5: Llama-7B LoRA step (32 layers, d_model 4096, d_ff 11008, vocab 32000), "
                    "frozen bf16 base, LoRA r16 on q/v/gate/up/down, 4x2048 tokens, AdamW, every "
                    "MLP FlashFFN int4 g64 + 1% outlier channels"),
}


@contextlib.contextmanager
def fused_attention_only():
    from torch.nn.attention import SDPBackend, sdpa_kernel
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        yield


def build_llama(cfg: dict, device, dtype=torch.bfloat16, seed: int = 0):
    """Random-initialised LlamaForCausalLM of `cfg` on `device` in `dtype`."""
    from transformers import LlamaConfig, LlamaForCausalLM
    lc = LlamaConfig(hidden_size=cfg["hidden"], intermediate_size=cfg["inter"],
                     num_hidden_layers=cfg["layers"], num_attention_heads=cfg["heads"],
                     num_key_value_heads=cfg["kv_heads"], vocab_size=cfg["vocab"],
                     max_position_embeddings=max(2048, cfg["seq"]), attn_implementation="sdpa")
    torch.manual_seed(seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        with torch.device(device):
            model = LlamaForCausalLM(lc)
    finally:
        torch.set_default_dtype(prev)
    return model


def prepare(cfg: dict, device, flash: bool = True, seed: int = 0):
    """(model, optimizer): LoRA injected when cfg asks for it, MLPs patched
    when `flash`."""
    model = build_llama(cfg, device, seed=seed)
    if cfg.get("lora"):
        inject_lora(model, cfg["lora"], cfg["lora_r"], cfg["lora_alpha"], b_std=0.01)
    if flash:
        n = apply_flash_ffn_v3(model, cfg["cache_mode"], cfg["group"],
                               outlier_ratio=cfg["outlier_ratio"])
        assert n == cfg["layers"], f"patched {n} of {cfg['layers']} MLPs"
    model.train()
    params = [p for p in model.parameters() if p.requires_grad]
    opt = torch.optim.AdamW(params, lr=1e-5, foreach=True)
    return model, opt


def random_batch(cfg: dict, device, seed: int = 0):
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randint(0, cfg["vocab"], (cfg["batch"], cfg["seq"]), device=device, generator=g)


def train_step(model, opt, ids) -> torch.Tensor:
    """One causal-LM step: forward, loss, backward, AdamW.  Returns the loss."""
    with fused_attention_only():
        out = model(input_ids=ids, labels=ids)
        out.loss.backward()
    opt.step()
    opt.zero_grad(set_to_none=True)
    return out.loss.detach()
