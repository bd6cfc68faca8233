"""Model-level patch (reference src/train_glue.py:810-876) on CPU: which MLPs
are patched, which wrappers are refused, and the PEFT-shaped LoRA injection.
The patched forward itself runs on the GPU (tests/test_gpu_model.py)."""

import pytest
import torch
import torch.nn as nn

from compact_amd import model_patch as MP
from tests.peft_like import SwiGLUMLP, adapter_wrap


def tiny_llama(layers=2):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(hidden_size=64, intermediate_size=192, num_hidden_layers=layers,
                      num_attention_heads=4, num_key_value_heads=2, vocab_size=128,
                      max_position_embeddings=64)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg)


def test_apply_patches_every_mlp():
    model = tiny_llama(3)
    assert MP.apply_flash_ffn_v3(model, "int8", 64) == 3
    for layer in model.model.layers:
        # the instance attribute shadows the class forward
        assert "forward" in layer.mlp.__dict__


def test_lora_injection_and_patch():
    model = tiny_llama(2)
    n = MP.inject_lora(model, ("q_proj", "v_proj", "gate_proj", "up_proj", "down_proj"), 8, 16.0)
    assert n == 2 * 5
    trainable = {k for k, p in model.named_parameters() if p.requires_grad}
    assert trainable and all("lora_" in k for k in trainable)
    assert MP.apply_flash_ffn_v3(model, "int4", 64, outlier_ratio=0.01) == 2
    from compact_amd import _v3_proj_kind
    assert _v3_proj_kind(model.model.layers[0].mlp.gate_proj) == "lora"


def test_adapter_families_patch():
    mlp = adapter_wrap(SwiGLUMLP(64, 192), "dora", 8, 16.0, which=("gate",))
    holder = nn.Module()
    holder.mlp = mlp
    assert MP.apply_flash_ffn_v3(holder, "int4") == 1


def test_unknown_wrapper_raises_value_error():
    mlp = SwiGLUMLP(64, 192)

    class Weird(nn.Module):
        def __init__(self):
            super().__init__()
            self.base_layer = nn.Linear(64, 192)

    mlp.up_proj = Weird()
    holder = nn.Module()
    holder.mlp = mlp
    with pytest.raises(ValueError):
        MP.apply_flash_ffn_v3(holder, "int8")


def test_bamboo_mlp_refused():
    mlp = SwiGLUMLP(64, 192)
    mlp.predictor = nn.Module()
    mlp.predictor.fc1 = nn.Linear(64, 8)
    mlp.predictor.fc2 = nn.Linear(8, 192)
    holder = nn.Module()
    holder.mlp = mlp
    with pytest.raises(ValueError):
        MP.apply_flash_ffn_v3(holder, "int8")


def test_mfma_layout_rule():
    """The engine takes 16-byte aligned rows: contiguous extent and row stride
    multiples of 8, the other extent free; degenerate rank-1 columns and
    ragged contiguous extents go elsewhere."""
    import torch
    from compact_amd.flashffn import _mfma
    bf = torch.bfloat16
    assert _mfma(torch.zeros(7, 256, dtype=bf))              # any token count
    assert _mfma(torch.zeros(7, 256, dtype=bf).t())          # transposed activation
    assert _mfma(torch.zeros(1, 256, dtype=bf))
    assert not _mfma(torch.zeros(256, 1, dtype=bf))          # a rank-1 factor
    assert not _mfma(torch.zeros(256, 4, dtype=bf))
    assert not _mfma(torch.zeros(256, 12, dtype=bf)[:, :8])  # rows 12 elements apart
    assert not _mfma(torch.zeros(8, 8, dtype=torch.float32))
    assert _mfma(torch.zeros(16, 768, dtype=bf)[:4])         # a row slice of a weight
    assert not _mfma(torch.zeros(4, 264, dtype=bf)[:, 1:257])  # rows 2 bytes off 16-byte alignment


def test_lora_fusable_rule():
    """Adapter ranks up to 16 ride in every GEMM epilogue; 17 to 32 only where
    every summed product runs on the 16x16x32 loop (k a positive multiple of
    64, n of 8); above 32 none."""
    from compact_amd import gemm as G
    from compact_amd.flashffn import _lora_ok
    for r in range(1, 17):
        assert G.lora_fusable(r, (136, 12))                  # the engine's shapes too
    assert not G.lora_fusable(0, (128, 64))
    for r in (17, 24, 30, 32):
        assert G.lora_fusable(r, (128, 264))
        assert G.lora_fusable(r, (4096, 11008), (11008, 4096))
        assert not G.lora_fusable(r, (136, 264))             # k not a multiple of 64
        assert not G.lora_fusable(r, (128, 260))             # n not a multiple of 8
        assert not G.lora_fusable(r, (128, 264), (136, 264))  # one product on the engine
        assert not G.lora_fusable(r, (0, 264))
        assert not G.lora_fusable(r)                         # no shapes given
    assert not G.lora_fusable(33, (128, 264))
    assert not G.lora_fusable(64, (4096, 11008))
    bf = torch.bfloat16
    a24, b24 = torch.zeros(24, 256, dtype=bf), torch.zeros(768, 24, dtype=bf)
    assert _lora_ok((a24, b24), dims=((256, 768), (768, 256)))
    assert not _lora_ok((a24, b24), dims=((264, 768),))
    a16 = torch.zeros(16, 256, dtype=bf)
    assert not _lora_ok((a16, torch.zeros(768, 16, dtype=bf)), (a24, b24), dims=((256, 768),))
    assert _lora_ok((None, None), dims=((136, 12),))
