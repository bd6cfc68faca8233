"""PEFT-shaped LoRA wrapper and a LLaMA-style MLP for tests (peft is not
installed here).  `_v3_proj_kind` / `_v3_extract_proj` are duck-typed on this
structure (reference src/flashffn.py:1605-1634,1798-1821): base_layer,
lora_A / lora_B ModuleDicts of nn.Linear, scaling dict, lora_dropout, and
active_adapters."""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F


class LoraLinear(nn.Module):
    def __init__(self, base: nn.Linear, r: int, alpha: float, name: str = "default",
                 b_std: float = 0.01, dropout: float = 0.0):
        super().__init__()
        self.base_layer = base
        self.lora_A = nn.ModuleDict({name: nn.Linear(base.in_features, r, bias=False)})
        self.lora_B = nn.ModuleDict({name: nn.Linear(r, base.out_features, bias=False)})
        self.lora_dropout = nn.ModuleDict({name: nn.Dropout(dropout) if dropout else nn.Identity()})
        self.scaling = {name: alpha / r}
        self.active_adapters = [name]
        nn.init.kaiming_uniform_(self.lora_A[name].weight, a=math.sqrt(5))
        nn.init.normal_(self.lora_B[name].weight, std=b_std)
        base.weight.requires_grad_(False)

    def get_base_layer(self):
        return self.base_layer

    def forward(self, x):
        n = self.active_adapters[0]
        return self.base_layer(x) + self.scaling[n] * self.lora_B[n](self.lora_A[n](x))


class SwiGLUMLP(nn.Module):
    """LLaMA MLP: down(silu(gate(x)) * up(x))."""

    def __init__(self, hidden: int, inter: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden, inter, bias=False)
        self.up_proj = nn.Linear(hidden, inter, bias=False)
        self.down_proj = nn.Linear(inter, hidden, bias=False)
        for lin in (self.gate_proj, self.up_proj, self.down_proj):
            nn.init.normal_(lin.weight, std=0.02)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


def lora_wrap(mlp: SwiGLUMLP, r: int = 16, alpha: float = 32.0, which=("gate", "up", "down")):
    for key in which:
        name = f"{key}_proj"
        setattr(mlp, name, LoraLinear(getattr(mlp, name), r, alpha))
    return mlp
