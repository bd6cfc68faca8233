"""Model-level patch: every SwiGLU MLP of a model runs FlashFFN v3.

`apply_flash_ffn_v3` mirrors the reference's `apply_flash_ffn_v3`
(src/train_glue.py:810-876): it walks the module tree, finds modules exposing
gate_proj / up_proj / down_proj, checks how each projection is wrapped
(plain nn.Linear, PEFT-shaped LoRA, DoRA, AdaLoRA, VeRA, DyLoRA) and replaces
the module's forward with `make_v3_forward`.  Unsupported wrappers raise
ValueError, dReLU/Bamboo MLPs raise ValueError: there is no silent fallback.

`LoraLinear` / `inject_lora` give a model PEFT's lora.Linear structure
(base_layer, lora_A / lora_B ModuleDicts, scaling, lora_dropout,
active_adapters), which is all the v3 path reads; PEFT itself is not a
dependency.
"""

from __future__ import annotations

import logging
import math

import torch.nn as nn

from .flashffn import _v3_proj_kind, make_v3_forward

logger = logging.getLogger(__name__)

_KIND_NAMES = {"dora": "DoRA", "adalora": "AdaLoRA", "dylora": "DyLoRA", "vera": "VeRA",
               "lora": "PEFT LoRA", "plain": "plain Linear"}


def _is_bamboo_mlp(module: nn.Module) -> bool:
    """TurboSparse / Bamboo dReLU MLP: gate/up/down plus a `predictor` sub-MLP
    with fc1 / fc2 (src/train_glue.py:610-620)."""
    return (hasattr(module, "gate_proj") and hasattr(module, "up_proj")
            and hasattr(module, "down_proj") and hasattr(module, "predictor")
            and hasattr(module.predictor, "fc1") and hasattr(module.predictor, "fc2"))


def apply_flash_ffn_v3(model: nn.Module, cache_mode: str, group_size: int = 64,
                       use_triton: bool = True, outlier_ratio: float = 0.0) -> int:
    """Patch every SwiGLU MLP of `model` with FlashFFN v3; returns how many.

    cache_mode: 'int4' | 'int8' | 'bf16' | 'recompute'.  outlier_ratio > 0
    keeps that fraction of h_gate / h_up channels in bf16 (int4/int8 caches,
    plain or LoRA projections only)."""
    converted = 0
    for name, module in model.named_modules():
        if not (hasattr(module, "gate_proj") and hasattr(module, "up_proj")
                and hasattr(module, "down_proj")):
            continue
        if _is_bamboo_mlp(module):
            raise ValueError(
                f"FlashFFN v3 does not support the dReLU/Bamboo (TurboSparse) architecture "
                f"(found at '{name}').")
        modes = []
        for proj_name in ("gate_proj", "up_proj", "down_proj"):
            proj = getattr(module, proj_name)
            kind = _v3_proj_kind(proj)
            if kind == "unknown":
                raise ValueError(
                    f"FlashFFN v3 does not support this wrapper ({type(proj).__name__}) on MLP "
                    f"projections (found at '{name}.{proj_name}'). Supported: PEFT LoRA, DoRA, "
                    f"AdaLoRA, DyLoRA, VeRA, plain nn.Linear (frozen or full-FT).")
            modes.append(_KIND_NAMES[kind])
        module.forward = make_v3_forward(module, cache_mode=cache_mode, group_size=group_size,
                                         use_triton=use_triton, outlier_ratio=outlier_ratio)
        logger.info("FlashFFN v3 applied (%s, cache_mode=%s) to: %s",
                    "/".join(sorted(set(modes))), cache_mode, name)
        converted += 1
    return converted


class LoraLinear(nn.Module):
    """PEFT lora.Linear's structure around an existing nn.Linear: the base
    weight is frozen; out = base(x) + scaling * B(A(x)), A kaiming-uniform
    (a = sqrt(5)) and B zero-initialised as PEFT does (pass b_std > 0 for a
    non-degenerate B)."""

    def __init__(self, base: nn.Linear, r: int, alpha: float, name: str = "default",
                 b_std: float = 0.0):
        super().__init__()
        self.base_layer = base
        dev, dt = base.weight.device, base.weight.dtype
        self.lora_A = nn.ModuleDict({name: nn.Linear(base.in_features, r, bias=False,
                                                     device=dev, dtype=dt)})
        self.lora_B = nn.ModuleDict({name: nn.Linear(r, base.out_features, bias=False,
                                                     device=dev, dtype=dt)})
        self.lora_dropout = nn.ModuleDict({name: nn.Identity()})
        self.scaling = {name: alpha / r}
        self.active_adapters = [name]
        nn.init.kaiming_uniform_(self.lora_A[name].weight, a=math.sqrt(5))
        if b_std > 0:
            nn.init.normal_(self.lora_B[name].weight, std=b_std)
        else:
            nn.init.zeros_(self.lora_B[name].weight)
        for p in base.parameters():
            p.requires_grad_(False)

    @property
    def in_features(self):
        return self.base_layer.in_features

    @property
    def out_features(self):
        return self.base_layer.out_features

    def get_base_layer(self):
        return self.base_layer

    def forward(self, x):
        n = self.active_adapters[0]
        return self.base_layer(x) + self.scaling[n] * self.lora_B[n](self.lora_A[n](x))


def inject_lora(model: nn.Module, target_modules, r: int, alpha: float,
                b_std: float = 0.0) -> int:
    """Freeze `model` and wrap every nn.Linear whose attribute name is in
    `target_modules` (e.g. q_proj, v_proj, gate_proj) with LoraLinear.
    Returns the number of wrapped layers."""
    for p in model.parameters():
        p.requires_grad_(False)
    targets = set(target_modules)
    wrapped = 0
    for parent in list(model.modules()):
        for attr, child in list(parent.named_children()):
            if attr in targets and isinstance(child, nn.Linear):
                setattr(parent, attr, LoraLinear(child, r, alpha, b_std=b_std))
                wrapped += 1
    return wrapped
