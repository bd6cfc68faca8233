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


# ---------------------------------------------------------------------------
# the other adapter families, structured as the wrappers the reference
# classifies (src/flashffn.py:1798-1821) and extracts (:1850-1921)
# ---------------------------------------------------------------------------

class _Magnitude(nn.Module):
    """PEFT's DoraLinearLayer keeps the magnitude as `.weight` [out]."""

    def __init__(self, m: torch.Tensor):
        super().__init__()
        self.weight = nn.Parameter(m)


class DoraLinear(LoraLinear):
    """PEFT lora.Linear with use_dora=True: out = c * (x W^T + s (x A^T) B^T),
    c = m / ||W + s B A||_2 (row norm, detached)."""

    def __init__(self, base: nn.Linear, r: int, alpha: float, name: str = "default",
                 b_std: float = 0.02, m_jitter: float = 0.2):
        super().__init__(base, r, alpha, name, b_std)
        with torch.no_grad():
            m = self._norm(name) * (1.0 + m_jitter * torch.randn(base.out_features))
        self.lora_magnitude_vector = nn.ModuleDict({name: _Magnitude(m)})

    def _norm(self, name):
        w = self.base_layer.weight.float()
        ba = self.lora_B[name].weight.float() @ self.lora_A[name].weight.float()
        return (w + self.scaling[name] * ba).norm(p=2, dim=1).detach()

    def forward(self, x):
        n = self.active_adapters[0]
        raw = self.base_layer(x) + self.scaling[n] * self.lora_B[n](self.lora_A[n](x))
        c = self.lora_magnitude_vector[n].weight / self._norm(n).to(x.dtype)
        return raw * c


class AdaLoraLinear(nn.Module):
    """PEFT AdaLoRA SVDLinear: out = x W^T + (x (A*E)^T) B^T * s / (ranknum + 1e-5)."""

    def __init__(self, base: nn.Linear, r: int, alpha: float, name: str = "default",
                 b_std: float = 0.02, e_std: float = 0.5):
        super().__init__()
        self.base_layer = base
        self.lora_A = nn.ParameterDict({name: nn.Parameter(torch.randn(r, base.in_features) * 0.02)})
        self.lora_B = nn.ParameterDict({name: nn.Parameter(torch.randn(base.out_features, r) * b_std)})
        self.lora_E = nn.ParameterDict({name: nn.Parameter(torch.randn(r, 1) * e_std)})
        self.ranknum = nn.ParameterDict({name: nn.Parameter(torch.tensor(float(r)),
                                                            requires_grad=False)})
        self.scaling = {name: float(alpha)}
        self.lora_dropout = nn.ModuleDict({name: nn.Identity()})
        self.active_adapters = [name]
        base.weight.requires_grad_(False)

    def get_base_layer(self):
        return self.base_layer

    def forward(self, x):
        n = self.active_adapters[0]
        a_eff = self.lora_A[n] * self.lora_E[n]
        return self.base_layer(x) + (x @ a_eff.t() @ self.lora_B[n].t()) * self.scaling[n] / (
            self.ranknum[n] + 1e-5)


class VeraLinear(nn.Module):
    """PEFT VeRA Linear: out = x W^T + lambda_b * ((x A^T) * lambda_d) B^T with
    frozen shared A [r, max_in], B [max_out, r] sliced to this layer."""

    def __init__(self, base: nn.Linear, vera_a: torch.Tensor, vera_b: torch.Tensor,
                 name: str = "default", d_initial: float = 0.1):
        super().__init__()
        r = vera_a.shape[0]
        self.base_layer = base
        self.in_features, self.out_features = base.in_features, base.out_features
        self.vera_A = {name: vera_a}
        self.vera_B = {name: vera_b}
        self.vera_lambda_d = nn.ParameterDict(
            {name: nn.Parameter(d_initial + 0.05 * torch.randn(r))})
        self.vera_lambda_b = nn.ParameterDict(
            {name: nn.Parameter(0.05 * torch.randn(base.out_features))})
        self.vera_dropout = nn.ModuleDict({name: nn.Identity()})
        self.active_adapters = [name]
        base.weight.requires_grad_(False)

    def get_base_layer(self):
        return self.base_layer

    def _apply(self, fn, *args, **kwargs):
        super()._apply(fn, *args, **kwargs)
        for d in (self.vera_A, self.vera_B):
            for k in d:
                d[k] = fn(d[k])
        return self

    def forward(self, x):
        n = self.active_adapters[0]
        a = self.vera_A[n][:, : self.in_features]
        b = self.vera_B[n][: self.out_features, :]
        u = F.linear(x, a) * self.vera_lambda_d[n]
        return self.base_layer(x) + F.linear(u, b) * self.vera_lambda_b[n]


class DyLoRALinear(nn.Module):
    """DyLoRA (reference src/dylora.py): rank b ~ U{1..r} per training
    forward from Python's `random`, r in eval; s = alpha / r."""

    def __init__(self, base: nn.Linear, r: int, alpha: float, b_std: float = 0.02):
        super().__init__()
        self.base_layer = base
        self.r = r
        self.scaling = alpha / r
        self.lora_A = nn.Parameter(torch.empty(r, base.in_features))
        nn.init.kaiming_uniform_(self.lora_A, a=math.sqrt(5))
        self.lora_B = nn.Parameter(torch.randn(base.out_features, r) * b_std)
        self.dropout = nn.Identity()
        base.weight.requires_grad_(False)

    def forward(self, x):
        import random
        b = random.randint(1, self.r) if self.training else self.r
        return self.base_layer(x) + self.scaling * F.linear(F.linear(x, self.lora_A[:b, :]),
                                                            self.lora_B[:, :b])


def adapter_wrap(mlp: SwiGLUMLP, kind: str, r: int = 8, alpha: float = 16.0,
                 which=("gate", "up", "down")):
    """Wrap the chosen projections of `mlp` with one adapter family."""
    if kind == "vera":
        h, d = mlp.gate_proj.in_features, mlp.gate_proj.out_features
        big = max(h, d)
        vera_a = torch.empty(r, big)
        vera_b = torch.empty(big, r)
        nn.init.kaiming_uniform_(vera_a, a=math.sqrt(5))
        nn.init.kaiming_uniform_(vera_b, a=math.sqrt(5))
    for key in which:
        name = f"{key}_proj"
        base = getattr(mlp, name)
        if kind == "lora":
            wrapped = LoraLinear(base, r, alpha, b_std=0.02)
        elif kind == "dora":
            wrapped = DoraLinear(base, r, alpha)
        elif kind == "adalora":
            wrapped = AdaLoraLinear(base, r, alpha)
        elif kind == "vera":
            wrapped = VeraLinear(base, vera_a, vera_b)
        elif kind == "dylora":
            wrapped = DyLoRALinear(base, r, alpha)
        else:
            raise ValueError(kind)
        setattr(mlp, name, wrapped)
    return mlp
