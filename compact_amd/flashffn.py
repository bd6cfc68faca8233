"""FlashFFN v3 on MI355X: LoRA-factored SwiGLU FFN whose backward cache is the
per-group absmax int4/int8 code of h_gate and h_up.

API kept from the reference (src/flashffn.py:1376-1694):
  FlashFFNv3Function.apply(x, w_gate, a_gate, b_gate, w_up, a_up, b_up,
                           w_down, a_down, b_down, s_gate=0.0, s_up=0.0,
                           s_down=0.0, cache_mode="int4", group_size=64,
                           use_triton=True)
  make_v3_forward(mlp, cache_mode="int4", group_size=64, use_triton=True)
  FlashFFNv3(mlp, cache_mode="int4", group_size=64, use_triton=True)

  out_P = x @ W_P^T + s_P * (x @ A_P^T) @ B_P^T  for P in {gate, up, down}
  h_mid = SiLU(h_gate) * h_up;  y = out_down(h_mid)

cache_mode: 'int4' / 'int8' save x + codes + fp16 scales of h_gate and h_up;
'bf16' saves h_gate and h_up; 'recompute' saves x only.  Adapters also save
the thin [N, r] products xA_g, xA_u, h_mid A_d^T.  `use_triton` keeps the
reference's name and meaning: use the fused device kernels (K1 forward, K2
backward) for int4/int8 bf16 caches; False runs the standalone codec kernels.
Every kernel is a HIP kernel of libcompact_amd.so; there is no CPU path.
"""

from __future__ import annotations

import warnings

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import gemm as G
from . import kernels as K
from .kernels import _V3_COUNTERS


def _bits(mode: str) -> int:
    return 4 if mode == "int4" else 8


_CACHE_CODE = {"int4": _lib.CACHE_INT4, "int8": _lib.CACHE_INT8, "bf16": _lib.CACHE_BF16,
               "recompute": _lib.CACHE_NONE}
_FUSED_GROUPS = (32, 64, 128)


def _mfma(*ts) -> bool:
    """The MFMA engine runs bf16 operands whose dims are multiples of 8."""
    for t in ts:
        if t is None:
            continue
        if t.dtype != torch.bfloat16 or any(d % 8 for d in t.shape):
            return False
    return True


def _mm(a, b, name):
    """a @ b: the MFMA engine for bf16, the library GEMM otherwise."""
    if _mfma(a, b) and a.shape[0] > 0:
        return G.mm(a, b, name)
    return a @ b


def _linear(x, w, name):
    if _mfma(x, w) and x.shape[0] > 0:
        return G.linear(x, w, name)
    return F.linear(x, w)


def _addmm(c, a, b, s, name):
    """c + s * (a @ b) in the reference's bf16 op order (product, scaling and
    sum each rounded): in place on the engine for bf16."""
    if _mfma(c, a, b) and a.shape[0] > 0 and c.stride(1) == 1:
        return G.addmm_(c, a, b, s, name)
    return c + s * (a @ b)


def _mm_scaled(a, b, s, name):
    """s * (a @ b) for the thin adapter gradients, which reduce over all
    tokens: split-K on the engine for bf16."""
    if _mfma(a, b) and a.shape[1] > 0:
        return G.mm_splitk(a, b, s, name=name)
    return s * (a @ b)


def _proj(x_2d, w, a, b, s, name):
    """out = x W^T (+ s * (x A^T) B^T) in PEFT op order (src/flashffn.py:1410-1420).
    Returns (out, xA | None)."""
    h = _linear(x_2d, w, name)
    xa = None
    if a is not None:
        xa = _mm(x_2d, a.t(), name + "_xa")
        h = _addmm(h, xa, b.t(), s, name + "_lora")
    return h, xa


class FlashFFNv3Function(torch.autograd.Function):
    """LoRA-factored SwiGLU FFN with a quantised GLU-cache backward
    (src/flashffn.py:1376-1602).  a_*/b_* may be None (pass s_*=0.0).

    bf16 without gate/up adapters runs the fused MFMA kernels: the forward
    gate/up GEMM carries SiLU*mul and the codec in its epilogue, the backward
    down-projection GEMM carries the dequantisation and the SwiGLU backward.
    Other cases compose the GEMM engine (or the library GEMM for non-bf16
    dtypes) with the standalone elementwise kernels in the reference's order.

    outlier_ratio > 0 (int4/int8 caches, this build's extension for config C3):
    per call, the int(D * ratio) columns of h_gate and of h_up with the largest
    L2 norm are kept in bf16 and left out of the per-group codec (HyC-LoRA's
    zero-and-overwrite semantics, hyclora/operators/compress_function.py:80-174)."""

    @staticmethod
    def forward(ctx, x, w_gate, a_gate, b_gate, w_up, a_up, b_up, w_down, a_down, b_down,
                s_gate=0.0, s_up=0.0, s_down=0.0, cache_mode="int4", group_size=64,
                use_triton=True, outlier_ratio=0.0):
        assert cache_mode in ("int4", "int8", "bf16", "recompute"), cache_mode
        _V3_COUNTERS["forward"] += 1
        K._require_device(x)
        orig_shape = x.shape
        hidden_dim = x.shape[-1]
        x_2d = x.reshape(-1, hidden_dim)
        if not x_2d.is_contiguous():
            x_2d = x_2d.contiguous()
        quant = cache_mode in ("int4", "int8")
        inter = w_gate.shape[0]
        k_out = int(inter * outlier_ratio) if (quant and outlier_ratio > 0) else 0
        assert k_out == 0 or x.dtype == torch.bfloat16, "outlier channels need bf16 activations"
        fusable = (a_gate is None and a_up is None and _mfma(x_2d, w_gate, w_up)
                   and x_2d.shape[0] > 0)

        c_gate = qs_gate = c_up = qs_up = None
        o_gate = o_up = slot_gate = slot_up = None
        h_gate = h_up = None
        xa_g = xa_u = None
        fused_quant = (quant and use_triton and x.dtype == torch.bfloat16)   # :1424-1426
        if fusable and fused_quant and k_out == 0 and group_size in _FUSED_GROUPS:
            # dual GEMM + GLU + codec in one kernel (K1 fused into the epilogue)
            h_mid, _, _, c_gate, qs_gate, c_up, qs_up = G.ffn_gate_up(
                x_2d, w_gate, w_up, _CACHE_CODE[cache_mode], group_size)
            _V3_COUNTERS["triton_quant_fwd"] += 1
        elif fusable and not fused_quant and k_out == 0:
            # h_gate/h_up are needed (bf16 cache, eager codec) or not (recompute)
            keep = cache_mode != "recompute"
            h_mid, h_gate, h_up, *_ = G.ffn_gate_up(
                x_2d, w_gate, w_up, _lib.CACHE_BF16 if keep else _lib.CACHE_NONE, group_size)
        else:
            if fusable:
                _, h_gate, h_up, *_ = G.ffn_gate_up(x_2d, w_gate, w_up, _lib.CACHE_BF16,
                                                    group_size, want_h_mid=False)
            else:
                h_gate, xa_g = _proj(x_2d, w_gate, a_gate, b_gate, s_gate, "gemm_fwd_gate")
                h_up, xa_u = _proj(x_2d, w_up, a_up, b_up, s_up, "gemm_fwd_up")
            if k_out > 0:
                slot_gate, _ = K.outlier_select(h_gate, k_out)
                slot_up, _ = K.outlier_select(h_up, k_out)
            if fused_quant and k_out > 0:
                h_mid, c_gate, qs_gate, o_gate, c_up, qs_up, o_up = K.silu_mul_quant_outlier(
                    h_gate, h_up, _bits(cache_mode), group_size, slot_gate, slot_up, k_out)
                h_gate = h_up = None
            elif fused_quant:
                h_mid, c_gate, qs_gate, c_up, qs_up = K.silu_mul_quant(
                    h_gate, h_up, _bits(cache_mode), group_size)
                h_gate = h_up = None
            else:
                h_mid = K.silu_mul(h_gate, h_up)

        y, ha_d = _proj(h_mid, w_down, a_down, b_down, s_down, "gemm_fwd_down")   # :1435-1439

        if not fused_quant:                                                # :1442-1451
            if quant and k_out > 0:
                c_gate, qs_gate, o_gate = K.v3_quantize_outlier(h_gate, _bits(cache_mode),
                                                                group_size, slot_gate, k_out)
                c_up, qs_up, o_up = K.v3_quantize_outlier(h_up, _bits(cache_mode), group_size,
                                                          slot_up, k_out)
            elif quant:
                c_gate, qs_gate = K.v3_quantize_group_absmax(h_gate, _bits(cache_mode),
                                                             group_size)
                c_up, qs_up = K.v3_quantize_group_absmax(h_up, _bits(cache_mode), group_size)
            elif cache_mode == "bf16":
                c_gate, c_up = h_gate, h_up
        del h_gate, h_up, h_mid

        ctx.save_for_backward(x, w_gate, a_gate, b_gate, w_up, a_up, b_up,
                              w_down, a_down, b_down, xa_g, xa_u, ha_d,
                              c_gate, qs_gate, c_up, qs_up, o_gate, o_up, slot_gate, slot_up)
        ctx.s = (s_gate, s_up, s_down)
        ctx.cache_mode = cache_mode
        ctx.group_size = group_size
        ctx.use_triton = fused_quant
        ctx.orig_shape = orig_shape
        ctx.in_dtype = x.dtype
        if len(orig_shape) == 3:
            y = y.view(orig_shape[0], orig_shape[1], hidden_dim)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        _V3_COUNTERS["backward"] += 1
        (x, w_gate, a_gate, b_gate, w_up, a_up, b_up, w_down, a_down, b_down,
         xa_g, xa_u, ha_d, c_gate, qs_gate, c_up, qs_up, o_gate, o_up, slot_gate,
         slot_up) = ctx.saved_tensors
        s_gate, s_up, s_down = ctx.s
        mode = ctx.cache_mode
        gs = ctx.group_size
        outl = o_gate is not None
        hidden_dim = ctx.orig_shape[-1]
        (need_x, need_wg, need_ag, need_bg, need_wu, need_au, need_bu,
         need_wd, need_ad, need_bd) = ctx.needs_input_grad[:10]
        gy = grad_y.reshape(-1, hidden_dim)
        if not gy.is_contiguous():
            gy = gy.contiguous()
        x_2d = x.reshape(-1, hidden_dim)
        if not x_2d.is_contiguous():
            x_2d = x_2d.contiguous()

        need_gate_path = (need_x or need_wg or need_ag or need_bg
                          or need_wu or need_au or need_bu)               # :1488-1489
        need_h_mid = need_wd or (a_down is not None and need_ad)          # :1490
        need_recon = need_gate_path or need_h_mid
        use_k2 = mode in ("int4", "int8") and ctx.use_triton and need_gate_path
        fusable = (a_down is None and _mfma(gy, w_down) and gy.shape[0] > 0 and not outl)
        fusable_gu = (a_gate is None and a_up is None and _mfma(x_2d, w_gate, w_up)
                      and x_2d.shape[0] > 0)

        hg = hu = None
        if need_recon and not use_k2:                                     # :1500-1516
            if mode == "recompute":
                if fusable_gu:
                    _, hg, hu, *_ = G.ffn_gate_up(x_2d, w_gate, w_up, _lib.CACHE_BF16, gs,
                                                  want_h_mid=False)
                else:
                    hg = _linear(x_2d, w_gate, "gemm_recompute_gate")
                    if a_gate is not None:
                        hg = _addmm(hg, xa_g, b_gate.t(), s_gate, "gemm_recompute_gate_lora")
                    hu = _linear(x_2d, w_up, "gemm_recompute_up")
                    if a_up is not None:
                        hu = _addmm(hu, xa_u, b_up.t(), s_up, "gemm_recompute_up_lora")
            elif mode == "bf16":
                hg, hu = c_gate, c_up
            elif outl:
                hg = K.v3_dequantize_outlier(c_gate, qs_gate, o_gate, slot_gate, _bits(mode), gs)
                hu = K.v3_dequantize_outlier(c_up, qs_up, o_up, slot_up, _bits(mode), gs)
            else:
                hg = K.v3_dequantize_group_absmax(c_gate, qs_gate, _bits(mode), gs, ctx.in_dtype)
                hu = K.v3_dequantize_group_absmax(c_up, qs_up, _bits(mode), gs, ctx.in_dtype)

        grad_w_down = grad_a_down = grad_b_down = None
        gyB_d = None
        if a_down is not None and (need_gate_path or need_ad):
            gyB_d = _mm(gy, b_down, "gemm_gyB_down")                      # :1521

        grad_h_gate = grad_h_up = h_mid_hat = None
        if need_gate_path:
            if use_k2 and fusable and gs in _FUSED_GROUPS:                # :1525-1533
                # dgrad GEMM with dequantise + SwiGLU backward in its epilogue
                grad_h_gate, grad_h_up, h_mid_hat = G.ffn_down_dgrad(
                    gy, w_down, _CACHE_CODE[mode], gs, c_gate, qs_gate, c_up, qs_up,
                    need_h_mid)
                _V3_COUNTERS["triton_dequant_bwd"] += 1
            elif (not use_k2) and fusable and hg is not None and _mfma(hg, hu):
                grad_h_gate, grad_h_up, h_mid_hat = G.ffn_down_dgrad(
                    gy, w_down, _lib.CACHE_BF16, gs, hg, None, hu, None, need_h_mid)
            else:
                grad_h_mid = _mm(gy, w_down, "gemm_dgrad_down")
                if a_down is not None:
                    grad_h_mid = _addmm(grad_h_mid, gyB_d, a_down, s_down, "gemm_dgrad_down_lora")
                if use_k2 and outl:
                    grad_h_gate, grad_h_up, h_mid_hat = K.dequant_swiglu_backward_outlier(
                        grad_h_mid, c_gate, qs_gate, o_gate, slot_gate, c_up, qs_up, o_up,
                        slot_up, _bits(mode), gs, want_h_mid=need_h_mid)
                elif use_k2:
                    grad_h_gate, grad_h_up, h_mid_hat = K.dequant_swiglu_backward(
                        grad_h_mid, c_gate, qs_gate, c_up, qs_up, _bits(mode), gs,
                        want_h_mid=need_h_mid)
                else:
                    grad_h_gate, grad_h_up, h_mid_hat = K.swiglu_backward_glu(
                        grad_h_mid, hg, hu, need_h_mid)
                del grad_h_mid

        if need_h_mid:                                                    # :1536-1543
            if h_mid_hat is None:
                h_mid_hat = K.silu_mul(hg, hu)
            if need_wd:
                grad_w_down = _mm(gy.t(), h_mid_hat, "gemm_wgrad_down")
            if need_ad:
                grad_a_down = _mm_scaled(gyB_d.t(), h_mid_hat, s_down, "gemm_grad_a_down")
            del h_mid_hat
        if need_bd:
            grad_b_down = _mm_scaled(gy.t(), ha_d, s_down, "gemm_grad_b_down")   # :1545

        grad_x = None
        grad_w_gate = grad_a_gate = grad_b_gate = None
        grad_w_up = grad_a_up = grad_b_up = None
        if need_gate_path:                                                # :1551-1587
            ghgB = None
            if a_gate is not None and (need_x or need_ag):
                ghgB = _mm(grad_h_gate, b_gate, "gemm_ghgB")
            ghuB = None
            if a_up is not None and (need_x or need_au):
                ghuB = _mm(grad_h_up, b_up, "gemm_ghuB")
            if need_x:
                if _mfma(grad_h_gate, w_gate, grad_h_up, w_up):
                    # dg @ W_g + du @ W_u as one K-concatenated GEMM
                    grad_x = G.mm2(grad_h_gate, w_gate, grad_h_up, w_up, "gemm_dgrad_x")
                else:
                    grad_x = grad_h_gate @ w_gate + grad_h_up @ w_up
                if a_gate is not None:
                    grad_x = _addmm(grad_x, ghgB, a_gate, s_gate, "gemm_dgrad_x_lora_gate")
                if a_up is not None:
                    grad_x = _addmm(grad_x, ghuB, a_up, s_up, "gemm_dgrad_x_lora_up")
            if need_bg:
                grad_b_gate = _mm_scaled(grad_h_gate.t(), xa_g, s_gate, "gemm_grad_b_gate")
            if need_ag:
                grad_a_gate = _mm_scaled(ghgB.t(), x_2d, s_gate, "gemm_grad_a_gate")
            if need_bu:
                grad_b_up = _mm_scaled(grad_h_up.t(), xa_u, s_up, "gemm_grad_b_up")
            if need_au:
                grad_a_up = _mm_scaled(ghuB.t(), x_2d, s_up, "gemm_grad_a_up")
            if need_wg:
                grad_w_gate = _mm(grad_h_gate.t(), x_2d, "gemm_wgrad_gate")
            if need_wu:
                grad_w_up = _mm(grad_h_up.t(), x_2d, "gemm_wgrad_up")

        # frozen weights => no dense [D_out, D_in] gradient was built (:1589-1593)
        if not (need_wg or need_wu or need_wd):
            assert grad_w_gate is None and grad_w_up is None and grad_w_down is None, \
                "FlashFFNv3 invariant violated: dense weight grad with frozen weights"
        if need_x and len(ctx.orig_shape) == 3:
            grad_x = grad_x.view(ctx.orig_shape)
        return (grad_x, grad_w_gate, grad_a_gate, grad_b_gate,
                grad_w_up, grad_a_up, grad_b_up,
                grad_w_down, grad_a_down, grad_b_down) + (None,) * (len(ctx.needs_input_grad) - 10)


# ---------------------------------------------------------------------------
# module-level API (src/flashffn.py:1605-1694)
# ---------------------------------------------------------------------------

def _is_lora(proj: nn.Module) -> bool:
    return (hasattr(proj, "base_layer")
            and isinstance(getattr(proj, "lora_A", None), nn.ModuleDict)
            and len(proj.lora_A) > 0)


def _v3_extract_proj(proj: nn.Module):
    """(W, A, B, s) from a plain nn.Linear or a PEFT-LoRA-shaped wrapper
    (src/flashffn.py:1605-1634).  Plain: (weight, None, None, 0.0).  Rejects
    DoRA / AdaLoRA / several active adapters; warns that dropout is ignored."""
    if not _is_lora(proj):
        return proj.weight, None, None, 0.0
    if len(getattr(proj, "lora_magnitude_vector", {}) or {}) > 0:
        raise NotImplementedError("FlashFFNv3 fast path does not support DoRA")
    if hasattr(proj, "lora_E"):
        raise NotImplementedError("FlashFFNv3 fast path does not support AdaLoRA")
    assert len(proj.active_adapters) == 1, "exactly one active adapter expected"
    name = proj.active_adapters[0]
    drop = proj.lora_dropout[name]
    p = float(getattr(drop, "p", 0.0))
    if p > 0.0:
        warnings.warn(f"FlashFFNv3 ignores LoRA dropout (p={p}); results differ from PEFT "
                      "forward when training with dropout.")
    w = proj.get_base_layer().weight
    return w, proj.lora_A[name].weight, proj.lora_B[name].weight, float(proj.scaling[name])


def _v3_proj_kind(proj: nn.Module) -> str:
    """Structural (duck-typed) classification of one MLP projection
    (src/flashffn.py:1798-1821): 'dora' | 'adalora' | 'vera' | 'dylora' |
    'lora' | 'plain' | 'unknown'."""
    if hasattr(proj, "base_layer"):
        if len(getattr(proj, "lora_magnitude_vector", None) or {}) > 0:
            return "dora"
        if len(getattr(proj, "lora_E", None) or {}) > 0:
            return "adalora"
        if len(getattr(proj, "vera_lambda_d", None) or {}) > 0:
            return "vera"
        if (isinstance(getattr(proj, "lora_A", None), nn.Parameter)
                and isinstance(getattr(proj, "lora_B", None), nn.Parameter)
                and hasattr(proj, "r") and hasattr(proj, "scaling")):
            return "dylora"
        if isinstance(getattr(proj, "lora_A", None), nn.ModuleDict) and len(proj.lora_A) > 0:
            return "lora"
        return "unknown"
    if hasattr(proj, "weight"):
        return "plain"
    return "unknown"


def make_v3_forward(mlp: nn.Module, cache_mode: str = "int4", group_size: int = 64,
                    use_triton: bool = True, outlier_ratio: float = 0.0):
    """Drop-in replacement for a LLaMA-style MLP forward (src/flashffn.py:1637-1678).
    `mlp` exposes gate_proj / up_proj / down_proj, each a plain nn.Linear or a
    PEFT-LoRA-shaped wrapper; factors are re-extracted on every call and cast
    to x's dtype through autograd.  Unknown wrappers raise NotImplementedError."""
    kinds = tuple(_v3_proj_kind(getattr(mlp, p)) for p in ("gate_proj", "up_proj", "down_proj"))
    if any(k == "unknown" for k in kinds):
        raise NotImplementedError(f"FlashFFNv3: unsupported projection wrapper(s) on MLP: {kinds}")
    if any(k not in ("plain", "lora") for k in kinds):
        raise NotImplementedError(f"FlashFFNv3: adapter kinds {kinds} need the adapter Function")

    def v3_forward(x):
        wg, ag, bg, sg = _v3_extract_proj(mlp.gate_proj)
        wu, au, bu, su = _v3_extract_proj(mlp.up_proj)
        wd, ad, bd, sd = _v3_extract_proj(mlp.down_proj)
        dt = x.dtype

        def cast(t):
            return t if (t is None or t.dtype == dt) else t.to(dt)

        return FlashFFNv3Function.apply(x, cast(wg), cast(ag), cast(bg), cast(wu), cast(au),
                                        cast(bu), cast(wd), cast(ad), cast(bd), sg, su, sd,
                                        cache_mode, group_size, use_triton, outlier_ratio)
    return v3_forward


class FlashFFNv3(nn.Module):
    """Module wrapper around make_v3_forward for an existing MLP (src/flashffn.py:1681-1694)."""

    def __init__(self, mlp: nn.Module, cache_mode: str = "int4", group_size: int = 64,
                 use_triton: bool = True, outlier_ratio: float = 0.0):
        super().__init__()
        self.mlp = mlp
        self.cache_mode = cache_mode
        self.group_size = group_size
        self.use_triton = use_triton
        self.outlier_ratio = outlier_ratio
        self._fwd = make_v3_forward(mlp, cache_mode, group_size, use_triton, outlier_ratio)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._fwd(x)
