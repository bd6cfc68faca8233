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

import random
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


def _private(mode: str, hg, hu) -> bool:
    """The backward's h_gate / h_up are its own buffers (recomputed or
    dequantised, not the saved bf16 cache), contiguous, so the SwiGLU
    backward may write its gradients over them."""
    return mode != "bf16" and hg.is_contiguous() and hu.is_contiguous()


_CACHE_CODE = {"int4": _lib.CACHE_INT4, "int8": _lib.CACHE_INT8, "bf16": _lib.CACHE_BF16,
               "recompute": _lib.CACHE_NONE}
_FUSED_GROUPS = (32, 64, 128)
# Cache formats whose codec runs in the gate/up dual GEMM's epilogue (K1 fused,
# only codes and h_mid leave the kernel), and from how many tokens.  Otherwise
# the forward runs the same dual GEMM with a bf16 epilogue and then the
# standalone K1; the two paths are bit-identical.  Measured on MI355X, fused
# against bf16 out + K1 (us, with and without LoRA terms in the epilogue):
#   d_model 2048, d_ff 5632:  2048 tokens int8 110.5 / 106.6, int4 109.2 / 105.6;
#                             4096 tokens int8 178.4 / 180.1, int4 177.6 / 175.9;
#                             8192 tokens int8 350.8 / 377.0, int4 348.7 / 366.3;
#   d_model 4096, d_ff 11008: fused faster at every count from 1024 to 16384
#                             (ratio 0.96-0.99; C2: 1141 / 1187 int8).
# Below that the codec epilogue's VALU work (one wavefront per SIMD, so the
# block's MFMAs idle meanwhile) costs more than K1 at HBM speed; a longer
# k-loop per tile (larger d_model) and more waves of tiles amortise it.
_F1_CODEC_MIN_TOKENS = {"int8": 4096, "int4": 8192}
_F1_CODEC_WIDE_D_MODEL = 4096      # from here on, at any token count


def _f1_codec_fused(cache_mode: str, tokens: int, d_model: int) -> bool:
    m = _F1_CODEC_MIN_TOKENS.get(cache_mode)
    return m is not None and (tokens >= m or d_model >= _F1_CODEC_WIDE_D_MODEL)


# Outlier channels (config C3) with a bf16 activation and d_model a multiple
# of 64.  True: the first sequence (which ranks the channels) runs the dual
# GEMM with a bf16 output, the selection and K1 with outliers, and every
# later row the dual GEMM with the outlier codec in its epilogue
# (G.ffn_gate_up_outlier), so only h_mid and the compressed cache of those
# rows reach HBM.  False (the default): the dual GEMM with a bf16 output for
# every row, then the selection and K1 with outliers.  The caches, outputs
# and gradients are bit-identical.  Measured at C3 on MI355X with the
# division-free quantiser: step 3.94 against 3.82 ms (the two dual GEMMs
# 1.286 ms plus 0.019 for the first sequence's K1, against 1.073 + 0.122 for
# one dual GEMM and K1): the int4 outlier codec inside the power-limited
# GEMM, and the first sequence's 1.34 waves of tiles, cost more than the
# 720 MB bf16 round trip at HBM speed.
_F1_OUTLIER_FUSED = False
# Group sizes whose dequantise + SwiGLU backward runs in the dgrad GEMM's
# epilogue (G.ffn_down_dgrad, on the 16x16x32 loop when d_model is a multiple
# of 64) instead of the dgrad GEMM followed by the K2 kernel.  Empty: on
# MI355X the fused epilogue (VALU work and 540 MB of writes while the block's
# MFMAs idle, one wavefront per SIMD) costs more than the standalone K2 at
# full occupancy.  On the 16x16x32 loop, inside the step: C2 0.816 ms fused
# against 0.555 + 0.148 ms (step 5.11 against 5.01 ms), C3 0.966 against
# 0.590 + 0.157 ms (step 4.11 against 3.89 ms).  The fused kernel stays
# available and tested; add group sizes here to route the Function through it.
_FUSED_DGRAD_GROUPS = ()
# The weight gradient of the down projection with the GLU decompressed in the
# GEMM's operand staging (G.wgrad_glu: h^ formed from the int cache as the TN
# GEMM stages its B tiles) instead of K2 writing h_mid^ for a plain TN GEMM.
# Off: each 256-column h^ tile is rebuilt by all hidden/256 = 16 row tiles,
# so the kernel is VALU-bound and measures slower than K2's h_mid^ plus the
# plain GEMM.  Both are bit-equal; set True to route the Function through it.
_FUSED_WGRAD_GLU = False
# The LoRA backward's two thin products of one tensor (grad_h B and
# s grad_h^T (x A^T); grad_y B_d and s grad_y^T (h_mid A_d^T)) in one pass
# over it (G.skinny_dual) instead of a projection and a token reduction that
# each read it.
_DUAL_SKINNY = True


def _mfma(*ts) -> bool:
    """The bf16 MFMA GEMMs take bf16 matrices with 16-byte aligned rows: the
    base address 16-byte aligned, the contiguous extent and the row stride
    multiples of 8.  The other extent (the token count of an activation, or
    of a transposed one) is free: the kernels mask rows and k past the edge.
    Everything else runs on the general-layout kernel (G.mm_any)."""
    for t in ts:
        if t is None:
            continue
        if t.dtype != torch.bfloat16 or t.dim() != 2 or t.data_ptr() % 16:
            return False
        rows, cols = t.shape
        if t.stride(1) == 1 and cols % 8 == 0 and t.stride(0) % 8 == 0:
            continue
        if t.stride(0) == 1 and rows % 8 == 0 and t.stride(1) % 8 == 0:
            continue
        return False
    return True


def _mm(a, b, name):
    """a @ b: the bf16 MFMA GEMMs, or the general-layout kernel for other
    dtypes and layouts."""
    if _mfma(a, b) and a.shape[0] > 0:
        return G.mm(a, b, name)
    return G.mm_any(a, b, name=name)


# The full fine-tune weight gradients dg^T x and du^T x read x with the token
# dimension as K.  From this many tokens they take x^T (one transpose kernel)
# as a K-major operand: at C2 (8192 x 4096, d_ff 11008) each product measured
# 531.5 against 567.8 us, and the transpose of x costs ~25 us.  Bit-identical.
_XT_MIN_TOKENS = 1024


def _xt_ok(x, *grads):
    return (x.shape[0] >= _XT_MIN_TOKENS and G.transpose_ok(x)
            and all(_mfma(g, x) for g in grads))


def _linear(x, w, name):
    return _mm(x, w.t(), name)


def _addmm(c, a, b, s, name):
    """c + s * (a @ b) in the reference's op order (product, scaling and sum
    each rounded to the dtype), in place on c."""
    if _mfma(c, a, b) and a.shape[0] > 0 and c.stride(1) == 1:
        return G.addmm_(c, a, b, s, name)
    return G.mm_any(a, b, s, G.ANY_ADD, out=c, name=name)


def _mm_scaled(a, b, s, name):
    """s * (a @ b) for the thin adapter gradients, which reduce over all
    tokens: split-K on the bf16 engine, or the general-layout kernel."""
    if _mfma(a, b) and a.shape[1] > 0:
        return G.mm_splitk(a, b, s, name=name)
    return G.mm_any(a, b, s, G.ANY_SCALE, name=name)


def _dual_ok(x, b, p) -> bool:
    """The projection x B and the reduction x^T p of one tensor go through
    G.skinny_dual (one pass over x): bf16 x [T, N] and B [N, r], p [T, r],
    rank a multiple of 8 up to 32, N a multiple of 8, at least one 512-column
    block of x (thinner tensors keep the separate kernels), when
    _DUAL_SKINNY is on."""
    return (_DUAL_SKINNY and x is not None and b is not None and p is not None
            and x.dim() == 2 and x.shape[1] >= 512 and x.shape[0] > 0
            and G.skinny_dual_ok(x, b.t(), p))


def _mm_sum(a, b, a2, b2, name):
    """a @ b + a2 @ b2: one K-concatenated accumulation on the bf16 engine, or
    the reference's two rounded products and their rounded sum."""
    if _mfma(a, b, a2, b2):
        return G.mm2(a, b, a2, b2, name)
    out = G.mm_any(a, b, name=name)
    return G.mm_any(a2, b2, 1.0, G.ANY_ADD, out=out, name=name)


def _lora_ok(*pairs, dims) -> bool:
    """The adapter terms (a, b) present ride in the epilogues of the GEMMs
    with the (k, n) `dims`: bf16 factors of one shared rank up to 16, or up to
    32 where those GEMMs run on the 16x16x32 loop (G.lora_fusable; the GEMM
    wrapper re-lays and zero-pads them for the kernel's 8-wide k chunks)."""
    ranks = {a.shape[0] for a, b in pairs if a is not None}
    return (len(ranks) <= 1 and all(G.lora_fusable(r, *dims) for r in ranks)
            and all(t.dtype == torch.bfloat16 and t.dim() == 2
                    for a, b in pairs if a is not None for t in (a, b)))


def outlier_stat_rows(shape) -> int:
    """Rows of the [N, D] activations whose column norms pick the outlier
    channels.  HyC-LoRA takes the norm over the first sample,
    `x_[0].abs().norm(dim=-2)` on a [B, S, D] tensor
    (src/hyclora/operators/compress_function.py:85): the first N / B rows for
    an input of 3 or more dims.  A 2-D input [N, D] is one sample: all rows."""
    n = 1
    for s in shape[:-1]:
        n *= int(s)
    if len(shape) >= 3 and int(shape[0]) > 0:
        return n // int(shape[0])
    return n


def _proj(x_2d, w, a, b, s, name):
    """out = x W^T (+ s * (x A^T) B^T) in PEFT op order (src/flashffn.py:1410-1420).
    Returns (out, xA | None)."""
    if (a is not None and _mfma(x_2d, w) and _lora_ok((a, b), dims=((w.shape[1], w.shape[0]),))
            and x_2d.shape[0] > 0):
        xa = _mm(x_2d, a.t(), name + "_xa")
        return G.linear_lora(x_2d, w, xa, b, s, name), xa
    h = _linear(x_2d, w, name)
    xa = None
    if a is not None:
        xa = _mm(x_2d, a.t(), name + "_xa")
        h = _addmm(h, xa, b.t(), s, name + "_lora")
    return h, xa


def _stackable(p, q) -> bool:
    """Two rank-r factors that one skinny product can take stacked: ranks up to
    32 together, the first a multiple of 8 (so the second's columns start on a
    16-byte boundary)."""
    return (p is not None and q is not None and p.dtype == q.dtype
            and p.shape[0] % 8 == 0 and p.shape[0] + q.shape[0] <= G.SKINNY_MAX_RANK)


def _gate_up_lora(x_2d, a_gate, b_gate, s_gate, a_up, b_up, s_up):
    """(xa_g | None, xa_u | None, ffn_gate_up keyword terms) for the fused
    gate/up GEMM.  With both adapters, x [A_g; A_u]^T is one pass over x: its
    column halves equal the two products bit for bit."""
    if _stackable(a_gate, a_up) and x_2d.shape[0] >= 256 and x_2d.shape[1] >= 256:
        r = a_gate.shape[0]
        xa = _mm(x_2d, torch.cat([a_gate, a_up]).t(), "gemm_fwd_gate_up_xa")
        xa_g, xa_u = xa[:, :r], xa[:, r:]
    else:
        xa_g = _mm(x_2d, a_gate.t(), "gemm_fwd_gate_xa") if a_gate is not None else None
        xa_u = _mm(x_2d, a_up.t(), "gemm_fwd_up_xa") if a_up is not None else None
    kw = dict(lora_gate=None if a_gate is None else (xa_g, b_gate, s_gate),
              lora_up=None if a_up is None else (xa_u, b_up, s_up))
    return xa_g, xa_u, kw


class FlashFFNv3Function(torch.autograd.Function):
    """LoRA-factored SwiGLU FFN with a quantised GLU-cache backward
    (src/flashffn.py:1376-1602).  a_*/b_* may be None (pass s_*=0.0).

    bf16 with 16-byte aligned rows runs the fused MFMA kernels: the forward
    gate/up GEMM carries the LoRA terms, SiLU*mul and the codec in its
    epilogue; the backward runs the dgrad GEMM, then the K2 kernel
    (dequantise + SwiGLU backward), or for bf16 / recompute caches the dgrad
    GEMM with the SwiGLU backward in its epilogue.  Other dtypes and layouts
    compose the general-layout GEMM kernel with the standalone elementwise
    kernels in the reference's order.

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
        # the dual gate/up kernel, with the gate/up LoRA terms in its epilogue
        fusable = (_mfma(x_2d, w_gate, w_up)
                   and _lora_ok((a_gate, b_gate), (a_up, b_up), dims=((hidden_dim, inter),))
                   and x_2d.shape[0] > 0)

        c_gate = qs_gate = c_up = qs_up = None
        o_gate = o_up = slot_gate = slot_up = None
        h_gate = h_up = None
        xa_g = xa_u = None
        lkw = {}
        if fusable:
            xa_g, xa_u, lkw = _gate_up_lora(x_2d, a_gate, b_gate, s_gate, a_up, b_up, s_up)
        fused_quant = (quant and use_triton and x.dtype == torch.bfloat16)   # :1424-1426
        if (fusable and fused_quant and k_out == 0 and group_size in _FUSED_GROUPS
                and _f1_codec_fused(cache_mode, x_2d.shape[0], hidden_dim)):
            # dual GEMM + GLU + codec in one kernel (K1 fused into the epilogue)
            h_mid, _, _, c_gate, qs_gate, c_up, qs_up = G.ffn_gate_up(
                x_2d, w_gate, w_up, _CACHE_CODE[cache_mode], group_size, **lkw)
            _V3_COUNTERS["triton_quant_fwd"] += 1
        elif (fusable and fused_quant and k_out > 0 and _F1_OUTLIER_FUSED
              and group_size in _FUSED_GROUPS and G.ffn_gate_up_outlier_fits(hidden_dim)
              and outlier_stat_rows(orig_shape) < x_2d.shape[0]):
            # outlier channels: the first sequence ranks them, so its rows get
            # the dual GEMM with a bf16 epilogue, the selection and K1 with
            # outliers; every later row runs the dual GEMM with the outlier
            # codec in its epilogue (only h_mid and the compressed cache reach
            # HBM for them)
            rows = outlier_stat_rows(orig_shape)
            n_all = x_2d.shape[0]
            lk_first, lk_rest = {}, {}
            for key, term in lkw.items():
                lk_first[key] = None if term is None else (term[0][:rows], term[1], term[2])
                lk_rest[key] = None if term is None else (term[0][rows:], term[1], term[2])
            _, hg1, hu1, *_ = G.ffn_gate_up(x_2d[:rows], w_gate, w_up, _lib.CACHE_BF16,
                                            group_size, want_h_mid=False, **lk_first)
            (slot_gate, _), (slot_up, _) = K.outlier_select_pair(hg1, hu1, k_out, rows)
            bits = _bits(cache_mode)
            dev = x.device
            qshape = (n_all, inter // 2) if bits == 4 else (n_all, inter)
            qdt = torch.uint8 if bits == 4 else torch.int8
            h_mid = torch.empty((n_all, inter), dtype=x.dtype, device=dev)
            c_gate = torch.empty(qshape, dtype=qdt, device=dev)
            c_up = torch.empty(qshape, dtype=qdt, device=dev)
            qs_gate = torch.empty((n_all, inter // group_size), dtype=torch.float16, device=dev)
            qs_up = torch.empty((n_all, inter // group_size), dtype=torch.float16, device=dev)
            o_gate = torch.empty((n_all, k_out), dtype=torch.bfloat16, device=dev)
            o_up = torch.empty((n_all, k_out), dtype=torch.bfloat16, device=dev)
            bufs = (h_mid, c_gate, qs_gate, o_gate, c_up, qs_up, o_up)
            K.silu_mul_quant_outlier(hg1, hu1, bits, group_size, slot_gate, slot_up, k_out,
                                     out=tuple(t[:rows] for t in bufs))
            del hg1, hu1
            G.ffn_gate_up_outlier(x_2d[rows:], w_gate, w_up, _CACHE_CODE[cache_mode], group_size,
                                  slot_gate, slot_up, k_out, tuple(t[rows:] for t in bufs),
                                  **lk_rest)
        elif fusable and not fused_quant and k_out == 0:
            # h_gate/h_up are needed (bf16 cache, eager codec) or not (recompute)
            keep = cache_mode != "recompute"
            h_mid, h_gate, h_up, *_ = G.ffn_gate_up(
                x_2d, w_gate, w_up, _lib.CACHE_BF16 if keep else _lib.CACHE_NONE, group_size,
                **lkw)
        else:
            if fusable:
                _, h_gate, h_up, *_ = G.ffn_gate_up(x_2d, w_gate, w_up, _lib.CACHE_BF16,
                                                    group_size, want_h_mid=False, **lkw)
            else:
                h_gate, xa_g = _proj(x_2d, w_gate, a_gate, b_gate, s_gate, "gemm_fwd_gate")
                h_up, xa_u = _proj(x_2d, w_up, a_up, b_up, s_up, "gemm_fwd_up")
            if k_out > 0:
                rows = outlier_stat_rows(orig_shape)
                (slot_gate, _), (slot_up, _) = K.outlier_select_pair(h_gate, h_up, k_out, rows)
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
        # grad_w_down from the cache itself: K2 then skips h_mid^ unless the
        # down adapter's gradient needs it
        use_wglu = (_FUSED_WGRAD_GLU and use_k2 and need_wd and not outl and gs in _FUSED_GROUPS
                    and _mfma(gy) and gy.shape[0] > 0)
        need_hm = need_h_mid and ((a_down is not None and need_ad) or not use_wglu)
        lora_d = _lora_ok((a_down, b_down), dims=((w_down.shape[0], w_down.shape[1]),))
        # the fused dgrad kernel restores outlier channels only for the
        # quantised caches (K2's path); bf16 / recompute caches carry none
        fusable = _mfma(gy, w_down) and lora_d and gy.shape[0] > 0 and (use_k2 or not outl)
        # F1's recompute (k d_model) and the K-concatenated grad_x product (k d_ff)
        d_ff, d_model = w_gate.shape
        fusable_gu = (_mfma(x_2d, w_gate, w_up)
                      and _lora_ok((a_gate, b_gate), (a_up, b_up),
                                   dims=((d_model, d_ff), (d_ff, d_model)))
                      and x_2d.shape[0] > 0)

        hg = hu = None
        if need_recon and not use_k2:                                     # :1500-1516
            if mode == "recompute":
                if fusable_gu:
                    # the forward's kernel and terms on the same inputs: bitwise equal
                    lkw = dict(lora_gate=None if a_gate is None else (xa_g, b_gate, s_gate),
                               lora_up=None if a_up is None else (xa_u, b_up, s_up))
                    _, hg, hu, *_ = G.ffn_gate_up(x_2d, w_gate, w_up, _lib.CACHE_BF16, gs,
                                                  want_h_mid=False, **lkw)
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
            if need_bd and _dual_ok(gy, b_down, ha_d):
                # grad_y B_d and s grad_y^T (h_mid A_d^T) in one pass over
                # grad_y (:1521,1545)
                gyB_d, grad_b_down = G.skinny_dual(gy, b_down.t(), ha_d, 1.0, s_down,
                                                   name="gemm_gyB_grad_b_down")
            else:
                gyB_d = _mm(gy, b_down, "gemm_gyB_down")                  # :1521

        # the down projection's LoRA term of grad_h_mid (:1527-1529) rides in
        # the dgrad GEMM's epilogue
        dlora = (gyB_d, a_down, s_down) if (a_down is not None and lora_d) else None
        grad_h_gate = grad_h_up = h_mid_hat = None
        if need_gate_path:
            if use_k2 and fusable and gs in _FUSED_DGRAD_GROUPS:          # :1525-1533
                # dgrad GEMM with dequantise + SwiGLU backward in its epilogue
                grad_h_gate, grad_h_up, h_mid_hat = G.ffn_down_dgrad(
                    gy, w_down, _CACHE_CODE[mode], gs, c_gate, qs_gate, c_up, qs_up,
                    need_hm, lora=dlora,
                    outliers=(slot_gate, o_gate, slot_up, o_up) if outl else None)
                _V3_COUNTERS["triton_dequant_bwd"] += 1
            elif (not use_k2) and fusable and hg is not None and _mfma(hg, hu):
                # grad_h_gate / grad_h_up are written over h_gate / h_up when
                # those are this backward's own (recomputed or dequantised)
                grad_h_gate, grad_h_up, h_mid_hat = G.ffn_down_dgrad(
                    gy, w_down, _lib.CACHE_BF16, gs, hg, None, hu, None, need_h_mid,
                    lora=dlora, inplace=_private(mode, hg, hu))
                hg = hu = None
            else:
                if dlora is not None and _mfma(gy, w_down) and gy.shape[0] > 0:
                    grad_h_mid = G.mm2(gy, w_down, name="gemm_dgrad_down", lora=[
                        (gyB_d, a_down, s_down)])
                else:
                    grad_h_mid = _mm(gy, w_down, "gemm_dgrad_down")
                    if a_down is not None:
                        grad_h_mid = _addmm(grad_h_mid, gyB_d, a_down, s_down,
                                            "gemm_dgrad_down_lora")
                # grad_h_mid is private: K2 writes grad_h_gate over it, and
                # the GLU backward writes over h_gate / h_up too when those
                # are private (3 live [N, D] buffers instead of 6,
                # src/flashffn.py:129-198)
                if use_k2 and outl:
                    grad_h_gate, grad_h_up, h_mid_hat = K.dequant_swiglu_backward_outlier(
                        grad_h_mid, c_gate, qs_gate, o_gate, slot_gate, c_up, qs_up, o_up,
                        slot_up, _bits(mode), gs, want_h_mid=need_h_mid, inplace=True)
                elif use_k2:
                    grad_h_gate, grad_h_up, h_mid_hat = K.dequant_swiglu_backward(
                        grad_h_mid, c_gate, qs_gate, c_up, qs_up, _bits(mode), gs,
                        want_h_mid=need_hm, inplace=True)
                else:
                    grad_h_gate, grad_h_up, h_mid_hat = K.swiglu_backward_glu(
                        grad_h_mid, hg, hu, need_h_mid,
                        inplace=_private(mode, hg, hu) and grad_h_mid.is_contiguous())
                    hg = hu = None
                del grad_h_mid

        if need_h_mid:                                                    # :1536-1543
            if h_mid_hat is None and need_hm:
                h_mid_hat = K.silu_mul(hg, hu)
            if need_wd and use_wglu:
                grad_w_down = G.wgrad_glu(gy, _CACHE_CODE[mode], gs, c_gate, qs_gate, c_up, qs_up,
                                          name="gemm_wgrad_down")
            elif need_wd:
                grad_w_down = _mm(gy.t(), h_mid_hat, "gemm_wgrad_down")
            if need_ad:
                grad_a_down = _mm_scaled(gyB_d.t(), h_mid_hat, s_down, "gemm_grad_a_down")
            del h_mid_hat
        if need_bd and grad_b_down is None:
            grad_b_down = _mm_scaled(gy.t(), ha_d, s_down, "gemm_grad_b_down")   # :1545

        grad_x = None
        grad_w_gate = grad_a_gate = grad_b_gate = None
        grad_w_up = grad_a_up = grad_b_up = None
        if need_gate_path:                                                # :1551-1587
            ghgB = ghuB = ghB = None
            # dg B_g and du B_u side by side in one [N, r_g + r_u] buffer, so
            # one token reduction over x gives both A gradients below
            stack = (_stackable(b_gate.t() if b_gate is not None else None,
                                b_up.t() if b_up is not None else None)
                     and (need_x or need_ag or need_au) and grad_h_gate.shape[0] >= 256
                     and _mfma(grad_h_gate, b_gate, grad_h_up, b_up)
                     and grad_h_gate.shape[1] >= 256)
            if stack:
                r = b_gate.shape[1]
                ghB = torch.empty((grad_h_gate.shape[0], r + b_up.shape[1]),
                                  dtype=grad_h_gate.dtype, device=grad_h_gate.device)
                # with the B gradient, both products of grad_h in one pass
                # (:1556-1557 with :1575-1582)
                if need_bg and _dual_ok(grad_h_gate, b_gate, xa_g):
                    _, grad_b_gate = G.skinny_dual(grad_h_gate, b_gate.t(), xa_g, 1.0, s_gate,
                                                   out_c=ghB[:, :r], name="gemm_ghgB_grad_b_gate")
                else:
                    G.skinny(grad_h_gate, b_gate.t(), 1.0, "gemm_ghgB", out=ghB[:, :r])
                if need_bu and _dual_ok(grad_h_up, b_up, xa_u):
                    _, grad_b_up = G.skinny_dual(grad_h_up, b_up.t(), xa_u, 1.0, s_up,
                                                 out_c=ghB[:, r:], name="gemm_ghuB_grad_b_up")
                else:
                    G.skinny(grad_h_up, b_up.t(), 1.0, "gemm_ghuB", out=ghB[:, r:])
                ghgB, ghuB = ghB[:, :r], ghB[:, r:]
            else:
                if a_gate is not None and (need_x or need_ag):
                    if need_bg and _dual_ok(grad_h_gate, b_gate, xa_g):
                        ghgB, grad_b_gate = G.skinny_dual(grad_h_gate, b_gate.t(), xa_g, 1.0,
                                                          s_gate, name="gemm_ghgB_grad_b_gate")
                    else:
                        ghgB = _mm(grad_h_gate, b_gate, "gemm_ghgB")
                if a_up is not None and (need_x or need_au):
                    if need_bu and _dual_ok(grad_h_up, b_up, xa_u):
                        ghuB, grad_b_up = G.skinny_dual(grad_h_up, b_up.t(), xa_u, 1.0, s_up,
                                                        name="gemm_ghuB_grad_b_up")
                    else:
                        ghuB = _mm(grad_h_up, b_up, "gemm_ghuB")
            if need_x:
                xl = [(ghgB, a_gate, s_gate) if a_gate is not None else None,
                      (ghuB, a_up, s_up) if a_up is not None else None]
                if _mfma(grad_h_gate, w_gate, grad_h_up, w_up) and fusable_gu:
                    # dg @ W_g + du @ W_u as one K-concatenated GEMM, the gate and up
                    # LoRA terms (:1561-1566) in its epilogue
                    grad_x = G.mm2(grad_h_gate, w_gate, grad_h_up, w_up, "gemm_dgrad_x",
                                   lora=[t for t in xl if t is not None] or None)
                else:
                    grad_x = _mm_sum(grad_h_gate, w_gate, grad_h_up, w_up, "gemm_dgrad_x")
                    if a_gate is not None:
                        grad_x = _addmm(grad_x, ghgB, a_gate, s_gate, "gemm_dgrad_x_lora_gate")
                    if a_up is not None:
                        grad_x = _addmm(grad_x, ghuB, a_up, s_up, "gemm_dgrad_x_lora_up")
            if need_bg and grad_b_gate is None:
                grad_b_gate = _mm_scaled(grad_h_gate.t(), xa_g, s_gate, "gemm_grad_b_gate")
            if ghB is not None and need_ag and need_au and s_gate == s_up:
                # s [dg B_g | du B_u]^T x: its row halves equal the two
                # reductions bit for bit (same token order per row)
                ga = _mm_scaled(ghB.t(), x_2d, s_gate, "gemm_grad_a_gate_up")
                grad_a_gate, grad_a_up = ga[:ghgB.shape[1]], ga[ghgB.shape[1]:]
            else:
                if need_ag:
                    grad_a_gate = _mm_scaled(ghgB.t(), x_2d, s_gate, "gemm_grad_a_gate")
                if need_au:
                    grad_a_up = _mm_scaled(ghuB.t(), x_2d, s_up, "gemm_grad_a_up")
            if need_bu and grad_b_up is None:
                grad_b_up = _mm_scaled(grad_h_up.t(), xa_u, s_up, "gemm_grad_b_up")
            if need_wg and need_wu and _xt_ok(x_2d, grad_h_gate, grad_h_up):
                # x^T once, so both products read it K-major (bit-identical)
                x_t = G.transpose(x_2d, "transpose_x").t()
                grad_w_gate = G.mm(grad_h_gate.t(), x_t, "gemm_wgrad_gate")   # :1585
                grad_w_up = G.mm(grad_h_up.t(), x_t, "gemm_wgrad_up")         # :1587
                x_t = None
            else:
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
# module-level API (src/flashffn.py:1605-1694, 1798-1921, 2211-2230)
#
# A projection of an MLP is a plain nn.Linear or a PEFT-shaped adapter
# wrapper (base_layer plus the family's own parameters).  The wrapper is
# recognised by which adapter parameters it carries (_WRAPPER_TESTS), and a
# per-family extractor (_EXTRACT) turns it into the factors the Functions
# take, re-read on every call so training updates and DyLoRA's rank draws are
# seen.  DoRA and AdaLoRA wrappers also carry LoRA's ModuleDicts, so the
# families with extra parameters are tested before plain LoRA.
# ---------------------------------------------------------------------------

_MLP_PROJS = ("gate_proj", "up_proj", "down_proj")
_FAMILY_NAME = {"dora": "DoRA", "adalora": "AdaLoRA", "vera": "VeRA", "dylora": "DyLoRA",
                "lora": "LoRA"}


def _holds_entries(proj: nn.Module, attr: str) -> bool:
    v = getattr(proj, attr, None)
    return v is not None and len(v) > 0


_WRAPPER_TESTS = (
    ("dora", lambda p: _holds_entries(p, "lora_magnitude_vector")),
    ("adalora", lambda p: _holds_entries(p, "lora_E")),
    ("vera", lambda p: _holds_entries(p, "vera_lambda_d")),
    # DyLoRA keeps its factors as bare Parameters with a rank bound r
    ("dylora", lambda p: all(isinstance(getattr(p, a, None), nn.Parameter)
                             for a in ("lora_A", "lora_B"))
     and hasattr(p, "r") and hasattr(p, "scaling")),
    ("lora", lambda p: isinstance(getattr(p, "lora_A", None), nn.ModuleDict)
     and len(p.lora_A) > 0),
)


def _v3_proj_kind(proj: nn.Module) -> str:
    """Structural classification of one MLP projection (src/flashffn.py:
    1798-1821): 'dora' | 'adalora' | 'vera' | 'dylora' | 'lora' | 'plain' |
    'unknown'."""
    if not hasattr(proj, "base_layer"):
        return "plain" if hasattr(proj, "weight") else "unknown"
    for kind, test in _WRAPPER_TESTS:
        if test(proj):
            return kind
    return "unknown"


def _active_adapter(proj: nn.Module) -> str:
    names = list(proj.active_adapters)
    assert len(names) == 1, "exactly one active adapter expected"
    return names[0]


def _warn_dropout(family: str, drop: nn.Module):
    """The fused path applies no adapter dropout: say so when it is on."""
    p = float(getattr(drop, "p", 0.0))
    if p > 0.0:
        warnings.warn(f"FlashFFNv3 ignores {family} dropout (p={p}); results differ from the "
                      f"reference forward when training with dropout.")


def _lora_factors(proj: nn.Module, family: str = "LoRA"):
    """(W, A, B, s) of a PEFT LoRA-style wrapper's active adapter."""
    name = _active_adapter(proj)
    _warn_dropout(family, proj.lora_dropout[name])
    return (proj.get_base_layer().weight, proj.lora_A[name].weight, proj.lora_B[name].weight,
            float(proj.scaling[name]))


def _v3_extract_proj(proj: nn.Module):
    """(W, A, B, s) from a plain nn.Linear (A = B = None, s = 0.0) or a PEFT
    LoRA wrapper (src/flashffn.py:1605-1634).  Other adapter families raise
    NotImplementedError: FlashFFNv3Function takes LoRA factors only."""
    kind = _v3_proj_kind(proj)
    if kind == "plain":
        return proj.weight, None, None, 0.0
    if kind != "lora":
        raise NotImplementedError(
            f"FlashFFNv3 fast path does not support {_FAMILY_NAME.get(kind, type(proj).__name__)}")
    return _lora_factors(proj)


def _to_dtype(t, dt):
    """Cast through autograd (gradients flow back to the stored parameter)."""
    return t if (t is None or t.dtype == dt) else t.to(dt)


def make_v3_forward(mlp: nn.Module, cache_mode: str = "int4", group_size: int = 64,
                    use_triton: bool = True, outlier_ratio: float = 0.0):
    """Drop-in replacement for a LLaMA-style MLP forward (src/flashffn.py:1637-1678).
    `mlp` exposes gate_proj / up_proj / down_proj, each a plain nn.Linear or an
    adapter wrapper.  Plain and LoRA projections run FlashFFNv3Function; any
    DoRA / AdaLoRA / VeRA / DyLoRA projection sends the MLP to the adapter
    Function (src/flashffn.py:1660-1661).  Unknown wrappers raise
    NotImplementedError."""
    projs = [getattr(mlp, name) for name in _MLP_PROJS]
    kinds = tuple(_v3_proj_kind(p) for p in projs)
    if "unknown" in kinds:
        raise NotImplementedError(f"FlashFFNv3: unsupported projection wrapper(s) on MLP: {kinds}")
    if not set(kinds) <= {"plain", "lora"}:
        assert outlier_ratio == 0.0, "outlier channels are not defined for the adapter Function"
        return make_v3_adapter_forward(mlp, cache_mode, group_size, use_triton)

    def v3_forward(x):
        factors = [_v3_extract_proj(p) for p in projs]
        tensors = [_to_dtype(t, x.dtype) for f in factors for t in f[:3]]
        scales = [f[3] for f in factors]
        return FlashFFNv3Function.apply(x, *tensors, *scales, cache_mode, group_size, use_triton,
                                        outlier_ratio)
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


# ---------------------------------------------------------------------------
# adapter families: DoRA / AdaLoRA / VeRA / DyLoRA (src/flashffn.py:1697-2230)
# ---------------------------------------------------------------------------

def _v3_dora_col_norm(w: torch.Tensor, a: torch.Tensor, b: torch.Tensor, s: float,
                      out_dtype=torch.float32) -> torch.Tensor:
    """DoRA's column norm ||W + s * B @ A||_2 over dim=1 without forming B @ A
    (src/flashffn.py:1824-1840): fp32 Gram identity on the device, detached.
    The reference returns float32; `out_dtype` folds its later `.to(dt)`."""
    with torch.no_grad():
        return K.dora_col_norm(w.detach(), a.detach(), b.detach(), s, out_dtype)


# Per-family factor extraction: proj -> (W, A, B, s, m, nu) in the stored
# dtype (the caller casts).  AdaLoRA's A*E and VeRA's lambda-scaled frozen
# factors are composed here, in autograd, so their chain rules run on [r, in]
# / [out, r] tensors; DyLoRA passes rank-b slices (b uniform in 1..r in
# training, r in eval); DoRA adds its magnitude m and the detached norm nu.

def _plain_adapter(proj):
    return proj.weight, None, None, 0.0, None, None


def _lora_adapter(proj):
    return _lora_factors(proj) + (None, None)


def _dylora_adapter(proj):
    _warn_dropout("DyLoRA", proj.dropout)
    rank = _rng_randint(1, proj.r) if proj.training else proj.r
    return (proj.base_layer.weight, proj.lora_A[:rank, :], proj.lora_B[:, :rank],
            float(proj.scaling), None, None)


def _adalora_adapter(proj):
    name = _active_adapter(proj)
    _warn_dropout("AdaLoRA", proj.lora_dropout[name])
    s_eff = float(proj.scaling[name]) / (float(proj.ranknum[name]) + 1e-5)
    return (proj.get_base_layer().weight, proj.lora_A[name] * proj.lora_E[name],
            proj.lora_B[name], s_eff, None, None)


def _vera_adapter(proj):
    name = _active_adapter(proj)
    _warn_dropout("VeRA", proj.vera_dropout[name])
    a_frozen = proj.vera_A[name][:, : proj.in_features]
    b_frozen = proj.vera_B[name][: proj.out_features, :]
    return (proj.get_base_layer().weight, proj.vera_lambda_d[name].unsqueeze(-1) * a_frozen,
            proj.vera_lambda_b[name].unsqueeze(-1) * b_frozen, 1.0, None, None)


def _dora_adapter(proj):
    w, a, b, s = _lora_factors(proj, "DoRA")
    return w, a, b, s, proj.lora_magnitude_vector[_active_adapter(proj)].weight, None


_EXTRACT = {"plain": _plain_adapter, "lora": _lora_adapter, "dylora": _dylora_adapter,
            "adalora": _adalora_adapter, "vera": _vera_adapter, "dora": _dora_adapter}


def _v3_extract_proj_adapter(proj: nn.Module, dt: torch.dtype):
    """(w, a, b, s, m, nu) of one projection in dtype dt, re-extracted per
    forward (src/flashffn.py:1850-1921).  DoRA's nu is computed from the
    cast factors; everything else is cast through autograd."""
    kind = _v3_proj_kind(proj)
    if kind not in _EXTRACT:
        raise NotImplementedError(
            f"FlashFFNv3 adapter path: unsupported projection wrapper ({type(proj).__name__}).")
    w, a, b, s, m, _ = _EXTRACT[kind](proj)
    w, a, b, m = (_to_dtype(t, dt) for t in (w, a, b, m))
    nu = _v3_dora_col_norm(w, a, b, s, out_dtype=dt) if m is not None else None
    return w, a, b, s, m, nu


def _rng_randint(lo: int, hi: int) -> int:
    """DyLoRA's per-forward rank draw from Python's global `random` stream,
    as the reference module draws it (src/dylora.py), so a seeded
    `random.seed` reproduces the same ranks in both."""
    return random.randint(lo, hi)


def _scaled(t, m, nu, inplace=False):
    """t * (m / nu) per column, or t when the projection has no magnitude."""
    if m is None:
        return t
    return K.dora_scale(t, m, nu, out=t if inplace else None)


class FlashFFNv3AdapterFunction(torch.autograd.Function):
    """Sibling of FlashFFNv3Function for DoRA / AdaLoRA / VeRA / DyLoRA
    projections (src/flashffn.py:1924-2208).  AdaLoRA, VeRA and DyLoRA arrive
    as composed or sliced thin factors (_v3_extract_proj_adapter), so every
    projection is the LoRA core, optionally with DoRA's magnitude: out =
    c * (z W^T + s (z A^T) B^T), c = m / nu, nu detached.

      apply(x, w_gate, a_gate, b_gate, m_gate, nu_gate,
            w_up, a_up, b_up, m_up, nu_up, w_down, a_down, b_down, m_down, nu_down,
            s_gate=0.0, s_up=0.0, s_down=0.0, cache_mode="int4", group_size=64,
            use_triton=True)

    The cache layer is FlashFFNv3Function's (h_gate / h_up cached after the
    scale c).  Backward: dL/draw = g * c feeds the LoRA-core grads; grad_m =
    sum_n g raw / nu with raw recomputed ('recompute' mode and the down
    projection, one extra GEMM) or sum_n g h / m from the cache."""

    @staticmethod
    def forward(ctx, x, w_gate, a_gate, b_gate, m_gate, nu_gate, w_up, a_up, b_up, m_up, nu_up,
                w_down, a_down, b_down, m_down, nu_down, s_gate=0.0, s_up=0.0, s_down=0.0,
                cache_mode="int4", group_size=64, use_triton=True):
        assert cache_mode in ("int4", "int8", "bf16", "recompute"), cache_mode
        _V3_COUNTERS["forward"] += 1
        _V3_COUNTERS["adapter_forward"] += 1
        K._require_device(x)
        orig_shape = x.shape
        hidden_dim = x.shape[-1]
        x_2d = x.reshape(-1, hidden_dim)
        if not x_2d.is_contiguous():
            x_2d = x_2d.contiguous()
        quant = cache_mode in ("int4", "int8")
        plain_gu = a_gate is None and a_up is None and m_gate is None and m_up is None
        fusable = plain_gu and _mfma(x_2d, w_gate, w_up) and x_2d.shape[0] > 0
        fused_quant = quant and use_triton and x.dtype == torch.bfloat16   # :1979-1981

        c_gate = qs_gate = c_up = qs_up = None
        h_gate = h_up = xa_g = xa_u = None
        if (fusable and fused_quant and group_size in _FUSED_GROUPS
                and _f1_codec_fused(cache_mode, x_2d.shape[0], hidden_dim)):
            h_mid, _, _, c_gate, qs_gate, c_up, qs_up = G.ffn_gate_up(
                x_2d, w_gate, w_up, _CACHE_CODE[cache_mode], group_size)
            _V3_COUNTERS["triton_quant_fwd"] += 1
        elif fusable and fused_quant:
            # the dual GEMM with a bf16 epilogue, then the standalone K1
            _, h_gate, h_up, *_ = G.ffn_gate_up(x_2d, w_gate, w_up, _lib.CACHE_BF16, group_size,
                                                want_h_mid=False)
            h_mid, c_gate, qs_gate, c_up, qs_up = K.silu_mul_quant(
                h_gate, h_up, _bits(cache_mode), group_size)
            h_gate = h_up = None
        elif fusable and not fused_quant:
            keep = cache_mode != "recompute"
            h_mid, h_gate, h_up, *_ = G.ffn_gate_up(
                x_2d, w_gate, w_up, _lib.CACHE_BF16 if keep else _lib.CACHE_NONE, group_size)
        else:
            h_gate, xa_g = _proj(x_2d, w_gate, a_gate, b_gate, s_gate, "gemm_fwd_gate")
            h_gate = _scaled(h_gate, m_gate, nu_gate, inplace=True)          # :1967
            h_up, xa_u = _proj(x_2d, w_up, a_up, b_up, s_up, "gemm_fwd_up")
            h_up = _scaled(h_up, m_up, nu_up, inplace=True)                   # :1975
            if fused_quant:
                h_mid, c_gate, qs_gate, c_up, qs_up = K.silu_mul_quant(
                    h_gate, h_up, _bits(cache_mode), group_size)
                h_gate = h_up = None
            else:
                h_mid = K.silu_mul(h_gate, h_up)

        y, ha_d = _proj(h_mid, w_down, a_down, b_down, s_down, "gemm_fwd_down")   # :1990-1994
        y = _scaled(y, m_down, nu_down, inplace=True)                              # :1996

        if not fused_quant:                                                         # :1998-2007
            if quant:
                c_gate, qs_gate = K.v3_quantize_group_absmax(h_gate, _bits(cache_mode), group_size)
                c_up, qs_up = K.v3_quantize_group_absmax(h_up, _bits(cache_mode), group_size)
            elif cache_mode == "bf16":
                c_gate, c_up = h_gate, h_up
        del h_gate, h_up, h_mid

        ctx.save_for_backward(x, w_gate, a_gate, b_gate, m_gate, nu_gate,
                              w_up, a_up, b_up, m_up, nu_up,
                              w_down, a_down, b_down, m_down, nu_down,
                              xa_g, xa_u, ha_d, c_gate, qs_gate, c_up, qs_up)
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
        _V3_COUNTERS["adapter_backward"] += 1
        (x, w_gate, a_gate, b_gate, m_gate, nu_gate, w_up, a_up, b_up, m_up, nu_up,
         w_down, a_down, b_down, m_down, nu_down,
         xa_g, xa_u, ha_d, cq_gate, qs_gate, cq_up, qs_up) = ctx.saved_tensors
        s_gate, s_up, s_down = ctx.s
        mode = ctx.cache_mode
        gs = ctx.group_size
        hidden_dim = ctx.orig_shape[-1]
        ng = ctx.needs_input_grad
        need_x = ng[0]
        need_wg, need_ag, need_bg, need_mg = ng[1], ng[2], ng[3], ng[4]
        need_wu, need_au, need_bu, need_mu = ng[6], ng[7], ng[8], ng[9]
        need_wd, need_ad, need_bd, need_md = ng[11], ng[12], ng[13], ng[14]
        gy = grad_y.reshape(-1, hidden_dim)
        if not gy.is_contiguous():
            gy = gy.contiguous()
        x_2d = x.reshape(-1, hidden_dim)
        if not x_2d.is_contiguous():
            x_2d = x_2d.contiguous()

        need_gate_path = (need_x or need_wg or need_ag or need_bg or need_mg
                          or need_wu or need_au or need_bu or need_mu)          # :2047-2048
        need_h_mid = need_wd or need_md or (a_down is not None and need_ad)
        need_recon = need_gate_path or need_h_mid
        use_k2 = mode in ("int4", "int8") and ctx.use_triton and need_gate_path
        plain_gu = a_gate is None and a_up is None and m_gate is None and m_up is None
        fusable_gu = plain_gu and _mfma(x_2d, w_gate, w_up) and x_2d.shape[0] > 0

        hg = hu = raw_g = raw_u = None
        if need_recon and not use_k2:                                           # :2055-2078
            if mode == "recompute":
                if fusable_gu:
                    # the forward's kernel and terms on the same inputs: bitwise equal
                    lkw = dict(lora_gate=None if a_gate is None else (xa_g, b_gate, s_gate),
                               lora_up=None if a_up is None else (xa_u, b_up, s_up))
                    _, hg, hu, *_ = G.ffn_gate_up(x_2d, w_gate, w_up, _lib.CACHE_BF16, gs,
                                                  want_h_mid=False, **lkw)
                else:
                    raw_g = _linear(x_2d, w_gate, "gemm_recompute_gate")
                    if a_gate is not None:
                        raw_g = _addmm(raw_g, xa_g, b_gate.t(), s_gate, "gemm_recompute_gate_lora")
                    hg = _scaled(raw_g, m_gate, nu_gate)
                    raw_u = _linear(x_2d, w_up, "gemm_recompute_up")
                    if a_up is not None:
                        raw_u = _addmm(raw_u, xa_u, b_up.t(), s_up, "gemm_recompute_up_lora")
                    hu = _scaled(raw_u, m_up, nu_up)
            elif mode == "bf16":
                hg, hu = cq_gate, cq_up
            else:
                hg = K.v3_dequantize_group_absmax(cq_gate, qs_gate, _bits(mode), gs, ctx.in_dtype)
                hu = K.v3_dequantize_group_absmax(cq_up, qs_up, _bits(mode), gs, ctx.in_dtype)
        elif use_k2 and (need_mg or need_mu):                                   # :2079-2089
            # grad_m needs h^ itself, which K2 never materialises
            if need_mg:
                hg = K.v3_dequantize_group_absmax(cq_gate, qs_gate, _bits(mode), gs, ctx.in_dtype)
            if need_mu:
                hu = K.v3_dequantize_group_absmax(cq_up, qs_up, _bits(mode), gs, ctx.in_dtype)

        g_eff_y = _scaled(gy, m_down, nu_down)                                  # :2094
        gyB_d = None
        if a_down is not None and (need_gate_path or need_ad):
            gyB_d = _mm(g_eff_y, b_down, "gemm_gyB_down")
        fusable_d = a_down is None and _mfma(g_eff_y, w_down) and g_eff_y.shape[0] > 0

        # the SwiGLU backward may write over h_gate / h_up when they are this
        # backward's own and no magnitude gradient reads them afterwards
        own = (hg is not None and hu is not None and m_gate is None and m_up is None
               and _private(mode, hg, hu))
        grad_h_gate = grad_h_up = h_mid_hat = None
        if need_gate_path:
            if use_k2 and fusable_d and gs in _FUSED_DGRAD_GROUPS:              # :2101-2110
                grad_h_gate, grad_h_up, h_mid_hat = G.ffn_down_dgrad(
                    g_eff_y, w_down, _CACHE_CODE[mode], gs, cq_gate, qs_gate, cq_up, qs_up,
                    need_h_mid)
                _V3_COUNTERS["triton_dequant_bwd"] += 1
            elif (not use_k2) and fusable_d and hg is not None and hu is not None \
                    and _mfma(hg, hu):
                grad_h_gate, grad_h_up, h_mid_hat = G.ffn_down_dgrad(
                    g_eff_y, w_down, _lib.CACHE_BF16, gs, hg, None, hu, None, need_h_mid,
                    inplace=own)
            else:
                grad_h_mid = _mm(g_eff_y, w_down, "gemm_dgrad_down")
                if a_down is not None:
                    grad_h_mid = _addmm(grad_h_mid, gyB_d, a_down, s_down, "gemm_dgrad_down_lora")
                if use_k2:
                    grad_h_gate, grad_h_up, h_mid_hat = K.dequant_swiglu_backward(
                        grad_h_mid, cq_gate, qs_gate, cq_up, qs_up, _bits(mode), gs,
                        want_h_mid=need_h_mid, inplace=True)
                else:
                    grad_h_gate, grad_h_up, h_mid_hat = K.swiglu_backward_glu(
                        grad_h_mid, hg, hu, need_h_mid,
                        inplace=own and grad_h_mid.is_contiguous())
                del grad_h_mid

        grad_w_down = grad_a_down = grad_b_down = grad_m_down = None
        if need_h_mid:                                                          # :2112-2131
            if h_mid_hat is None:
                h_mid_hat = K.silu_mul(hg, hu)
            if need_wd:
                grad_w_down = _mm(g_eff_y.t(), h_mid_hat, "gemm_wgrad_down")
            if need_ad:
                grad_a_down = _mm_scaled(gyB_d.t(), h_mid_hat, s_down, "gemm_grad_a_down")
            if need_md:
                # raw_d is never stored: one extra GEMM recomputes it
                raw_d, _ = _proj(h_mid_hat, w_down, None, None, 0.0, "gemm_recompute_down")
                if a_down is not None:
                    raw_d = _addmm(raw_d, ha_d, b_down.t(), s_down, "gemm_recompute_down_lora")
                grad_m_down = K.col_dot_div(gy, raw_d, nu_down)
                del raw_d
            del h_mid_hat
        if need_bd:
            grad_b_down = _mm_scaled(g_eff_y.t(), ha_d, s_down, "gemm_grad_b_down")

        grad_x = None
        grad_w_gate = grad_a_gate = grad_b_gate = grad_m_gate = None
        grad_w_up = grad_a_up = grad_b_up = grad_m_up = None
        if need_gate_path:                                                      # :2134-2191
            if need_mg:
                grad_m_gate = (K.col_dot_div(grad_h_gate, raw_g, nu_gate) if raw_g is not None
                               else K.col_dot_div(grad_h_gate, hg, m_gate))
            if need_mu:
                grad_m_up = (K.col_dot_div(grad_h_up, raw_u, nu_up) if raw_u is not None
                             else K.col_dot_div(grad_h_up, hu, m_up))
            # h = c * raw  =>  dL/draw = grad_h * c (grad_h is private here)
            g_eff_g = _scaled(grad_h_gate, m_gate, nu_gate, inplace=True)
            g_eff_u = _scaled(grad_h_up, m_up, nu_up, inplace=True)
            ghgB = None
            if a_gate is not None and (need_x or need_ag):
                ghgB = _mm(g_eff_g, b_gate, "gemm_ghgB")
            ghuB = None
            if a_up is not None and (need_x or need_au):
                ghuB = _mm(g_eff_u, b_up, "gemm_ghuB")
            if need_x:
                grad_x = _mm_sum(g_eff_g, w_gate, g_eff_u, w_up, "gemm_dgrad_x")
                if a_gate is not None:
                    grad_x = _addmm(grad_x, ghgB, a_gate, s_gate, "gemm_dgrad_x_lora_gate")
                if a_up is not None:
                    grad_x = _addmm(grad_x, ghuB, a_up, s_up, "gemm_dgrad_x_lora_up")
            if need_bg:
                grad_b_gate = _mm_scaled(g_eff_g.t(), xa_g, s_gate, "gemm_grad_b_gate")
            if need_ag:
                grad_a_gate = _mm_scaled(ghgB.t(), x_2d, s_gate, "gemm_grad_a_gate")
            if need_bu:
                grad_b_up = _mm_scaled(g_eff_u.t(), xa_u, s_up, "gemm_grad_b_up")
            if need_au:
                grad_a_up = _mm_scaled(ghuB.t(), x_2d, s_up, "gemm_grad_a_up")
            if need_wg:
                grad_w_gate = _mm(g_eff_g.t(), x_2d, "gemm_wgrad_gate")
            if need_wu:
                grad_w_up = _mm(g_eff_u.t(), x_2d, "gemm_wgrad_up")

        # frozen weights => no dense [D_out, D_in] gradient was built (:2194-2197)
        if not (need_wg or need_wu or need_wd):
            assert grad_w_gate is None and grad_w_up is None and grad_w_down is None, \
                "FlashFFNv3 invariant violated: dense weight grad with frozen weights"
        if need_x and len(ctx.orig_shape) == 3:
            grad_x = grad_x.view(ctx.orig_shape)
        return (grad_x,
                grad_w_gate, grad_a_gate, grad_b_gate, grad_m_gate, None,
                grad_w_up, grad_a_up, grad_b_up, grad_m_up, None,
                grad_w_down, grad_a_down, grad_b_down, grad_m_down, None,
                ) + (None,) * (len(ctx.needs_input_grad) - 16)


def make_v3_adapter_forward(mlp: nn.Module, cache_mode: str = "int4", group_size: int = 64,
                            use_triton: bool = True):
    """Adapter-factored v3 forward for an MLP whose projections may be DoRA /
    AdaLoRA / VeRA / DyLoRA wrapped, mixed with plain or LoRA ones
    (src/flashffn.py:2211-2230).  Factors, the DoRA norm and DyLoRA's rank
    are re-extracted on every call."""
    projs = [getattr(mlp, name) for name in _MLP_PROJS]

    def v3_adapter_forward(x):
        per = [_v3_extract_proj_adapter(p, x.dtype) for p in projs]
        tensors = [t for w, a, b, _, m, nu in per for t in (w, a, b, m, nu)]
        scales = [f[3] for f in per]
        return FlashFFNv3AdapterFunction.apply(x, *tensors, *scales, cache_mode, group_size,
                                               use_triton)
    return v3_adapter_forward


# ---------------------------------------------------------------------------
# v1/v2 API: FlashFFNFunction with top-K compression, FlashFFN, StandardFFN
# (src/flashffn.py:300-519)
# ---------------------------------------------------------------------------

def _gate_up(x_2d, w_gate, w_up, keep: bool):
    """(h_mid, h_gate | None, h_up | None): the fused dual GEMM + GLU on the
    engine for bf16, the general-layout GEMMs + the GLU kernel otherwise."""
    if _mfma(x_2d, w_gate, w_up) and x_2d.shape[0] > 0:
        h_mid, hg, hu, *_ = G.ffn_gate_up(x_2d, w_gate, w_up,
                                          _lib.CACHE_BF16 if keep else _lib.CACHE_NONE, 64)
        return h_mid, hg, hu
    hg = _linear(x_2d, w_gate, "gemm_fwd_gate")
    hu = _linear(x_2d, w_up, "gemm_fwd_up")
    return K.silu_mul(hg, hu), (hg if keep else None), (hu if keep else None)


def _glu_backward(gy, w_down, hg, hu, inplace=False):
    """(grad_h_gate, grad_h_up) of h_mid = SiLU(hg) * hu through y = h_mid W_d^T;
    `inplace` writes them over hg / hu (private, contiguous)."""
    if _mfma(gy, w_down, hg, hu) and gy.shape[0] > 0:
        dg, du, _ = G.ffn_down_dgrad(gy, w_down, _lib.CACHE_BF16, 64, hg, None, hu, None, False,
                                     inplace=inplace)
        return dg, du
    ghm = _mm(gy, w_down, "gemm_dgrad_down")
    if inplace and ghm.is_contiguous():
        dg, du, _ = K.swiglu_backward_glu(ghm, hg, hu, False, inplace=True)
        return dg, du
    return K.swiglu_backward(ghm, hg, hu)


def _dgrad_x(dg, w_gate, du, w_up):
    return _mm_sum(dg, w_gate, du, w_up, "gemm_dgrad_x")


class FlashFFNFunction(torch.autograd.Function):
    """SwiGLU FFN with top-K activation compression (src/flashffn.py:300-449).

    The mode follows the weights' requires_grad, as in the reference:
      'recompute' (some weight trains): saves x and, per token, the
          k = max(1, int(D * k_fraction)) entries of h_mid with the largest
          magnitude (values + int16 columns).  Backward: grad_w_down from the
          sparse h_mid (approximate by design), every other grad exact from
          recomputed h_gate / h_up;
      'activations' (all weights frozen): saves h_gate and h_up; backward
          returns grad_x only.
    Device path: the fused dual GEMM + GLU forward and the fused dgrad GEMM +
    SwiGLU backward on the MFMA engine (bf16), the top-K select and scatter
    kernels; the general-layout GEMMs + the GLU kernels for other dtypes."""

    @staticmethod
    def forward(ctx, x, w_gate, w_up, w_down, k_fraction=0.3):
        K._require_device(x)
        orig_shape = x.shape
        hidden_dim = x.shape[-1]
        inter = w_gate.shape[0]
        x_2d = x.reshape(-1, hidden_dim)
        if not x_2d.is_contiguous():
            x_2d = x_2d.contiguous()
        weights_need_grad = w_gate.requires_grad or w_up.requires_grad or w_down.requires_grad
        h_mid, h_gate, h_up = _gate_up(x_2d, w_gate, w_up, keep=not weights_need_grad)
        y = _linear(h_mid, w_down, "gemm_fwd_down")
        if weights_need_grad:                                              # :349-361
            k = max(1, int(inter * k_fraction))
            values, indices = K.topk_abs(h_mid, k)
            ctx.save_for_backward(x, w_gate, w_up, w_down, values, indices)
            ctx.save_mode = "recompute"
            ctx.k = k
            ctx.intermediate_dim = inter
        else:                                                              # :362-366
            ctx.save_for_backward(h_gate, h_up, w_gate, w_up, w_down)
            ctx.save_mode = "activations"
        del h_mid
        ctx.orig_shape = orig_shape
        if len(orig_shape) == 3:
            y = y.view(orig_shape[0], orig_shape[1], hidden_dim)
        return y

    @staticmethod
    def backward(ctx, grad_output):
        orig_shape = ctx.orig_shape
        hidden_dim = orig_shape[-1]
        gy = grad_output.reshape(-1, hidden_dim)
        if not gy.is_contiguous():
            gy = gy.contiguous()
        if ctx.save_mode == "activations":                                 # :386-405
            h_gate, h_up, w_gate, w_up, w_down = ctx.saved_tensors
            dg, du = _glu_backward(gy, w_down, h_gate, h_up)
            grad_x = _dgrad_x(dg, w_gate, du, w_up)
            if len(orig_shape) == 3:
                grad_x = grad_x.view(orig_shape)
            return grad_x, None, None, None, None

        x, w_gate, w_up, w_down, values, indices = ctx.saved_tensors      # :407-449
        x_2d = x.reshape(-1, hidden_dim)
        if not x_2d.is_contiguous():
            x_2d = x_2d.contiguous()
        need_x, need_wg, need_wu, need_wd = ctx.needs_input_grad[:4]
        grad_w_down = None
        if need_wd:
            h_mid_sparse = K.topk_scatter(values, indices, ctx.intermediate_dim)
            grad_w_down = _mm(gy.t(), h_mid_sparse, "gemm_wgrad_down")
            del h_mid_sparse
        grad_x = grad_w_gate = grad_w_up = None
        if need_x or need_wg or need_wu:
            _, hg, hu = _gate_up(x_2d, w_gate, w_up, keep=True)
            dg, du = _glu_backward(gy, w_down, hg, hu,
                                   inplace=hg.is_contiguous() and hu.is_contiguous())
            del hg, hu
            if need_wg:
                grad_w_gate = _mm(dg.t(), x_2d, "gemm_wgrad_gate")
            if need_wu:
                grad_w_up = _mm(du.t(), x_2d, "gemm_wgrad_up")
            if need_x:
                grad_x = _dgrad_x(dg, w_gate, du, w_up)
        if need_x and len(orig_shape) == 3:
            grad_x = grad_x.view(orig_shape)
        return grad_x, grad_w_gate, grad_w_up, grad_w_down, None


class FlashFFN(nn.Module):
    """SwiGLU FFN module over FlashFFNFunction (src/flashffn.py:456-496).
    As in the reference, `bias` creates bias parameters that the compressed
    forward does not use."""

    def __init__(self, hidden_dim: int, intermediate_dim: int, k_fraction: float = 0.3,
                 bias: bool = False):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.intermediate_dim = intermediate_dim
        self.k_fraction = k_fraction
        self.gate_proj = nn.Linear(hidden_dim, intermediate_dim, bias=bias)
        self.up_proj = nn.Linear(hidden_dim, intermediate_dim, bias=bias)
        self.down_proj = nn.Linear(intermediate_dim, hidden_dim, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return FlashFFNFunction.apply(x, self.gate_proj.weight, self.up_proj.weight,
                                      self.down_proj.weight, self.k_fraction)


class StandardFFN(nn.Module):
    """The unfused SwiGLU FFN the reference compares against
    (src/flashffn.py:499-519): torch modules and autograd, no compression."""

    def __init__(self, hidden_dim: int, intermediate_dim: int, bias: bool = False):
        super().__init__()
        self.gate_proj = nn.Linear(hidden_dim, intermediate_dim, bias=bias)
        self.up_proj = nn.Linear(hidden_dim, intermediate_dim, bias=bias)
        self.down_proj = nn.Linear(intermediate_dim, hidden_dim, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h_gate = self.gate_proj(x)
        h_up = self.up_proj(x)
        return self.down_proj(F.silu(h_gate) * h_up)
