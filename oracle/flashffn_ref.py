"""torch-CPU restatement of the FlashFFN v3 autograd Function (CPU oracle).

TEST INFRASTRUCTURE ONLY -- imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline, never by the product.

Contents
  kernel contracts with the reference's wrapper names and torch in/out:
    triton_silu_mul (flashffn.py:205-220), triton_swiglu_backward (:223-239),
    triton_swiglu_backward_glu (:259-293), v3_quantize_group_absmax
    (:1055-1088), v3_dequantize_group_absmax (:1091-1110),
    triton_silu_mul_quant (:1314-1340), triton_dequant_swiglu_backward
    (:1343-1373); all computed by oracle/codec.py.
  OracleFlashFFNv3Function: FlashFFNv3Function.forward/backward
    (:1395-1602) in the reference's op order, on CPU tensors of any float dtype;
    with outlier_ratio > 0 (this build's C3 extension, parity unpinned against
    the reference) the int4/int8 cache keeps HyC-LoRA outlier channels.
  ref_grads_fp32: the fp32 plain-autograd reference of the same factored
    computation (src/verify_flashffn_v3.py:294-327).
  count_saved_bytes / int4_saved_bytes_closed_form: the reference's
    saved-activation accounting (src/verify_flashffn_v3.py:523-543,594-600).

Parity status: OracleFlashFFNv3Function is pinned against ref_grads_fp32 (in
'recompute' and 'bf16' cache modes the two agree to float32 rounding in fp32,
which fails on any dropped term, wrong transpose or wrong scale in the
reassociated backward) and against the reference's own V2 cosine thresholds in
the quantised modes (tests/test_oracle_function.py).  GEMM outputs are not
bit-pinnable against the reference (cuBLAS), as in the reference's own gates.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import codec

# ---------------------------------------------------------------------------
# torch <-> numpy with exact bf16 handling
# ---------------------------------------------------------------------------


def to_f32(t: torch.Tensor) -> np.ndarray:
    """Exact widening of a bf16/fp16/fp32 tensor to a float32 numpy array."""
    return t.detach().cpu().to(torch.float32).contiguous().numpy()


def from_f32(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    """Round a float32 array to `dtype` with round-to-nearest-even."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    if dtype == torch.bfloat16:
        return torch.from_numpy(codec.f32_to_bf16_bits(a).view(np.int16)).view(torch.bfloat16)
    if dtype == torch.float16:
        return torch.from_numpy(a.astype(np.float16))
    if dtype == torch.float32:
        return torch.from_numpy(a.copy())
    raise TypeError(f"unsupported dtype {dtype}")


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


# ---------------------------------------------------------------------------
# kernel contracts (torch in / torch out)
# ---------------------------------------------------------------------------


def v3_quantize_group_absmax(t: torch.Tensor, bits: int, group_size: int = 64):
    """flashffn.py:1055-1088 -> (payload uint8 [N,D/2] | int8 [N,D], scales fp16 [N,G])."""
    q, s = codec.quantize_group_absmax(to_f32(t), bits, group_size)
    return torch.from_numpy(q), torch.from_numpy(s)


def v3_dequantize_group_absmax(payload, scales, bits, group_size=64, dtype=torch.bfloat16):
    """flashffn.py:1091-1110."""
    f = codec.dequantize_group_absmax_f32(payload.cpu().numpy(), scales.cpu().numpy(),
                                          bits, group_size)
    return from_f32(f, dtype)


def triton_silu_mul(h_gate, h_up):
    """flashffn.py:205-220: output in the input dtype."""
    return from_f32(codec.silu_mul(to_f32(h_gate), to_f32(h_up)), h_gate.dtype).reshape(h_gate.shape)


def triton_swiglu_backward(grad_h_mid, h_gate, h_up):
    """flashffn.py:223-239 -> (grad_h_gate, grad_h_up) in h_gate's dtype."""
    dg, du = codec.swiglu_backward(to_f32(grad_h_mid), to_f32(h_gate), to_f32(h_up))
    dt = h_gate.dtype
    return from_f32(dg, dt).reshape(h_gate.shape), from_f32(du, dt).reshape(h_gate.shape)


def triton_swiglu_backward_glu(grad_h_mid, h_gate, h_up, want_h_mid):
    """flashffn.py:259-293 values (aliasing is a memory property, not a value one)."""
    dg, du = triton_swiglu_backward(grad_h_mid, h_gate, h_up)
    hm = triton_silu_mul(h_gate, h_up) if want_h_mid else None
    return dg, du, hm


def triton_silu_mul_quant(h_gate, h_up, bits, group_size=64):
    """flashffn.py:1314-1340 contract -> (h_mid, q_gate, s_gate, q_up, s_up)."""
    g, u = to_f32(h_gate), to_f32(h_up)
    hm, qg, sg, qu, su = codec.silu_mul_quant(g, u, bits, group_size)
    return (from_f32(hm, h_gate.dtype), torch.from_numpy(qg), torch.from_numpy(sg),
            torch.from_numpy(qu), torch.from_numpy(su))


def triton_dequant_swiglu_backward(grad_h_mid, q_gate, s_gate, q_up, s_up, bits,
                                   group_size=64, want_h_mid=False):
    """flashffn.py:1343-1373 contract -> (grad_h_gate, grad_h_up, h_mid_hat | None)."""
    dg, du, hm = codec.dequant_swiglu_backward(
        to_f32(grad_h_mid), q_gate.numpy(), s_gate.numpy(), q_up.numpy(), s_up.numpy(),
        bits, group_size, want_h_mid)
    dt = grad_h_mid.dtype
    return from_f32(dg, dt), from_f32(du, dt), (from_f32(hm, dt) if want_h_mid else None)


def outlier_select(h, ratio, rows=None):
    """Outlier columns of the bf16 tensor h (codec.outlier_channels spec),
    ranked by the column norms of its first `rows` rows."""
    return codec.outlier_channels(to_f32(h), ratio, rows)


def stat_rows(shape):
    """The first sample's row count: HyC-LoRA ranks channels on x_[0] of a
    [B, S, D] input (compress_function.py:85), i.e. N / B rows; a 2-D input is
    a single sample."""
    n = int(np.prod([int(s) for s in shape[:-1]])) if len(shape) > 1 else 1
    return n // int(shape[0]) if len(shape) >= 3 and int(shape[0]) > 0 else n


def v3_quantize_outlier(h, bits, group_size, idx):
    v = to_f32(h)
    q, s, o = codec.outlier_quantize(v, codec.f32_to_bf16_bits(v), idx, bits, group_size)
    return torch.from_numpy(q), torch.from_numpy(s), torch.from_numpy(o.view(np.int16)).view(torch.bfloat16)


def v3_dequantize_outlier(payload, scales, outliers, idx, bits, group_size):
    ob = outliers.contiguous().view(torch.int16).numpy().view(np.uint16)
    bits_out = codec.outlier_dequantize_bf16(payload.numpy(), scales.numpy(), ob, idx, bits,
                                             group_size)
    return torch.from_numpy(bits_out.view(np.int16)).view(torch.bfloat16)


# ---------------------------------------------------------------------------
# FlashFFNv3Function restated
# ---------------------------------------------------------------------------


class OracleFlashFFNv3Function(torch.autograd.Function):
    """CPU restatement of FlashFFNv3Function (flashffn.py:1376-1602).

    Same argument list:
      apply(x, w_gate, a_gate, b_gate, w_up, a_up, b_up, w_down, a_down, b_down,
            s_gate, s_up, s_down, cache_mode, group_size, use_triton)
    The Triton kernels are replaced by their oracle contracts; the GEMMs are
    torch CPU F.linear/@ in the tensors' dtype, as the reference runs them.

    Two trailing arguments serve the tests that check a device run on a
    sample of its rows or against its own cache (neither changes the
    algorithm, only where one of its inputs comes from):
      outlier_idx = (idx_gate, idx_up): the outlier channels to keep, instead
          of ranking this call's rows (a row sample does not hold the first
          sequence those channels are ranked on);
      cache_override = (c_gate, qs_gate, c_up, qs_up): the int4/int8 cache to
          save instead of quantising this call's h_gate / h_up (which a CPU
          GEMM rounds differently from the device's).
    """

    @staticmethod
    def forward(ctx, x, w_gate, a_gate, b_gate, w_up, a_up, b_up, w_down, a_down, b_down,
                s_gate=0.0, s_up=0.0, s_down=0.0, cache_mode="int4", group_size=64,
                use_triton=True, outlier_ratio=0.0, outlier_idx=None, cache_override=None):
        assert cache_mode in ("int4", "int8", "bf16", "recompute"), cache_mode
        orig_shape = x.shape
        hidden_dim = x.shape[-1]
        x_2d = x.reshape(-1, hidden_dim)

        h_gate = F.linear(x_2d, w_gate)                                  # :1410
        xa_g = None
        if a_gate is not None:
            xa_g = F.linear(x_2d, a_gate)                                # :1413
            h_gate = h_gate + s_gate * F.linear(xa_g, b_gate)            # :1414
        h_up = F.linear(x_2d, w_up)                                      # :1416
        xa_u = None
        if a_up is not None:
            xa_u = F.linear(x_2d, a_up)
            h_up = h_up + s_up * F.linear(xa_u, b_up)                    # :1420

        c_gate = qs_gate = c_up = qs_up = None
        o_gate = o_up = idx_gate = idx_up = None
        fused_quant = (cache_mode in ("int4", "int8") and use_triton
                       and h_gate.dtype == torch.bfloat16)               # :1424-1426
        k_out = (int(h_gate.shape[1] * outlier_ratio)
                 if cache_mode in ("int4", "int8") and outlier_ratio > 0 else 0)
        if k_out > 0:
            # this build's C3 extension: HyC-LoRA outlier channels on the v3 codec
            bits = 4 if cache_mode == "int4" else 8
            if outlier_idx is not None:
                idx_gate, idx_up = (np.asarray(i, dtype=np.int64) for i in outlier_idx)
            else:
                rows = stat_rows(orig_shape)
                idx_gate = outlier_select(h_gate, outlier_ratio, rows)
                idx_up = outlier_select(h_up, outlier_ratio, rows)
            c_gate, qs_gate, o_gate = v3_quantize_outlier(h_gate, bits, group_size, idx_gate)
            c_up, qs_up, o_up = v3_quantize_outlier(h_up, bits, group_size, idx_up)
            h_mid = triton_silu_mul(h_gate, h_up)
        elif fused_quant:
            bits = 4 if cache_mode == "int4" else 8
            h_mid, c_gate, qs_gate, c_up, qs_up = triton_silu_mul_quant(
                h_gate, h_up, bits, group_size)                          # :1429
        else:
            h_mid = triton_silu_mul(h_gate, h_up)                        # :1433

        y = F.linear(h_mid, w_down)                                      # :1435
        ha_d = None
        if a_down is not None:
            ha_d = F.linear(h_mid, a_down)                               # :1438
            y = y + s_down * F.linear(ha_d, b_down)                      # :1439

        if not fused_quant and k_out == 0:
            if cache_mode in ("int4", "int8"):
                bits = 4 if cache_mode == "int4" else 8
                c_gate, qs_gate = v3_quantize_group_absmax(h_gate, bits, group_size)
                c_up, qs_up = v3_quantize_group_absmax(h_up, bits, group_size)
            elif cache_mode == "bf16":
                c_gate, c_up = h_gate, h_up
        if cache_override is not None:
            assert cache_mode in ("int4", "int8") and k_out == 0
            c_gate, qs_gate, c_up, qs_up = cache_override
        ctx.save_for_backward(x, w_gate, a_gate, b_gate, w_up, a_up, b_up,
                              w_down, a_down, b_down, xa_g, xa_u, ha_d,
                              c_gate, qs_gate, c_up, qs_up)              # :1454-1458
        ctx.outliers = (o_gate, o_up, idx_gate, idx_up)
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
        (x, w_gate, a_gate, b_gate, w_up, a_up, b_up, w_down, a_down, b_down,
         xa_g, xa_u, ha_d, c_gate, qs_gate, c_up, qs_up) = ctx.saved_tensors
        s_gate, s_up, s_down = ctx.s
        mode = ctx.cache_mode
        hidden_dim = ctx.orig_shape[-1]
        (need_x, need_wg, need_ag, need_bg, need_wu, need_au, need_bu,
         need_wd, need_ad, need_bd) = ctx.needs_input_grad[:10]
        gy = grad_y.reshape(-1, hidden_dim)
        x_2d = x.reshape(-1, hidden_dim)

        need_gate_path = (need_x or need_wg or need_ag or need_bg
                          or need_wu or need_au or need_bu)              # :1488-1489
        need_h_mid = need_wd or (a_down is not None and need_ad)         # :1490
        need_recon = need_gate_path or need_h_mid
        use_k2 = (mode in ("int4", "int8") and ctx.use_triton and need_gate_path
                  and ctx.outliers[0] is None)

        hg = hu = None
        if need_recon and not use_k2:                                    # :1500-1516
            if mode == "recompute":
                hg = F.linear(x_2d, w_gate)
                if a_gate is not None:
                    hg = hg + s_gate * F.linear(xa_g, b_gate)
                hu = F.linear(x_2d, w_up)
                if a_up is not None:
                    hu = hu + s_up * F.linear(xa_u, b_up)
            elif mode == "bf16":
                hg, hu = c_gate, c_up
            elif ctx.outliers[0] is not None:
                bits = 4 if mode == "int4" else 8
                o_gate, o_up, idx_gate, idx_up = ctx.outliers
                hg = v3_dequantize_outlier(c_gate, qs_gate, o_gate, idx_gate, bits, ctx.group_size)
                hu = v3_dequantize_outlier(c_up, qs_up, o_up, idx_up, bits, ctx.group_size)
            else:
                bits = 4 if mode == "int4" else 8
                hg = v3_dequantize_group_absmax(c_gate, qs_gate, bits, ctx.group_size,
                                                ctx.in_dtype)
                hu = v3_dequantize_group_absmax(c_up, qs_up, bits, ctx.group_size,
                                                ctx.in_dtype)

        grad_w_down = grad_a_down = grad_b_down = None
        gyB_d = None
        if a_down is not None and (need_gate_path or need_ad):
            gyB_d = gy @ b_down                                          # :1521

        grad_h_gate = grad_h_up = h_mid_hat = None
        if use_k2:                                                       # :1525-1533
            bits = 4 if mode == "int4" else 8
            grad_h_mid = gy @ w_down
            if a_down is not None:
                grad_h_mid = grad_h_mid + s_down * (gyB_d @ a_down)
            grad_h_gate, grad_h_up, h_mid_hat = triton_dequant_swiglu_backward(
                grad_h_mid, c_gate, qs_gate, c_up, qs_up, bits, ctx.group_size,
                want_h_mid=need_h_mid)

        if need_h_mid:                                                   # :1536-1543
            if h_mid_hat is None:
                h_mid_hat = triton_silu_mul(hg, hu)
            if need_wd:
                grad_w_down = gy.t() @ h_mid_hat
            if need_ad:
                grad_a_down = s_down * (gyB_d.t() @ h_mid_hat)
        if need_bd:
            grad_b_down = s_down * (gy.t() @ ha_d)                       # :1545

        grad_x = None
        grad_w_gate = grad_a_gate = grad_b_gate = None
        grad_w_up = grad_a_up = grad_b_up = None
        if need_gate_path:                                               # :1551-1587
            if grad_h_gate is None:
                grad_h_mid = gy @ w_down
                if a_down is not None:
                    grad_h_mid = grad_h_mid + s_down * (gyB_d @ a_down)
                grad_h_gate, grad_h_up = triton_swiglu_backward(grad_h_mid, hg, hu)
            ghgB = None
            if a_gate is not None and (need_x or need_ag):
                ghgB = grad_h_gate @ b_gate
            ghuB = None
            if a_up is not None and (need_x or need_au):
                ghuB = grad_h_up @ b_up
            if need_x:
                grad_x = grad_h_gate @ w_gate
                if a_gate is not None:
                    grad_x = grad_x + s_gate * (ghgB @ a_gate)
                grad_x = grad_x + grad_h_up @ w_up
                if a_up is not None:
                    grad_x = grad_x + s_up * (ghuB @ a_up)
            if need_bg:
                grad_b_gate = s_gate * (grad_h_gate.t() @ xa_g)
            if need_ag:
                grad_a_gate = s_gate * (ghgB.t() @ x_2d)
            if need_bu:
                grad_b_up = s_up * (grad_h_up.t() @ xa_u)
            if need_au:
                grad_a_up = s_up * (ghuB.t() @ x_2d)
            if need_wg:
                grad_w_gate = grad_h_gate.t() @ x_2d
            if need_wu:
                grad_w_up = grad_h_up.t() @ x_2d

        if need_x and len(ctx.orig_shape) == 3:
            grad_x = grad_x.view(ctx.orig_shape)
        return (grad_x, grad_w_gate, grad_a_gate, grad_b_gate,
                grad_w_up, grad_a_up, grad_b_up,
                grad_w_down, grad_a_down, grad_b_down) + (None,) * (len(ctx.needs_input_grad) - 10)


# ---------------------------------------------------------------------------
# fp32 plain-autograd reference and test helpers
# ---------------------------------------------------------------------------

PROJ = ("gate", "up", "down")


def ref_grads_fp32(ps: dict, x: torch.Tensor, gy: torch.Tensor):
    """src/verify_flashffn_v3.py:294-327: plain autograd in float32 of the SAME
    factored computation, from the SAME (possibly bf16) inputs upcast.
    Returns ({name: grad}, y)."""
    def leaf(t, rg):
        return None if t is None else t.detach().float().requires_grad_(rg)

    xl = x.detach().float().requires_grad_(True)
    t = {}
    for key in PROJ:
        t[f"w_{key}"] = leaf(ps[f"w_{key}"], ps["train_w"])
        has = ps[f"a_{key}"] is not None
        t[f"a_{key}"] = leaf(ps[f"a_{key}"], has)
        t[f"b_{key}"] = leaf(ps[f"b_{key}"], has)

    def proj(z, key):
        out = F.linear(z, t[f"w_{key}"])
        if t[f"a_{key}"] is not None:
            out = out + ps[f"s_{key}"] * F.linear(F.linear(z, t[f"a_{key}"]), t[f"b_{key}"])
        return out

    h_mid = F.silu(proj(xl, "gate")) * proj(xl, "up")
    y = proj(h_mid, "down")
    y.backward(gy.detach().float())
    grads = {"grad_x": xl.grad}
    for k, tt in t.items():
        if tt is not None and tt.requires_grad:
            grads[k] = tt.grad
    return grads, y.detach()


def run_function_grads(fn_apply, ps: dict, x, gy, mode: str, group_size: int,
                       use_triton: bool = True, outlier_ratio: float = 0.0, *extra):
    """Run an FFN v3 Function (oracle or product) on leaf clones of `ps`.
    Mirrors src/verify_flashffn_v3.py:259-291.  `extra` are further trailing
    arguments of the Function (the oracle's outlier_idx / cache_override).
    Returns ({name: grad}, y)."""
    def leaf(t, rg):
        return None if t is None else t.detach().clone().requires_grad_(rg)

    xl = x.detach().clone().requires_grad_(True)
    t = {}
    for key in PROJ:
        t[f"w_{key}"] = leaf(ps[f"w_{key}"], ps["train_w"])
        has = ps[f"a_{key}"] is not None
        t[f"a_{key}"] = leaf(ps[f"a_{key}"], has)
        t[f"b_{key}"] = leaf(ps[f"b_{key}"], has)
    y = fn_apply(xl, t["w_gate"], t["a_gate"], t["b_gate"],
                 t["w_up"], t["a_up"], t["b_up"],
                 t["w_down"], t["a_down"], t["b_down"],
                 ps["s_gate"], ps["s_up"], ps["s_down"], mode, group_size, use_triton,
                 outlier_ratio, *extra)
    y.backward(gy)
    grads = {"grad_x": xl.grad}
    for k, tt in t.items():
        if tt is not None and tt.requires_grad:
            grads[k] = tt.grad
    return grads, y.detach()


def synthetic_param_set(config: str, h: int, d: int, rank: int, scaling: float,
                        seed: int, dtype=torch.bfloat16, device="cpu",
                        b_std: float = 0.02, peft_init: bool = False):
    """Seeded parameters after src/verify_flashffn_v3.py:150-182.

    config: 'all' (LoRA on gate/up/down) | 'gateup' | 'none' | 'fullft'.
    W ~ N(0, 0.02).  Adapters: A ~ randn/sqrt(in) (reference gate) or, with
    peft_init, kaiming-uniform(a=sqrt(5)) as nn.Linear/PEFT initialise it;
    B ~ N(0, b_std)."""
    g = torch.Generator().manual_seed(seed)
    ps = {"train_w": config == "fullft"}
    ps["w_gate"] = (torch.randn(d, h, generator=g) * 0.02).to(device, dtype)
    ps["w_up"] = (torch.randn(d, h, generator=g) * 0.02).to(device, dtype)
    ps["w_down"] = (torch.randn(h, d, generator=g) * 0.02).to(device, dtype)
    has = {"gate": config in ("all", "gateup"), "up": config in ("all", "gateup"),
           "down": config == "all"}
    for key, d_in, d_out in (("gate", h, d), ("up", h, d), ("down", d, h)):
        if has[key]:
            if peft_init:
                bound = 1.0 / np.sqrt(d_in)     # kaiming_uniform_(a=sqrt(5)) on [r, in]
                a = (torch.rand(rank, d_in, generator=g) * 2 - 1) * bound
            else:
                a = torch.randn(rank, d_in, generator=g) / np.sqrt(d_in)
            ps[f"a_{key}"] = a.to(device, dtype)
            ps[f"b_{key}"] = (torch.randn(d_out, rank, generator=g) * b_std).to(device, dtype)
            ps[f"s_{key}"] = scaling
        else:
            ps[f"a_{key}"] = ps[f"b_{key}"] = None
            ps[f"s_{key}"] = 0.0
    return ps


def tensor_cos(a, b) -> float:
    a, b = a.detach(), b.detach()
    return float(F.cosine_similarity(a.double().flatten(), b.double().flatten(), dim=0))


def rel_frob(a, b) -> float:
    a, b64 = a.detach(), b.detach().double()
    den = b64.norm()
    return float((a.double() - b64).norm() / den) if den > 0 else float((a.double()).norm())


def count_saved_bytes(forward_fn, param_ptrs):
    """src/verify_flashffn_v3.py:523-543: non-parameter bytes saved for
    backward, deduplicated by (data_ptr, nbytes).  Returns (total, entries)."""
    seen = set()
    entries = []
    total = 0

    def pack(t):
        nonlocal total
        key = (t.data_ptr(), t.nbytes)
        if t.data_ptr() in param_ptrs or key in seen:
            return t
        seen.add(key)
        total += t.nbytes
        entries.append({"shape": list(t.shape), "dtype": str(t.dtype), "bytes": t.nbytes})
        return t

    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        y = forward_fn()
    del y
    return total, entries


def int4_saved_bytes_closed_form(n: int, h: int, d: int, rank: int, group: int = 64,
                                 n_thin: int = 3, x_bytes_per: int = 2):
    """src/verify_flashffn_v3.py:598-600: x + 2*N*D/2 + 2*N*(D/g)*2 + 3*N*r*2."""
    return (n * h * x_bytes_per + 2 * (n * d // 2) + 2 * (n * (d // group) * 2)
            + n_thin * (n * rank * 2))


def saved_bytes_closed_form(n: int, h: int, d: int, bits: int, group: int,
                            n_thin: int = 0, rank: int = 0, x_bytes_per: int = 2,
                            n_outlier: int = 0):
    """Generalisation of the int4 closed form to int8 and outlier channels:
    x + 2 payloads + 2 fp16 scale arrays + thin [N,r] + 2 bf16 outlier blocks."""
    payload = n * d // 2 if bits == 4 else n * d
    return (n * h * x_bytes_per + 2 * payload + 2 * n * (d // group) * 2
            + n_thin * n * rank * 2 + 2 * n * n_outlier * 2)


# ---------------------------------------------------------------------------
# adapter families (src/flashffn.py:1697-2230)
# ---------------------------------------------------------------------------


@torch.no_grad()
def dora_col_norm(w, a, b, s):
    """src/flashffn.py:1824-1840: ||W + s*B@A||_2 over dim=1 through the
    Gram identity, in float32, without forming B@A."""
    wf, af, bf = w.float(), a.float(), b.float()
    w2 = (wf * wf).sum(dim=1)
    wa = wf @ af.t()
    cross = (2.0 * s) * (bf * wa).sum(dim=1)
    gram = af @ af.t()
    quad = (s * s) * ((bf @ gram) * bf).sum(dim=1)
    return (w2 + cross + quad).clamp_min_(0.0).sqrt_()


def dora_scale(h, m, nu):
    """src/flashffn.py:1967-1975: h * (m / nu).unsqueeze(0) in h's dtype."""
    return h * (m / nu).unsqueeze(0)


def col_dot_div(a, b, den):
    """src/flashffn.py:2086-2089: ((a * b).sum(0, fp32) / den.float()).to(den.dtype)."""
    return ((a * b).sum(0, dtype=torch.float32) / den.float()).to(den.dtype)


class OracleFlashFFNv3AdapterFunction(torch.autograd.Function):
    """CPU restatement of FlashFFNv3AdapterFunction (src/flashffn.py:1924-2208):
    the LoRA core plus DoRA's per-output-channel magnitude c = m / nu applied
    after the bypass.  Same argument list:
      apply(x, w_gate, a_gate, b_gate, m_gate, nu_gate,
            w_up, a_up, b_up, m_up, nu_up, w_down, a_down, b_down, m_down, nu_down,
            s_gate, s_up, s_down, cache_mode, group_size, use_triton)"""

    @staticmethod
    def forward(ctx, x, w_gate, a_gate, b_gate, m_gate, nu_gate, w_up, a_up, b_up, m_up, nu_up,
                w_down, a_down, b_down, m_down, nu_down, s_gate=0.0, s_up=0.0, s_down=0.0,
                cache_mode="int4", group_size=64, use_triton=True):
        assert cache_mode in ("int4", "int8", "bf16", "recompute"), cache_mode
        # torch's CPU bf16 matrix-vector product ignores the row stride of a
        # strided [K, 1] right operand (a DyLoRA rank-1 slice B[:, :1]);
        # contiguous copies of the thin factors keep their values and avoid it
        a_gate, b_gate, a_up, b_up, a_down, b_down = (
            None if t is None else t.contiguous()
            for t in (a_gate, b_gate, a_up, b_up, a_down, b_down))
        orig_shape = x.shape
        hidden_dim = x.shape[-1]
        x_2d = x.reshape(-1, hidden_dim)

        h_gate = F.linear(x_2d, w_gate)                                  # :1962-1967
        xa_g = None
        if a_gate is not None:
            xa_g = F.linear(x_2d, a_gate)
            h_gate = h_gate + s_gate * F.linear(xa_g, b_gate)
        if m_gate is not None:
            h_gate = dora_scale(h_gate, m_gate, nu_gate)
        h_up = F.linear(x_2d, w_up)                                      # :1969-1975
        xa_u = None
        if a_up is not None:
            xa_u = F.linear(x_2d, a_up)
            h_up = h_up + s_up * F.linear(xa_u, b_up)
        if m_up is not None:
            h_up = dora_scale(h_up, m_up, nu_up)

        c_gate = qs_gate = c_up = qs_up = None
        fused_quant = (cache_mode in ("int4", "int8") and use_triton
                       and h_gate.dtype == torch.bfloat16)               # :1979-1981
        if fused_quant:
            bits = 4 if cache_mode == "int4" else 8
            h_mid, c_gate, qs_gate, c_up, qs_up = triton_silu_mul_quant(
                h_gate, h_up, bits, group_size)
        else:
            h_mid = triton_silu_mul(h_gate, h_up)

        y = F.linear(h_mid, w_down)                                      # :1990-1996
        ha_d = None
        if a_down is not None:
            ha_d = F.linear(h_mid, a_down)
            y = y + s_down * F.linear(ha_d, b_down)
        if m_down is not None:
            y = dora_scale(y, m_down, nu_down)

        if not fused_quant:                                              # :1998-2007
            if cache_mode in ("int4", "int8"):
                bits = 4 if cache_mode == "int4" else 8
                c_gate, qs_gate = v3_quantize_group_absmax(h_gate, bits, group_size)
                c_up, qs_up = v3_quantize_group_absmax(h_up, bits, group_size)
            elif cache_mode == "bf16":
                c_gate, c_up = h_gate, h_up

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
        (x, w_gate, a_gate, b_gate, m_gate, nu_gate, w_up, a_up, b_up, m_up, nu_up,
         w_down, a_down, b_down, m_down, nu_down,
         xa_g, xa_u, ha_d, cq_gate, qs_gate, cq_up, qs_up) = ctx.saved_tensors
        s_gate, s_up, s_down = ctx.s
        mode = ctx.cache_mode
        hidden_dim = ctx.orig_shape[-1]
        ng = ctx.needs_input_grad
        need_x = ng[0]
        need_wg, need_ag, need_bg, need_mg = ng[1], ng[2], ng[3], ng[4]
        need_wu, need_au, need_bu, need_mu = ng[6], ng[7], ng[8], ng[9]
        need_wd, need_ad, need_bd, need_md = ng[11], ng[12], ng[13], ng[14]
        gy = grad_y.reshape(-1, hidden_dim)
        x_2d = x.reshape(-1, hidden_dim)
        bits = 4 if mode == "int4" else 8

        need_gate_path = (need_x or need_wg or need_ag or need_bg or need_mg
                          or need_wu or need_au or need_bu or need_mu)   # :2047-2048
        need_h_mid = need_wd or need_md or (a_down is not None and need_ad)
        need_recon = need_gate_path or need_h_mid
        use_k2 = mode in ("int4", "int8") and ctx.use_triton and need_gate_path

        hg = hu = raw_g = raw_u = None
        if need_recon and not use_k2:                                    # :2055-2078
            if mode == "recompute":
                raw_g = F.linear(x_2d, w_gate)
                if a_gate is not None:
                    raw_g = raw_g + s_gate * F.linear(xa_g, b_gate)
                hg = dora_scale(raw_g, m_gate, nu_gate) if m_gate is not None else raw_g
                raw_u = F.linear(x_2d, w_up)
                if a_up is not None:
                    raw_u = raw_u + s_up * F.linear(xa_u, b_up)
                hu = dora_scale(raw_u, m_up, nu_up) if m_up is not None else raw_u
            elif mode == "bf16":
                hg, hu = cq_gate, cq_up
            else:
                hg = v3_dequantize_group_absmax(cq_gate, qs_gate, bits, ctx.group_size,
                                                ctx.in_dtype)
                hu = v3_dequantize_group_absmax(cq_up, qs_up, bits, ctx.group_size,
                                                ctx.in_dtype)
        elif use_k2 and (need_mg or need_mu):                            # :2079-2089
            if need_mg:
                hg = v3_dequantize_group_absmax(cq_gate, qs_gate, bits, ctx.group_size,
                                                ctx.in_dtype)
            if need_mu:
                hu = v3_dequantize_group_absmax(cq_up, qs_up, bits, ctx.group_size,
                                                ctx.in_dtype)

        g_eff_y = dora_scale(gy, m_down, nu_down) if m_down is not None else gy   # :2094
        gyB_d = None
        if a_down is not None and (need_gate_path or need_ad):
            gyB_d = g_eff_y @ b_down

        grad_h_gate = grad_h_up = h_mid_hat = None
        if use_k2:                                                       # :2101-2110
            grad_h_mid = g_eff_y @ w_down
            if a_down is not None:
                grad_h_mid = grad_h_mid + s_down * (gyB_d @ a_down)
            grad_h_gate, grad_h_up, h_mid_hat = triton_dequant_swiglu_backward(
                grad_h_mid, cq_gate, qs_gate, cq_up, qs_up, bits, ctx.group_size,
                want_h_mid=need_h_mid)

        grad_w_down = grad_a_down = grad_b_down = grad_m_down = None
        if need_h_mid:                                                   # :2112-2131
            if h_mid_hat is None:
                h_mid_hat = triton_silu_mul(hg, hu)
            if need_wd:
                grad_w_down = g_eff_y.t() @ h_mid_hat
            if need_ad:
                grad_a_down = s_down * (gyB_d.t() @ h_mid_hat)
            if need_md:
                raw_d = F.linear(h_mid_hat, w_down)
                if a_down is not None:
                    raw_d = raw_d + s_down * F.linear(ha_d, b_down)
                grad_m_down = col_dot_div(gy, raw_d, nu_down)
        if need_bd:
            grad_b_down = s_down * (g_eff_y.t() @ ha_d)

        grad_x = None
        grad_w_gate = grad_a_gate = grad_b_gate = grad_m_gate = None
        grad_w_up = grad_a_up = grad_b_up = grad_m_up = None
        if need_gate_path:                                               # :2134-2191
            if grad_h_gate is None:
                grad_h_mid = g_eff_y @ w_down
                if a_down is not None:
                    grad_h_mid = grad_h_mid + s_down * (gyB_d @ a_down)
                grad_h_gate, grad_h_up = triton_swiglu_backward(grad_h_mid, hg, hu)
            if need_mg:
                grad_m_gate = (col_dot_div(grad_h_gate, raw_g, nu_gate) if raw_g is not None
                               else col_dot_div(grad_h_gate, hg, m_gate))
            if need_mu:
                grad_m_up = (col_dot_div(grad_h_up, raw_u, nu_up) if raw_u is not None
                             else col_dot_div(grad_h_up, hu, m_up))
            g_eff_g = dora_scale(grad_h_gate, m_gate, nu_gate) if m_gate is not None else grad_h_gate
            g_eff_u = dora_scale(grad_h_up, m_up, nu_up) if m_up is not None else grad_h_up
            ghgB = g_eff_g @ b_gate if a_gate is not None and (need_x or need_ag) else None
            ghuB = g_eff_u @ b_up if a_up is not None and (need_x or need_au) else None
            if need_x:
                grad_x = g_eff_g @ w_gate
                if a_gate is not None:
                    grad_x = grad_x + s_gate * (ghgB @ a_gate)
                grad_x = grad_x + g_eff_u @ w_up
                if a_up is not None:
                    grad_x = grad_x + s_up * (ghuB @ a_up)
            if need_bg:
                grad_b_gate = s_gate * (g_eff_g.t() @ xa_g)
            if need_ag:
                grad_a_gate = s_gate * (ghgB.t() @ x_2d)
            if need_bu:
                grad_b_up = s_up * (g_eff_u.t() @ xa_u)
            if need_au:
                grad_a_up = s_up * (ghuB.t() @ x_2d)
            if need_wg:
                grad_w_gate = g_eff_g.t() @ x_2d
            if need_wu:
                grad_w_up = g_eff_u.t() @ x_2d

        if need_x and len(ctx.orig_shape) == 3:
            grad_x = grad_x.view(ctx.orig_shape)
        return (grad_x,
                grad_w_gate, grad_a_gate, grad_b_gate, grad_m_gate, None,
                grad_w_up, grad_a_up, grad_b_up, grad_m_up, None,
                grad_w_down, grad_a_down, grad_b_down, grad_m_down, None,
                ) + (None,) * (len(ctx.needs_input_grad) - 16)


ADAPTER_KINDS = ("dora", "adalora", "vera", "dylora")


def synthetic_adapter_set(kind: str, h: int, d: int, rank: int, alpha: float, seed: int,
                          dtype=torch.bfloat16):
    """Seeded raw parameters of one adapter family on gate/up/down, after the
    reference's non-degenerate initialisation (src/verify_v3_adapters.py:101-149):
    W ~ N(0, 0.02); B ~ N(0, 0.02); DoRA m = ||W_j|| * (1 + 0.2 N(0, 1));
    AdaLoRA E ~ N(0, 0.5), ranknum = rank; VeRA lambda_d = 0.1 + 0.05 N,
    lambda_b ~ N(0, 0.05) with shared frozen A, B; DyLoRA ranks b per projection."""
    g = torch.Generator().manual_seed(seed)
    ps = {"kind": kind}
    dims = {"gate": (h, d), "up": (h, d), "down": (d, h)}
    for key, (d_in, d_out) in dims.items():
        w = torch.randn(d_out, d_in, generator=g) * 0.02
        p = {"w": w.to(dtype)}
        bound = 1.0 / np.sqrt(d_in)
        a = (torch.rand(rank, d_in, generator=g) * 2 - 1) * bound
        b = torch.randn(d_out, rank, generator=g) * 0.02
        if kind == "dora":
            p["a"], p["b"], p["s"] = a.to(dtype), b.to(dtype), alpha / rank
            m = w.to(dtype).float().norm(dim=1) * (1.0 + 0.2 * torch.randn(d_out, generator=g))
            p["m"] = m.to(dtype)
        elif kind == "adalora":
            p["a"], p["b"] = a.to(dtype), b.to(dtype)
            p["e"] = (torch.randn(rank, 1, generator=g) * 0.5).to(dtype)
            p["s_eff"] = (alpha / rank) / (float(rank) + 1e-5)
        elif kind == "vera":
            p["a_frozen"], p["b_frozen"] = a.to(dtype), b.to(dtype)
            p["lam_d"] = (0.1 + 0.05 * torch.randn(rank, generator=g)).to(dtype)
            p["lam_b"] = (torch.randn(d_out, generator=g) * 0.05).to(dtype)
        elif kind == "dylora":
            p["a"], p["b"], p["s"] = a.to(dtype), b.to(dtype), alpha / rank
            p["b_rank"] = int(torch.randint(1, rank + 1, (1,), generator=g))
        else:
            raise ValueError(kind)
        ps[key] = p
    return ps


def adapter_trainables(ps):
    """name -> tensor of every trainable adapter parameter (reference
    src/verify_v3_adapters.py:153-176)."""
    names = {"dora": ("a", "b", "m"), "adalora": ("a", "e", "b"), "vera": ("lam_d", "lam_b"),
             "dylora": ("a", "b")}[ps["kind"]]
    return {f"{key}.{n}": ps[key][n] for key in PROJ for n in names}


def adapter_factors(p, kind, leaves):
    """The Function's factored arguments (w, a, b, s, m, nu) of one
    projection from leaf tensors, composed in autograd like
    _v3_extract_proj_adapter (src/flashffn.py:1850-1921).  `leaves` maps the
    raw names of `p` to (possibly grad-tracking) tensors."""
    w = p["w"]
    if kind == "dora":
        a, b, s, m = leaves["a"], leaves["b"], p["s"], leaves["m"]
        nu = dora_col_norm(w, a.detach(), b.detach(), s).to(w.dtype)
        return w, a, b, s, m, nu
    if kind == "adalora":
        return w, leaves["a"] * leaves["e"], leaves["b"], p["s_eff"], None, None
    if kind == "vera":
        a_eff = leaves["lam_d"].unsqueeze(-1) * p["a_frozen"]
        b_eff = leaves["lam_b"].unsqueeze(-1) * p["b_frozen"]
        return w, a_eff, b_eff, 1.0, None, None
    if kind == "dylora":
        r = p["b_rank"]
        return w, leaves["a"][:r, :], leaves["b"][:, :r], p["s"], None, None
    raise ValueError(kind)


def run_adapter_grads(fn_apply, ps, x, gy, mode: str, group_size: int, use_triton: bool = True):
    """Run an adapter Function (oracle or product) on leaf clones of the
    trainables of `ps` (their device is x's).  Returns ({name: grad}, y)."""
    kind = ps["kind"]
    xl = x.detach().clone().requires_grad_(True)
    leaves, args = {}, []
    for key in PROJ:
        p = {k: (v.to(x.device) if isinstance(v, torch.Tensor) else v) for k, v in ps[key].items()}
        lv = {n: p[n].detach().clone().requires_grad_(True)
              for n in ("a", "b", "m", "e", "lam_d", "lam_b") if n in p
              and not (kind == "vera" and n in ("a", "b"))}
        for n, t in lv.items():
            leaves[f"{key}.{n}"] = t
        w, a, b, s, m, nu = adapter_factors(p, kind, lv)
        args.append((w, a, b, m, nu, s))
    (wg, ag, bg, mg, nug, sg), (wu, au, bu, mu, nuu, su), (wd, ad, bd, md, nud, sd) = args
    y = fn_apply(xl, wg, ag, bg, mg, nug, wu, au, bu, mu, nuu, wd, ad, bd, md, nud,
                 sg, su, sd, mode, group_size, use_triton)
    y.backward(gy)
    grads = {"grad_x": xl.grad}
    for k, t in leaves.items():
        grads[k] = t.grad
    return grads, y.detach()


def ref_adapter_grads_fp32(ps, x, gy):
    """fp32 plain autograd of the adapter families' own forward
    (src/verify_v3_adapters.py:204-258): DoRA c = m / ||W + s B A||.detach()
    (PEFT DoraLinearLayer), AdaLoRA (A*E) with s / (ranknum + 1e-5), VeRA
    lambda_b * ((x A^T) * lambda_d) B^T, DyLoRA rank-b slices."""
    kind = ps["kind"]
    xl = x.detach().float().requires_grad_(True)
    leaves = {}

    def leaf(key, n):
        t = ps[key][n].detach().float().requires_grad_(True)
        leaves[f"{key}.{n}"] = t
        return t

    def proj(z, key):
        p = ps[key]
        w = p["w"].float()
        if kind == "dora":
            a, b, m = leaf(key, "a"), leaf(key, "b"), leaf(key, "m")
            nu = (w + p["s"] * (b @ a)).detach().norm(p=2, dim=1)
            raw = F.linear(z, w) + p["s"] * F.linear(F.linear(z, a), b)
            return raw * (m / nu).unsqueeze(0)
        if kind == "adalora":
            a, e, b = leaf(key, "a"), leaf(key, "e"), leaf(key, "b")
            return F.linear(z, w) + p["s_eff"] * F.linear(F.linear(z, a * e), b)
        if kind == "vera":
            ld, lb = leaf(key, "lam_d"), leaf(key, "lam_b")
            u = F.linear(z, p["a_frozen"].float()) * ld
            return F.linear(z, w) + F.linear(u, p["b_frozen"].float()) * lb
        if kind == "dylora":
            a, b = leaf(key, "a"), leaf(key, "b")
            r = p["b_rank"]
            return F.linear(z, w) + p["s"] * F.linear(F.linear(z, a[:r, :]), b[:, :r])
        raise ValueError(kind)

    h_mid = F.silu(proj(xl, "gate")) * proj(xl, "up")
    y = proj(h_mid, "down")
    y.backward(gy.detach().float())
    grads = {"grad_x": xl.grad}
    grads.update({k: t.grad for k, t in leaves.items()})
    return grads, y.detach()


# ---------------------------------------------------------------------------
# v1/v2 API with top-K compression (src/flashffn.py:300-519)
# ---------------------------------------------------------------------------


def topk_abs(t: torch.Tensor, k: int):
    """Per row: the k entries of largest |t| in ascending column order, ties
    at the k-th magnitude to the lowest columns (a fixed choice of
    `torch.topk(t.abs(), k, sorted=False)`, src/flashffn.py:353-356).
    Returns (values in t's dtype, indices int16)."""
    a = to_f32(t)
    n, d = a.shape
    mag = np.abs(a)
    cols = np.broadcast_to(np.arange(d), (n, d))
    # descending magnitude, then ascending column (lexsort: last key is primary)
    order = np.lexsort((cols, -mag), axis=1)[:, :k]
    order.sort(axis=1)
    vals = np.take_along_axis(t.detach().cpu().contiguous().view(-1, d).numpy()
                              if t.dtype == torch.float32 else
                              t.detach().cpu().contiguous().view(torch.int16).numpy(),
                              order, axis=1)
    values = torch.from_numpy(np.ascontiguousarray(vals))
    if t.dtype != torch.float32:
        values = values.view(t.dtype)
    return values, torch.from_numpy(order.astype(np.int16))


def topk_scatter(values: torch.Tensor, indices: torch.Tensor, d: int):
    """src/flashffn.py:410-415: zeros [N, d] with values scattered at indices."""
    out = torch.zeros(values.shape[0], d, dtype=values.dtype)
    out.scatter_(-1, indices.long(), values)
    return out


class OracleFlashFFNFunction(torch.autograd.Function):
    """CPU restatement of FlashFFNFunction (src/flashffn.py:300-449): mode by
    the weights' requires_grad; 'recompute' keeps the top-K of h_mid and
    recomputes h_gate / h_up, 'activations' keeps h_gate / h_up."""

    @staticmethod
    def forward(ctx, x, w_gate, w_up, w_down, k_fraction=0.3):
        orig_shape = x.shape
        hidden_dim = x.shape[-1]
        inter = w_gate.shape[0]
        x_2d = x.reshape(-1, hidden_dim)
        h_gate = F.linear(x_2d, w_gate)
        h_up = F.linear(x_2d, w_up)
        h_mid = triton_silu_mul(h_gate, h_up)
        y = F.linear(h_mid, w_down)
        if w_gate.requires_grad or w_up.requires_grad or w_down.requires_grad:
            k = max(1, int(inter * k_fraction))
            values, indices = topk_abs(h_mid, k)
            ctx.save_for_backward(x, w_gate, w_up, w_down, values, indices)
            ctx.save_mode = "recompute"
            ctx.intermediate_dim = inter
        else:
            ctx.save_for_backward(h_gate, h_up, w_gate, w_up, w_down)
            ctx.save_mode = "activations"
        ctx.orig_shape = orig_shape
        if len(orig_shape) == 3:
            y = y.view(orig_shape[0], orig_shape[1], hidden_dim)
        return y

    @staticmethod
    def backward(ctx, grad_output):
        orig_shape = ctx.orig_shape
        hidden_dim = orig_shape[-1]
        gy = grad_output.reshape(-1, hidden_dim)
        if ctx.save_mode == "activations":
            h_gate, h_up, w_gate, w_up, w_down = ctx.saved_tensors
            dg, du = triton_swiglu_backward(gy @ w_down, h_gate, h_up)
            grad_x = dg @ w_gate + du @ w_up
            if len(orig_shape) == 3:
                grad_x = grad_x.view(orig_shape)
            return grad_x, None, None, None, None
        x, w_gate, w_up, w_down, values, indices = ctx.saved_tensors
        x_2d = x.reshape(-1, hidden_dim)
        need_x, need_wg, need_wu, need_wd = ctx.needs_input_grad[:4]
        grad_w_down = None
        if need_wd:
            grad_w_down = gy.t() @ topk_scatter(values, indices, ctx.intermediate_dim)
        grad_x = grad_w_gate = grad_w_up = None
        if need_x or need_wg or need_wu:
            dg, du = triton_swiglu_backward(gy @ w_down, F.linear(x_2d, w_gate),
                                            F.linear(x_2d, w_up))
            grad_w_gate = dg.t() @ x_2d if need_wg else None
            grad_w_up = du.t() @ x_2d if need_wu else None
            grad_x = dg @ w_gate + du @ w_up if need_x else None
        if need_x and len(orig_shape) == 3:
            grad_x = grad_x.view(orig_shape)
        return grad_x, grad_w_gate, grad_w_up, grad_w_down, None
