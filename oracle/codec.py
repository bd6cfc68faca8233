"""numpy restatement of the FlashFFN v3 codec and GLU math (CPU oracle).

TEST INFRASTRUCTURE ONLY -- imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline, never by the product.

Every function states the reference lines it restates (paths relative to the
reference repo root, SDMuhsin/CompAct).  Arithmetic is float32 throughout, as
in the reference: numpy's float32 `/` is IEEE correctly rounded (the
reference's `torch` division and Triton `div_rn`), `np.rint` is
round-half-to-even (`torch.round`, libdevice `rint`), and `astype(float16)` is
round-to-nearest-even with subnormals and overflow to +-inf (`.to(float16)`).
bf16 has no numpy dtype: bf16 tensors travel as their uint16 bit patterns and
are rounded by `f32_to_bf16_bits` (RNE, NaN -> 0x7FC0, torch's convention).

Parity status (how each function is pinned; see tests/test_oracle_codec.py):
  quantize_group_absmax / dequantize_group_absmax  pinned: hand-computed
      known-answer vectors (half-even ties, nibble order, fp16-rounded scale,
      fp16-subnormal scale + clamp, fp16 overflow), exact-rational brute force
      (oracle/exact.py), and bit-exact agreement with the independent C
      restatement (oracle/codec_ref.c).
  silu_mul / swiglu_backward   pinned to float64 autograd of silu(g)*u.
  silu_mul_quant / dequant_swiglu_backward   compositions of the above (the
      reference's own K1/K2 contract, flashffn.py:1129-1137).
  outlier_* (zero-and-overwrite outlier channels)   the reference has no
      combination of per-group codec + outlier channels; the semantics are
      this build's specification (HyC-LoRA zero-and-overwrite,
      hyclora/operators/compress_function.py:80-105,147-174), pinned by
      invariants (outlier columns round-trip bit-exactly, the rest equals the
      plain codec of the zeroed tensor) -- parity unpinned against the reference.
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# bit-level helpers
# ---------------------------------------------------------------------------


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Widen bf16 bit patterns (uint16) to float32 exactly."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 (round-to-nearest-even), returning uint16 bits.

    NaN maps to 0x7FC0 as in c10::BFloat16's round_to_nearest_even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = 0x7FC0
    return r


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 -> float32 round trip."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def _qmax(bits: int) -> np.float32:
    return np.float32(2 ** (bits - 1) - 1)


def check_codec_args(shape, bits: int, group_size: int, need_pow2: bool = False):
    """The reference's argument contract: the eager codec asserts bits in
    {4, 8} and D divisible by group_size (flashffn.py:1070-1072); the fused
    K1/K2 wrappers also require a power-of-two group_size (:1303-1311)."""
    assert bits in (4, 8), f"unsupported bits={bits}"
    assert len(shape) == 2, "expected [N, D]"
    n, d = shape
    assert d % group_size == 0, f"D={d} not divisible by group_size={group_size}"
    if need_pow2:
        assert group_size > 0 and (group_size & (group_size - 1)) == 0, \
            f"group_size={group_size} must be a power of two"
    return n, d, d // group_size


# ---------------------------------------------------------------------------
# a1 / a2: per-group absmax codec
# ---------------------------------------------------------------------------


def quantize_group_absmax(t: np.ndarray, bits: int, group_size: int = 64):
    """Restates `v3_quantize_group_absmax` (flashffn.py:1055-1088).

    t: float32 [N, D] (the input already widened to fp32, `.float()` at :1075).
    Returns (payload, scales):
      bits=4: uint8 [N, D/2], code q+8 of the even column in the low nibble and
              of the odd column in the high nibble (:1081-1085);
      bits=8: int8 [N, D] (:1087);
      scales: float16 [N, D/group_size] = fp16(fp32(absmax / qmax)) (:1076-1077).
    Codes are rint(fp32(t / safe)) clamped to +-qmax, where safe is the
    fp16-rounded scale widened to fp32, or 1 where that scale is 0 (:1078-1080).
    """
    t = np.ascontiguousarray(t, dtype=np.float32)
    n, d, g = check_codec_args(t.shape, bits, group_size)
    qmax = _qmax(bits)
    tg = t.reshape(n, g, group_size)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        absmax = np.abs(tg).max(axis=-1, keepdims=True) if n * d else \
            np.zeros((n, g, 1), np.float32)
        scales = (absmax / qmax).astype(np.float16)
        safe = scales.astype(np.float32)
        safe = np.where(safe > 0, safe, np.float32(1.0))
        q = np.rint(tg / safe)
        q = np.clip(q, -qmax, qmax)
    if bits == 4:
        q8 = (q.reshape(n, d) + np.float32(8.0)).astype(np.uint8)
        payload = (q8[:, 0::2] | (q8[:, 1::2] << 4)).astype(np.uint8)
    else:
        payload = q.reshape(n, d).astype(np.int8)
    return payload, scales.reshape(n, g)


def unpack_codes(payload: np.ndarray, bits: int) -> np.ndarray:
    """Signed integer codes [N, D] from a payload (inverse of the packing)."""
    if bits == 8:
        return payload.astype(np.int32)
    lo = (payload & 0x0F).astype(np.int32) - 8
    hi = (payload >> 4).astype(np.int32) - 8
    return np.stack((lo, hi), axis=-1).reshape(payload.shape[0], -1)


def dequantize_group_absmax_f32(payload: np.ndarray, scales: np.ndarray,
                                bits: int, group_size: int = 64) -> np.ndarray:
    """Restates `v3_dequantize_group_absmax` up to (not including) its final
    `.to(dtype)` (flashffn.py:1099-1109): code * fp32(scale), in float32."""
    if bits == 4:
        n, half = payload.shape
        d = 2 * half
        lo = (payload & 0x0F).astype(np.float32) - np.float32(8.0)
        hi = (payload >> 4).astype(np.float32) - np.float32(8.0)
        q = np.stack((lo, hi), axis=-1).reshape(n, d)
    else:
        n, d = payload.shape
        q = payload.astype(np.float32)
    g = d // group_size
    with np.errstate(invalid="ignore", over="ignore"):
        deq = q.reshape(n, g, group_size) * scales.reshape(n, g, 1).astype(np.float32)
    return deq.reshape(n, d)


def dequantize_group_absmax_bf16(payload, scales, bits, group_size=64):
    """`v3_dequantize_group_absmax(..., dtype=bf16)` (flashffn.py:1110): the
    float32 product rounded to bf16 (uint16 bits)."""
    return f32_to_bf16_bits(dequantize_group_absmax_f32(payload, scales, bits, group_size))


# ---------------------------------------------------------------------------
# a5: GLU elementwise math (float32, reference op order)
# ---------------------------------------------------------------------------


def sigmoid_f32(x: np.ndarray) -> np.ndarray:
    """tl.sigmoid(x) = 1 / (1 + exp(-x)) in float32."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (np.float32(1.0) / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """`_silu_mul_fwd_kernel` arithmetic (flashffn.py:71-76): act = g*sigmoid(g);
    result = act*u, float32 (the caller rounds to the storage dtype)."""
    g = np.asarray(g, dtype=np.float32)
    u = np.asarray(u, dtype=np.float32)
    act = g * sigmoid_f32(g)
    return (act * u).astype(np.float32)


def swiglu_backward(dh: np.ndarray, g: np.ndarray, u: np.ndarray):
    """`_swiglu_bwd_kernel` arithmetic (flashffn.py:109-123), float32.
    Returns (grad_h_gate, grad_h_up)."""
    dh = np.asarray(dh, dtype=np.float32)
    g = np.asarray(g, dtype=np.float32)
    u = np.asarray(u, dtype=np.float32)
    one = np.float32(1.0)
    sig = sigmoid_f32(g)
    h_act = g * sig
    grad_h_act = dh * u
    grad_h_up = dh * h_act
    dsilu = sig * (one + g * (one - sig))
    grad_h_gate = grad_h_act * dsilu
    return grad_h_gate.astype(np.float32), grad_h_up.astype(np.float32)


# ---------------------------------------------------------------------------
# a3 / a4: the K1 / K2 contracts
# ---------------------------------------------------------------------------


def silu_mul_quant(g: np.ndarray, u: np.ndarray, bits: int, group_size: int = 64):
    """K1 contract (flashffn.py:1116-1122,1314-1319): h_mid = silu_mul(g, u)
    plus the codec of BOTH g and u.  g, u: float32 values of the bf16 inputs.
    Returns (h_mid_f32, q_gate, s_gate, q_up, s_up); the caller rounds h_mid."""
    check_codec_args(np.shape(g), bits, group_size, need_pow2=True)
    qg, sg = quantize_group_absmax(g, bits, group_size)
    qu, su = quantize_group_absmax(u, bits, group_size)
    return silu_mul(g, u), qg, sg, qu, su


def dequant_swiglu_backward(gmid: np.ndarray, qg, sg, qu, su, bits: int,
                            group_size: int = 64, want_h_mid: bool = False):
    """K2 contract (flashffn.py:1123-1127,1343-1349): dequantize both caches
    rounding through bf16 (:1251-1253), then swiglu_backward, and optionally
    h_mid^ = silu_mul(hg^, hu^).  gmid: float32 values of bf16 grad_h_mid.
    Returns float32 (grad_h_gate, grad_h_up, h_mid_hat | None)."""
    hg = bf16_bits_to_f32(dequantize_group_absmax_bf16(qg, sg, bits, group_size))
    hu = bf16_bits_to_f32(dequantize_group_absmax_bf16(qu, su, bits, group_size))
    dg, du = swiglu_backward(gmid, hg, hu)
    hm = silu_mul(hg, hu) if want_h_mid else None
    return dg, du, hm


# ---------------------------------------------------------------------------
# Outlier-channel extension (config C3): this build's specification.
# ---------------------------------------------------------------------------


def outlier_channels(h: np.ndarray, ratio: float, rows: int | None = None) -> np.ndarray:
    """Channel selection after HyC-LoRA's `get_statistics_channel_base`
    (hyclora/operators/compress_function.py:80-88): the int(D*ratio) channels
    with the largest L2 norm over the first sample's tokens,
    `x_[0].abs().norm(dim=-2)` (:85).  h is the [N, D] matrix; `rows` is the
    first sample's row count (None: all rows, a 2-D input being one sample).
    Spec of this build where HyC-LoRA leaves it open: the norm is taken in
    float64; ties go to the lower channel index; the result is sorted
    ascending (slot i of the outlier buffer holds channel idx[i])."""
    h = np.asarray(h, dtype=np.float64)
    k = int(h.shape[1] * ratio)
    if k == 0:
        return np.zeros((0,), np.int32)
    if rows is not None:
        h = h[:rows]
    norms = np.sqrt((h * h).sum(axis=0))
    order = np.lexsort((np.arange(h.shape[1]), -norms))
    return np.sort(order[:k]).astype(np.int32)


def outlier_quantize(t: np.ndarray, t_bf16_bits: np.ndarray, idx: np.ndarray,
                     bits: int, group_size: int):
    """Zero-and-store outlier codec (spec; compress_function.py:111-143 for
    the zeroing): columns `idx` are copied out as bf16 [N, k] and set to 0,
    then the per-group absmax codec runs on the result.
    Returns (payload, scales, outlier_bits uint16 [N, k])."""
    t = np.array(t, dtype=np.float32, copy=True)
    out = np.ascontiguousarray(np.asarray(t_bf16_bits, np.uint16)[:, idx])
    t[:, idx] = 0.0
    q, s = quantize_group_absmax(t, bits, group_size)
    return q, s, out


def outlier_dequantize_bf16(payload, scales, outlier_bits, idx, bits, group_size):
    """Inverse (spec; compress_function.py:147-174 for the overwrite):
    dequantize through bf16, then overwrite columns `idx` with the stored
    bf16 values.  Returns uint16 bf16 bits [N, D]."""
    deq = dequantize_group_absmax_bf16(payload, scales, bits, group_size)
    deq[:, idx] = outlier_bits
    return deq
