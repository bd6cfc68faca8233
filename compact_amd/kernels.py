"""torch-facing wrappers of the HIP kernels, with the reference's names and
argument contracts (src/flashffn.py:205-293, 1055-1110, 1303-1373).

Each wrapper validates its arguments the way the reference does (assert),
allocates its outputs with torch on the input's device (the C ABI never
allocates), and launches on torch's current stream.  Inputs must be HIP
device tensors: there is no CPU path.

The reference's Triton-era names (`triton_silu_mul_quant`, ...) are kept as
aliases so callers of the reference swap in unchanged; `use_triton` in the
Function API keeps its meaning "use the fused device kernels".
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import check

_DT = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}

# Honesty counters (src/flashffn.py:1040-1042): prove which path ran.
# quant_fwd / dequant_bwd count executions of the fused K1 / K2 kernels.
_V3_COUNTERS = {"forward": 0, "backward": 0,
                "triton_quant_fwd": 0, "triton_dequant_bwd": 0,
                "adapter_forward": 0, "adapter_backward": 0}


def v3_reset_counters():
    for k in _V3_COUNTERS:
        _V3_COUNTERS[k] = 0


def _stream(t: torch.Tensor):
    return torch.cuda.current_stream(t.device).cuda_stream


class KernelTimer:
    """Opt-in per-kernel timing with HIP events recorded on the stream each
    kernel is launched on.  `with KernelTimer() as kt: ...` collects
    (start, end) event pairs per kernel name; `kt.avg_ms()` reads them after
    a synchronize.  Disabled (zero events) outside the context."""

    active = None

    def __init__(self):
        self.events = {}

    def __enter__(self):
        KernelTimer.active = self
        return self

    def __exit__(self, *exc):
        KernelTimer.active = None

    def avg_ms(self):
        out = {}
        for name, pairs in self.events.items():
            ts = [a.elapsed_time(b) for a, b in pairs]
            out[name] = {"calls": len(ts), "avg_ms": sum(ts) / len(ts), "total_ms": sum(ts)}
        return out


class _timed:
    __slots__ = ("name", "ev")

    def __init__(self, name):
        self.name = name
        self.ev = None

    def __enter__(self):
        if KernelTimer.active is not None:
            self.ev = torch.cuda.Event(enable_timing=True)
            self.ev.record(torch.cuda.current_stream())
        return self

    def __exit__(self, *exc):
        kt = KernelTimer.active
        if self.ev is not None and kt is not None:
            end = torch.cuda.Event(enable_timing=True)
            end.record(torch.cuda.current_stream())
            kt.events.setdefault(self.name, []).append((self.ev, end))


def _ptr(t):
    return None if t is None else t.data_ptr()


def _require_device(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("compact_amd kernels run on the HIP device only; got a CPU tensor")


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype not in _DT:
        raise AssertionError(f"unsupported dtype {t.dtype}")
    return _DT[t.dtype]


# ---------------------------------------------------------------------------
# GLU elementwise (src/flashffn.py:205-293)
# ---------------------------------------------------------------------------

def silu_mul(h_gate: torch.Tensor, h_up: torch.Tensor) -> torch.Tensor:
    """SiLU(h_gate) * h_up in float32, stored in h_gate's dtype
    (`triton_silu_mul`, src/flashffn.py:205-220)."""
    _require_device(h_gate, h_up)
    assert h_up.shape == h_gate.shape and h_up.dtype == h_gate.dtype
    h_gate, h_up = h_gate.contiguous(), h_up.contiguous()
    out = torch.empty_like(h_gate)
    check(_lib.lib().cpt_silu_mul(h_gate.data_ptr(), h_up.data_ptr(), out.data_ptr(),
                                  h_gate.numel(), _dtype_code(h_gate), _stream(h_gate)),
          "silu_mul")
    return out


def swiglu_backward(grad_h_mid, h_gate, h_up):
    """(grad_h_gate, grad_h_up) through h_mid = SiLU(h_gate)*h_up
    (`triton_swiglu_backward`, src/flashffn.py:223-239)."""
    _require_device(grad_h_mid, h_gate, h_up)
    assert h_gate.shape == h_up.shape == grad_h_mid.shape
    assert h_gate.dtype == h_up.dtype == grad_h_mid.dtype
    grad_h_mid, h_gate, h_up = grad_h_mid.contiguous(), h_gate.contiguous(), h_up.contiguous()
    dg = torch.empty_like(h_gate)
    du = torch.empty_like(h_up)
    check(_lib.lib().cpt_swiglu_backward(grad_h_mid.data_ptr(), h_gate.data_ptr(),
                                         h_up.data_ptr(), dg.data_ptr(), du.data_ptr(),
                                         h_gate.numel(), _dtype_code(h_gate), _stream(h_gate)),
          "swiglu_backward")
    return dg, du


def swiglu_backward_glu(grad_h_mid, h_gate, h_up, want_h_mid, inplace=False):
    """SwiGLU backward plus the h_mid rematerialisation in one pass
    (`triton_swiglu_backward_glu`, src/flashffn.py:259-293).  `inplace=True`
    writes grad_h_gate over h_gate, grad_h_up over h_up and h_mid over
    grad_h_mid (inputs must be contiguous and private to the caller).
    Returns (grad_h_gate, grad_h_up, h_mid | None)."""
    _require_device(grad_h_mid, h_gate, h_up)
    assert h_gate.shape == h_up.shape == grad_h_mid.shape
    assert h_gate.dtype == h_up.dtype == grad_h_mid.dtype
    if inplace:
        assert grad_h_mid.is_contiguous() and h_gate.is_contiguous() and h_up.is_contiguous()
        dg, du = h_gate, h_up
        hm = grad_h_mid if want_h_mid else None
    else:
        grad_h_mid, h_gate, h_up = grad_h_mid.contiguous(), h_gate.contiguous(), h_up.contiguous()
        dg = torch.empty_like(h_gate)
        du = torch.empty_like(h_up)
        hm = torch.empty_like(h_gate) if want_h_mid else None
    check(_lib.lib().cpt_swiglu_backward_glu(grad_h_mid.data_ptr(), h_gate.data_ptr(),
                                             h_up.data_ptr(), dg.data_ptr(), du.data_ptr(),
                                             _ptr(hm), h_gate.numel(), _dtype_code(h_gate),
                                             _stream(h_gate)),
          "swiglu_backward_glu")
    return dg, du, hm


# ---------------------------------------------------------------------------
# codec (src/flashffn.py:1055-1110)
# ---------------------------------------------------------------------------

def v3_quantize_group_absmax(t: torch.Tensor, bits: int, group_size: int = 64):
    """Per-group absmax quantisation along the last dim
    (src/flashffn.py:1055-1088).  t: [N, D] float tensor.  Returns
    (payload uint8 [N, D/2] | int8 [N, D], scales fp16 [N, D/group_size])."""
    assert bits in (4, 8), f"unsupported bits={bits}"
    _require_device(t)
    n, d = t.shape
    assert d % group_size == 0, f"D={d} not divisible by group_size={group_size}"
    t = t.contiguous()
    g = d // group_size
    if bits == 4:
        payload = torch.empty((n, d // 2), dtype=torch.uint8, device=t.device)
    else:
        payload = torch.empty((n, d), dtype=torch.int8, device=t.device)
    scales = torch.empty((n, g), dtype=torch.float16, device=t.device)
    check(_lib.lib().cpt_v3_quantize_group_absmax(t.data_ptr(), _dtype_code(t), n, d, bits,
                                                  group_size, payload.data_ptr(),
                                                  scales.data_ptr(), _stream(t)),
          "v3_quantize_group_absmax")
    return payload, scales


def v3_dequantize_group_absmax(payload, scales, bits, group_size=64, dtype=torch.bfloat16):
    """Inverse of v3_quantize_group_absmax (src/flashffn.py:1091-1110):
    out_dtype(fp32(code) * fp32(scale)), [N, D]."""
    assert bits in (4, 8), f"unsupported bits={bits}"
    _require_device(payload, scales)
    n = payload.shape[0]
    d = payload.shape[1] * (2 if bits == 4 else 1)
    assert d % group_size == 0, f"D={d} not divisible by group_size={group_size}"
    assert tuple(scales.shape) == (n, d // group_size) and scales.dtype == torch.float16
    payload, scales = payload.contiguous(), scales.contiguous()
    out = torch.empty((n, d), dtype=dtype, device=payload.device)
    check(_lib.lib().cpt_v3_dequantize_group_absmax(payload.data_ptr(), scales.data_ptr(), n, d,
                                                    bits, group_size, out.data_ptr(),
                                                    _DT[dtype], _stream(payload)),
          "v3_dequantize_group_absmax")
    return out


def _check_quant_shapes(t, bits, group_size):
    """src/flashffn.py:1303-1311."""
    assert bits in (4, 8), f"unsupported bits={bits}"
    assert t.dim() == 2 and t.is_contiguous(), "expected contiguous [N, D]"
    assert t.dtype == torch.bfloat16, f"fused v3 kernels are bf16-only, got {t.dtype}"
    n, d = t.shape
    assert d % group_size == 0, f"D={d} not divisible by group_size={group_size}"
    assert group_size > 0 and (group_size & (group_size - 1)) == 0, \
        f"group_size={group_size} must be a power of two"
    return n, d, d // group_size


def silu_mul_quant(h_gate, h_up, bits, group_size=64):
    """K1 (src/flashffn.py:1314-1340): returns (h_mid, q_gate, s_gate, q_up, s_up);
    h_mid equals silu_mul(h_gate, h_up) and payloads/scales equal
    v3_quantize_group_absmax of each input, bit for bit."""
    _require_device(h_gate, h_up)
    n, d, g = _check_quant_shapes(h_gate, bits, group_size)
    assert h_up.shape == h_gate.shape and h_up.is_contiguous() and h_up.dtype == h_gate.dtype
    dev = h_gate.device
    h_mid = torch.empty_like(h_gate)
    s_gate = torch.empty((n, g), dtype=torch.float16, device=dev)
    s_up = torch.empty((n, g), dtype=torch.float16, device=dev)
    if bits == 4:
        q_gate = torch.empty((n, d // 2), dtype=torch.uint8, device=dev)
        q_up = torch.empty((n, d // 2), dtype=torch.uint8, device=dev)
    else:
        q_gate = torch.empty((n, d), dtype=torch.int8, device=dev)
        q_up = torch.empty((n, d), dtype=torch.int8, device=dev)
    with _timed("silu_mul_quant"):
        rc = _lib.lib().cpt_silu_mul_quant(h_gate.data_ptr(), h_up.data_ptr(), n, d, bits,
                                           group_size, h_mid.data_ptr(), q_gate.data_ptr(),
                                           s_gate.data_ptr(), q_up.data_ptr(), s_up.data_ptr(),
                                           _stream(h_gate))
    check(rc, "silu_mul_quant")
    _V3_COUNTERS["triton_quant_fwd"] += 1
    return h_mid, q_gate, s_gate, q_up, s_up


def dequant_swiglu_backward(grad_h_mid, q_gate, s_gate, q_up, s_up, bits, group_size=64,
                            want_h_mid=False, inplace=False):
    """K2 (src/flashffn.py:1343-1373): returns (grad_h_gate, grad_h_up,
    h_mid_hat | None), equal to dequantise-through-bf16 + swiglu_backward
    (+ silu_mul) without materialising the dequantised caches.
    `inplace=True` writes grad_h_gate over grad_h_mid (which must be private
    to the caller): one [N, D] buffer fewer at the backward's peak."""
    _require_device(grad_h_mid, q_gate, s_gate, q_up, s_up)
    assert grad_h_mid.dim() == 2 and grad_h_mid.is_contiguous()
    assert grad_h_mid.dtype == torch.bfloat16, \
        f"fused v3 kernels are bf16-only, got {grad_h_mid.dtype}"
    assert bits in (4, 8), f"unsupported bits={bits}"
    n, d = grad_h_mid.shape
    assert d % group_size == 0, f"D={d} not divisible by group_size={group_size}"
    assert group_size > 0 and (group_size & (group_size - 1)) == 0, \
        f"group_size={group_size} must be a power of two"
    g = d // group_size
    assert tuple(s_gate.shape) == (n, g) and tuple(s_up.shape) == (n, g)
    expect = (n, d // 2) if bits == 4 else (n, d)
    assert tuple(q_gate.shape) == expect and tuple(q_up.shape) == expect, \
        f"payload shape {tuple(q_gate.shape)} != expected {expect}"
    q_gate, s_gate, q_up, s_up = (t.contiguous() for t in (q_gate, s_gate, q_up, s_up))
    grad_h_gate = grad_h_mid if inplace else torch.empty_like(grad_h_mid)
    grad_h_up = torch.empty_like(grad_h_mid)
    h_mid_hat = torch.empty_like(grad_h_mid) if want_h_mid else None
    with _timed("dequant_swiglu_backward"):
        rc = _lib.lib().cpt_dequant_swiglu_backward(
            grad_h_mid.data_ptr(), q_gate.data_ptr(), s_gate.data_ptr(), q_up.data_ptr(),
            s_up.data_ptr(), n, d, bits, group_size, grad_h_gate.data_ptr(),
            grad_h_up.data_ptr(), _ptr(h_mid_hat), _stream(grad_h_mid))
    check(rc, "dequant_swiglu_backward")
    _V3_COUNTERS["triton_dequant_bwd"] += 1
    return grad_h_gate, grad_h_up, h_mid_hat


# The reference's names and signatures (src/flashffn.py:205,223,259,1314,1343),
# kept for drop-in use.  `digest` belongs to the fused decoder block's
# rematerialisation certificate, which is outside this path.

def triton_silu_mul(h_gate, h_up, digest=False):
    """src/flashffn.py:205-220."""
    if digest:
        raise NotImplementedError("digest witnesses belong to the fused decoder block")
    return silu_mul(h_gate, h_up)


triton_swiglu_backward = swiglu_backward


def triton_swiglu_backward_glu(grad_h_mid, h_gate, h_up, want_h_mid, inplace, digest=False):
    """src/flashffn.py:259-293: returns (grad_h_gate, grad_h_up, h_mid | None, None)."""
    if digest:
        raise NotImplementedError("digest witnesses belong to the fused decoder block")
    dg, du, hm = swiglu_backward_glu(grad_h_mid, h_gate, h_up, want_h_mid, inplace)
    return dg, du, hm, None


triton_silu_mul_quant = silu_mul_quant
triton_dequant_swiglu_backward = dequant_swiglu_backward


# ---------------------------------------------------------------------------
# outlier channels (config C3; HyC-LoRA zero-and-overwrite on the v3 codec,
# hyclora/operators/compress_function.py:80-174)
# ---------------------------------------------------------------------------

def outlier_select(t: torch.Tensor, k: int, rows: int | None = None):
    """The k columns of t [N, D] with the largest L2 norm over the first `rows`
    rows (all rows when None; ties to the lower column).  HyC-LoRA takes the
    norm over the first sample's tokens, `x_[0].abs().norm(dim=-2)`
    (src/hyclora/operators/compress_function.py:85-86): pass that sample's
    row count.  Returns (slot int16 [D]: -1 or the column's position among the
    selected in ascending order, idx int32 [k] ascending)."""
    _require_device(t)
    t = t.contiguous()
    n, d = t.shape
    if rows is not None:
        assert 0 <= rows <= n, f"rows={rows} outside [0, {n}]"
        n = rows
    dev = t.device
    chunks = max(1, (n + 63) // 64)            # 64-row fp64 partial sums
    partial = torch.empty((chunks, d), dtype=torch.float64, device=dev)
    sumsq = torch.empty((d,), dtype=torch.float64, device=dev)
    slot = torch.empty((d,), dtype=torch.int16, device=dev)
    idx = torch.empty((max(k, 1),), dtype=torch.int32, device=dev)
    check(_lib.lib().cpt_outlier_select(t.data_ptr(), _dtype_code(t), n, d, k, partial.data_ptr(),
                                        sumsq.data_ptr(), slot.data_ptr(), idx.data_ptr(),
                                        _stream(t)), "outlier_select")
    return slot, idx[:k]


def outlier_select_pair(t0: torch.Tensor, t1: torch.Tensor, k: int, rows: int | None = None):
    """outlier_select of t0 and of t1 (same shape and dtype) in the same
    launches.  Returns ((slot0, idx0), (slot1, idx1)), each equal to
    outlier_select on that tensor."""
    _require_device(t0, t1)
    t0, t1 = t0.contiguous(), t1.contiguous()
    assert t0.shape == t1.shape and t0.dtype == t1.dtype, \
        f"pair of {tuple(t0.shape)} {t0.dtype} and {tuple(t1.shape)} {t1.dtype}"
    n, d = t0.shape
    if rows is not None:
        assert 0 <= rows <= n, f"rows={rows} outside [0, {n}]"
        n = rows
    dev = t0.device
    chunks = max(1, (n + 63) // 64)            # 64-row fp64 partial sums
    partial = torch.empty((2, chunks, d), dtype=torch.float64, device=dev)
    sumsq = torch.empty((2, d), dtype=torch.float64, device=dev)
    slot = torch.empty((2, d), dtype=torch.int16, device=dev)
    idx = torch.empty((2, max(k, 1)), dtype=torch.int32, device=dev)
    check(_lib.lib().cpt_outlier_select_pair(
        t0.data_ptr(), t1.data_ptr(), _dtype_code(t0), n, d, k, partial.data_ptr(),
        sumsq.data_ptr(), slot[0].data_ptr(), idx[0].data_ptr(), slot[1].data_ptr(),
        idx[1].data_ptr(), _stream(t0)), "outlier_select_pair")
    return (slot[0], idx[0, :k]), (slot[1], idx[1, :k])


def _outlier_buf(n, k, dev):
    return torch.empty((n, k), dtype=torch.bfloat16, device=dev)


def v3_quantize_outlier(t, bits, group_size, slot, k):
    """Codec of t with the slot columns extracted first.  Returns
    (payload, scales, outliers bf16 [N, k])."""
    assert bits in (4, 8), f"unsupported bits={bits}"
    _require_device(t, slot)
    t = t.contiguous()
    n, d = t.shape
    assert d % group_size == 0, f"D={d} not divisible by group_size={group_size}"
    dev = t.device
    payload = torch.empty((n, d // 2) if bits == 4 else (n, d),
                          dtype=torch.uint8 if bits == 4 else torch.int8, device=dev)
    scales = torch.empty((n, d // group_size), dtype=torch.float16, device=dev)
    out = _outlier_buf(n, k, dev)
    check(_lib.lib().cpt_v3_quantize_outlier(t.data_ptr(), _dtype_code(t), n, d, bits, group_size,
                                             slot.data_ptr(), k, out.data_ptr(), payload.data_ptr(),
                                             scales.data_ptr(), _stream(t)), "v3_quantize_outlier")
    return payload, scales, out


def v3_dequantize_outlier(payload, scales, outliers, slot, bits, group_size):
    """Dequantise through bf16 and write the outlier columns back -> bf16 [N, D]."""
    _require_device(payload, scales, outliers, slot)
    n = payload.shape[0]
    d = payload.shape[1] * (2 if bits == 4 else 1)
    out = torch.empty((n, d), dtype=torch.bfloat16, device=payload.device)
    k = outliers.shape[1]
    check(_lib.lib().cpt_v3_dequantize_outlier(payload.data_ptr(), scales.data_ptr(),
                                               slot.data_ptr(), k, outliers.data_ptr(), n, d, bits,
                                               group_size, out.data_ptr(), _stream(payload)),
          "v3_dequantize_outlier")
    return out


def silu_mul_quant_outlier(h_gate, h_up, bits, group_size, slot_gate, slot_up, k, out=None):
    """K1 with outlier channels.  Returns
    (h_mid, q_gate, s_gate, o_gate, q_up, s_up, o_up), written into `out`
    (the same seven, preallocated and contiguous) when given."""
    _require_device(h_gate, h_up, slot_gate, slot_up)
    n, d, g = _check_quant_shapes(h_gate, bits, group_size)
    assert h_up.shape == h_gate.shape and h_up.is_contiguous()
    dev = h_gate.device
    shape = (n, d // 2) if bits == 4 else (n, d)
    qdt = torch.uint8 if bits == 4 else torch.int8
    if out is not None:
        h_mid, qg, sg, og, qu, su, ou = out
        for t, shp, dt in ((h_mid, (n, d), h_gate.dtype), (qg, shape, qdt), (qu, shape, qdt),
                           (sg, (n, g), torch.float16), (su, (n, g), torch.float16),
                           (og, (n, k), torch.bfloat16), (ou, (n, k), torch.bfloat16)):
            assert tuple(t.shape) == shp and t.dtype == dt and t.is_contiguous()
    else:
        h_mid = torch.empty_like(h_gate)
        qg = torch.empty(shape, dtype=qdt, device=dev)
        qu = torch.empty(shape, dtype=qdt, device=dev)
        sg = torch.empty((n, g), dtype=torch.float16, device=dev)
        su = torch.empty((n, g), dtype=torch.float16, device=dev)
        og, ou = _outlier_buf(n, k, dev), _outlier_buf(n, k, dev)
    with _timed("silu_mul_quant_outlier"):
        rc = _lib.lib().cpt_silu_mul_quant_outlier(
            h_gate.data_ptr(), h_up.data_ptr(), n, d, bits, group_size, slot_gate.data_ptr(),
            slot_up.data_ptr(), k, h_mid.data_ptr(), qg.data_ptr(), sg.data_ptr(), og.data_ptr(),
            qu.data_ptr(), su.data_ptr(), ou.data_ptr(), _stream(h_gate))
    check(rc, "silu_mul_quant_outlier")
    _V3_COUNTERS["triton_quant_fwd"] += 1
    return h_mid, qg, sg, og, qu, su, ou


def dequant_swiglu_backward_outlier(grad_h_mid, q_gate, s_gate, o_gate, slot_gate, q_up, s_up,
                                    o_up, slot_up, bits, group_size, want_h_mid=False,
                                    inplace=False):
    """K2 with the outlier columns restored.  Returns (grad_h_gate, grad_h_up,
    h_mid^ | None); `inplace=True` writes grad_h_gate over grad_h_mid."""
    _require_device(grad_h_mid, q_gate, s_gate, o_gate, slot_gate, q_up, s_up, o_up, slot_up)
    assert grad_h_mid.dtype == torch.bfloat16 and grad_h_mid.is_contiguous()
    n, d = grad_h_mid.shape
    dg = grad_h_mid if inplace else torch.empty_like(grad_h_mid)
    du = torch.empty_like(grad_h_mid)
    hm = torch.empty_like(grad_h_mid) if want_h_mid else None
    k = o_gate.shape[1]
    with _timed("dequant_swiglu_backward_outlier"):
        rc = _lib.lib().cpt_dequant_swiglu_backward_outlier(
            grad_h_mid.data_ptr(), q_gate.data_ptr(), s_gate.data_ptr(), slot_gate.data_ptr(),
            o_gate.data_ptr(), q_up.data_ptr(), s_up.data_ptr(), slot_up.data_ptr(),
            o_up.data_ptr(), k, n, d, bits, group_size, dg.data_ptr(), du.data_ptr(), _ptr(hm),
            _stream(grad_h_mid))
    check(rc, "dequant_swiglu_backward_outlier")
    _V3_COUNTERS["triton_dequant_bwd"] += 1
    return dg, du, hm


# ---------------------------------------------------------------------------
# DoRA magnitude (src/flashffn.py:1824-1840, 1967-1975, 2054, 2086-2130)
# ---------------------------------------------------------------------------

def dora_scale(x: torch.Tensor, m: torch.Tensor, nu: torch.Tensor, out=None) -> torch.Tensor:
    """x * (m / nu).unsqueeze(0) with the reference's eager rounding: the
    column scale c = m / nu is rounded to x's dtype, then x * c.  x [N, D],
    m / nu [D], one dtype.  `out` may be x itself (in place)."""
    _require_device(x, m, nu)
    assert x.dim() == 2 and m.shape == nu.shape == (x.shape[1],), \
        f"dora_scale: x {tuple(x.shape)}, m {tuple(m.shape)}, nu {tuple(nu.shape)}"
    assert x.dtype == m.dtype == nu.dtype, "dora_scale: x, m and nu share one dtype"
    x, m, nu = x.contiguous(), m.contiguous(), nu.contiguous()
    if out is None:
        out = torch.empty_like(x)
    assert out.is_contiguous() and out.shape == x.shape and out.dtype == x.dtype
    n, d = x.shape
    with _timed("dora_scale"):
        rc = _lib.lib().cpt_dora_scale(x.data_ptr(), m.data_ptr(), nu.data_ptr(), n, d,
                                       _dtype_code(x), out.data_ptr(), _stream(x))
    check(rc, "dora_scale")
    return out


def col_dot_div(a: torch.Tensor, b: torch.Tensor, den: torch.Tensor) -> torch.Tensor:
    """((a * b).sum(0, dtype=float32) / den.float()).to(den.dtype) for a, b
    [N, D] and den [D] of one dtype; deterministic fp32 summation."""
    _require_device(a, b, den)
    assert a.dim() == 2 and a.shape == b.shape and den.shape == (a.shape[1],)
    assert a.dtype == b.dtype == den.dtype, "col_dot_div: one dtype expected"
    a, b, den = a.contiguous(), b.contiguous(), den.contiguous()
    n, d = a.shape
    L = _lib.lib()
    ws = torch.empty((max(1, L.cpt_col_dot_workspace_bytes(n, d)) + 3) // 4,
                     dtype=torch.float32, device=a.device)
    out = torch.empty((d,), dtype=a.dtype, device=a.device)
    with _timed("col_dot_div"):
        rc = L.cpt_col_dot_div(a.data_ptr(), b.data_ptr(), den.data_ptr(), n, d, _dtype_code(a),
                               ws.data_ptr(), out.data_ptr(), _stream(a))
    check(rc, "col_dot_div")
    return out


def dora_col_norm(w: torch.Tensor, a: torch.Tensor, b: torch.Tensor, s: float,
                  out_dtype=torch.float32) -> torch.Tensor:
    """||W + s * B @ A||_2 over dim=1 (the DoRA weight norm) without forming
    B @ A: fp32 Gram identity (src/flashffn.py:1824-1840).  w [out, in],
    a [r, in], b [out, r], one dtype.  Returns [out] in out_dtype."""
    _require_device(w, a, b)
    assert w.dim() == 2 and a.dim() == 2 and b.dim() == 2
    rows, cols = w.shape
    r = a.shape[0]
    assert a.shape == (r, cols) and b.shape == (rows, r), \
        f"dora_col_norm: w {tuple(w.shape)}, a {tuple(a.shape)}, b {tuple(b.shape)}"
    assert w.dtype == a.dtype == b.dtype, "dora_col_norm: one dtype expected"
    w, a, b = w.contiguous(), a.contiguous(), b.contiguous()
    L = _lib.lib()
    ws = torch.empty((L.cpt_dora_col_norm_workspace_bytes(rows, r) + 3) // 4 + 1,
                     dtype=torch.float32, device=w.device)
    nu = torch.empty((rows,), dtype=out_dtype, device=w.device)
    with _timed("dora_col_norm"):
        rc = L.cpt_dora_col_norm(w.data_ptr(), a.data_ptr(), b.data_ptr(), rows, cols, r,
                                 float(s), _dtype_code(w), ws.data_ptr(), nu.data_ptr(),
                                 _DT[out_dtype], _stream(w))
    check(rc, "dora_col_norm")
    return nu


# ---------------------------------------------------------------------------
# top-K activation compression (FlashFFN v1/v2, src/flashffn.py:349-356,410-415)
# ---------------------------------------------------------------------------

def topk_abs(t: torch.Tensor, k: int):
    """Per row of t [N, D]: the k entries of largest |t| -> (values [N, k] in
    t's dtype, indices int16 [N, k]) in ascending column order, ties at the
    k-th magnitude resolved to the lowest columns (torch.topk's sorted=False
    order and tie choice are unspecified; this fixes both)."""
    _require_device(t)
    assert t.dim() == 2, "topk_abs expects [N, D]"
    t = t.contiguous()
    n, d = t.shape
    assert 0 <= k <= d, f"k={k} out of range for D={d}"
    values = torch.empty((n, k), dtype=t.dtype, device=t.device)
    indices = torch.empty((n, k), dtype=torch.int16, device=t.device)
    with _timed("topk_abs"):
        rc = _lib.lib().cpt_topk_abs(t.data_ptr(), _dtype_code(t), n, d, k, values.data_ptr(),
                                     indices.data_ptr(), _stream(t))
    check(rc, "topk_abs")
    return values, indices


def topk_scatter(values: torch.Tensor, indices: torch.Tensor, d: int) -> torch.Tensor:
    """Dense [N, d] rows with `values` at `indices` and zeros elsewhere
    (`zeros(...).scatter_(-1, indices.long(), values)`)."""
    _require_device(values, indices)
    assert values.shape == indices.shape and indices.dtype == torch.int16
    values, indices = values.contiguous(), indices.contiguous()
    n, k = values.shape
    out = torch.empty((n, d), dtype=values.dtype, device=values.device)
    with _timed("topk_scatter"):
        rc = _lib.lib().cpt_topk_scatter(values.data_ptr(), indices.data_ptr(),
                                         _dtype_code(values), n, d, k, out.data_ptr(),
                                         _stream(values))
    check(rc, "topk_scatter")
    return out
