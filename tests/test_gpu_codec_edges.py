"""GPU codec against the oracle on inputs built to hit the quantiser's two
fast paths at their edges:

- scales: fp16(fp32(absmax / qmax)) is computed as absmax * fp32(1/qmax)
  unless that product lies near an fp16 rounding midpoint.  Group maxima are
  swept across fp32 values whose quotient sits within +-8 fp32 ulp of fp16
  midpoints over the whole normal range, around the fp16 subnormal and
  overflow boundaries, and at random; every scale must equal numpy's
  correctly rounded division converted to fp16, bit for bit.
- codes: rint(v * (1/safe)) decides unless some quotient of the 8 a thread
  owns lies near a half-integer.  Groups of exact half-integer multiples of
  an exact scale (round-half-even ties) and of their fp32 neighbours must
  give the oracle's codes.
"""

import numpy as np
import pytest
import torch

from oracle import codec

pytestmark = pytest.mark.gpu


def _cpt():
    import compact_amd
    return compact_amd


def _midpoint_maxima(qmax, rng, n_mid=6000, ulps=8):
    """fp32 group maxima whose fp32 quotient by qmax lies within +-ulps of an
    fp16 midpoint (fp16 normal exponents -14 .. 15), plus random ones."""
    e = rng.integers(-14, 16, n_mid)
    mant = rng.integers(0, 1024, n_mid)
    mid = ((1024 + mant + 0.5) * np.exp2(e - 10.0)).astype(np.float32)   # fp16 midpoints
    a = (mid.astype(np.float64) * qmax).astype(np.float32)
    bits = a.view(np.int32)[:, None] + np.arange(-ulps, ulps + 1, dtype=np.int32)[None, :]
    near = bits.reshape(-1).view(np.float32)
    edges = np.array([0.0, 2.0 ** -24, 2.0 ** -14, 65504.0, 65519.0, 65520.0, 65536.0,
                      np.inf], np.float64) * qmax
    eb = edges.astype(np.float32).view(np.int32)
    around = (eb[:, None] + np.arange(-3, 4, dtype=np.int32)[None, :]).reshape(-1).view(np.float32)
    rand = np.exp2(rng.uniform(-30, 24, 20000)).astype(np.float32)
    out = np.concatenate([near, around, rand])
    return out[np.isfinite(out) & (out >= 0)]


@pytest.mark.parametrize("bits", [4, 8])
def test_scales_at_fp16_midpoints(device, bits):
    cpt = _cpt()
    qmax = 7 if bits == 4 else 127
    rng = np.random.default_rng(bits)
    amax = _midpoint_maxima(qmax, rng)
    gs = 8
    t = np.zeros((amax.size, gs), np.float32)
    t[:, 0] = amax
    t[:, 1] = -0.5 * amax
    pad = (-amax.size) % 64
    t = np.concatenate([t, np.zeros((pad, gs), np.float32)]).reshape(-1, 64 * gs)
    q, s = cpt.v3_quantize_group_absmax(torch.from_numpy(t).to(device), bits, gs)
    rq, rs = codec.quantize_group_absmax(t, bits, gs)
    got = s.cpu().numpy().view(np.uint16)
    assert np.array_equal(got, rs.view(np.uint16))
    with np.errstate(over="ignore"):              # maxima past fp16's range give inf
        want = (np.abs(t.reshape(-1, gs)).max(1) / np.float32(qmax)).astype(np.float16)
    assert np.array_equal(got.reshape(-1), want.view(np.uint16))
    assert np.array_equal(q.cpu().numpy().view(np.uint8), rq.view(np.uint8))


@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 128), (8, 32)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_codes_at_half_integer_ties(device, bits, gs, dtype):
    """v = (k + 1/2) * scale exactly with an exact fp16 scale (absmax =
    qmax * 2^-3), so every quotient is a tie; fp32 runs also take the
    neighbouring values (ties broken the other way by 1 ulp)."""
    cpt = _cpt()
    qmax = 7 if bits == 4 else 127
    scale = 0.125
    rng = np.random.default_rng(gs + bits)
    rows = 64
    k = rng.integers(-qmax, qmax, size=(rows, 1024)).astype(np.float32)
    v = ((k + 0.5) * scale).astype(np.float32)
    if dtype == torch.float32:
        nudge = rng.integers(-1, 2, size=v.shape).astype(np.int32)
        v = (v.view(np.int32) + nudge * (v != 0)).view(np.float32)
    v = v.reshape(rows, -1, gs)
    v[:, :, 0] = qmax * scale                    # the group's absmax: scale exactly 0.125
    v = v.reshape(rows, -1)
    tv = torch.from_numpy(v).to(dtype)
    q, s = cpt.v3_quantize_group_absmax(tv.to(device), bits, gs)
    rq, rs = codec.quantize_group_absmax(tv.float().numpy(), bits, gs)
    assert np.array_equal(s.cpu().numpy().view(np.uint16), rs.view(np.uint16))
    assert np.array_equal(q.cpu().numpy().view(np.uint8), rq.view(np.uint8))
    if dtype == torch.bfloat16:
        # K1 takes the same path for the gate and the up tensor
        hm, qg, sg, qu, su = cpt.silu_mul_quant(tv.to(device), tv.to(device), bits, gs)
        assert torch.equal(qg.cpu().view(torch.uint8), torch.from_numpy(rq.view(np.uint8)))
        assert torch.equal(qu.cpu().view(torch.uint8), torch.from_numpy(rq.view(np.uint8)))
