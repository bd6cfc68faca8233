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


def _bf16_round(x):
    """float64 -> nearest bf16 (round-half-even), as float32."""
    f = np.asarray(x, np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 128)])
def test_bf16_codes_near_ties_over_scales(device, bits, gs):
    """bf16 inputs take the division-free code rule (two roundings of v *
    rcp(safe)).  Sweep every bf16 group maximum over 40 binades (fp16-
    subnormal, normal and large scales), and fill each group with the bf16
    values nearest to half-integer multiples of its scale and their bf16
    neighbours: exact ties where representable, the closest non-ties
    otherwise.  Codes and scales of the quantiser and of K1 (both tensors)
    must equal the oracle's."""
    cpt = _cpt()
    qmax = 7 if bits == 4 else 127
    rng = np.random.default_rng(100 + bits)
    mant = np.arange(128, dtype=np.uint32)
    exps = np.arange(127 - 28, 127 + 12, dtype=np.uint32)     # 2^-28 .. 2^11
    amax = ((exps[:, None] << 23) | (mant[None, :] << 16)).reshape(-1).view(np.float32)
    s = (amax / np.float32(qmax)).astype(np.float16).astype(np.float64)
    safe = np.where(s > 0, s, 1.0)
    k = rng.integers(-qmax - 1, qmax + 1, size=(amax.size, gs))
    near = _bf16_round((k + 0.5) * safe[:, None])
    step = rng.integers(-1, 2, size=near.shape).astype(np.int32) << 16   # bf16 neighbours
    v = (near.view(np.int32) + step * (near != 0)).view(np.float32)
    v = np.clip(v, -amax[:, None], amax[:, None])
    v[:, 0] = amax
    v[:, 1] = -amax * rng.choice([0.0, 0.5, 1.0], size=amax.size).astype(np.float32)
    v = _bf16_round(v)
    rows = 64
    pad = (-v.shape[0]) % rows
    v = np.concatenate([v, np.zeros((pad, gs), np.float32)]).reshape(rows, -1)
    tv = torch.from_numpy(v).to(torch.bfloat16)
    assert torch.equal(tv.float(), torch.from_numpy(v))                   # exact bf16 values
    rq, rs = codec.quantize_group_absmax(v, bits, gs)
    q, sc = cpt.v3_quantize_group_absmax(tv.to(device), bits, gs)
    assert np.array_equal(sc.cpu().numpy().view(np.uint16), rs.view(np.uint16))
    assert np.array_equal(q.cpu().numpy().view(np.uint8), rq.view(np.uint8))
    u = torch.flip(tv, dims=[1]).contiguous()
    rqu, rsu = codec.quantize_group_absmax(u.float().numpy(), bits, gs)
    hm, qg, sg, qu, su = cpt.silu_mul_quant(tv.to(device), u.to(device), bits, gs)
    assert np.array_equal(qg.cpu().numpy().view(np.uint8), rq.view(np.uint8))
    assert np.array_equal(sg.cpu().numpy().view(np.uint16), rs.view(np.uint16))
    assert np.array_equal(qu.cpu().numpy().view(np.uint8), rqu.view(np.uint8))
    assert np.array_equal(su.cpu().numpy().view(np.uint16), rsu.view(np.uint16))
