"""Pins the CPU oracle's codec (oracle/codec.py) before anything is checked
against it.

Three independent lines of evidence, each chosen so that a plausible mistake
fails at least one of them:
  * hand-computed known-answer vectors for the reference's codec
    (src/flashffn.py:1071-1088): half-even ties, int4 nibble order, division by
    the fp16-ROUNDED scale, fp16-subnormal scales with clamping, fp16 overflow;
  * exact-rational brute force (oracle/exact.py) on tiny inputs;
  * bit-exact agreement with the plain-C restatement (oracle/codec_ref.c),
    which carries its own bit-level fp16/bf16 rounding.
"""

import numpy as np
import pytest
import torch

from oracle import c_codec, codec, exact
from oracle.flashffn_ref import to_f32
from tests.inputs import KINDS, make_pair


def q1(vals, bits, group=4):
    """Quantise one row of float32 values with the oracle."""
    q, s = codec.quantize_group_absmax(np.array([vals], np.float32), bits, group)
    return codec.unpack_codes(q, bits)[0].tolist(), s.view(np.uint16)[0].tolist(), q


# --------------------------------------------------------------------------
# known-answer vectors
# --------------------------------------------------------------------------

def test_kat_int8_half_even_ties():
    # absmax 127 -> scale fp16(1.0) = 0x3C00; ties 0.5 -> 0, 1.5 -> 2, -2.5 -> -2
    codes, sc, _ = q1([127.0, 0.5, 1.5, -2.5], 8)
    assert codes == [127, 0, 2, -2]
    assert sc == [0x3C00]


def test_kat_int4_nibble_order():
    # absmax 7 -> scale 1.0; codes 7, 4 (3.5 ties to even), -4, 0
    codes, sc, payload = q1([7.0, 3.5, -3.5, 0.5], 4)
    assert codes == [7, 4, -4, 0]
    # offset-8 nibbles 15, 12, 4, 8: even column in the low nibble
    assert payload[0].tolist() == [0xCF, 0x84]


def test_kat_divides_by_fp16_rounded_scale():
    # scale = fp16(1/127) = 1032 * 2^-17 (0x2008), not 1/127.  0.7913*127 =
    # 100.495 would round to 100; 0.7913 / 0.00787353515625 = 100.501 -> 101.
    codes, sc, _ = q1([1.0, 0.7913, 0.0, 0.0], 8)
    assert sc == [0x2008]
    assert codes == [127, 101, 0, 0]


def test_kat_subnormal_scale_clamps():
    # 1e-4/127 lands in fp16 subnormals: 13 * 2^-24 (0x000D); 1e-4/scale = 129.05
    # is clamped to 127 and 5e-5/scale = 64.53 -> 65.
    codes, sc, _ = q1([1e-4, 5e-5, 0.0, 0.0], 8)
    assert sc == [0x000D]
    assert codes == [127, 65, 0, 0]


def test_kat_negative_absmax():
    codes, sc, _ = q1([-5.0, 1.0, 2.0, 3.0], 8)
    assert sc == [0x290A]
    assert codes == [-127, 25, 51, 76]


@pytest.mark.parametrize("bits,big", [(8, 1e7), (4, 1e6)])
def test_kat_fp16_scale_overflow(bits, big):
    # absmax/qmax > 65504 -> fp16 +inf; safe = inf, every code 0 and the
    # dequantised group is 0 * inf = NaN (the reference's arithmetic).
    codes, sc, q = q1([big, 1.0, 0.0, 0.0], bits)
    assert sc == [0x7C00]
    assert codes == [0, 0, 0, 0]
    s = np.array([[0x7C00]], np.uint16).view(np.float16)
    deq = codec.dequantize_group_absmax_f32(q, s, bits, 4)
    assert np.isnan(deq).all()


def test_kat_zero_group():
    codes, sc, q = q1([0.0, 0.0, 0.0, 0.0], 4)
    assert sc == [0] and codes == [0, 0, 0, 0]
    assert q[0].tolist() == [0x88, 0x88]


def test_ragged_and_bad_args_assert():
    t = np.zeros((2, 96), np.float32)
    with pytest.raises(AssertionError):
        codec.quantize_group_absmax(t, 4, 64)           # ragged last group
    with pytest.raises(AssertionError):               # fused path: power of two only
        codec.silu_mul_quant(t, t, 4, 48)
    q, s = codec.quantize_group_absmax(t, 4, 48)       # eager codec accepts 48
    assert q.shape == (2, 48) and s.shape == (2, 2)
    with pytest.raises(AssertionError):
        codec.quantize_group_absmax(np.zeros((2, 64), np.float32), 3, 64)


# --------------------------------------------------------------------------
# exact-rational brute force
# --------------------------------------------------------------------------

@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("bits", [4, 8])
def test_brute_force_matches_exact(kind, bits):
    group = 8
    a, b = make_pair(kind, 3, 32, group=group, seed=7)
    for t in (a, b):
        vals = to_f32(t)
        q, s = codec.quantize_group_absmax(vals, bits, group)
        codes_e, scales_e = exact.quantize_exact(vals.tolist(), bits, group)
        assert codec.unpack_codes(q, bits).tolist() == codes_e
        got = s.astype(np.float64).tolist()
        want = [[float(x) for x in row] for row in scales_e]
        assert got == want


def test_brute_force_ties_and_boundaries():
    # values constructed to sit exactly on rounding ties after division
    rng = np.random.default_rng(3)
    rows = []
    for _ in range(20):
        amax = float(np.float32(rng.uniform(0.5, 2.0)))
        s = float(np.float16(np.float32(amax) / np.float32(127)))
        row = [amax] + [float(np.float32((k + 0.5) * s)) for k in rng.integers(-120, 120, 7)]
        rows.append(row)
    vals = np.array(rows, np.float32)
    q, sc = codec.quantize_group_absmax(vals, 8, 8)
    codes_e, scales_e = exact.quantize_exact(vals.tolist(), 8, 8)
    assert codec.unpack_codes(q, 8).tolist() == codes_e


# --------------------------------------------------------------------------
# agreement with the C restatement
# --------------------------------------------------------------------------

@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("bits,group", [(4, 64), (8, 128), (8, 64), (4, 32), (8, 48)])
def test_c_restatement_bit_exact(kind, bits, group):
    d = 1024 if 1024 % group == 0 else 960
    a, b = make_pair(kind, 64, d, group=group, seed=11)
    for t in (a, b):
        vals = to_f32(t)
        q_np, s_np = codec.quantize_group_absmax(vals, bits, group)
        q_c, s_c = c_codec.quantize(vals, bits, group)
        assert np.array_equal(q_np, q_c)
        assert np.array_equal(s_np.view(np.uint16), s_c.view(np.uint16))
        d_np = codec.dequantize_group_absmax_bf16(q_np, s_np, bits, group)
        d_c = c_codec.dequantize_bf16(q_c, s_c, bits, group)
        nan_np = (d_np & 0x7FFF) > 0x7F80
        nan_c = (d_c & 0x7FFF) > 0x7F80
        assert np.array_equal(nan_np, nan_c)
        assert np.array_equal(d_np[~nan_np], d_c[~nan_c])


def test_fp32_inputs_c_vs_numpy():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((32, 512)) * np.exp(rng.uniform(-20, 10, (32, 512)))).astype(np.float32)
    for bits in (4, 8):
        q_np, s_np = codec.quantize_group_absmax(x, bits, 64)
        q_c, s_c = c_codec.quantize(x, bits, 64)
        assert np.array_equal(q_np, q_c)
        assert np.array_equal(s_np.view(np.uint16), s_c.view(np.uint16))


def test_conversions_match_numpy_and_torch():
    rng = np.random.default_rng(9)
    specials = [0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.98e-8, 2.9802322387695312e-08,
                5.96e-8, 6.1e-5, 6.103515625e-05, 1.0, 1.0009765625, 1.00048828125, 3e38]
    bits = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)
    vals = np.concatenate([np.array(specials, np.float32), bits.view(np.float32)])
    vals = vals[np.isfinite(vals)]
    c16 = np.array([c_codec.f32_to_f16_bits(v) for v in vals], np.uint16)
    with np.errstate(over="ignore"):        # overflow to +-inf is part of what is checked
        n16 = vals.astype(np.float16)
    assert np.array_equal(c16, n16.view(np.uint16))
    cb = np.array([c_codec.f32_to_bf16_bits(v) for v in vals], np.uint16)
    tb = torch.from_numpy(vals.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(cb, tb)
    assert np.array_equal(codec.f32_to_bf16_bits(vals), tb)


# --------------------------------------------------------------------------
# invariants on random data
# --------------------------------------------------------------------------

@pytest.mark.parametrize("bits,group", [(4, 64), (8, 128)])
def test_codec_invariants(bits, group):
    a, _ = make_pair("random", 128, 2048, group=group, seed=13)
    v = to_f32(a)
    q, s = codec.quantize_group_absmax(v, bits, group)
    qmax = 2 ** (bits - 1) - 1
    codes = codec.unpack_codes(q, bits)
    assert codes.min() >= -qmax and codes.max() <= qmax
    if bits == 4:
        nib = np.concatenate([(q & 0xF).ravel(), (q >> 4).ravel()])
        assert nib.min() >= 1 and nib.max() <= 15
    absmax = np.abs(v.reshape(128, -1, group)).max(-1)
    assert np.array_equal(s, (absmax / np.float32(qmax)).astype(np.float16))
    deq = codec.dequantize_group_absmax_f32(q, s, bits, group)
    err = np.abs(deq - v).reshape(128, -1, group).max(-1)
    sf = s.astype(np.float32)
    # |error| <= scale/2 up to the fp16 rounding of the scale (relative 2^-11 * qmax)
    assert (err <= sf * 0.5 + absmax * (qmax * 2.0 ** -11) + 1e-30).all()


def test_outlier_codec_spec():
    a, _ = make_pair("random", 64, 512, seed=17)
    a = a.clone()
    a[:, [3, 100, 257]] *= 50          # three hot channels
    v = to_f32(a)
    bitsv = a.view(torch.int16).numpy().view(np.uint16)
    idx = codec.outlier_channels(v, 3 / 512 + 1e-9)
    assert idx.tolist() == [3, 100, 257]
    q, s, ob = codec.outlier_quantize(v, bitsv, idx, 4, 64)
    z = v.copy()
    z[:, idx] = 0
    q2, s2 = codec.quantize_group_absmax(z, 4, 64)
    assert np.array_equal(q, q2) and np.array_equal(s.view(np.uint16), s2.view(np.uint16))
    deq = codec.outlier_dequantize_bf16(q, s, ob, idx, 4, 64)
    assert np.array_equal(deq[:, idx], bitsv[:, idx])
    # outliers stored exactly improve the reconstruction over the plain codec
    plain = codec.bf16_bits_to_f32(codec.dequantize_group_absmax_bf16(
        *codec.quantize_group_absmax(v, 4, 64), 4, 64))
    with_o = codec.bf16_bits_to_f32(deq)
    assert np.linalg.norm(with_o - v) < np.linalg.norm(plain - v)


@pytest.mark.parametrize("b,s,d,ratio", [(2, 64, 512, 0.01), (4, 32, 1024, 0.05), (1, 48, 256, 0.02)])
def test_outlier_channels_rank_the_first_sample(b, s, d, ratio):
    """Channel selection follows HyC-LoRA's `get_statistics_channel_base`
    (src/hyclora/operators/compress_function.py:85-86): the top int(D*ratio)
    of `x_[0].abs().norm(dim=-2)` on the [B, S, D] tensor, i.e. the first
    sample's S rows of the [N, D] matrix.  The later samples carry other hot
    channels, so ranking all rows would pick a different set."""
    g = torch.Generator().manual_seed(b * 1000 + d)
    x = torch.randn(b, s, d, generator=g)
    k = int(d * ratio)
    hot0 = torch.randperm(d, generator=g)[:k]
    x[0][:, hot0] *= 8.0
    if b > 1:
        other = torch.randperm(d, generator=g)[:k]
        x[1:][:, :, other] *= 80.0
    v = x.reshape(-1, d).numpy()
    got = codec.outlier_channels(v, ratio, rows=s)
    want = torch.topk(x[0].abs().norm(dim=-2), k, largest=True).indices
    assert got.tolist() == sorted(want.tolist())
    assert sorted(got.tolist()) == sorted(hot0.tolist())
    if b > 1:
        assert codec.outlier_channels(v, ratio).tolist() != got.tolist()
    # a 2-D input is one sample: rows=None ranks every row
    assert codec.outlier_channels(v[:s], ratio).tolist() == got.tolist()


def test_outlier_stat_rows_product_equals_oracle():
    from compact_amd.flashffn import outlier_stat_rows
    from oracle.flashffn_ref import stat_rows
    for shape, want in (((256, 64), 256), ((2, 128, 64), 128), ((4, 2, 8, 64), 16),
                        ((0, 5, 64), 0), ((1, 7, 64), 7), ((0, 64), 0)):
        assert outlier_stat_rows(shape) == want == stat_rows(shape), shape
