"""GPU tests of the LoRA adapter terms carried by the GEMM epilogues
(PEFT's `h + s * B(A(x))`, src/flashffn.py:1414,1420,1439,1529,1558-1566):

  * a plain GEMM with one or two terms against the fp32 reference of the
    same bf16 inputs, with PEFT's rounding (the product and its scaling are
    rounded to bf16 before the sum, so the bar is relative to the terms), and
    against the composition GEMM + thin adapter add (equal up to the fp32
    summation order of the rank-sized dot products: at most a few elements,
    each within one bf16 step);
  * the fused gate/up and down-dgrad kernels with their terms against the
    plain GEMM with the same terms followed by the standalone K1 / K2 kernels:
    bitwise, since both apply the terms with the same instructions;
  * an absent term (adapter on gate only, or up only) leaves its columns
    bitwise equal to the adapter-free kernel;
  * ranks 17 to 32 (a second MFMA over k 16..31) on the 16x16x32 loop, and
    their refusal where a product would leave it (the engine, and the
    stream-K kernels, carry ranks up to 16).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _cpt():
    import compact_amd
    from compact_amd import _lib, gemm
    return compact_amd, gemm, _lib


def rnd(shape, seed, device, scale=1.0):
    g = torch.Generator(device=device).manual_seed(seed)
    return (torch.randn(*shape, device=device, generator=g) * scale).to(torch.bfloat16)


def peft_ref(h_f32, terms):
    """fp32 value of out = h + sum_t s_t * (p_t @ q_t) and the size of the terms
    the bf16 roundings are relative to."""
    out, mag = h_f32.clone(), h_f32.abs().clone()
    for p, q, s in terms:
        l = s * (p.float().cpu() @ q.float().cpu())
        out += l
        mag += l.abs()
    return out, mag


def bits16(t):
    return t.contiguous().view(torch.int16)


@pytest.mark.parametrize("rank", [8, 16, 24, 32])
@pytest.mark.parametrize("bk", [True, False])
@pytest.mark.parametrize("q_kmajor", [True, False])
@pytest.mark.parametrize("nterms", [1, 2])
@pytest.mark.parametrize("mnk", [(300, 264, 136), (512, 768, 128), (300, 264, 128)])
# the engine (K 136), the 16x16x32 loop on whole tiles and on ragged ones
def test_mm2_lora_terms(device, rank, bk, q_kmajor, nterms, mnk):
    _, G, _ = _cpt()
    m, n, k = mnk
    if not G.lora_fusable(rank, (k, n)):
        pytest.skip("ranks above 16 ride on the 16x16x32 loop only (K a multiple of 64)")
    a = rnd((m, k), 1, device)
    b = rnd((n, k), 2, device).t() if bk else rnd((k, n), 2, device)
    terms = []
    for t in range(nterms):
        p = rnd((m, rank), 10 + t, device)
        q = rnd((n, rank), 20 + t, device, 0.1).t() if q_kmajor else rnd((rank, n), 20 + t, device, 0.1)
        terms.append((p, q, 2.0 if t == 0 else -0.5))
    got = G.mm2(a, b, lora=terms)
    # fp32 reference with PEFT's roundings
    base = G.mm(a, b)
    ref, mag = peft_ref(base.float().cpu(), terms)
    tol = nterms * 2 ** -7 * mag + 1e-6
    assert not ((got.float().cpu() - ref).abs() > tol).any()
    # the composition through the thin adapter add
    comp = base.clone()
    for p, q, s in terms:
        comp = G.addmm_(comp, p, q, s)
    diff = bits16(got) != bits16(comp)
    assert diff.float().mean().item() < 1e-3, int(diff.sum())


def plain_like_f1(G, x, w):
    """x . w^T in the summation order of F1: the 16x16x32 loop when d_model is
    a multiple of 64 (ffn_nt16_fits in gemm.hip), where the plain product then
    runs too (nt16_fits); else the engine."""
    if x.shape[1] % 64 == 0:
        assert x.shape[1] < 1024 and w.shape[0] > 32, "mm would leave the 16x16x32 loop"
        return G.linear(x, w)
    return G.mm_engine(x, w.t())


@pytest.mark.parametrize("cache,bits,group", [("int4", 4, 64), ("int8", 8, 128), ("bf16", 0, 64),
                                              ("none", 0, 64)])
@pytest.mark.parametrize("which", ["both", "gate", "up"])
@pytest.mark.parametrize("rank", [8, 16, 24, 32])
@pytest.mark.parametrize("n_tok,hid,inter", [(300, 128, 384), (512, 128, 512), (300, 136, 384)])
def test_gate_up_lora_fused_equals_composed(device, cache, bits, group, which, rank, n_tok, hid,
                                            inter):
    """F1 with adapter terms equals the plain product of the same main loop
    (the 16x16x32 loop for d_model 128, the engine for 136) with the same
    terms, then K1, bit for bit."""
    cpt, G, _lib = _cpt()
    if not G.lora_fusable(rank, (hid, inter)):
        pytest.skip("ranks above 16 ride on the 16x16x32 loop only (d_model a multiple of 64)")
    code = {"int4": _lib.CACHE_INT4, "int8": _lib.CACHE_INT8, "bf16": _lib.CACHE_BF16,
            "none": _lib.CACHE_NONE}[cache]
    x = rnd((n_tok, hid), 30, device)
    wg, wu = rnd((inter, hid), 31, device, 0.05), rnd((inter, hid), 32, device, 0.05)
    xa_g, xa_u = rnd((n_tok, rank), 33, device), rnd((n_tok, rank), 34, device)
    bg, bu = rnd((inter, rank), 35, device, 0.05), rnd((inter, rank), 36, device, 0.05)
    lg = (xa_g, bg, 2.0) if which in ("both", "gate") else None
    lu = (xa_u, bu, 2.0) if which in ("both", "up") else None
    hm, hg, hu, qg, sg, qu, su = G.ffn_gate_up(x, wg, wu, code, group, lora_gate=lg, lora_up=lu)
    hg_ref = G.mm2(x, wg.t(), lora=[(xa_g, bg.t(), 2.0)]) if lg else plain_like_f1(G, x, wg)
    hu_ref = G.mm2(x, wu.t(), lora=[(xa_u, bu.t(), 2.0)]) if lu else plain_like_f1(G, x, wu)
    assert torch.equal(bits16(hm), bits16(cpt.silu_mul(hg_ref, hu_ref)))
    if cache == "bf16":
        assert torch.equal(bits16(hg), bits16(hg_ref))
        assert torch.equal(bits16(hu), bits16(hu_ref))
    if bits:
        _, rqg, rsg, rqu, rsu = cpt.silu_mul_quant(hg_ref, hu_ref, bits, group)
        assert torch.equal(qg.view(torch.uint8), rqg.view(torch.uint8))
        assert torch.equal(qu.view(torch.uint8), rqu.view(torch.uint8))
        assert torch.equal(bits16(sg), bits16(rsg))
        assert torch.equal(bits16(su), bits16(rsu))


@pytest.mark.parametrize("cache,bits,group,inter", [("bf16", 0, 64, 264), ("none", 0, 64, 264),
                                                    ("int8", 8, 64, 320), ("int4", 4, 32, 320)])
@pytest.mark.parametrize("which", ["both", "gate"])
@pytest.mark.parametrize("rank", [8, 16, 32])
def test_gate_up_lora_ragged_dff(device, cache, bits, group, inter, which, rank):
    """The adapter terms on a partial last d_ff tile: the Q rows (B's rows)
    past d_ff read zero and those columns are never stored."""
    test_gate_up_lora_fused_equals_composed(device, cache, bits, group, which, rank, 300, 128,
                                            inter)


def test_absent_term_is_a_no_op(device):
    """Adapter on gate only: h_up must equal the adapter-free kernel's bit for
    bit (zero rows of x included)."""
    _, G, _lib = _cpt()
    n_tok, hid, inter, rank = 64, 64, 256, 16
    x = rnd((n_tok, hid), 40, device)
    x[::3] = -0.0
    wg, wu = rnd((inter, hid), 41, device, 0.05), rnd((inter, hid), 42, device, 0.05)
    xa_g, bg = rnd((n_tok, rank), 43, device), rnd((inter, rank), 44, device, 0.05)
    _, hg, hu, *_ = G.ffn_gate_up(x, wg, wu, _lib.CACHE_BF16, 64, lora_gate=(xa_g, bg, 2.0))
    _, hg0, hu0, *_ = G.ffn_gate_up(x, wg, wu, _lib.CACHE_BF16, 64)
    assert torch.equal(bits16(hu), bits16(hu0))


@pytest.mark.parametrize("cache,bits,group", [("int4", 4, 64), ("int8", 8, 128), ("bf16", 0, 64)])
@pytest.mark.parametrize("want_h_mid", [True, False])
@pytest.mark.parametrize("rank", [8, 16, 24, 32])
def test_down_dgrad_lora_fused_equals_composed(device, cache, bits, group, want_h_mid, rank):
    cpt, G, _lib = _cpt()
    code = {"int4": _lib.CACHE_INT4, "int8": _lib.CACHE_INT8, "bf16": _lib.CACHE_BF16}[cache]
    n_tok, hid, inter = 300, 128, 384
    hg, hu = rnd((n_tok, inter), 50, device, 3.0), rnd((n_tok, inter), 51, device, 2.0)
    gy, wd = rnd((n_tok, hid), 52, device), rnd((hid, inter), 53, device, 0.05)
    gyb, ad = rnd((n_tok, rank), 54, device), rnd((rank, inter), 55, device, 0.05)
    lora = (gyb, ad, 2.0)
    gmid = G.mm2(gy, wd, lora=[lora])
    if bits:
        _, qg, sg, qu, su = cpt.silu_mul_quant(hg, hu, bits, group)
        dg, du, hm = G.ffn_down_dgrad(gy, wd, code, group, qg, sg, qu, su, want_h_mid, lora=lora)
        rdg, rdu, rhm = cpt.dequant_swiglu_backward(gmid, qg, sg, qu, su, bits, group,
                                                    want_h_mid=want_h_mid)
    else:
        dg, du, hm = G.ffn_down_dgrad(gy, wd, code, group, hg, None, hu, None, want_h_mid,
                                      lora=lora)
        rdg, rdu, rhm = cpt.swiglu_backward_glu(gmid, hg, hu, want_h_mid)
    assert torch.equal(bits16(dg), bits16(rdg))
    assert torch.equal(bits16(du), bits16(rdu))
    if want_h_mid:
        assert torch.equal(bits16(hm), bits16(rhm))


def test_rank_not_a_multiple_of_8_is_zero_padded(device):
    """A rank that is not a multiple of 8 is passed to the epilogue
    zero-padded to the next multiple: the extra products are exact zeros, so
    the result equals the caller-padded call bit for bit."""
    _, G, _ = _cpt()
    a, b = rnd((64, 64), 60, device), rnd((64, 64), 61, device)
    for r, rp in ((4, 8), (12, 16), (17, 24), (30, 32)):
        p, q = rnd((64, r), 62, device), rnd((r, 64), 63, device)
        pp = torch.nn.functional.pad(p, (0, rp - r))
        qp = torch.nn.functional.pad(q, (0, 0, 0, rp - r))
        got = G.mm2(a, b, lora=[(p, q, 1.0)])
        ref = G.mm2(a, b, lora=[(pp, qp, 1.0)])
        assert torch.equal(bits16(got), bits16(ref))


def test_rank_outside_epilogue_set_raises(device):
    _, G, _ = _cpt()
    a, b = rnd((64, 64), 60, device), rnd((64, 64), 61, device)
    p, q = rnd((64, 40), 62, device), rnd((40, 64), 63, device)
    with pytest.raises(AssertionError):
        G.mm2(a, b, lora=[(p, q, 1.0)])
    # rank 24 on a product the engine would run (K not a multiple of 64)
    a = rnd((64, 72), 64, device)
    b = rnd((72, 64), 65, device)
    p, q = rnd((64, 24), 62, device), rnd((24, 64), 63, device)
    with pytest.raises(AssertionError):
        G.mm2(a, b, lora=[(p, q, 1.0)])


@pytest.mark.parametrize("rank", [16, 24, 32])
def test_high_rank_term_equals_two_low_rank_terms(device, rank):
    """Ranks 17 to 32 go through two MFMAs, k 0..15 then k 16..31, accumulated
    in fp32: the term over k 0..15 plus the term over k 16..r-1 in one fp32
    sum.  Against the fp32 reference with PEFT's roundings (the bar of
    test_mm2_lora_terms) and, with the first half of the factors zero, against
    the rank-(r - 16) call bit for bit (the zero half adds exact zeros)."""
    _, G, _ = _cpt()
    m, n, k = 300, 264, 128
    a, b = rnd((m, k), 70, device), rnd((k, n), 71, device)
    p, q = rnd((m, rank), 72, device), rnd((rank, n), 73, device, 0.1)
    got = G.mm2(a, b, lora=[(p, q, 2.0)])
    base = G.mm(a, b)
    ref, mag = peft_ref(base.float().cpu(), [(p, q, 2.0)])
    assert not ((got.float().cpu() - ref).abs() > 2 ** -7 * mag + 1e-6).any()
    if rank > 16:
        pz, qz = p.clone(), q.clone()
        pz[:, :16] = 0
        qz[:16] = 0
        lo = G.mm2(a, b, lora=[(pz, qz, 2.0)])
        hi = G.mm2(a, b, lora=[(p[:, 16:].contiguous(), q[16:].contiguous(), 2.0)])
        assert torch.equal(bits16(lo), bits16(hi))


def test_high_rank_stream_k_shape(device):
    """A product whose tile count would take the stream-K schedule: with a
    rank-32 term it runs data-parallel (the stream-K kernels carry ranks up
    to 16) and its rows match the same product computed in row blocks that
    the stream-K plan leaves alone."""
    _, G, _ = _cpt()
    # 8 x 43 = 344 tiles of 256 x 256 on 256 CUs: a part-empty second wave
    m, n, k = 2048, 11008, 1024
    a, b = rnd((m, k), 80, device), rnd((n, k), 81, device, 0.05).t()
    p, q = rnd((m, 32), 82, device), rnd((32, n), 83, device, 0.1)
    got = G.mm2(a, b, lora=[(p, q, 0.5)])
    for r0 in range(0, m, 256):
        part = G.mm2(a[r0:r0 + 256], b, lora=[(p[r0:r0 + 256], q, 0.5)])
        assert torch.equal(bits16(got[r0:r0 + 256]), bits16(part)), r0
