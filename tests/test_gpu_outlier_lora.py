"""GPU tests of the C3 pieces: outlier channels (this build's specification
of HyC-LoRA zero-and-overwrite on the v3 codec -- parity unpinned against the
reference, which has no such combination, so the oracle's specification is
the bar) and the LoRA terms on the GEMM engine.

Bars: outlier selection, codes, scales, stored outliers and dequantised values
bit-exact against the oracle; fused (K1/K2) == standalone bitwise; LoRA GEMM
paths within the bf16 output rounding of an fp32 reference; the C3-shaped
Function within rel 2e-2 of the oracle Function and above the reference's V2
cosine floors against fp32 autograd.
"""

import numpy as np
import pytest
import torch

from oracle import codec
from oracle import flashffn_ref as R
from oracle.flashffn_ref import to_f32
from tests.inputs import make_pair

pytestmark = pytest.mark.gpu


def _cpt():
    import compact_amd
    from compact_amd import gemm
    return compact_amd, gemm


def _hot(n, d, seed, hot=(3, 100, 257, 1000)):
    a, b = make_pair("random", n, d, seed=seed)
    a, b = a.clone(), b.clone()
    for j, c in enumerate(hot):
        if c < d:
            a[:, c] *= 40 + j
            b[:, (c * 7) % d] *= 30 + j
    return a, b


@pytest.mark.parametrize("ratio", [0.005, 0.01, 0.05])
@pytest.mark.parametrize("rows", [None, 128, 1])
def test_outlier_select_matches_oracle(device, ratio, rows):
    """rows: the first sample's row count that ranks the channels (None: all)."""
    cpt, _ = _cpt()
    a, b = _hot(384, 2048, 5)
    if rows is not None:
        # later rows carry other hot channels: ranking all rows would differ
        a[rows:, 1500:1600] *= 60
    for t in (a, b):
        k = int(t.shape[1] * ratio)
        slot, idx = cpt.outlier_select(t.to(device), k, rows)
        want = codec.outlier_channels(to_f32(t), ratio, rows)
        assert idx.cpu().numpy().tolist() == want.tolist()
        s = slot.cpu().numpy()
        assert (s >= 0).sum() == k
        assert s[want].tolist() == list(range(k))


@pytest.mark.parametrize("n,d,ratio,rows", [(384, 2048, 0.01, 128), (384, 2048, 0.05, None),
                                            (1, 1024, 0.01, None), (300, 11008, 0.01, 100),
                                            (64, 512, 0.0, None)])
def test_outlier_select_pair_equals_singles(device, n, d, ratio, rows):
    """Both tensors selected in the same launches: each result bit-equal to
    its own single selection and to the oracle."""
    cpt, _ = _cpt()
    a, b = _hot(n, d, 15)
    ga, gb = a.to(device), b.to(device)
    k = int(d * ratio)
    (s0, i0), (s1, i1) = cpt.outlier_select_pair(ga, gb, k, rows)
    for t, s, i in ((ga, s0, i0), (gb, s1, i1)):
        rs, ri = cpt.outlier_select(t, k, rows)
        assert torch.equal(s, rs) and torch.equal(i, ri)
        want = codec.outlier_channels(to_f32(t.cpu()), ratio, rows)
        assert i.cpu().numpy().tolist() == want.tolist()


def test_outlier_select_pair_rejects_mismatch(device):
    cpt, _ = _cpt()
    a = torch.zeros(8, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(AssertionError):
        cpt.outlier_select_pair(a, torch.zeros(8, 128, dtype=torch.bfloat16, device=device), 1)
    with pytest.raises(AssertionError):
        cpt.outlier_select_pair(a, a.float(), 1)


@pytest.mark.parametrize("bits,group", [(4, 64), (8, 128), (4, 32)])
def test_outlier_codec_bit_exact(device, bits, group):
    cpt, _ = _cpt()
    a, _ = _hot(256, 2048, 7)
    k = int(2048 * 0.01)
    slot, idx = cpt.outlier_select(a.to(device), k)
    q, s, o = cpt.v3_quantize_outlier(a.to(device), bits, group, slot, k)
    ridx = codec.outlier_channels(to_f32(a), 0.01)
    bits16 = a.view(torch.int16).numpy().view(np.uint16)
    rq, rs, ro = codec.outlier_quantize(to_f32(a), bits16, ridx, bits, group)
    assert np.array_equal(q.cpu().numpy().view(np.uint8), rq.view(np.uint8))
    assert np.array_equal(s.cpu().numpy().view(np.uint16), rs.view(np.uint16))
    assert np.array_equal(o.cpu().view(torch.int16).numpy().view(np.uint16), ro)
    deq = cpt.v3_dequantize_outlier(q, s, o, slot, bits, group)
    rdeq = codec.outlier_dequantize_bf16(rq, rs, ro, ridx, bits, group)
    assert np.array_equal(deq.cpu().view(torch.int16).numpy().view(np.uint16), rdeq)


@pytest.mark.parametrize("bits,group,n,d,ratio", [
    (4, 64, 256, 1024, 0.01), (8, 128, 256, 1024, 0.01), (4, 64, 7, 1024, 0.01),
    (8, 512, 258, 2048, 0.01), (4, 8, 1, 1024, 0.01), (8, 32, 5, 1024, 0.01),
    (4, 64, 300, 4096, 0.01), (4, 64, 3, 11008, 0.01), (8, 128, 513, 2048, 0.0625),
    (4, 64, 300, 4096, 0.05), (8, 128, 130, 2048, 0.0)])
def test_outlier_k1_k2_equal_standalone(device, bits, group, n, d, ratio):
    """K1 / K2 with outlier channels against the standalone codec and GLU
    kernels, bit for bit: groups of 1 to 64 lanes, one row, ragged row counts
    (a part-empty last block), and both K2 forms: the block's outlier rows
    staged in LDS (k <= 128 with D / 8 >= 256, k = 128 at the limit) and read
    from HBM (k = 204; D / 8 < 256); no outliers at all (k = 0)."""
    cpt, _ = _cpt()
    a, b = _hot(n, d, 9)
    ga, gb = a.to(device), b.to(device)
    k = int(d * ratio)
    sg_, _ = cpt.outlier_select(ga, k)
    su_, _ = cpt.outlier_select(gb, k)
    hm, qg, sg, og, qu, su, ou = cpt.silu_mul_quant_outlier(ga, gb, bits, group, sg_, su_, k)
    q2, s2, o2 = cpt.v3_quantize_outlier(ga, bits, group, sg_, k)
    q3, s3, o3 = cpt.v3_quantize_outlier(gb, bits, group, su_, k)
    assert torch.equal(qg.view(torch.uint8), q2.view(torch.uint8))
    assert torch.equal(qu.view(torch.uint8), q3.view(torch.uint8))
    assert torch.equal(sg.view(torch.int16), s2.view(torch.int16))
    assert torch.equal(og.view(torch.int16), o2.view(torch.int16))
    assert torch.equal(ou.view(torch.int16), o3.view(torch.int16))
    assert torch.equal(hm.view(torch.int16), cpt.silu_mul(ga, gb).view(torch.int16))
    gm = torch.randn(n, d, device=device).to(torch.bfloat16)
    dg, du, h = cpt.dequant_swiglu_backward_outlier(gm, qg, sg, og, sg_, qu, su, ou, su_, bits,
                                                    group, want_h_mid=True)
    hg = cpt.v3_dequantize_outlier(qg, sg, og, sg_, bits, group)
    hu = cpt.v3_dequantize_outlier(qu, su, ou, su_, bits, group)
    rdg, rdu, rh = cpt.swiglu_backward_glu(gm, hg, hu, True)
    for x, y in ((dg, rdg), (du, rdu), (h, rh)):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))


@pytest.mark.parametrize("bits,group", [(4, 64), (8, 128)])
@pytest.mark.parametrize("with_lora", [False, 16, 32])
@pytest.mark.parametrize("want_h_mid", [True, False])
def test_outlier_fused_dgrad_equals_unfused(device, bits, group, with_lora, want_h_mid):
    """The dgrad GEMM with dequantise + outlier restore + SwiGLU backward in
    its epilogue equals the GEMM (with the down projection's LoRA term, rank
    16, or 32 on the kernels for ranks above 16) and the standalone outlier
    K2, bit for bit."""
    cpt, G = _cpt()
    n, hdim, d = 384, 256, 1024
    a, b = _hot(n, d, 11)
    ga, gb = a.to(device), b.to(device)
    k = int(d * 0.01)
    sg_, _ = cpt.outlier_select(ga, k)
    su_, _ = cpt.outlier_select(gb, k)
    _, qg, sg, og, qu, su, ou = cpt.silu_mul_quant_outlier(ga, gb, bits, group, sg_, su_, k)
    gen = torch.Generator(device=device).manual_seed(12)
    gy = torch.randn(n, hdim, device=device, generator=gen).to(torch.bfloat16)
    wd = (torch.randn(hdim, d, device=device, generator=gen) * 0.05).to(torch.bfloat16)
    lora = None
    if with_lora:
        r = with_lora
        gyb = (torch.randn(n, r, device=device, generator=gen) * 0.1).to(torch.bfloat16)
        a_d = (torch.randn(r, d, device=device, generator=gen) * 0.05).to(torch.bfloat16)
        lora = (gyb, a_d, 2.0)
    dg, du, hm = G.ffn_down_dgrad(gy, wd, bits, group, qg, sg, qu, su, want_h_mid, lora=lora,
                                  outliers=(sg_, og, su_, ou))
    # B1 runs on the 16x16x32 loop at d_model 256, as G.mm2 does
    gmid = G.mm2(gy, wd, lora=[lora]) if with_lora else G.mm2(gy, wd)
    rdg, rdu, rhm = cpt.dequant_swiglu_backward_outlier(gmid, qg, sg, og, sg_, qu, su, ou, su_,
                                                        bits, group, want_h_mid=want_h_mid)
    assert torch.equal(dg.view(torch.int16), rdg.view(torch.int16))
    assert torch.equal(du.view(torch.int16), rdu.view(torch.int16))
    if want_h_mid:
        assert torch.equal(hm.view(torch.int16), rhm.view(torch.int16))
    else:
        assert hm is None


def _close(got, ref):
    got = got.float().cpu()
    tol = 1e-2 * ref.abs() + 1e-3 * ref.abs().max()
    assert not ((got - ref).abs() > tol).any(), float((got - ref).abs().max())


def test_lora_addmm_matches_peft_order(device):
    _, G = _cpt()
    g = torch.Generator(device=device).manual_seed(3)
    h = torch.randn(300, 512, device=device, generator=g).to(torch.bfloat16)
    xa = torch.randn(300, 16, device=device, generator=g).to(torch.bfloat16)
    bt = (torch.randn(512, 16, device=device, generator=g) * 0.1).to(torch.bfloat16)
    want = h + 2.0 * (xa @ bt.t())          # torch bf16: same three roundings
    got = G.addmm_(h.clone(), xa, bt.t(), 2.0)
    assert (got.float() - want.float()).abs().max() <= 2 * 2 ** -7 * want.float().abs().max()
    lora = 2.0 * (xa.float().cpu() @ bt.float().cpu().t())
    ref = h.float().cpu() + lora
    # the product and its scaling are rounded to bf16 before the sum: the
    # error is relative to the terms, not to their (possibly cancelling) sum
    tol = 2 ** -7 * (h.float().cpu().abs() + lora.abs()) + 1e-6
    assert not ((got.float().cpu() - ref).abs() > tol).any()


@pytest.mark.parametrize("mnk", [(16, 4096, 8192), (4096, 16, 8192), (24, 264, 1000)])
def test_splitk_matches_fp32(device, mnk):
    _, G = _cpt()
    m, n, k = mnk
    g = torch.Generator(device=device).manual_seed(4)
    a = torch.randn(k, m, device=device, generator=g).to(torch.bfloat16).t()   # token-major
    b = torch.randn(k, n, device=device, generator=g).to(torch.bfloat16)
    got = G.mm_splitk(a, b, 0.5)
    ref = 0.5 * (a.float().cpu() @ b.float().cpu())
    _close(got, ref)


H, D, RANK, S, N = 256, 768, 16, 2.0, 256


@pytest.mark.parametrize("ratio,batch", [(0.0, None), (0.01, None), (0.01, 2)])
def test_c3_function_vs_oracle(device, ratio, batch):
    """C3 shape in miniature: LoRA r16 (s=2) on gate/up/down, frozen base,
    int4 g64 cache, top-1% outlier channels.  batch: x as [batch, N / batch, H],
    whose first sample ranks the outlier channels."""
    cpt, _ = _cpt()
    ps = R.synthetic_param_set("all", H, D, RANK, S, seed=21, dtype=torch.bfloat16,
                               peft_init=True, b_std=0.01)
    gen = torch.Generator().manual_seed(22)
    x = torch.randn(N, H, generator=gen).to(torch.bfloat16)
    gy = torch.randn(N, H, generator=gen).to(torch.bfloat16)
    if batch:
        x, gy = x.view(batch, N // batch, H), gy.view(batch, N // batch, H)
    psd = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in ps.items()}
    got, y = R.run_function_grads(cpt.FlashFFNv3Function.apply, psd, x.to(device), gy.to(device),
                                  "int4", 64, True, ratio)
    ora, y_o = R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, x, gy, "int4", 64,
                                    True, ratio)
    ref, _ = R.ref_grads_fp32(ps, x, gy)
    assert R.rel_frob(y.cpu(), y_o) < 1e-2
    assert set(got) == set(ref)
    for k in ref:
        assert R.rel_frob(got[k].cpu(), ora[k]) < 2e-2, k
        c = R.tensor_cos(got[k].cpu(), ref[k])
        assert c >= (0.99 if k == "grad_x" else 0.98), (k, c)
    eager, _ = R.run_function_grads(cpt.FlashFFNv3Function.apply, psd, x.to(device),
                                    gy.to(device), "int4", 64, False, ratio)
    for k in got:
        assert torch.equal(got[k], eager[k]), k


def test_c3_saved_bytes(device):
    cpt, _ = _cpt()
    ps = {k: (v.to(device) if isinstance(v, torch.Tensor) else v)
          for k, v in R.synthetic_param_set("all", H, D, RANK, S, seed=23).items()}
    params = [v for v in ps.values() if isinstance(v, torch.Tensor)]
    for p in params:
        p.requires_grad_(True)
    x = torch.randn(N, H, device=device).to(torch.bfloat16).requires_grad_(True)
    ptrs = {p.data_ptr() for p in params} | {x.data_ptr()}
    got, entries = R.count_saved_bytes(
        lambda: cpt.FlashFFNv3Function.apply(
            x, ps["w_gate"], ps["a_gate"], ps["b_gate"], ps["w_up"], ps["a_up"], ps["b_up"],
            ps["w_down"], ps["a_down"], ps["b_down"], S, S, S, "int4", 64, True, 0.01), ptrs)
    got += x.nbytes
    k = int(D * 0.01)
    want = R.saved_bytes_closed_form(N, H, D, 4, 64, n_thin=3, rank=RANK, n_outlier=k)
    assert got == want + 2 * D * 2, entries     # + the two int16 slot tables


@pytest.mark.parametrize("ratio,rank,s_up,mode", [(0.01, 16, 2.0, "int4"), (0.0, 16, 2.0, "int8"),
                                                  (0.0, 8, 2.0, "bf16"), (0.01, 16, 1.0, "int4")])
def test_stacked_adapter_products_bitwise(device, monkeypatch, ratio, rank, s_up, mode):
    """Gate and up adapters stacked into one skinny product: x [A_g; A_u]^T in
    the forward, [dg B_g | du B_u] and its one token reduction over x in the
    backward (when s_gate == s_up).  Every output and gradient equals the
    unstacked route bit for bit."""
    cpt, _ = _cpt()
    from compact_amd import flashffn as F
    n, h, d = 512, 256, 768
    ps = R.synthetic_param_set("all", h, d, rank, 2.0, seed=31, dtype=torch.bfloat16,
                               peft_init=True, b_std=0.05)
    ps["s_up"] = s_up
    psd = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in ps.items()}
    gen = torch.Generator().manual_seed(32)
    x = torch.randn(2, n // 2, h, generator=gen).to(torch.bfloat16).to(device)
    gy = torch.randn(2, n // 2, h, generator=gen).to(torch.bfloat16).to(device)
    calls = []
    real = F._stackable
    monkeypatch.setattr(F, "_stackable", lambda p, q: calls.append(1) or real(p, q))
    got, y = R.run_function_grads(cpt.FlashFFNv3Function.apply, psd, x, gy, mode, 64, True, ratio)
    assert calls and real(psd["a_gate"], psd["a_up"])
    monkeypatch.setattr(F, "_stackable", lambda p, q: False)
    want, y2 = R.run_function_grads(cpt.FlashFFNv3Function.apply, psd, x, gy, mode, 64, True,
                                    ratio)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    assert set(got) == set(want)
    for k in want:
        assert torch.equal(got[k].view(torch.int16), want[k].view(torch.int16)), k


@pytest.mark.parametrize("bits,group", [(4, 64), (4, 32), (8, 128)])
@pytest.mark.parametrize("with_lora", [False, 16, 32])
@pytest.mark.parametrize("n,hdim,d", [(384, 256, 1024), (300, 128, 320)])
def test_gate_up_outlier_epilogue_equals_k1(device, bits, group, with_lora, n, hdim, d):
    """F1 with the outlier channels in its codec epilogue equals the dual GEMM
    with a bf16 output (same loop, same accumulators) followed by K1 with
    outliers, bit for bit: h_mid, codes, scales and outlier blocks, with LoRA
    terms of rank 16 or 32 (the kernels for ranks above 16).  The
    (300, 128, 320) case has ragged token and d_ff tiles."""
    if d % group:
        pytest.skip("d_ff not a multiple of the group")
    cpt, G = _cpt()
    from compact_amd import _lib
    gen = torch.Generator(device=device).manual_seed(21)
    x = torch.randn(n, hdim, device=device, generator=gen).to(torch.bfloat16)
    wg = (torch.randn(d, hdim, device=device, generator=gen) * 0.05).to(torch.bfloat16)
    wu = (torch.randn(d, hdim, device=device, generator=gen) * 0.05).to(torch.bfloat16)
    wg[7] *= 30
    wu[(d * 3) // 4] *= 25            # hot channels, as in a trained model
    lk = {}
    if with_lora:
        r = with_lora
        xa_g = (torch.randn(n, r, device=device, generator=gen) * 0.3).to(torch.bfloat16)
        xa_u = (torch.randn(n, r, device=device, generator=gen) * 0.3).to(torch.bfloat16)
        bg = (torch.randn(d, r, device=device, generator=gen) * 0.05).to(torch.bfloat16)
        bu = (torch.randn(d, r, device=device, generator=gen) * 0.05).to(torch.bfloat16)
        lk = dict(lora_gate=(xa_g, bg, 2.0), lora_up=(xa_u, bu, 2.0))
    k = max(1, int(d * 0.01))
    _, hg, hu, *_ = G.ffn_gate_up(x, wg, wu, _lib.CACHE_BF16, group, want_h_mid=False, **lk)
    (slot_g, _), (slot_u, _) = cpt.outlier_select_pair(hg, hu, k)
    ref = cpt.silu_mul_quant_outlier(hg, hu, bits, group, slot_g, slot_u, k)
    out = tuple(torch.empty_like(t) for t in ref)
    code = _lib.CACHE_INT4 if bits == 4 else _lib.CACHE_INT8
    G.ffn_gate_up_outlier(x, wg, wu, code, group, slot_g, slot_u, k, out, **lk)
    for got, want in zip(out, ref):
        assert torch.equal(got.view(torch.uint8), want.view(torch.uint8))


@pytest.mark.parametrize("mode,group", [("int4", 64), ("int8", 128)])
def test_function_outlier_epilogue_route(device, mode, group):
    """The Function's two routes for outlier channels (the rows after the
    first sequence through the outlier-codec epilogue, or every row through a
    bf16 dual GEMM + K1) give the same y, gradients and saved cache bit for
    bit, with LoRA on gate/up/down and a [4, 96, 256] input (first sequence:
    96 rows)."""
    cpt, _ = _cpt()
    from compact_amd import flashffn as FF
    default = FF._F1_OUTLIER_FUSED
    ps = R.synthetic_param_set("all", 256, 512, 16, 2.0, seed=23, dtype=torch.bfloat16,
                               device=device, peft_init=True, b_std=0.01)
    gen = torch.Generator(device=device).manual_seed(24)
    x = torch.randn(4, 96, 256, device=device, generator=gen).to(torch.bfloat16)
    gy = torch.randn(4, 96, 256, device=device, generator=gen).to(torch.bfloat16)
    res = {}
    for fused in (True, False):
        FF._F1_OUTLIER_FUSED = fused
        saved = []

        def pack(t):
            saved.append(t.detach().clone())
            return t
        with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
            got, y = R.run_function_grads(cpt.FlashFFNv3Function.apply, ps, x, gy, mode, group,
                                          True, 0.01)
        res[fused] = (got, y, saved)
    FF._F1_OUTLIER_FUSED = default
    (g1, y1, s1), (g0, y0, s0) = res[True], res[False]
    assert torch.equal(y1.view(torch.int16), y0.view(torch.int16))
    assert set(g1) == set(g0)
    for kk in g1:
        assert torch.equal(g1[kk].view(torch.int16), g0[kk].view(torch.int16)), kk
    assert len(s1) == len(s0)
    for a, b in zip(s1, s0):
        assert a.shape == b.shape and a.dtype == b.dtype
        assert torch.equal(a.view(torch.uint8) if a.dtype != torch.bool else a,
                           b.view(torch.uint8) if b.dtype != torch.bool else b)
