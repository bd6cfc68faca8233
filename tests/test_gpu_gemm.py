"""GPU tests of the MFMA GEMM engine and its fused FlashFFN epilogues.

GEMM numerics are compared with a float32 reference of the same bf16 inputs
(fp32 GEMMs run on the CPU: torch's bf16 batched products are avoided as a
reference); the bar is the bf16 rounding of the output: elementwise
|got - ref| <= 1e-2 |ref| + 1e-3 max|ref|.  Fused kernels must equal their
unfused composition (the same GEMM engine with a plain bf16 store, then the
standalone K1 / K2 kernel) bit for bit: the accumulation order is the same.
Products with K a multiple of 64 (F1 with d_model a multiple of 64) run on a
second main loop (16x16x32 MFMAs, another fp32 summation order); each
composition uses the plain product of the same loop (plain_like_f1,
G.mm_engine).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _cpt():
    import compact_amd
    from compact_amd import gemm
    return compact_amd, gemm


def ref_mm(a, b):
    return a.float().cpu() @ b.float().cpu()


def assert_gemm_close(got, ref):
    got = got.float().cpu()
    tol = 1e-2 * ref.abs() + 1e-3 * ref.abs().max()
    bad = (got - ref).abs() > tol
    assert not bad.any(), f"{int(bad.sum())} elements off; max err {(got - ref).abs().max():.3e}"


def rnd(shape, seed, device, scale=1.0):
    g = torch.Generator(device=device).manual_seed(seed)
    return (torch.randn(*shape, device=device, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("ak", [True, False])
@pytest.mark.parametrize("bk", [True, False])
@pytest.mark.parametrize("mnk", [(256, 256, 64), (300, 264, 136), (8, 512, 512),
                                 (1000, 96, 1024), (512, 1024, 8)])
def test_mm_layouts(device, ak, bk, mnk):
    _, G = _cpt()
    m, n, k = mnk
    a = rnd((m, k), 1, device) if ak else rnd((k, m), 1, device).t()
    b = rnd((n, k), 2, device).t() if bk else rnd((k, n), 2, device)
    got = G.mm(a, b)
    assert got.shape == (m, n)
    assert_gemm_close(got, ref_mm(a, b))


def test_mm_two_pairs(device):
    _, G = _cpt()
    a, b = rnd((384, 256), 3, device), rnd((256, 520), 4, device)
    a2, b2 = rnd((384, 128), 5, device), rnd((128, 520), 6, device)
    got = G.mm2(a, b, a2, b2)
    assert_gemm_close(got, ref_mm(a, b) + ref_mm(a2, b2))


def test_mm_deterministic_and_k_tail(device):
    _, G = _cpt()
    a, b = rnd((512, 200), 7, device), rnd((200, 256), 8, device)
    c1, c2 = G.mm(a, b), G.mm(a, b)
    assert torch.equal(c1, c2)
    assert_gemm_close(c1, ref_mm(a, b))


# Products with K a multiple of 64 and N of 8 run on the 16x16x32 direct-to-LDS
# loop (mm sends products of < 128 tiles with K >= 1024 to split-K instead):
# one k-tile, two (the prologue's pair only), odd tile counts, a last group of
# fewer than 4 tile rows (M 2560), ragged M and N (the last tile row and column
# masked at the store), and operands whose rows are longer than their extent
# (sub-views of wider tensors).
@pytest.mark.parametrize("ak", [True, False])
@pytest.mark.parametrize("bk", [True, False])
@pytest.mark.parametrize("m,n,k,pad", [(256, 256, 64, 0), (256, 512, 128, 0), (768, 256, 192, 8),
                                       (2560, 2304, 960, 0), (4096, 2048, 4096, 64),
                                       (300, 264, 128, 0), (8, 520, 64, 8), (1000, 96, 192, 0),
                                       (257, 1032, 256, 16)])
def test_mm_nt16_loop(device, ak, bk, m, n, k, pad):
    """Every operand layout (K-major: rows of K; MN-major: rows of M or N,
    transposing LDS reads); pad > 0 makes rows longer than their extent."""
    _, G = _cpt()
    a = rnd((m, k + pad), 40, device)[:, :k] if ak else rnd((k, m + pad), 40, device)[:, :m].t()
    b = rnd((n, k + pad), 41, device, 0.05)[:, :k].t() if bk else \
        rnd((k, n + pad), 41, device, 0.05)[:, :n]
    got = G.mm(a, b)
    assert_gemm_close(got, ref_mm(a, b))
    assert torch.equal(got, G.mm(a, b))
    # the engine's product of the same operands: same bf16 rounding of an
    # fp32 sum in another order, so all but a few elements agree exactly
    eng = G.mm_engine(a, b)
    assert_gemm_close(eng, ref_mm(a, b))
    diff = (got.view(torch.int16) != eng.view(torch.int16)).float().mean().item()
    assert diff < 0.05, diff


@pytest.mark.parametrize("ak,bk", [(True, False), (True, True), (False, False)])
@pytest.mark.parametrize("k1,k2", [(64, 64), (192, 320), (1024, 2048)])
def test_mm2_nt16_two_pairs(device, ak, bk, k1, k2):
    """A K-concatenated pair (dg W_g + du W_u) on the 16x16x32 loop: the
    k-tiles switch operand pairs at k1, and the sum is one fp32 accumulation."""
    _, G = _cpt()
    m, n = 512, 768

    def op_a(k, seed):
        return rnd((m, k), seed, device) if ak else rnd((k, m), seed, device).t()

    def op_b(k, seed):
        return rnd((n, k), seed, device, 0.05).t() if bk else rnd((k, n), seed, device, 0.05)

    a, b, a2, b2 = op_a(k1, 50), op_b(k1, 51), op_a(k2, 52), op_b(k2, 53)
    got = G.mm2(a, b, a2, b2)
    ref = ref_mm(a, b) + ref_mm(a2, b2)
    assert_gemm_close(got, ref)
    # the same sum as one product over the concatenated K
    cat = G.mm2(torch.cat([a, a2], 1), torch.cat([b, b2], 0))
    assert torch.equal(got.view(torch.int16), cat.view(torch.int16))


def plain_like_f1(G, x, w):
    """x . w^T in the summation order of F1 without adapter terms: the
    16x16x32 loop when F1 runs on it (ffn_nt16_fits in gemm.hip: d_model a
    multiple of 64), which is also where the plain product runs then (nt16_fits:
    K a multiple of 64, N of 8; these shapes stay off split-K and the skinny
    kernel); else the engine."""
    n, k = x.shape
    if k % 64 == 0:
        assert k < 1024 and w.shape[0] > 32, "mm would leave the 16x16x32 loop"
        return G.linear(x, w)
    return G.mm_engine(x, w.t())


@pytest.mark.parametrize("cache,bits,group", [("int4", 4, 64), ("int8", 8, 128), ("int8", 8, 64),
                                              ("int4", 4, 32), ("bf16", 0, 64),
                                              ("none", 0, 64)])
@pytest.mark.parametrize("n_tok,hid,inter", [(512, 256, 512), (512, 128, 384), (300, 128, 384),
                                             (7, 64, 256)])
def test_gate_up_fused_equals_unfused(device, cache, bits, group, n_tok, hid, inter):
    cpt, G = _cpt()
    from compact_amd import _lib
    code = {"int4": _lib.CACHE_INT4, "int8": _lib.CACHE_INT8, "bf16": _lib.CACHE_BF16,
            "none": _lib.CACHE_NONE}[cache]
    x = rnd((n_tok, hid), 10, device)
    wg = rnd((inter, hid), 11, device, 0.05)
    wu = rnd((inter, hid), 12, device, 0.05)
    hm, hg, hu, qg, sg, qu, su = G.ffn_gate_up(x, wg, wu, code, group)
    # the plain product in the fused kernel's summation order
    hg_ref = plain_like_f1(G, x, wg)
    hu_ref = plain_like_f1(G, x, wu)
    assert_gemm_close(hg_ref, ref_mm(x, wg.t()))
    hm_ref = cpt.silu_mul(hg_ref, hu_ref)
    assert torch.equal(hm.view(torch.int16), hm_ref.view(torch.int16))
    if cache == "bf16":
        assert torch.equal(hg.view(torch.int16), hg_ref.view(torch.int16))
        assert torch.equal(hu.view(torch.int16), hu_ref.view(torch.int16))
    if bits:
        _, rqg, rsg, rqu, rsu = cpt.silu_mul_quant(hg_ref, hu_ref, bits, group)
        assert torch.equal(qg.view(torch.uint8), rqg.view(torch.uint8))
        assert torch.equal(qu.view(torch.uint8), rqu.view(torch.uint8))
        assert torch.equal(sg.view(torch.int16), rsg.view(torch.int16))
        assert torch.equal(su.view(torch.int16), rsu.view(torch.int16))


@pytest.mark.parametrize("cache,bits,group,inter", [("bf16", 0, 64, 264), ("none", 0, 64, 264),
                                                    ("int8", 8, 64, 320), ("int4", 4, 32, 320),
                                                    ("int8", 8, 32, 288)])
@pytest.mark.parametrize("n_tok,hid", [(300, 128), (7, 64)])
def test_gate_up_fused_ragged_dff(device, cache, bits, group, inter, n_tok, hid):
    """F1 with a partial last d_ff tile (d_ff not a multiple of the 128 gate
    columns a tile holds): the interleaved gate/up source rows past d_ff read
    zero and glu_finish masks those columns; the result equals the plain
    product of the same loop, then K1, bit for bit."""
    test_gate_up_fused_equals_unfused(device, cache, bits, group, n_tok, hid, inter)


@pytest.mark.parametrize("cache,bits,group", [("int8", 8, 128), ("int4", 4, 64), ("int4", 4, 32)])
def test_gate_up_codec_mixed_scale_ranges(device, cache, bits, group):
    """F1's codec epilogue over every scale range: rows scaled by 1e-4 give
    fp16-subnormal scales (quotients up to 1.5 qmax, which the clamp
    decides), zero rows scale 0, and the rest normal scales, mixed within
    wavefronts and alone in others.  Codes and scales equal the plain
    product's through K1."""
    cpt, G = _cpt()
    from compact_amd import _lib
    code = {"int4": _lib.CACHE_INT4, "int8": _lib.CACHE_INT8}[cache]
    n_tok, hid, inter = 512, 256, 512
    x = rnd((n_tok, hid), 13, device)
    r = torch.arange(n_tok, device=device)
    f = torch.where((r // 2) % 3 == 0, 1e-4, 1.0)            # mixed within wavefronts
    f = torch.where((r >= 256) & (r < 320), 1e-4, f)          # tiny-only wavefronts
    f = torch.where((r % 37) == 5, 0.0, f)                    # zero rows: scale 0
    x = (x.float() * f[:, None]).to(torch.bfloat16)
    wg = rnd((inter, hid), 14, device, 0.05)
    wu = rnd((inter, hid), 15, device, 0.05)
    hm, _, _, qg, sg, qu, su = G.ffn_gate_up(x, wg, wu, code, group)
    hg_ref = plain_like_f1(G, x, wg)
    hu_ref = plain_like_f1(G, x, wu)
    _, rqg, rsg, rqu, rsu = cpt.silu_mul_quant(hg_ref, hu_ref, bits, group)
    sub = ((rsg.view(torch.int16) > 0) & (rsg.view(torch.int16) < 0x0400)).sum().item()
    zero = (rsg.view(torch.int16) == 0).sum().item()
    assert sub > 100 and zero > 10, (sub, zero)
    assert torch.equal(qg.view(torch.uint8), rqg.view(torch.uint8))
    assert torch.equal(qu.view(torch.uint8), rqu.view(torch.uint8))
    assert torch.equal(sg.view(torch.int16), rsg.view(torch.int16))
    assert torch.equal(su.view(torch.int16), rsu.view(torch.int16))


def plain_like_b1(G, gy, wd):
    """gy . W_d in the summation order of B1 (the dgrad GEMM with the K2
    epilogue): the 16x16x32 loop when d_model is a multiple of 64
    (dgrad_nt16_fits in gemm.hip), where the plain product also runs then
    (these shapes stay off split-K, the skinny kernel and stream-K), else the
    engine."""
    if gy.shape[1] % 64 == 0:
        assert gy.shape[1] < 1024, "mm would leave the 16x16x32 loop"
        return G.mm(gy, wd)
    return G.mm_engine(gy, wd)


@pytest.mark.parametrize("cache,bits,group", [("int4", 4, 64), ("int8", 8, 128), ("int4", 4, 32),
                                              ("bf16", 0, 64)])
@pytest.mark.parametrize("want_h_mid", [True, False])
@pytest.mark.parametrize("n_tok,hid,inter", [(512, 256, 512), (300, 128, 384), (300, 136, 384)])
def test_down_dgrad_fused_equals_unfused(device, cache, bits, group, want_h_mid, n_tok, hid,
                                         inter):
    cpt, G = _cpt()
    from compact_amd import _lib
    code = {"int4": _lib.CACHE_INT4, "int8": _lib.CACHE_INT8, "bf16": _lib.CACHE_BF16}[cache]
    hg = rnd((n_tok, inter), 20, device, 3.0)
    hu = rnd((n_tok, inter), 21, device, 2.0)
    gy = rnd((n_tok, hid), 22, device)
    wd = rnd((hid, inter), 23, device, 0.05)
    if bits:
        _, qg, sg, qu, su = cpt.silu_mul_quant(hg, hu, bits, group)
        dg, du, hm = G.ffn_down_dgrad(gy, wd, code, group, qg, sg, qu, su, want_h_mid)
        gmid = plain_like_b1(G, gy, wd)
        rdg, rdu, rhm = cpt.dequant_swiglu_backward(gmid, qg, sg, qu, su, bits, group,
                                                    want_h_mid=want_h_mid)
    else:
        dg, du, hm = G.ffn_down_dgrad(gy, wd, code, group, hg, None, hu, None, want_h_mid)
        gmid = plain_like_b1(G, gy, wd)
        rdg, rdu, rhm = cpt.swiglu_backward_glu(gmid, hg, hu, want_h_mid)
    assert_gemm_close(gmid, ref_mm(gy, wd))
    assert torch.equal(dg.view(torch.int16), rdg.view(torch.int16))
    assert torch.equal(du.view(torch.int16), rdu.view(torch.int16))
    if want_h_mid:
        assert torch.equal(hm.view(torch.int16), rhm.view(torch.int16))
    else:
        assert hm is None


@pytest.mark.parametrize("cache,bits,group,inter", [("bf16", 0, 64, 264), ("int8", 8, 64, 320),
                                                    ("int4", 4, 32, 320)])
@pytest.mark.parametrize("want_h_mid", [True, False])
def test_down_dgrad_fused_ragged_dff(device, cache, bits, group, inter, want_h_mid):
    """B1 with a partial last d_ff tile: the W_d columns past d_ff read zero
    and dglu_finish masks them."""
    test_down_dgrad_fused_equals_unfused(device, cache, bits, group, want_h_mid, 300, 128, inter)


def test_c2_shapes_gemm_numerics(device):
    """The C2 GEMM shapes (8192 x 4096 x 11008), checked on sampled rows
    against an fp32 product of the same bf16 operands."""
    _, G = _cpt()
    n, h, d = 8192, 4096, 11008
    x = rnd((n, h), 30, device)
    w = rnd((d, h), 31, device, 0.02)
    y = G.linear(x, w)
    rows = torch.arange(0, n, 997, device=device)
    ref = x[rows].float() @ w.float().t()
    assert_gemm_close(y[rows], ref.cpu())
    gy = rnd((n, h), 32, device)
    dw = G.mm(gy.t(), y)            # TN: [H, D] = gy^T @ y, both token-major
    cols = torch.arange(0, d, 1009, device=device)
    ref2 = gy.float().t() @ y[:, cols].float()
    assert_gemm_close(dw[:, cols], ref2.cpu())
    # the forward down projection, K = 11008 (the 16x16x32 NT loop)
    hm = rnd((n, d), 33, device)
    wd = rnd((h, d), 34, device, 0.02)
    yd = G.linear(hm, wd)
    ref3 = hm[rows].float() @ wd.float().t()
    assert_gemm_close(yd[rows], ref3.cpu())


@pytest.mark.parametrize("m,r,k", [(8192, 16, 4096), (8192, 16, 11008), (300, 8, 264),
                                   (1000, 32, 1032), (257, 20, 4104), (64, 16, 256)])
def test_skinny_matches_reference(device, m, r, k):
    """The skinny adapter product (K split across blocks, fp32 partials in a
    fixed order) against an fp32 product of the same bf16 operands; repeated
    calls are bit-identical."""
    _, G = _cpt()
    a = rnd((m, k), 70, device)
    q = rnd((r, k), 71, device, 0.05)
    got = G.skinny(a, q, 2.0)
    assert got.shape == (m, r)
    rows = torch.arange(0, m, max(1, m // 64), device=device)
    assert_gemm_close(got[rows], 2.0 * (a[rows].float().cpu() @ q.float().cpu().t()))
    assert torch.equal(got.view(torch.int16), G.skinny(a, q, 2.0).view(torch.int16))


@pytest.mark.parametrize("m,r,k,splits", [(777, 24, 1096, 3), (8192, 16, 4160, 5), (130, 16, 96, 1),
                                          (300, 32, 2080, 2), (64, 8, 8, 1), (1000, 8, 328, 1)])
def test_skinny_splits_cover_every_k_pass(device, m, r, k, splits):
    """Explicit split counts through the C ABI: each block's k range runs
    k-256 passes through LDS, then single k-64 steps, then k-32 steps whose
    last 8-wide chunks may fall past K (they read zero).  Every shape here
    leaves a different mix of the three, for ranks up to 16 and above."""
    from compact_amd import _lib
    a = rnd((m, k), 72, device)
    q = rnd((r, k), 73, device, 0.05)
    c = torch.empty((m, r), dtype=torch.bfloat16, device=device)
    ws = torch.empty(splits * m * r + 16, dtype=torch.float32, device=device)
    rc = _lib.lib().cpt_gemm_bf16_skinny(a.data_ptr(), k, q.data_ptr(), k, c.data_ptr(), r, m, r, k,
                                         0.5, splits, ws.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    assert_gemm_close(c, 0.5 * (a.float().cpu() @ q.float().cpu().t()))


def test_mm_routes_thin_products_to_skinny(device):
    """mm() with N <= 32 on a row-major A gives the skinny kernel's result,
    including a transposed [K, r] weight view (B = W^T of an [r, K] weight)
    and a [K, r] B factor."""
    _, G = _cpt()
    x = rnd((2048, 4096), 72, device)
    a_w = rnd((16, 4096), 73, device, 0.02)       # LoRA A [r, in]
    b_w = rnd((4096, 16), 74, device, 0.02)       # LoRA B [out, r]
    assert torch.equal(G.mm(x, a_w.t()).view(torch.int16), G.skinny(x, a_w).view(torch.int16))
    got = G.mm(x, b_w)
    assert torch.equal(got.view(torch.int16), G.skinny(x, b_w.t().contiguous()).view(torch.int16))
    assert_gemm_close(got, ref_mm(x, b_w))


@pytest.mark.parametrize("t,n,r", [(8192, 11008, 16), (8192, 4096, 16), (1000, 264, 8),
                                   (300, 136, 32), (4097, 1024, 24)])
@pytest.mark.parametrize("trans", [False, True])
def test_skinny_t_matches_reference(device, t, n, r, trans):
    """The token reduction of the adapter gradients, alpha * x^T p (or its
    transpose), against an fp32 product of the same bf16 operands; repeated
    calls are bit-identical."""
    _, G = _cpt()
    x = rnd((t, n), 80, device)
    p = rnd((t, r), 81, device, 0.05)
    got = G.skinny_t(x, p, 2.0, trans=trans)
    assert got.shape == ((r, n) if trans else (n, r))
    cols = torch.arange(0, n, max(1, n // 48), device=device)
    ref = 2.0 * (x[:, cols].float().cpu().t() @ p.float().cpu())
    sub = got[:, cols].t() if trans else got[cols]
    assert_gemm_close(sub, ref)
    assert torch.equal(got.view(torch.int16), G.skinny_t(x, p, 2.0, trans=trans).view(torch.int16))


def test_mm_splitk_routes_adapter_gradients(device):
    """mm_splitk on the two adapter-gradient patterns (s (gB)^T x and
    s gy^T (xA)) gives the token-reduction kernel's result."""
    _, G = _cpt()
    x = rnd((2048, 1024), 82, device)
    gb = rnd((2048, 16), 83, device, 0.1)
    got = G.mm_splitk(gb.t(), x, 0.5)
    assert torch.equal(got.view(torch.int16), G.skinny_t(x, gb, 0.5, trans=True).view(torch.int16))
    got2 = G.mm_splitk(x.t(), gb, 0.5)
    assert torch.equal(got2.view(torch.int16), G.skinny_t(x, gb, 0.5).view(torch.int16))
    assert_gemm_close(got2, 0.5 * ref_mm(x.t(), gb))


@pytest.mark.parametrize("shape", [0, 1])
def test_mfma_probe_runs_and_scales_with_iters(device, shape):
    """The register-only MFMA probe behind the achievable-peak figure: each
    wavefront's partial grows linearly with the round count (the rounds
    repeat the same products), and invalid arguments are rejected."""
    from compact_amd import _lib
    lib = _lib.lib()
    out1 = torch.empty(8 * 4, dtype=torch.float32, device=device)
    out3 = torch.empty_like(out1)
    s = torch.cuda.current_stream().cuda_stream
    assert lib.cpt_probe_mfma_rate(shape, 8, 1, 0.5, out1.data_ptr(), s) == 0
    assert lib.cpt_probe_mfma_rate(shape, 8, 3, 0.5, out3.data_ptr(), s) == 0
    torch.cuda.synchronize()
    assert torch.isfinite(out1).all() and out1.abs().sum() > 0
    torch.testing.assert_close(out3, 3 * out1, rtol=1e-4, atol=1e-3)
    assert lib.cpt_probe_mfma_rate(shape, 0, 1, 0.5, out1.data_ptr(), s) != 0
    assert lib.cpt_probe_mfma_rate(shape, 8, 0, 0.5, out1.data_ptr(), s) != 0
    assert lib.cpt_probe_mfma_rate(2, 8, 1, 0.5, out1.data_ptr(), s) != 0


@pytest.mark.parametrize("rows,cols", [(8, 8), (64, 64), (136, 200), (1024, 4096), (8200, 264)])
def test_transpose_bf16(device, rows, cols):
    """cpt_transpose_bf16 against torch's transposed copy, bit for bit:
    whole and partial 64 x 64 tiles, and a strided source (row stride past
    the column count)."""
    _, G = _cpt()
    x = rnd((rows, cols), 31, device)
    assert torch.equal(G.transpose(x), x.t().contiguous())
    wide = rnd((rows, cols + 24), 32, device)
    v = wide[:, 8:8 + cols]
    assert torch.equal(G.transpose(v), v.t().contiguous())


@pytest.mark.parametrize("mode", ["int8", "bf16"])
def test_wgrad_transposed_x_route_bitwise(device, monkeypatch, mode):
    """The full fine-tune weight gradients dg^T x and du^T x read x^T as a
    K-major operand from _XT_MIN_TOKENS tokens on: forced either way at one
    shape, every output and gradient is bit-identical."""
    from compact_amd import flashffn as FF
    from oracle import flashffn_ref as R
    cpt, _ = _cpt()
    ps = R.synthetic_param_set("fullft", 256, 768, 16, 2.0, seed=7, dtype=torch.bfloat16)
    ps = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in ps.items()}
    x = rnd((520, 256), 33, device)
    gy = rnd((520, 256), 34, device)
    out = {}
    for threshold in (0, 10 ** 9):
        monkeypatch.setattr(FF, "_XT_MIN_TOKENS", threshold)
        out[threshold] = R.run_function_grads(cpt.FlashFFNv3Function.apply, ps, x, gy, mode, 64,
                                              True)
    (g0, y0), (g1, y1) = out[0], out[10 ** 9]
    assert torch.equal(y0, y1)
    assert set(g0) == set(g1) and "w_gate" in g0 and "w_up" in g0
    for k in g0:
        assert torch.equal(g0[k], g1[k]), k
