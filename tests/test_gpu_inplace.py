"""In-place GLU backward (the reference's memory lever, src/flashffn.py:129-198,
259-293, 3368-3392): gradients written over buffers private to the backward.

  * kernel level: K2 with grad_h_gate over grad_h_mid, the fused dgrad GEMM
    with grad_h_gate / grad_h_up over a bf16 cache, and the GLU backward over
    its inputs each equal their out-of-place call bit for bit;
  * Function level: the 'recompute' cache (whose recomputed h_gate / h_up the
    backward overwrites) gives gradients bitwise equal to the 'bf16' cache
    (the same values, saved and therefore never overwritten);
  * memory: at config C2's size in 'recompute' mode the backward's peak stays
    within 3 live [N, D] buffers plus the gradients it returns.
"""

import pytest
import torch

from oracle import flashffn_ref as R

pytestmark = pytest.mark.gpu


def _mods():
    import compact_amd
    from compact_amd import _lib, gemm, kernels
    return compact_amd, _lib, gemm, kernels


def _bits_equal(a, b):
    assert a.shape == b.shape and a.dtype == b.dtype
    assert torch.equal(a.view(torch.int16) if a.element_size() == 2 else a.view(torch.int32),
                       b.view(torch.int16) if b.element_size() == 2 else b.view(torch.int32))


@pytest.mark.parametrize("bits,gs,outl", [(8, 128, False), (4, 64, False), (4, 64, True)])
def test_k2_over_grad_h_mid(device, bits, gs, outl):
    _, _, _, K = _mods()
    gen = torch.Generator(device=device).manual_seed(1)
    n, d = 300, 1024
    hg = torch.randn(n, d, device=device, generator=gen).to(torch.bfloat16)
    hu = torch.randn(n, d, device=device, generator=gen).to(torch.bfloat16)
    ghm = torch.randn(n, d, device=device, generator=gen).to(torch.bfloat16)
    if outl:
        k = 10
        slot_g, _ = K.outlier_select(hg, k, n)
        slot_u, _ = K.outlier_select(hu, k, n)
        qg, sg, og = K.v3_quantize_outlier(hg, bits, gs, slot_g, k)
        qu, su, ou = K.v3_quantize_outlier(hu, bits, gs, slot_u, k)
        ref = K.dequant_swiglu_backward_outlier(ghm, qg, sg, og, slot_g, qu, su, ou, slot_u,
                                                bits, gs, want_h_mid=True)
        buf = ghm.clone()
        got = K.dequant_swiglu_backward_outlier(buf, qg, sg, og, slot_g, qu, su, ou, slot_u,
                                                bits, gs, want_h_mid=True, inplace=True)
    else:
        qg, sg = K.v3_quantize_group_absmax(hg, bits, gs)
        qu, su = K.v3_quantize_group_absmax(hu, bits, gs)
        ref = K.dequant_swiglu_backward(ghm, qg, sg, qu, su, bits, gs, want_h_mid=True)
        buf = ghm.clone()
        got = K.dequant_swiglu_backward(buf, qg, sg, qu, su, bits, gs, want_h_mid=True,
                                        inplace=True)
    assert got[0].data_ptr() == buf.data_ptr()
    for a, b in zip(got, ref):
        _bits_equal(a, b)


@pytest.mark.parametrize("lora", [False, True])
def test_fused_dgrad_over_bf16_cache(device, lora):
    _, L, G, _ = _mods()
    gen = torch.Generator(device=device).manual_seed(2)
    n, h, d, r = 512, 256, 768, 16
    gy = torch.randn(n, h, device=device, generator=gen).to(torch.bfloat16)
    wd = (torch.randn(h, d, device=device, generator=gen) * 0.02).to(torch.bfloat16)
    hg = torch.randn(n, d, device=device, generator=gen).to(torch.bfloat16)
    hu = torch.randn(n, d, device=device, generator=gen).to(torch.bfloat16)
    lt = None
    if lora:
        p = torch.randn(n, r, device=device, generator=gen).to(torch.bfloat16)
        a = (torch.randn(r, d, device=device, generator=gen) * 0.05).to(torch.bfloat16)
        lt = (p, a, 2.0)
    ref = G.ffn_down_dgrad(gy, wd, L.CACHE_BF16, 64, hg, None, hu, None, True, lora=lt)
    bg, bu = hg.clone(), hu.clone()
    got = G.ffn_down_dgrad(gy, wd, L.CACHE_BF16, 64, bg, None, bu, None, True, lora=lt,
                           inplace=True)
    assert got[0].data_ptr() == bg.data_ptr() and got[1].data_ptr() == bu.data_ptr()
    for a_, b_ in zip(got, ref):
        _bits_equal(a_, b_)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_glu_backward_over_inputs(device, dtype):
    _, _, _, K = _mods()
    gen = torch.Generator(device=device).manual_seed(3)
    n = 1000 * 8 + 5                            # a ragged tail past the 8-wide chunks
    ghm, hg, hu = (torch.randn(n, device=device, generator=gen).to(dtype) for _ in range(3))
    ref = K.swiglu_backward_glu(ghm, hg, hu, True)
    b = [t.clone() for t in (ghm, hg, hu)]
    got = K.swiglu_backward_glu(b[0], b[1], b[2], True, inplace=True)
    assert got[0].data_ptr() == b[1].data_ptr() and got[2].data_ptr() == b[0].data_ptr()
    for a_, b_ in zip(got, ref):
        assert torch.equal(a_, b_)


@pytest.mark.parametrize("config", ["all", "fullft", "gateup"])
@pytest.mark.parametrize("dtype,hd", [(torch.bfloat16, (256, 768)), (torch.float32, (64, 200)),
                                      (torch.bfloat16, (64, 200))])
def test_recompute_equals_bf16_cache_bitwise(device, config, dtype, hd):
    """'recompute' rebuilds h_gate / h_up with the forward's own kernel and
    then overwrites them; 'bf16' reads the saved values and does not: the
    gradients agree bit for bit.  (64, 200) is off the bf16 engine's 8-wide
    layout, so it runs the unfused GLU backward over its inputs."""
    cpt, _, _, _ = _mods()
    h, d = hd
    ps = R.synthetic_param_set(config, h, d, 16, 2.0, seed=5, dtype=dtype)
    psd = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in ps.items()}
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(129, h, generator=gen).to(dtype).to(device)
    gy = torch.randn(129, h, generator=gen).to(dtype).to(device)
    g_re, y_re = R.run_function_grads(cpt.FlashFFNv3Function.apply, psd, x, gy, "recompute", 64)
    g_bf, y_bf = R.run_function_grads(cpt.FlashFFNv3Function.apply, psd, x, gy, "bf16", 64)
    assert torch.equal(y_re, y_bf)
    assert set(g_re) == set(g_bf)
    for k in g_re:
        assert torch.equal(g_re[k], g_bf[k]), k


def test_recompute_backward_peak_at_c2(device):
    """C2 (8192 x 4096 x 11008, full-FT) in 'recompute' mode.  The backward
    recomputes h_gate / h_up (2 [N, D]), writes grad_h_gate / grad_h_up over
    them and h_mid^ next to them (3 live [N, D]), then returns grad_x [N, H]
    and three [D, H] weight gradients.  Without the in-place writes it would
    hold 5 [N, D] at once."""
    cpt, _, _, _ = _mods()
    n, h, d = 8192, 4096, 11008
    gen = torch.Generator(device=device).manual_seed(7)
    x = torch.randn(n, h, device=device, generator=gen).to(torch.bfloat16).requires_grad_()
    gy = torch.randn(n, h, device=device, generator=gen).to(torch.bfloat16)
    ws = [(torch.randn(*s, device=device, generator=gen) * 0.02).to(torch.bfloat16)
          .requires_grad_() for s in ((d, h), (d, h), (h, d))]
    y = cpt.FlashFFNv3Function.apply(x, ws[0], None, None, ws[1], None, None, ws[2], None, None,
                                     0.0, 0.0, 0.0, "recompute", 64)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    y.backward(gy)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base
    nd, grads = n * d * 2, 3 * d * h * 2 + n * h * 2
    assert peak <= 3 * nd + grads + (32 << 20), (peak / 1e6, (3 * nd + grads) / 1e6)
    assert peak < 5 * nd, peak / 1e6
