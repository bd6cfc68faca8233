"""The down projection's weight gradient with the GLU decompressed in the
GEMM's operand staging (cpt_gemm_wgrad_glu): grad_y^T . h^ with h^ built
from the int4/int8 cache as the B tiles are staged.  h^ is K2's h_mid^ bit for
bit, and the GEMM's accumulation order is the plain TN GEMM's, so the result
equals gy^T @ K2's h_mid^ bit for bit; the Function routed through it gives
the same gradients bit for bit."""

import pytest
import torch

from oracle import flashffn_ref as R

pytestmark = pytest.mark.gpu


def _mods():
    import compact_amd
    from compact_amd import _lib, gemm, kernels
    return compact_amd, _lib, gemm, kernels


@pytest.mark.parametrize("bits,gs", [(8, 128), (8, 64), (8, 32), (4, 64), (4, 32), (4, 128)])
@pytest.mark.parametrize("n,h,d", [(8192, 4096, 11008), (300, 256, 768), (129, 64, 256),
                                   (1, 256, 512)])
def test_wgrad_glu_equals_k2_then_gemm(device, bits, gs, n, h, d):
    _, L, G, K = _mods()
    if d % gs:
        pytest.skip("group must divide d_ff")
    gen = torch.Generator(device=device).manual_seed(n + h + d + bits + gs)
    hg = (torch.randn(n, d, device=device, generator=gen) * 3).to(torch.bfloat16)
    hu = (torch.randn(n, d, device=device, generator=gen) * 2).to(torch.bfloat16)
    gm = torch.randn(n, d, device=device, generator=gen).to(torch.bfloat16)
    gy = torch.randn(n, h, device=device, generator=gen).to(torch.bfloat16)
    _, qg, sg, qu, su = K.silu_mul_quant(hg, hu, bits, gs)
    _, _, hm = K.dequant_swiglu_backward(gm, qg, sg, qu, su, bits, gs, want_h_mid=True)
    ref = G.mm_engine(gy.t(), hm)   # the fused kernel runs on the engine
    cache = L.CACHE_INT8 if bits == 8 else L.CACHE_INT4
    got = G.wgrad_glu(gy, cache, gs, qg, sg, qu, su)
    assert got.shape == (h, d)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_wgrad_glu_rejects_bad_arguments(device):
    _, L, G, K = _mods()
    gy = torch.zeros(16, 64, dtype=torch.bfloat16, device=device)
    q = torch.zeros(16, 96, dtype=torch.int8, device=device)
    s = torch.zeros(16, 1, dtype=torch.float16, device=device)
    with pytest.raises(AssertionError):              # 96 columns: no whole group of 128
        G.wgrad_glu(gy, L.CACHE_INT8, 128, q, s, q, s)
    with pytest.raises(AssertionError):              # no fused kernel for groups of 16
        G.wgrad_glu(gy, L.CACHE_INT8, 16, q, torch.zeros(16, 6, dtype=torch.float16,
                                                         device=device), q, s)


@pytest.mark.parametrize("config,mode,gs", [("fullft", "int8", 128), ("all", "int4", 64),
                                            ("fullft", "int4", 32)])
def test_function_through_wgrad_glu_is_bitwise_equal(device, monkeypatch, config, mode, gs):
    """The Function with grad_w_down from the cache equals the default route
    (K2's h_mid^ and the plain GEMM) bit for bit; with LoRA on the down
    projection K2 still writes h_mid^ for the adapter gradient."""
    cpt, _, _, _ = _mods()
    from compact_amd import flashffn
    ps = R.synthetic_param_set(config, 256, 768, 16, 2.0, seed=7, dtype=torch.bfloat16)
    psd = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in ps.items()}
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(300, 256, generator=gen).to(torch.bfloat16).to(device)
    gy = torch.randn(300, 256, generator=gen).to(torch.bfloat16).to(device)
    base, y0 = R.run_function_grads(cpt.FlashFFNv3Function.apply, psd, x, gy, mode, gs)
    monkeypatch.setattr(flashffn, "_FUSED_WGRAD_GLU", True)
    from compact_amd.kernels import KernelTimer
    with KernelTimer() as kt:
        got, y1 = R.run_function_grads(cpt.FlashFFNv3Function.apply, psd, x, gy, mode, gs)
    assert "gemm_wgrad_down_glu" not in kt.events          # named as the GEMM it replaces
    assert torch.equal(y0, y1)
    for k in base:
        assert torch.equal(base[k], got[k]), k
