"""The allocation-free entry point cpt_gemm_bf16_skinny_t_noalloc, called
through the C ABI: its output equals cpt_gemm_bf16_skinny_t's (same kernels,
same split order, partials in the library's fixed per-GPU scratch instead of
a torch workspace) bit for bit, on two calls in a row, the second smaller
(the scratch keeps the first call's partials, which the second must not
see); a call whose partials exceed the scratch is refused before any launch.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _noalloc(x, p, alpha, trans, splits):
    from compact_amd import _lib
    T, N = x.shape
    R = p.shape[1]
    out = torch.empty((R, N) if trans else (N, R), dtype=torch.bfloat16, device=x.device)
    rc = _lib.lib().cpt_gemm_bf16_skinny_t_noalloc(
        x.data_ptr(), x.stride(0), p.data_ptr(), p.stride(0), out.data_ptr(), out.stride(0),
        1 if trans else 0, T, N, R, alpha, splits, torch.cuda.current_stream().cuda_stream)
    return rc, out


def test_noalloc_equals_workspace_entry_point(device):
    from compact_amd import _lib
    from compact_amd import gemm as G
    gen = torch.Generator(device=device).manual_seed(3)
    for T, N, R, alpha, trans in ((8192, 11008, 16, 2.0, False), (300, 4096, 8, 0.5, True)):
        x = torch.randn(T, N, device=device, generator=gen).to(torch.bfloat16)
        p = torch.randn(T, R, device=device, generator=gen).to(torch.bfloat16)
        ref = G.skinny_t(x, p, alpha, trans)
        rc, got = _noalloc(x, p, alpha, trans, G.skinny_t_splits(T, N))
        assert rc == _lib.OK, _lib.lib().cpt_status_string(rc)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (T, N, R)
        exact = alpha * (x.double().t() @ p.double())
        exact = exact.t() if trans else exact
        scale = alpha * (x.double().abs().t() @ p.double().abs())
        scale = scale.t() if trans else scale
        assert ((got.double() - exact).abs() <= 2 ** -8 * exact.abs() + 1e-5 * scale).all()


def test_noalloc_wrapper_and_size_limit(device):
    from compact_amd import _lib
    from compact_amd import gemm as G
    gen = torch.Generator(device=device).manual_seed(4)
    x = torch.randn(512, 1024, device=device, generator=gen).to(torch.bfloat16)
    p = torch.randn(512, 16, device=device, generator=gen).to(torch.bfloat16)
    out = torch.empty(1024, 16, dtype=torch.bfloat16, device=device)
    assert G.skinny_t_noalloc(x, p, out, 1.5) is out
    assert torch.equal(out, G.skinny_t(x, p, 1.5))
    # 64 splits x 11008 x 32 fp32 partials = 90 MB > the 16 MiB scratch
    xb = torch.zeros(8192, 11008, dtype=torch.bfloat16, device=device)
    pb = torch.zeros(8192, 32, dtype=torch.bfloat16, device=device)
    rc, _ = _noalloc(xb, pb, 1.0, False, 64)
    assert rc == _lib.ERR_TOO_LARGE
    with pytest.raises(AssertionError, match="scratch"):
        G.skinny_t_noalloc(xb, pb, torch.empty(11008, 32, dtype=torch.bfloat16, device=device),
                           splits=64)
