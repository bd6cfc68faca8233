"""The LoRA backward's two thin products of one tensor in one pass
(cpt_gemm_bf16_skinny_dual): C = x Q^T (the projection) and Z = x^T P (the
token reduction), checked against float32 products of the same bf16
operands (bf16 output rounding: 2^-7 relative plus an fp32 summation
allowance), against the separate skinny kernels within the same bound, for
determinism, and for the Function routed through it against the separate
kernels."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _G():
    from compact_amd import gemm
    return gemm


def rnd(shape, seed, device, scale=1.0):
    g = torch.Generator(device=device).manual_seed(seed)
    return (torch.randn(*shape, device=device, generator=g) * scale).to(torch.bfloat16)


def _close(got, ref, scale):
    got = got.float().cpu()
    tol = 2 ** -7 * ref.abs() + 1e-5 * scale
    return bool(((got - ref).abs() <= tol).all()), float((got - ref).abs().max())


@pytest.mark.parametrize("q_as_b", [False, True])
@pytest.mark.parametrize("T,N,R", [(8192, 11008, 16), (300, 520, 8), (1000, 4096, 32),
                                   (64, 1024, 24), (33, 512, 16)])
def test_skinny_dual_against_fp32(device, T, N, R, q_as_b):
    """q_as_b: Q given as the transposed view of a B factor [N, R] (read in
    place) instead of rank rows [R, N]; same bits either way."""
    G = _G()
    x = rnd((T, N), 1, device)
    q = rnd((R, N), 2, device, 0.05)
    if q_as_b:
        q = q.t().contiguous().t()
    p = rnd((T, R), 3, device, 0.5)
    c, z = G.skinny_dual(x, q, p, 1.0, 2.0)
    c2, z2 = G.skinny_dual(x, q, p, 1.0, 2.0)
    assert torch.equal(c.view(torch.int16), c2.view(torch.int16))
    assert torch.equal(z.view(torch.int16), z2.view(torch.int16))
    xd, qd, pd = x.double().cpu(), q.double().cpu(), p.double().cpu()
    ref_c = xd @ qd.t()
    ref_z = 2.0 * (xd.t() @ pd)
    ok, err = _close(c, ref_c, (xd.abs() @ qd.abs().t()))
    assert ok, err
    ok, err = _close(z, ref_z, 2.0 * (xd.abs().t() @ pd.abs()))
    assert ok, err
    # the separate kernels, within the same bound of each other's reference
    c_sep = G.skinny(x, q, 1.0)
    z_sep = G.skinny_t(x, p, 2.0)
    assert _close(c_sep, ref_c, xd.abs() @ qd.abs().t())[0]
    assert _close(z_sep, ref_z, 2.0 * (xd.abs().t() @ pd.abs()))[0]


def test_skinny_dual_into_a_column_half(device):
    """C written into the column half of a wider buffer (the Function's
    [grad_h_gate B_g | grad_h_up B_u] block); the other half is untouched."""
    G = _G()
    T, N, R = 700, 1536, 16
    x, q, p = rnd((T, N), 4, device), rnd((R, N), 5, device, 0.05), rnd((T, R), 6, device)
    buf = torch.full((T, 2 * R), 7.0, dtype=torch.bfloat16, device=device)
    c, _ = G.skinny_dual(x, q, p, out_c=buf[:, R:])
    alone, _ = G.skinny_dual(x, q, p)
    assert torch.equal(buf[:, R:].view(torch.int16), alone.view(torch.int16))
    assert (buf[:, :R] == 7.0).all()


@pytest.mark.parametrize("mode,group", [("int4", 64), ("int8", 128)])
def test_function_dual_route_matches_separate(device, mode, group):
    """FlashFFNv3Function with LoRA on gate/up/down: the backward through the
    one-pass kernel against the separate projection and reduction kernels:
    y bit-identical (the forward is the same), the B gradients within the
    bf16 rounding of each other, and grad_x and the A gradients (which take
    the projection through further products) within rel 1e-2."""
    import compact_amd
    from compact_amd import flashffn as FF
    from oracle import flashffn_ref as R
    ps = R.synthetic_param_set("all", 1024, 2048, 16, 2.0, seed=7, dtype=torch.bfloat16,
                               device=device, peft_init=True, b_std=0.01)
    gen = torch.Generator(device=device).manual_seed(8)
    x = torch.randn(2, 512, 1024, device=device, generator=gen).to(torch.bfloat16)
    gy = torch.randn(2, 512, 1024, device=device, generator=gen).to(torch.bfloat16)
    res = {}
    for dual in (True, False):
        FF._DUAL_SKINNY = dual
        res[dual] = R.run_function_grads(compact_amd.FlashFFNv3Function.apply, ps, x, gy, mode,
                                         group, True, 0.01)
    FF._DUAL_SKINNY = True
    (g1, y1), (g0, y0) = res[True], res[False]
    assert torch.equal(y1.view(torch.int16), y0.view(torch.int16))
    for k in g1:
        if k.startswith("b_"):
            diff = (g1[k].float() - g0[k].float()).abs()
            assert (diff <= 2 ** -7 * g0[k].float().abs() + 1e-3 * g0[k].float().abs().max()).all(), k
        else:
            rel = ((g1[k].float() - g0[k].float()).norm() / g0[k].float().norm()).item()
            assert rel < 1e-2, (k, rel)
