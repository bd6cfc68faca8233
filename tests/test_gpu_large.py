"""Operands beyond 2 GiB: ~100k tokens at d_ff 11008 make every [N, d_ff]
bf16 tensor 2.2 GB, past the reach of one 32-bit buffer offset.  The
kernels start each block's buffer resource where its reads start, and the
host splits the long-k products (weight and adapter gradients) into ranges
that fit.

Inputs repeat one block of rows R times, so the checks need no CPU pass over
the full size:
- row-wise outputs (GEMM rows, y, grad_x, codes) of the last block, which lie
  past 2 GiB, equal the first block's bit for bit (same row content, same
  kernel, same accumulation order: these tests run without the stream-K
  schedule, whose shared tiles sum k in another order; one test repeats its
  product with it and checks the last block within a bf16 rounding);
- reductions over the tokens (weight and adapter gradients) equal R times
  the oracle's value on one block, within the bf16 / fp32 split-sum
  tolerance written in each test.
"""

import pytest
import torch

from oracle import flashffn_ref as R

# the bitwise row checks need every row summed in one order: no stream-K
pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("no_stream_k")]

BLOCK = 512
REPS = 196                    # 100352 tokens
D_FF = 11008                  # [100352, 11008] bf16 = 2.21 GB


def _cpt():
    import compact_amd
    from compact_amd import gemm
    return compact_amd, gemm


def _rep(t, reps=REPS):
    return t.repeat(reps, 1)


def _same_rows(t, rows=BLOCK):
    assert torch.equal(t[-rows:].view(torch.int16), t[:rows].view(torch.int16))


def test_kmajor_operand_over_2gib(device):
    """x [100352, 11008] @ W^T: the A panel of the last row tiles starts past
    2 GiB."""
    _, G = _cpt()
    gen = torch.Generator(device=device).manual_seed(31)
    ab = torch.randn(BLOCK, D_FF, device=device, generator=gen).to(torch.bfloat16)
    w = (torch.randn(384, D_FF, device=device, generator=gen) * 0.02).to(torch.bfloat16)
    a = _rep(ab)
    assert a.numel() * 2 > (1 << 31)
    c = G.linear(a, w)
    _same_rows(c)
    ref = ab.float().cpu() @ w.float().cpu().t()
    got = c[:BLOCK].float().cpu()
    assert ((got - ref).abs() <= 2 ** -7 * ref.abs() + 1e-3).all()
    # with stream-K (784 tiles: the last 272 share their k-iterations)
    G.set_stream_k(True)
    c_sk = G.linear(a, w)
    G.set_stream_k(False)
    last = c_sk[-BLOCK:].float().cpu()
    assert ((last - ref).abs() <= 2 ** -7 * ref.abs() + 1e-3).all()
    assert ((c_sk.float() - c.float()).abs() <= 2 ** -7 * c.float().abs() + 1e-3).all()
    del a, c, c_sk


@pytest.mark.parametrize("m", [4096, 256])
def test_transposed_long_k_over_2gib(device, m):
    """g^T @ h over 100352 tokens with h [100352, 11008]: the host splits k so
    each block's range of the transposed operand stays within 32-bit
    offsets.  m = 4096 takes the 256x256-tile path, m = 256 the thin one."""
    _, G = _cpt()
    gen = torch.Generator(device=device).manual_seed(32)
    gb = torch.randn(BLOCK, m, device=device, generator=gen).to(torch.bfloat16)
    hb = torch.randn(BLOCK, D_FF, device=device, generator=gen).to(torch.bfloat16)
    g, h = _rep(gb), _rep(hb)
    dw = G.mm(g.t(), h)
    ref = REPS * (gb.double().cpu().t() @ hb.double().cpu())
    # bf16 output rounding plus fp32 accumulation over 100352 terms
    tol = 2 ** -7 * ref.abs() + 1e-4 * (gb.double().cpu().t().abs() @ hb.double().cpu().abs()) * REPS
    assert ((dw.double().cpu() - ref).abs() <= tol).all()
    del g, h


def test_adapter_products_over_2gib(device):
    """The rank-16 adapter kernels over 100352 tokens of d_ff 11008: the
    projection h_mid A^T (rows past 2 GiB) and the token reduction
    h_mid^T (gy B) (splits forced by the operand size)."""
    _, G = _cpt()
    gen = torch.Generator(device=device).manual_seed(33)
    hb = torch.randn(BLOCK, D_FF, device=device, generator=gen).to(torch.bfloat16)
    a_d = (torch.randn(16, D_FF, device=device, generator=gen) * 0.01).to(torch.bfloat16)
    pb = torch.randn(BLOCK, 16, device=device, generator=gen).to(torch.bfloat16)
    h, p = _rep(hb), _rep(pb)
    proj = G.skinny(h, a_d)
    _same_rows(proj)
    ref = hb.double().cpu() @ a_d.double().cpu().t()
    assert ((proj[:BLOCK].double().cpu() - ref).abs() <= 2 ** -7 * ref.abs() + 1e-3).all()
    red = G.skinny_t(h, p)                  # [11008, 16] = h^T p
    ref = REPS * (hb.double().cpu().t() @ pb.double().cpu())
    scale = REPS * (hb.double().cpu().t().abs() @ pb.double().cpu().abs())
    assert ((red.double().cpu() - ref).abs() <= 2 ** -7 * ref.abs() + 1e-4 * scale).all()
    del h, p


@pytest.mark.parametrize("cfg,mode,gs,ratio", [("fullft", "int8", 128, 0.0),
                                                ("all", "int4", 64, 0.01)])
def test_function_over_2gib(device, cfg, mode, gs, ratio):
    """FlashFFNv3Function at 100352 tokens, d_model 512, d_ff 11008: every
    [N, d_ff] activation, cache payload and gradient exceeds or nears 2 GiB.
    Row outputs of the last block equal the first block's bitwise and the
    oracle's within the usual tolerance; token reductions equal REPS times
    the oracle's on one block."""
    cpt, _ = _cpt()
    h = 512
    ps = R.synthetic_param_set(cfg, h, D_FF, 16, 2.0, seed=34, dtype=torch.bfloat16,
                               peft_init=True, b_std=0.01)
    gen = torch.Generator().manual_seed(35)
    xb = torch.randn(BLOCK, h, generator=gen).to(torch.bfloat16)
    gyb = torch.randn(BLOCK, h, generator=gen).to(torch.bfloat16)
    psd = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in ps.items()}
    x, gy = _rep(xb.to(device)), _rep(gyb.to(device))
    got, y = R.run_function_grads(cpt.FlashFFNv3Function.apply, psd, x, gy, mode, gs, True,
                                  ratio)
    _same_rows(y)
    _same_rows(got["grad_x"])
    ora, y_o = R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, xb, gyb, mode, gs,
                                    True, ratio)
    assert R.rel_frob(y[:BLOCK].cpu(), y_o) < 1e-2
    assert R.rel_frob(got["grad_x"][:BLOCK].cpu(), ora["grad_x"]) < 2e-2
    for k in ora:
        if k == "grad_x":
            continue
        assert R.rel_frob(got[k].cpu().double() / REPS, ora[k]) < 2e-2, k
