"""GPU parity of the v1/v2 FlashFFN API (src/flashffn.py:300-519):

  kernels   topk_abs and topk_scatter bit-exact against the oracle (same
            values, same int16 columns, same order: the tie rule is fixed),
            on random, heavily tied and edge-sized rows;
  Function  FlashFFNFunction against OracleFlashFFNFunction in both modes
            (bf16 rel 2e-2 -- the top-K set follows h_mid's bf16 bits, which
            the GPU and CPU GEMMs round differently near the threshold;
            float32 1e-5 with k_fraction = 1);
  modules   FlashFFN against StandardFFN on the same weights.
"""

import pytest
import torch

from oracle import flashffn_ref as R

pytestmark = pytest.mark.gpu


def _cpt():
    import compact_amd
    return compact_amd


def _bits(t):
    return t.contiguous().view(torch.int16) if t.dtype != torch.float32 else t


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("kind", ["random", "ties"])
@pytest.mark.parametrize("n,d,k", [(64, 5632, 1689), (33, 100, 7), (8, 300, 300), (5, 37, 1),
                                   (3, 1, 1), (16, 11008, 3302)])
def test_topk_abs_bitexact(device, dtype, kind, n, d, k):
    cpt = _cpt()
    g = torch.Generator().manual_seed(n * d + k)
    if kind == "random":
        t = torch.randn(n, d, generator=g).to(dtype)
    else:
        t = torch.randint(-3, 4, (n, d), generator=g).to(dtype)
    v_o, i_o = R.topk_abs(t, k)
    v, i = cpt.topk_abs(t.to(device), k)
    assert torch.equal(i.cpu(), i_o)
    assert torch.equal(_bits(v.cpu()), _bits(v_o))
    dense = cpt.topk_scatter(v, i, d).cpu()
    assert torch.equal(_bits(dense), _bits(R.topk_scatter(v_o, i_o, d)))


def test_topk_rejects_bad_sizes(device):
    cpt = _cpt()
    t = torch.zeros(2, 40000, dtype=torch.bfloat16, device=device)
    with pytest.raises(AssertionError):
        cpt.topk_abs(t, 10)                     # int16 columns
    with pytest.raises(AssertionError):
        cpt.topk_abs(t[:, :100], 101)


H, D, N = 256, 768, 512


def _params(dtype, seed):
    g = torch.Generator().manual_seed(seed)
    w = [(torch.randn(*s, generator=g) * 0.05).to(dtype) for s in ((D, H), (D, H), (H, D))]
    x = torch.randn(N, H, generator=g).to(dtype)
    gy = torch.randn(N, H, generator=g).to(dtype)
    return w, x, gy


def _run(fn, w, x, gy, k_fraction, train_w):
    ws = [t.detach().clone().requires_grad_(train_w) for t in w]
    xl = x.detach().clone().requires_grad_(True)
    y = fn(xl, *ws, k_fraction)
    y.backward(gy)
    return y.detach().cpu(), xl.grad.cpu(), [None if t.grad is None else t.grad.cpu() for t in ws]


@pytest.mark.parametrize("train_w", [True, False])
@pytest.mark.parametrize("k_fraction", [0.3, 1.0])
def test_flashffn_function_vs_oracle_bf16(device, train_w, k_fraction):
    cpt = _cpt()
    w, x, gy = _params(torch.bfloat16, 41)
    got = _run(cpt.FlashFFNFunction.apply, [t.to(device) for t in w], x.to(device),
               gy.to(device), k_fraction, train_w)
    ora = _run(R.OracleFlashFFNFunction.apply, w, x, gy, k_fraction, train_w)
    assert R.rel_frob(got[0], ora[0]) < 1e-2
    assert R.rel_frob(got[1], ora[1]) < 2e-2
    for g, o in zip(got[2], ora[2]):
        assert (g is None) == (o is None)
        if g is not None:
            assert R.rel_frob(g, o) < 2e-2


@pytest.mark.parametrize("train_w", [True, False])
def test_flashffn_function_vs_oracle_fp32(device, train_w):
    torch.backends.cuda.matmul.allow_tf32 = False
    cpt = _cpt()
    w, x, gy = _params(torch.float32, 42)
    got = _run(cpt.FlashFFNFunction.apply, [t.to(device) for t in w], x.to(device),
               gy.to(device), 1.0, train_w)
    ora = _run(R.OracleFlashFFNFunction.apply, w, x, gy, 1.0, train_w)
    assert R.rel_frob(got[0], ora[0]) < 1e-5 and R.rel_frob(got[1], ora[1]) < 1e-5
    for g, o in zip(got[2], ora[2]):
        if g is not None:
            assert R.rel_frob(g, o) < 1e-5


def test_flashffn_module_vs_standard(device):
    cpt = _cpt()
    torch.manual_seed(5)
    std = cpt.StandardFFN(H, D).to(device=device, dtype=torch.bfloat16)
    fl = cpt.FlashFFN(H, D, k_fraction=0.3).to(device=device, dtype=torch.bfloat16)
    fl.load_state_dict(std.state_dict())
    x = torch.randn(2, 64, H, device=device).to(torch.bfloat16)
    y_s, y_f = std(x).float(), fl(x)
    assert y_f.shape == x.shape
    assert R.rel_frob(y_f.float().cpu(), y_s.cpu()) < 1e-2
    y_f.float().pow(2).mean().backward()
    assert all(p.grad is not None for p in fl.parameters())
