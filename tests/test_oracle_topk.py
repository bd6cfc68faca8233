"""CPU pins of the oracle's v1/v2 FlashFFN restatement (src/flashffn.py:300-519):

  * topk_abs against torch.topk on the same rows: the same multiset of
    magnitudes, values read from their columns, unique ascending columns;
    ties at the k-th magnitude go to the lowest columns; k = 1 is the first
    argmax and k = D is every column;
  * OracleFlashFFNFunction against float32 autograd of the plain SwiGLU FFN
    (StandardFFN's math): the 'activations' mode and, with k_fraction = 1 (the
    top-K keeps every entry), the 'recompute' mode must match it to float32
    rounding; with k_fraction < 1 only grad_w_down changes, to gy^T times h_mid
    restricted to each row's top-K columns.
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import flashffn_ref as R


def _ref_topk_check(t, k, values, indices):
    n, d = t.shape
    assert values.shape == indices.shape == (n, k)
    idx = indices.long()
    assert bool((idx[:, 1:] > idx[:, :-1]).all()) if k > 1 else True
    assert torch.equal(torch.gather(t, 1, idx), values)
    ref = torch.topk(t.float().abs(), k, dim=-1).values
    assert torch.equal(values.float().abs().sort(dim=1).values, ref.sort(dim=1).values)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,d,k", [(8, 100, 30), (5, 64, 1), (3, 17, 17), (6, 256, 77)])
def test_topk_matches_torch_topk(dtype, n, d, k):
    t = torch.randn(n, d, generator=torch.Generator().manual_seed(d + k)).to(dtype)
    values, indices = R.topk_abs(t, k)
    _ref_topk_check(t, k, values, indices)


def test_topk_ties_take_lowest_columns():
    t = torch.tensor([[1.0, -2.0, 2.0, 0.5, -2.0, 2.0, 3.0]])
    values, indices = R.topk_abs(t, 3)
    assert indices.tolist() == [[1, 2, 6]]
    assert values.tolist() == [[-2.0, 2.0, 3.0]]
    g = torch.Generator().manual_seed(3)
    t = torch.randint(-2, 3, (10, 300), generator=g).to(torch.bfloat16)   # heavy ties
    values, indices = R.topk_abs(t, 101)
    _ref_topk_check(t, 101, values, indices)
    for row in range(10):
        kept = set(indices[row].tolist())
        thr = values[row].float().abs().min()
        # every entry above the threshold is kept; equal ones fill the lowest columns
        above = {c for c in range(300) if abs(float(t[row, c])) > thr}
        assert above <= kept
        eq = [c for c in range(300) if abs(float(t[row, c])) == thr]
        assert sorted(kept - above) == eq[:len(kept - above)]


def test_topk_scatter_inverse():
    t = torch.randn(7, 50, generator=torch.Generator().manual_seed(5))
    values, indices = R.topk_abs(t, 12)
    dense = R.topk_scatter(values, indices, 50)
    mask = torch.zeros_like(t, dtype=torch.bool).scatter_(1, indices.long(), True)
    assert torch.equal(dense[mask], t[mask]) and bool((dense[~mask] == 0).all())


H, D, N = 48, 160, 64


def _params(dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    w = [(torch.randn(*s, generator=g) * 0.1).to(dtype) for s in ((D, H), (D, H), (H, D))]
    x = torch.randn(N, H, generator=g).to(dtype)
    gy = torch.randn(N, H, generator=g).to(dtype)
    return w, x, gy


def _run(fn, w, x, gy, k_fraction, train_w):
    ws = [t.detach().clone().requires_grad_(train_w) for t in w]
    xl = x.detach().clone().requires_grad_(True)
    y = fn(xl, *ws, k_fraction)
    y.backward(gy)
    return y.detach(), xl.grad, [t.grad for t in ws]


def _autograd(w, x, gy, mask=None):
    ws = [t.detach().float().requires_grad_(True) for t in w]
    xl = x.detach().float().requires_grad_(True)
    h_mid = F.silu(F.linear(xl, ws[0])) * F.linear(xl, ws[1])
    y = F.linear(h_mid, ws[2])
    y.backward(gy.float())
    gwd = None
    if mask is not None:
        gwd = gy.float().t() @ (h_mid.detach() * mask)
    return y.detach(), xl.grad, [t.grad for t in ws], gwd


def test_activations_mode_matches_autograd():
    w, x, gy = _params()
    y, gx, gw = _run(R.OracleFlashFFNFunction.apply, w, x, gy, 0.3, train_w=False)
    y_r, gx_r, _, _ = _autograd(w, x, gy)
    assert R.rel_frob(y, y_r) < 1e-5 and R.rel_frob(gx, gx_r) < 1e-5
    assert all(g is None for g in gw)


def test_recompute_mode_full_k_matches_autograd():
    w, x, gy = _params(seed=1)
    y, gx, gw = _run(R.OracleFlashFFNFunction.apply, w, x, gy, 1.0, train_w=True)
    y_r, gx_r, gw_r, _ = _autograd(w, x, gy)
    assert R.rel_frob(y, y_r) < 1e-5 and R.rel_frob(gx, gx_r) < 1e-5
    for g, r in zip(gw, gw_r):
        assert R.rel_frob(g, r) < 1e-5


def test_recompute_mode_topk_grad_w_down():
    w, x, gy = _params(seed=2)
    y, gx, gw = _run(R.OracleFlashFFNFunction.apply, w, x, gy, 0.25, train_w=True)
    with torch.no_grad():
        h_mid = F.silu(F.linear(x, w[0])) * F.linear(x, w[1])
        k = int(D * 0.25)
        top = torch.topk(h_mid.abs(), k, dim=-1).indices
        mask = torch.zeros_like(h_mid).scatter_(1, top, 1.0)
    y_r, gx_r, gw_r, gwd = _autograd(w, x, gy, mask)
    assert R.rel_frob(gx, gx_r) < 1e-5
    assert R.rel_frob(gw[0], gw_r[0]) < 1e-5 and R.rel_frob(gw[1], gw_r[1]) < 1e-5
    assert R.rel_frob(gw[2], gwd) < 1e-5
    assert R.rel_frob(gw[2], gw_r[2]) > 1e-3          # the compression is lossy


def test_three_d_input_shape():
    w, x, gy = _params(seed=3)
    x3 = x.view(4, N // 4, H)
    y, gx, _ = _run(R.OracleFlashFFNFunction.apply, w, x3, gy.view(4, N // 4, H), 0.3, True)
    assert y.shape == x3.shape and gx.shape == x3.shape
