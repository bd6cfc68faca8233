"""The general-layout GEMM (cpt_gemm_any): float32 / float16 / bfloat16
operands of any strides, ragged sizes and every epilogue, against a float64
product of the same inputs on the CPU.

Bounds, with S = |A| . |B| (the sum of absolute products) and u the unit
roundoff of the output dtype:
  fp32 accumulation over K terms:   |acc - exact| <= K * 2^-24 * S  (a loose,
                                     order-independent bound; typical error is
                                     far smaller)
  each rounding to the dtype:        u * |value|, or half the subnormal
                                     spacing below the normal range
so STORE is checked at  |c - exact| <= u |exact| + K 2^-24 S + tiny,  and the
ADD / SCALE epilogues against the same op order restated in float64 with
each step rounded to the dtype.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

U = {torch.float32: 2.0 ** -24, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}
# half the subnormal spacing: the absolute rounding error below the normal range
TINY = {torch.float32: 2.0 ** -150, torch.float16: 2.0 ** -25, torch.bfloat16: 2.0 ** -134}


def _G():
    from compact_amd import gemm
    return gemm


def _rd(t, dt):
    return t.to(dt).double()


def _operand(shape, layout, dt, gen, device):
    """A [rows, cols] device operand of the given layout."""
    r, c = shape
    if layout == "row":
        return torch.randn(r, c, generator=gen).to(dt).to(device)
    if layout == "col":                        # transposed view
        return torch.randn(c, r, generator=gen).to(dt).to(device).t()
    if layout == "strided":                    # every other column of a wider matrix
        return torch.randn(r, 2 * c + 3, generator=gen).to(dt).to(device)[:, 1:2 * c + 1:2]
    if layout == "offset":                     # rows one element off the aligned start
        return torch.randn(r, c + 9, generator=gen).to(dt).to(device)[:, 1:c + 1]
    raise ValueError(layout)


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("la,lb", [("row", "row"), ("row", "col"), ("col", "row"),
                                   ("col", "col"), ("strided", "offset"), ("offset", "strided")])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (7, 130, 33), (257, 100, 300), (300, 257, 1),
                                   (64, 5, 1000)])
def test_store_vs_float64(device, dt, la, lb, M, N, K):
    G = _G()
    gen = torch.Generator().manual_seed(M * 7 + N * 3 + K)
    a = _operand((M, K), la, dt, gen, device)
    b = _operand((K, N), lb, dt, gen, device)
    c = G.mm_any(a, b)
    assert c.shape == (M, N) and c.dtype == dt
    a64, b64 = a.cpu().double(), b.cpu().double()
    exact = a64 @ b64
    s = a64.abs() @ b64.abs()
    err = (c.cpu().double() - exact).abs()
    assert (err <= U[dt] * exact.abs() + K * 2.0 ** -24 * s + TINY[dt]).all()


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["add", "scale"])
def test_add_and_scale_epilogues(device, dt, mode):
    """PEFT's h + s * F.linear(xa, b) and s * (a @ b), each step rounded."""
    G = _G()
    gen = torch.Generator().manual_seed(5)
    M, N, K, s = 200, 96, 1, 2.0              # a rank-1 adapter term
    a = torch.randn(M, K, generator=gen).to(dt).to(device)
    b = torch.randn(K, N, generator=gen).to(dt).to(device)
    h = torch.randn(M, N, generator=gen).to(dt).to(device)
    prod = _rd(a.cpu().double() @ b.cpu().double(), dt)      # K = 1: the product is exact
    if mode == "add":
        ref = _rd(h.cpu().double() + _rd(s * prod, dt), dt)
        out = G.mm_any(a, b, s, G.ANY_ADD, out=h)
        assert out.data_ptr() == h.data_ptr()
    else:
        ref = _rd(s * prod, dt)
        out = G.mm_any(a, b, s, G.ANY_SCALE)
    assert torch.equal(out.cpu().double(), ref)


def test_empty_and_k0(device):
    G = _G()
    a = torch.zeros(0, 8, device=device)
    b = torch.zeros(8, 5, device=device)
    assert G.mm_any(a, b).shape == (0, 5)
    a = torch.zeros(4, 0, device=device)
    b = torch.zeros(0, 5, device=device)
    assert torch.equal(G.mm_any(a, b).cpu(), torch.zeros(4, 5))


def test_fp32_function_uses_no_torch_gemm(device, monkeypatch):
    """C1's float32 FlashFFNv3Function runs every product on this build's
    kernels: torch's matmul entry points are poisoned for the call."""
    import compact_amd as cpt
    from oracle import flashffn_ref as R

    def boom(*a, **k):
        raise AssertionError("a torch GEMM ran on the product path")
    for name in ("matmul", "mm", "addmm", "bmm"):
        monkeypatch.setattr(torch, name, boom)
    monkeypatch.setattr(torch.Tensor, "__matmul__", boom)
    monkeypatch.setattr(torch.nn.functional, "linear", boom)
    ps = R.synthetic_param_set("all", 64, 256, 1, 2.0, seed=9, dtype=torch.float32)
    psd = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in ps.items()}
    gen = torch.Generator().manual_seed(10)
    x = torch.randn(33, 64, generator=gen).to(device)
    gy = torch.randn(33, 64, generator=gen).to(device)
    got, y = R.run_function_grads(cpt.FlashFFNv3Function.apply, psd, x, gy, "int8", 128)
    assert torch.isfinite(y).all() and all(torch.isfinite(g).all() for g in got.values())
