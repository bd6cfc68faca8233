"""GPU parity of the adapter families (DoRA / AdaLoRA / VeRA / DyLoRA) on the
FlashFFN v3 cache against the CPU oracle and float32 autograd, after the
reference's verify_v3_adapters.py (src/verify_v3_adapters.py:1-32):

  kernels  dora_scale bit-exact against the reference's eager op
           `h * (m / nu).unsqueeze(0)` on the CPU; col_dot_div within one
           rounding of the output dtype (the fp32 summation order differs);
           the DoRA norm within 1e-5 of the float64 definition;
  Function y and every grad against OracleFlashFFNv3AdapterFunction (bf16:
           rel 1e-2 / 2e-2; float32: 1e-5, int8 1e-3), and against float32
           autograd of each family's own forward with the reference's cosine
           gates (int4 0.98 / grad_x 0.99, otherwise 0.999; r-entry vectors
           0.9, as the oracle's own tests explain);
  fused    use_triton fused == standalone codec, bitwise, with counters;
  module   make_v3_forward on wrapped MLPs routes to the adapter Function
           (counters), matches the module forward within
           max(2e-2, 4 ulp(max|y|)) and reaches every trainable parameter.
"""

import random

import pytest
import torch

from oracle import flashffn_ref as R
from tests.peft_like import SwiGLUMLP, adapter_wrap
from tests.test_oracle_adapters import cos_floor

pytestmark = pytest.mark.gpu

H, D, N, RANK, ALPHA = 256, 768, 256, 8, 16.0
GH, GD, GN, VERA_R = 128, 384, 1024, 256


def _cpt():
    import compact_amd
    return compact_amd


def _bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16)


# ---------------------------------------------------------------------------
# kernels
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("n,d", [(64, 768), (33, 200), (5, 37)])
def test_dora_scale_bitexact(device, dtype, n, d):
    cpt = _cpt()
    g = torch.Generator().manual_seed(n * d)
    x = (torch.randn(n, d, generator=g) * 3).to(dtype)
    m = (torch.rand(d, generator=g) + 0.5).to(dtype)
    nu = (torch.rand(d, generator=g) * 2 + 0.1).to(dtype)
    ref = R.dora_scale(x, m, nu)
    got = cpt.dora_scale(x.to(device), m.to(device), nu.to(device)).cpu()
    if dtype == torch.float32:
        assert torch.equal(got, ref)
    else:
        assert torch.equal(_bits16(got), _bits16(ref))
    xi = x.to(device)
    out = cpt.dora_scale(xi, m.to(device), nu.to(device), out=xi)
    assert out.data_ptr() == xi.data_ptr() and torch.equal(out.cpu(), got)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,d", [(1024, 768), (300, 200), (7, 37), (0, 64)])
def test_col_dot_div(device, dtype, n, d):
    cpt = _cpt()
    g = torch.Generator().manual_seed(n + d)
    a = torch.randn(n, d, generator=g).to(dtype)
    b = torch.randn(n, d, generator=g).to(dtype)
    den = (torch.rand(d, generator=g) + 0.5).to(dtype)
    ref = R.col_dot_div(a, b, den).double()
    got = cpt.col_dot_div(a.to(device), b.to(device), den.to(device)).cpu().double()
    # exact products per dtype; the fp32 sum order differs -> bounded by
    # 1e-6 * sum|a b| / den, then one rounding of the output dtype
    mag = (a.double() * b.double()).abs().sum(0) / den.double()
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -22
    assert bool(((got - ref).abs() <= 1e-6 * mag + ulp * ref.abs() + 1e-30).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,cols,r,s", [(768, 256, 8, 2.0), (256, 768, 16, -0.5),
                                           (100, 37, 3, 1.0), (64, 64, 0, 1.0)])
def test_dora_col_norm(device, dtype, rows, cols, r, s):
    cpt = _cpt()
    g = torch.Generator().manual_seed(rows + cols + r)
    w = (torch.randn(rows, cols, generator=g) * 0.02).to(dtype)
    a = (torch.randn(r, cols, generator=g) / cols ** 0.5).to(dtype)
    b = (torch.randn(rows, r, generator=g) * 0.05).to(dtype)
    got = cpt.dora_col_norm(w.to(device), a.to(device), b.to(device), s).cpu()
    assert got.dtype == torch.float32
    direct = (w.double() + s * (b.double() @ a.double())).norm(dim=1)
    assert float(((got.double() - direct).abs() / direct).max()) < 1e-5
    if r > 0:
        assert float(((got - R.dora_col_norm(w, a, b, s)).abs() / direct).max()) < 1e-5
    nu_dt = cpt.dora_col_norm(w.to(device), a.to(device), b.to(device), s, out_dtype=dtype).cpu()
    assert torch.equal(nu_dt, got.to(dtype))


# ---------------------------------------------------------------------------
# Function
# ---------------------------------------------------------------------------

def _run_both(ps, x, gy, mode, group, device, use_triton=True):
    got, y = R.run_adapter_grads(_cpt().FlashFFNv3AdapterFunction.apply, ps, x.to(device),
                                 gy.to(device), mode, group, use_triton)
    return {k: v.cpu() for k, v in got.items()}, y.cpu()


@pytest.mark.parametrize("kind", R.ADAPTER_KINDS)
@pytest.mark.parametrize("mode,group", [("int4", 64), ("int8", 128), ("bf16", 64),
                                        ("recompute", 64)])
def test_adapter_function_vs_oracle_bf16(device, kind, mode, group):
    ps = R.synthetic_adapter_set(kind, H, D, RANK, ALPHA, seed=21)
    gen = torch.Generator().manual_seed(22)
    x = torch.randn(N, H, generator=gen).to(torch.bfloat16)
    gy = torch.randn(N, H, generator=gen).to(torch.bfloat16)
    cpt = _cpt()
    cpt.v3_reset_counters()
    got, y = _run_both(ps, x, gy, mode, group, device)
    assert cpt._V3_COUNTERS["adapter_forward"] == 1 and cpt._V3_COUNTERS["adapter_backward"] == 1
    ora, y_o = R.run_adapter_grads(R.OracleFlashFFNv3AdapterFunction.apply, ps, x, gy, mode,
                                   group)
    assert R.rel_frob(y, y_o) < 1e-2
    assert set(got) == set(ora)
    for k in ora:
        assert R.rel_frob(got[k], ora[k]) < 2e-2, k


@pytest.mark.parametrize("kind", R.ADAPTER_KINDS)
@pytest.mark.parametrize("n", [7, 100])
def test_adapter_function_odd_token_counts(device, kind, n):
    """Token counts that are not multiples of 8 run on the same kernels for
    every adapter family (int4 g64 cache), against the oracle."""
    ps = R.synthetic_adapter_set(kind, H, D, RANK, ALPHA, seed=23)
    gen = torch.Generator().manual_seed(n)
    x = torch.randn(n, H, generator=gen).to(torch.bfloat16)
    gy = torch.randn(n, H, generator=gen).to(torch.bfloat16)
    got, y = _run_both(ps, x, gy, "int4", 64, device)
    ora, y_o = R.run_adapter_grads(R.OracleFlashFFNv3AdapterFunction.apply, ps, x, gy, "int4", 64)
    assert R.rel_frob(y, y_o) < 1e-2
    assert set(got) == set(ora)
    for k in ora:
        assert R.rel_frob(got[k], ora[k]) < 2e-2, k


@pytest.mark.parametrize("kind", R.ADAPTER_KINDS)
@pytest.mark.parametrize("mode", ["int4", "recompute", "bf16"])
def test_adapter_function_gates_vs_fp32(device, kind, mode):
    """The reference's V2-style gates against float32 autograd of the family's
    own forward, at the oracle tests' gate size."""
    ps = R.synthetic_adapter_set(kind, GH, GD, VERA_R if kind == "vera" else RANK, ALPHA,
                                 seed=23)
    gen = torch.Generator().manual_seed(24)
    x = torch.randn(GN, GH, generator=gen).to(torch.bfloat16)
    gy = torch.randn(GN, GH, generator=gen).to(torch.bfloat16)
    got, y = _run_both(ps, x, gy, mode, 64, device)
    ref, y_ref = R.ref_adapter_grads_fp32(ps, x, gy)
    tol = max(2e-2, 4 * 2.0 ** -8 * float(y_ref.abs().max()))
    assert float((y.float() - y_ref).abs().max()) <= tol
    for k in ref:
        c = R.tensor_cos(got[k], ref[k])
        assert c >= cos_floor(mode, k, ref[k].numel()), (k, c)


@pytest.mark.parametrize("kind", R.ADAPTER_KINDS)
@pytest.mark.parametrize("mode", ["recompute", "bf16", "int8"])
def test_adapter_function_vs_oracle_fp32(device, kind, mode):
    torch.backends.cuda.matmul.allow_tf32 = False
    ps = R.synthetic_adapter_set(kind, H, D, RANK, ALPHA, seed=25, dtype=torch.float32)
    gen = torch.Generator().manual_seed(26)
    x = torch.randn(N, H, generator=gen)
    gy = torch.randn(N, H, generator=gen)
    got, y = _run_both(ps, x, gy, mode, 128, device)
    ora, y_o = R.run_adapter_grads(R.OracleFlashFFNv3AdapterFunction.apply, ps, x, gy, mode, 128)
    assert R.rel_frob(y, y_o) < 1e-5
    # int8: a value on a rounding tie of the CPU/GPU GEMMs flips one code
    tol = 1e-5 if mode != "int8" else 1e-3
    for k in ora:
        assert R.rel_frob(got[k], ora[k]) < tol, k


@pytest.mark.parametrize("kind", ["dora", "vera"])
@pytest.mark.parametrize("mode", ["int4", "int8"])
def test_adapter_fused_equals_unfused_bitwise(device, kind, mode):
    cpt = _cpt()
    ps = R.synthetic_adapter_set(kind, H, D, RANK, ALPHA, seed=27)
    gen = torch.Generator().manual_seed(28)
    x = torch.randn(N, H, generator=gen).to(torch.bfloat16)
    gy = torch.randn(N, H, generator=gen).to(torch.bfloat16)
    cpt.v3_reset_counters()
    fused, yf = _run_both(ps, x, gy, mode, 64, device, use_triton=True)
    assert cpt._V3_COUNTERS["triton_quant_fwd"] == 1
    assert cpt._V3_COUNTERS["triton_dequant_bwd"] == 1
    cpt.v3_reset_counters()
    eager, ye = _run_both(ps, x, gy, mode, 64, device, use_triton=False)
    assert cpt._V3_COUNTERS["triton_quant_fwd"] == 0
    assert cpt._V3_COUNTERS["triton_dequant_bwd"] == 0
    assert torch.equal(yf, ye)
    for k in fused:
        assert torch.equal(fused[k], eager[k]), k


# ---------------------------------------------------------------------------
# module patch
# ---------------------------------------------------------------------------

def _trainables(mlp):
    return {n: p for n, p in mlp.named_parameters() if p.requires_grad}


@pytest.mark.parametrize("kind", R.ADAPTER_KINDS)
@pytest.mark.parametrize("mode", ["int4", "recompute"])
def test_make_v3_forward_routes_adapters(device, kind, mode):
    cpt = _cpt()
    torch.manual_seed(31)
    mlp = adapter_wrap(SwiGLUMLP(H, D), kind, VERA_R if kind == "vera" else RANK, ALPHA)
    mlp = mlp.to(device=device, dtype=torch.bfloat16).train()
    x = torch.randn(2, 128, H, generator=torch.Generator().manual_seed(32))
    x = x.to(torch.bfloat16).to(device)
    with torch.no_grad():
        random.seed(1234)
        y_mod = mlp(x).float()
    fwd = cpt.make_v3_forward(mlp, mode)
    cpt.v3_reset_counters()
    random.seed(1234)
    y = fwd(x)
    assert cpt._V3_COUNTERS["adapter_forward"] == 1
    assert y.shape == x.shape
    tol = max(2e-2, 4 * 2.0 ** -8 * float(y_mod.detach().abs().max()))
    assert float((y.detach().float() - y_mod.detach()).abs().max()) <= tol
    y.float().pow(2).mean().backward()
    assert cpt._V3_COUNTERS["adapter_backward"] == 1
    tr = _trainables(mlp)
    assert tr and all(p.grad is not None for p in tr.values()), \
        [n for n, p in tr.items() if p.grad is None]


def test_mixed_projection_kinds(device):
    """DoRA gate, plain up, LoRA down in one MLP: the adapter Function with
    per-projection None factors."""
    cpt = _cpt()
    torch.manual_seed(33)
    mlp = SwiGLUMLP(H, D)
    adapter_wrap(mlp, "dora", RANK, ALPHA, which=("gate",))
    adapter_wrap(mlp, "lora", RANK, ALPHA, which=("down",))
    mlp = mlp.to(device=device, dtype=torch.bfloat16)
    x = torch.randn(N, H, generator=torch.Generator().manual_seed(34)).to(torch.bfloat16)
    x = x.to(device)
    with torch.no_grad():
        y_mod = mlp(x).float()
    y = cpt.make_v3_forward(mlp, "int8", 128)(x)
    tol = max(2e-2, 4 * 2.0 ** -8 * float(y_mod.detach().abs().max()))
    assert float((y.detach().float() - y_mod.detach()).abs().max()) <= tol
    y.float().sum().backward()
    tr = _trainables(mlp)
    assert all(p.grad is not None for p in tr.values())
    assert mlp.up_proj.weight.grad is not None        # plain projection: full fine-tune


def test_dylora_rank_sampling_matches_module(device):
    """Seeded random draws give the same per-projection ranks as the module,
    and eval mode uses the full rank."""
    cpt = _cpt()
    torch.manual_seed(35)
    mlp = adapter_wrap(SwiGLUMLP(H, D), "dylora", RANK, ALPHA)
    mlp = mlp.to(device=device, dtype=torch.bfloat16)
    x = torch.randn(N, H, generator=torch.Generator().manual_seed(36)).to(torch.bfloat16)
    x = x.to(device)
    fwd = cpt.make_v3_forward(mlp, "bf16")
    for train in (True, False):
        mlp.train(train)
        with torch.no_grad():
            random.seed(99)
            y_mod = mlp(x).float()
            random.seed(99)
            y = fwd(x).float()
        tol = max(2e-2, 4 * 2.0 ** -8 * float(y_mod.detach().abs().max()))
        assert float((y - y_mod).abs().max()) <= tol
