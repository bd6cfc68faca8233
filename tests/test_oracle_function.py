"""Pins the CPU oracle's GLU math and its FlashFFNv3Function restatement.

GLU: closed forms against float64 autograd of silu(g)*u (a wrong sign or a
dropped term in dsilu fails).  Function: in the cache modes without
quantisation the restated reassociated backward must equal plain fp32 autograd
of the factored forward to float32 rounding (src/verify_flashffn_v3.py:294-327
is the reference's own oracle of this kind); a planted mistake must fail it.
Quantised modes are held to the reference's V2 cosine thresholds
(src/verify_flashffn_v3.py:456-467) and V1's "y identical across cache modes".
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import codec
from oracle import flashffn_ref as R

H, D, RANK, S = 128, 256, 8, 2.0


def test_silu_mul_closed_form():
    g = np.random.default_rng(0).standard_normal(4096).astype(np.float32) * 4
    u = np.random.default_rng(1).standard_normal(4096).astype(np.float32) * 3
    ref = (F.silu(torch.from_numpy(g).double()) * torch.from_numpy(u).double()).numpy()
    got = codec.silu_mul(g, u)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


def test_swiglu_backward_matches_autograd():
    rng = np.random.default_rng(2)
    g = rng.standard_normal(4096).astype(np.float32) * 4
    u = rng.standard_normal(4096).astype(np.float32) * 3
    dh = rng.standard_normal(4096).astype(np.float32)
    gt = torch.from_numpy(g).double().requires_grad_(True)
    ut = torch.from_numpy(u).double().requires_grad_(True)
    (F.silu(gt) * ut).backward(torch.from_numpy(dh).double())
    dg, du = codec.swiglu_backward(dh, g, u)
    assert np.abs(dg - gt.grad.numpy()).max() <= 1e-5 * np.abs(gt.grad.numpy()).max()
    assert np.abs(du - ut.grad.numpy()).max() <= 1e-5 * np.abs(ut.grad.numpy()).max()


def _grads_vs_ref(config, mode, dtype, n=64, seed=0):
    ps = R.synthetic_param_set(config, H, D, RANK, S, seed, dtype=dtype)
    g = torch.Generator().manual_seed(seed + 7)
    x = torch.randn(n, H, generator=g).to(dtype)
    gy = torch.randn(n, H, generator=g).to(dtype)
    ref, y_ref = R.ref_grads_fp32(ps, x, gy)
    got, y = R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, x, gy, mode, 64)
    assert set(got) == set(ref)
    return got, ref, y, y_ref


@pytest.mark.parametrize("config", ["all", "gateup", "none", "fullft"])
@pytest.mark.parametrize("mode", ["recompute", "bf16"])
def test_function_fp32_equals_autograd(config, mode):
    got, ref, y, y_ref = _grads_vs_ref(config, mode, torch.float32)
    assert R.rel_frob(y, y_ref) < 1e-5
    for k in ref:
        assert R.rel_frob(got[k], ref[k]) < 1e-5, k


def test_planted_mistake_is_caught(monkeypatch):
    """Drop the gate adapter's terms from the backward (s_gate -> 0 there
    only): the fp32 gate must fail (the comparison has teeth)."""
    orig = R.OracleFlashFFNv3Function.backward

    def broken(ctx, gy):
        ctx.s = (0.0,) + tuple(ctx.s[1:])
        return orig(ctx, gy)

    monkeypatch.setattr(R.OracleFlashFFNv3Function, "backward", staticmethod(broken))
    got, ref, _, _ = _grads_vs_ref("all", "recompute", torch.float32)
    assert R.rel_frob(got["grad_x"], ref["grad_x"]) > 1e-5


@pytest.mark.parametrize("config", ["all", "gateup", "fullft"])
@pytest.mark.parametrize("mode", ["int4", "int8", "bf16", "recompute"])
def test_function_bf16_v2_thresholds(config, mode):
    got, ref, y, y_ref = _grads_vs_ref(config, mode, torch.bfloat16, n=128)
    cos = {k: R.tensor_cos(got[k], ref[k]) for k in ref}
    if mode in ("recompute", "bf16"):
        assert all(c >= 0.999 for c in cos.values()), cos
    elif mode == "int8":
        assert all(c >= 0.999 for c in cos.values()), cos
    else:
        ad = [c for k, c in cos.items() if k.startswith(("a_", "b_"))]
        assert all(c >= 0.98 for c in ad) and cos["grad_x"] >= 0.99, cos


def test_forward_identical_across_cache_modes():
    ps = R.synthetic_param_set("all", H, D, RANK, S, 1, dtype=torch.bfloat16)
    x = torch.randn(4, 16, H, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    ys = []
    for mode in ("int4", "int8", "bf16", "recompute"):
        with torch.no_grad():
            ys.append(R.OracleFlashFFNv3Function.apply(
                x, ps["w_gate"], ps["a_gate"], ps["b_gate"], ps["w_up"], ps["a_up"],
                ps["b_up"], ps["w_down"], ps["a_down"], ps["b_down"], S, S, S, mode, 64, True))
    assert ys[0].shape == x.shape
    assert all(torch.equal(ys[0], y) for y in ys)


@pytest.mark.parametrize("mode,bits", [("int4", 4), ("int8", 8)])
def test_saved_bytes_closed_form(mode, bits):
    n = 96
    ps = R.synthetic_param_set("all", H, D, RANK, S, 2, dtype=torch.bfloat16)
    params = [ps[k] for k in ps if isinstance(ps[k], torch.Tensor)]
    for p in params:
        p.requires_grad_(True)
    x = torch.randn(n, H, dtype=torch.bfloat16).requires_grad_(True)
    ptrs = {p.data_ptr() for p in params} | {x.data_ptr()}
    got, entries = R.count_saved_bytes(
        lambda: R.OracleFlashFFNv3Function.apply(
            x, ps["w_gate"], ps["a_gate"], ps["b_gate"], ps["w_up"], ps["a_up"],
            ps["b_up"], ps["w_down"], ps["a_down"], ps["b_down"], S, S, S, mode, 64, True),
        ptrs)
    got += x.nbytes
    want = R.saved_bytes_closed_form(n, H, D, bits, 64, n_thin=3, rank=RANK)
    assert got == want, entries
    if bits == 4:
        assert got == R.int4_saved_bytes_closed_form(n, H, D, RANK, 64)


def test_outlier_cache_function_invariants():
    """C3 extension (parity unpinned against the reference, which has no
    per-group + outlier combination): with outlier channels the int4 grads are
    at least as close to the bf16-cache grads as without, and at ratio 0 the
    path is the plain codec."""
    ps = R.synthetic_param_set("all", H, D, RANK, S, 11, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(96, H, generator=g).to(torch.bfloat16)
    x[:, :4] *= 20                                       # hot input features -> hot h channels
    gy = torch.randn(96, H, generator=g).to(torch.bfloat16)
    ref, _ = R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, x, gy, "bf16", 64)
    plain, _ = R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, x, gy, "int4", 64)
    outl, _ = R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, x, gy, "int4", 64,
                                   outlier_ratio=0.05)
    zero, _ = R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, x, gy, "int4", 64,
                                   outlier_ratio=0.001)      # int(256 * 0.001) == 0
    for k in ref:
        assert torch.equal(zero[k], plain[k]), k
    err_plain = sum(R.rel_frob(plain[k], ref[k]) for k in ref)
    err_outl = sum(R.rel_frob(outl[k], ref[k]) for k in ref)
    assert err_outl <= err_plain


@pytest.mark.parametrize("dtype,mode,gs,ratio", [(torch.float32, "int8", 128, 0.0),
                                                 (torch.bfloat16, "int4", 64, 0.0),
                                                 (torch.bfloat16, "int4", 64, 0.05)])
def test_oracle_injection_arguments_keep_the_algorithm(dtype, mode, gs, ratio):
    """outlier_idx / cache_override given the values the oracle would compute
    itself leave every output and gradient bit-identical, so a test that
    injects the device's own channels or cache checks the same algorithm."""
    ps = R.synthetic_param_set("all", 32, 128, 4, 2.0, seed=21, dtype=dtype)
    g = torch.Generator().manual_seed(22)
    x = torch.randn(2, 24, 32, generator=g).to(dtype)
    gy = torch.randn(2, 24, 32, generator=g).to(dtype)
    base, y0 = R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, x, gy, mode, gs,
                                    True, ratio)
    x2 = x.reshape(-1, 32)
    hg = F.linear(x2, ps["w_gate"]) + ps["s_gate"] * F.linear(F.linear(x2, ps["a_gate"]),
                                                            ps["b_gate"])
    hu = F.linear(x2, ps["w_up"]) + ps["s_up"] * F.linear(F.linear(x2, ps["a_up"]), ps["b_up"])
    bits = 4 if mode == "int4" else 8
    if ratio > 0:
        rows = R.stat_rows(x.shape)
        extra = ((R.outlier_select(hg, ratio, rows), R.outlier_select(hu, ratio, rows)), None)
    else:
        qg, sg = R.v3_quantize_group_absmax(hg, bits, gs)
        qu, su = R.v3_quantize_group_absmax(hu, bits, gs)
        extra = (None, (qg, sg, qu, su))
    got, y1 = R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, x, gy, mode, gs, True,
                                   ratio, *extra)
    assert torch.equal(y0, y1)
    for k in base:
        assert torch.equal(base[k], got[k]), k
