"""Parity at every BASELINE config's own size (configs C1..C5), on the device
path that bench.py times.

Row outputs are independent given the weights, so y, grad_x and the cache
are checked on a sample of rows (spread over every tile boundary kind: the
first and last rows, 256-row tile edges, random rows) against the CPU oracle
run on those rows alone.  Codes and scales are checked bit for bit against
the oracle codec applied to the engine's own bf16 h_gate / h_up for those
rows (the same dual-GEMM kernel on the same rows gives the same
accumulators).  Weight gradients are sums over all tokens:
  C2  a column sample: the sub-FFN restricted to whole quantisation groups of
      d_ff has exactly the full FFN's weight-gradient rows / columns for those
      channels, so the oracle runs it over all 8192 tokens;
  C3  a second run whose input repeats one 512-row block 16 times: every
      token reduction equals 16 times the oracle's on the block;
  C1  float32 is small enough for the whole oracle on the CPU.
Every gradient is also checked at full size against float32 autograd of the
plain FFN on the device (the reference's V2 cosine gates,
src/verify_flashffn_v3.py:456-467), and saved bytes against the closed form
(src/verify_flashffn_v3.py:594-605).
C4 / C5 run the whole-model training step at full size.  Each MLP's input,
output, upstream gradient and input gradient are recorded in the patched
step, and every layer is checked against float32 autograd of the stock MLP on
its own recorded inputs (y rel-Frobenius 1e-2, gradients by the V2 cosine
gates), its trainable gradients also against the unpatched model's step on
the same weights and tokens; C5's layer-0 outlier channels against the
oracle's ranking of that layer's first sequence; saved bytes against the
closed form per layer.

Tolerances (north star: rel <= 1e-2 in bf16, <= 1e-5 in fp32):
  bf16  y rel-Frobenius 1e-2; gradients 2e-2 where the oracle derives its
        own cache from CPU GEMMs (a code can flip), 1e-2 where it takes the
        engine's cache;
  fp32  1e-5 with the engine's cache (C1).
"""

import numpy as np
import pytest
import torch

from oracle import codec
from oracle import flashffn_ref as R

pytestmark = pytest.mark.gpu

H7, D7 = 4096, 11008          # Llama-7B FFN (C2, C3)
N7 = 8 * 1024


def _mods():
    import compact_amd
    from compact_amd import _lib, gemm
    return compact_amd, _lib, gemm


def _rows(n, k=32, seed=0):
    fixed = {0, 1, 255, 256, 257, n // 2 - 1, n // 2, n - 257, n - 256, n - 1}
    rng = np.random.default_rng(seed)
    rest = rng.choice(n, size=k, replace=False).tolist()
    return torch.tensor(sorted(fixed | set(rest)))


def _capture(fn):
    """fn() with every tensor it saves for backward recorded (in order)."""
    saved = []

    def pack(t):
        saved.append(t)
        return t
    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        out = fn()
    return out, saved


def _saved_bytes(saved, params, x):
    """The reference's accounting (src/verify_flashffn_v3.py:523-543):
    deduplicated by storage, parameters excluded, x counted once."""
    skip = {p.data_ptr() for p in params} | {x.data_ptr()}
    seen, total = set(), 0
    for t in saved:
        key = (t.data_ptr(), t.nbytes)
        if t.data_ptr() in skip or key in seen:
            continue
        seen.add(key)
        total += t.nbytes
    return total + x.nbytes


def _of(saved, dtype, shape):
    return [t for t in saved if t.dtype == dtype and tuple(t.shape) == tuple(shape)]


def _cos_gates(got, ref, floors):
    for k, g in got.items():
        c = R.tensor_cos(g.float(), ref[k])
        assert c >= floors(k), (k, c)


def _lora(r, d_in, d_out, gen, device):
    bound = 1.0 / d_in ** 0.5     # kaiming_uniform_(a=sqrt(5)) on [r, d_in]
    a = ((torch.rand(r, d_in, device=device, generator=gen) * 2 - 1) * bound).to(torch.bfloat16)
    b = (torch.randn(d_out, r, device=device, generator=gen) * 0.01).to(torch.bfloat16)
    return a, b


def _weights(h, d, gen, device, dtype=torch.bfloat16):
    return [(torch.randn(*s, device=device, generator=gen) * 0.02).to(dtype)
            for s in ((d, h), (d, h), (h, d))]


def _fp32_ref(ps_dev, x, gy):
    with torch.enable_grad():
        return R.ref_grads_fp32(ps_dev, x, gy)


# --------------------------------------------------------------------------
# C2: bf16, 8192 x 4096 x 11008, int8 g128, full fine-tune
# --------------------------------------------------------------------------

def test_c2_full_size(device):
    cpt, L, G = _mods()
    gen = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(N7, H7, device=device, generator=gen).to(torch.bfloat16)
    gy = torch.randn(N7, H7, device=device, generator=gen).to(torch.bfloat16)
    wg, wu, wd = _weights(H7, D7, gen, device)
    leaves = [t.clone().requires_grad_() for t in (x, wg, wu, wd)]
    xl, wgl, wul, wdl = leaves
    y, saved = _capture(lambda: cpt.FlashFFNv3Function.apply(
        xl.view(8, 1024, H7), wgl, None, None, wul, None, None, wdl, None, None,
        0.0, 0.0, 0.0, "int8", 128))
    y.backward(gy.view(8, 1024, H7))
    y = y.detach().view(N7, H7)
    got = {"grad_x": xl.grad, "w_gate": wgl.grad, "w_up": wul.grad, "w_down": wdl.grad}
    assert all(torch.isfinite(g).all() for g in got.values())
    qs = _of(saved, torch.int8, (N7, D7))
    ss = _of(saved, torch.float16, (N7, D7 // 128))
    assert len(qs) == 2 and len(ss) == 2
    assert _saved_bytes(saved, leaves[1:], xl) == R.saved_bytes_closed_form(N7, H7, D7, 8, 128)

    # codes and scales of sampled rows, bit for bit
    rows = _rows(N7)
    rd = rows.to(device)
    _, hg, hu, *_ = G.ffn_gate_up(x[rd].contiguous(), wg, wu, L.CACHE_BF16, 128,
                                  want_h_mid=False)
    for h, q, s in ((hg, qs[0], ss[0]), (hu, qs[1], ss[1])):
        rq, rs = codec.quantize_group_absmax(R.to_f32(h.cpu()), 8, 128)
        assert np.array_equal(q[rd].cpu().numpy(), rq)
        assert np.array_equal(s[rd].cpu().numpy().view(np.uint16), rs.view(np.uint16))

    # y and grad_x of the sampled rows: the oracle on those rows with their cache
    wc = [w.cpu() for w in (wg, wu, wd)]
    ps = dict(train_w=True, w_gate=wc[0], w_up=wc[1], w_down=wc[2], a_gate=None, b_gate=None,
              a_up=None, b_up=None, a_down=None, b_down=None, s_gate=0.0, s_up=0.0, s_down=0.0)
    cache = tuple(t[rd].cpu() for t in (qs[0], ss[0], qs[1], ss[1]))
    ora, y_o = R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, x[rd].cpu(),
                                    gy[rd].cpu(), "int8", 128, True, 0.0, None, cache)
    assert R.rel_frob(y[rd].cpu(), y_o) < 1e-2
    assert R.rel_frob(got["grad_x"][rd].cpu(), ora["grad_x"]) < 1e-2

    # weight gradients of three whole groups of channels over all tokens
    groups = (0, D7 // 128 // 2, D7 // 128 - 1)
    cols = torch.cat([torch.arange(g * 128, (g + 1) * 128) for g in groups])
    cd = cols.to(device)
    gi = torch.tensor(groups, device=device)
    ps_sub = dict(ps, w_gate=wc[0][cols], w_up=wc[1][cols], w_down=wc[2][:, cols].contiguous())
    cache = tuple(t.cpu().contiguous() for t in (qs[0][:, cd], ss[0][:, gi], qs[1][:, cd],
                                                 ss[1][:, gi]))
    sub, _ = R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps_sub, x.cpu(), gy.cpu(),
                                  "int8", 128, True, 0.0, None, cache)
    assert R.rel_frob(got["w_gate"][cd].cpu(), sub["w_gate"]) < 1e-2
    assert R.rel_frob(got["w_up"][cd].cpu(), sub["w_up"]) < 1e-2
    assert R.rel_frob(got["w_down"][:, cd].cpu(), sub["w_down"]) < 1e-2

    # every gradient at full size: the V2 gates against float32 autograd
    ps_dev = dict(ps, w_gate=wg, w_up=wu, w_down=wd)
    ref, y_ref = _fp32_ref(ps_dev, x, gy)
    assert R.tensor_cos(y.float(), y_ref) >= 0.999
    _cos_gates(got, ref, lambda k: 0.999)


# --------------------------------------------------------------------------
# C3: C2 + LoRA r16 (s = 2) on gate/up/down, frozen base, int4 g64, 1 % outliers
# --------------------------------------------------------------------------

def _c3_params(device, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    wg, wu, wd = _weights(H7, D7, gen, device)
    ag, bg = _lora(16, H7, D7, gen, device)
    au, bu = _lora(16, H7, D7, gen, device)
    ad, bd = _lora(16, D7, H7, gen, device)
    return dict(train_w=False, w_gate=wg, w_up=wu, w_down=wd, a_gate=ag, b_gate=bg, a_up=au,
                b_up=bu, a_down=ad, b_down=bd, s_gate=2.0, s_up=2.0, s_down=2.0), gen


def _run_c3(ps, x, gy):
    """The product Function on leaves of ps: (grads, y [N, H], saved, leaves)."""
    cpt, _, _ = _mods()
    xl = x.view(8, 1024, H7).clone().requires_grad_()
    t = {k: ps[k].clone().requires_grad_(k[0] in "ab")
         for k in ps if isinstance(ps[k], torch.Tensor)}
    y, saved = _capture(lambda: cpt.FlashFFNv3Function.apply(
        xl, t["w_gate"], t["a_gate"], t["b_gate"], t["w_up"], t["a_up"], t["b_up"],
        t["w_down"], t["a_down"], t["b_down"], 2.0, 2.0, 2.0, "int4", 64, True, 0.01))
    y.backward(gy.view(8, 1024, H7))
    got = {"grad_x": xl.grad}
    got.update({k: v.grad for k, v in t.items() if v.requires_grad})
    return got, y.detach().view(N7, H7), saved, [xl] + list(t.values())


def test_c3_full_size(device):
    cpt, L, G = _mods()
    ps, gen = _c3_params(device, 1)
    x = torch.randn(N7, H7, device=device, generator=gen).to(torch.bfloat16)
    gy = torch.randn(N7, H7, device=device, generator=gen).to(torch.bfloat16)
    got, y, saved, leaves = _run_c3(ps, x, gy)
    got["grad_x"] = got["grad_x"].reshape(N7, H7)
    assert set(got) == {"grad_x", "a_gate", "b_gate", "a_up", "b_up", "a_down", "b_down"}
    assert all(torch.isfinite(g).all() for g in got.values())
    k = int(D7 * 0.01)
    qs = _of(saved, torch.uint8, (N7, D7 // 2))
    ss = _of(saved, torch.float16, (N7, D7 // 64))
    os_ = _of(saved, torch.bfloat16, (N7, k))
    slots = _of(saved, torch.int16, (D7,))
    assert len(qs) == 2 and len(ss) == 2 and len(os_) == 2 and len(slots) == 2
    closed = R.saved_bytes_closed_form(N7, H7, D7, 4, 64, n_thin=3, rank=16, n_outlier=k)
    assert _saved_bytes(saved, leaves[1:], leaves[0]) == closed + 2 * D7 * 2   # + slot maps

    # the engine's h_gate / h_up of given rows (the Function's own x A^T terms)
    xa_g = G.mm(x, ps["a_gate"].t())
    xa_u = G.mm(x, ps["a_up"].t())

    def h_rows(rd):
        _, hg, hu, *_ = G.ffn_gate_up(
            x[rd].contiguous(), ps["w_gate"], ps["w_up"], L.CACHE_BF16, 64, want_h_mid=False,
            lora_gate=(xa_g[rd].contiguous(), ps["b_gate"], 2.0),
            lora_up=(xa_u[rd].contiguous(), ps["b_up"], 2.0))
        return hg.cpu(), hu.cpu()

    # outlier channels: ranked on the first sequence's 1024 rows, bit for bit
    hg1, hu1 = h_rows(torch.arange(1024, device=device))
    idx = []
    for h1, slot in ((hg1, slots[0]), (hu1, slots[1])):
        ref_idx = np.asarray(R.outlier_select(h1, 0.01, 1024))
        got_idx = torch.nonzero(slot >= 0).flatten().cpu().numpy()
        assert np.array_equal(np.sort(ref_idx), got_idx)
        assert np.array_equal(slot[slot >= 0].cpu().numpy(), np.arange(k))
        idx.append(got_idx)

    # codes, scales and outlier blocks of sampled rows, bit for bit
    rows = _rows(N7, seed=1)
    rd = rows.to(device)
    hg, hu = h_rows(rd)
    for h, q, s, o, ix in ((hg, qs[0], ss[0], os_[0], idx[0]), (hu, qs[1], ss[1], os_[1], idx[1])):
        rq, rs, ro = R.v3_quantize_outlier(h, 4, 64, ix)
        assert torch.equal(q[rd].cpu(), rq)
        assert torch.equal(s[rd].cpu().view(torch.int16), rs.view(torch.int16))
        assert torch.equal(o[rd].cpu().view(torch.int16), ro.view(torch.int16))

    # y and grad_x of the sampled rows against the oracle on those rows
    psc = {kk: (v.cpu() if isinstance(v, torch.Tensor) else v) for kk, v in ps.items()}
    ora, y_o = R.run_function_grads(R.OracleFlashFFNv3Function.apply, psc, x[rd].cpu(),
                                    gy[rd].cpu(), "int4", 64, True, 0.01, tuple(idx))
    assert R.rel_frob(y[rd].cpu(), y_o) < 1e-2
    assert R.rel_frob(got["grad_x"][rd].cpu(), ora["grad_x"]) < 2e-2

    # every gradient at full size: the int4 V2 gates against float32 autograd
    ref, y_ref = _fp32_ref(ps, x, gy)
    assert R.tensor_cos(y.float(), y_ref) >= 0.99
    _cos_gates(got, ref, lambda kk: 0.99 if kk == "grad_x" else 0.98)


def test_c3_token_reductions_repeated_block(device, no_stream_k):
    """The adapter gradients reduce over all 8192 tokens: with the input one
    512-row block repeated 16 times they equal 16 x the oracle's on the
    block.  The first sequence (1024 rows) is two copies of the block, so it
    ranks the outlier channels as the block alone does.  Without stream-K, so
    the last block's rows are summed in the first block's order (bitwise
    equal)."""
    ps, gen = _c3_params(device, 2)
    reps, blk = 16, 512
    xb = torch.randn(blk, H7, device=device, generator=gen).to(torch.bfloat16)
    gyb = torch.randn(blk, H7, device=device, generator=gen).to(torch.bfloat16)
    got, y, _, _ = _run_c3(ps, xb.repeat(reps, 1), gyb.repeat(reps, 1))
    gx = got.pop("grad_x").reshape(N7, H7)
    assert torch.equal(y[-blk:].view(torch.int16), y[:blk].view(torch.int16))
    assert torch.equal(gx[-blk:].view(torch.int16), gx[:blk].view(torch.int16))
    psc = {kk: (v.cpu() if isinstance(v, torch.Tensor) else v) for kk, v in ps.items()}
    ora, y_o = R.run_function_grads(R.OracleFlashFFNv3Function.apply, psc, xb.cpu(), gyb.cpu(),
                                    "int4", 64, True, 0.01)
    assert R.rel_frob(y[:blk].cpu(), y_o) < 1e-2
    assert R.rel_frob(gx[:blk].cpu(), ora["grad_x"]) < 2e-2
    for kk, g in got.items():
        assert R.rel_frob(g.cpu().double() / reps, ora[kk]) < 2e-2, kk


# --------------------------------------------------------------------------
# C1: float32, 4 x 512 tokens, 2048 x 5632 (TinyLlama), int8 g128, full fine-tune
# --------------------------------------------------------------------------

def test_c1_full_size_fp32(device):
    cpt, _, G = _mods()
    n, h, d = 2048, 2048, 5632
    g = torch.Generator().manual_seed(0)                 # C1's seed 0, on the CPU
    x = torch.randn(4, 512, h, generator=g)
    wg, wu, wd = [torch.randn(*s, generator=g) * 0.02 for s in ((d, h), (d, h), (h, d))]
    gy = torch.randn(4, 512, h, generator=g)
    ps = dict(train_w=True, w_gate=wg, w_up=wu, w_down=wd, a_gate=None, b_gate=None, a_up=None,
              b_up=None, a_down=None, b_down=None, s_gate=0.0, s_up=0.0, s_down=0.0)
    psd = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in ps.items()}
    (got, y), saved = _capture(lambda: R.run_function_grads(
        cpt.FlashFFNv3Function.apply, psd, x.to(device), gy.to(device), "int8", 128))
    qs = _of(saved, torch.int8, (n, d))
    ss = _of(saved, torch.float16, (n, d // 128))
    assert len(qs) == 2 and len(ss) == 2
    # the cache is the oracle codec of the engine's own float32 h_gate / h_up
    x2 = x.reshape(n, h).to(device)
    for w, q, s in ((psd["w_gate"], qs[0], ss[0]), (psd["w_up"], qs[1], ss[1])):
        hh = G.mm_any(x2, w.t())
        rq, rs = codec.quantize_group_absmax(hh.cpu().numpy(), 8, 128)
        assert np.array_equal(q.cpu().numpy(), rq)
        assert np.array_equal(s.cpu().numpy().view(np.uint16), rs.view(np.uint16))
    # the whole C1 oracle on the CPU, given that cache: 1e-5
    cache = tuple(t.cpu() for t in (qs[0], ss[0], qs[1], ss[1]))
    ora, y_o = R.run_function_grads(R.OracleFlashFFNv3Function.apply, ps, x, gy, "int8", 128,
                                    True, 0.0, None, cache)
    assert R.rel_frob(y.cpu(), y_o) < 1e-5
    assert set(got) == set(ora)
    for k in ora:
        assert R.rel_frob(got[k].cpu(), ora[k]) < 1e-5, k


# --------------------------------------------------------------------------
# C4 / C5: whole-model training steps at full size
# --------------------------------------------------------------------------

def _mlp_params(mlp):
    """(w, a, b, s) of each projection of a stock LlamaMLP, plain or LoRA."""
    from compact_amd.flashffn import _v3_extract_proj
    ps = {}
    for key in R.PROJ:
        w, a, b, s = _v3_extract_proj(getattr(mlp, f"{key}_proj"))
        ps[f"w_{key}"], ps[f"a_{key}"], ps[f"b_{key}"], ps[f"s_{key}"] = w, a, b, s
    ps["train_w"] = ps["w_gate"].requires_grad
    return ps


def _mlp_trainables(mlp):
    """{oracle grad name: parameter} of one MLP's trainable tensors."""
    ps = _mlp_params(mlp)
    return {k: ps[k] for k in ps if isinstance(ps[k], torch.Tensor) and ps[k].requires_grad}


@pytest.mark.parametrize("name", ["c4", "c5"])
def test_model_step_full_size(device, name):
    """The whole-model step at full size, every MLP checked on its own inputs:
      - the unpatched model's step on the same weights and tokens gives the
        reference gradients (bf16 autograd, stock MLPs);
      - in the patched step every MLP's input x_l, output y_l, upstream
        gradient gy_l and input gradient gx_l are recorded;
      - per layer, float32 autograd of the stock MLP on (x_l, gy_l) must give
        y_l (rel-Frobenius 1e-2), gx_l and the MLP's trainable gradients
        under the reference's V2 cosine gates (src/verify_flashffn_v3.py:456-467:
        0.999 for an int8 cache; int4: adapter factors 0.98, grad_x 0.99);
      - the MLP trainables of the patched step must also match the unpatched
        model's gradients.  With an int8 cache (C4) every layer meets the
        0.999 gate.  With an int4 cache (C5) each layer's codec error in its
        grad_x (cos 0.99 against exact, the V2 gate) reaches every layer below
        it through the residual stream, so against the unpatched model only
        the last layer, which no other codec feeds, is held to the V2 gates,
        and the rest to 0.9 (measured 0.95-0.96 at layer 0).  To show that
        this gap is the codec's and not the model plumbing's, C5 also runs the
        patched model with the lossless bf16 cache (same fused LoRA kernels),
        whose MLP gradients must meet 0.995 against the unpatched model in
        every layer (measured 0.9975).  The unpatched model is itself a bf16
        computation with its own roundings: C4's last layer measures 0.9993
        against it and 0.99997 against float32 on the same inputs, so the
        float32 per-layer gates above are the precise ones;
      - C5: the outlier channels of layer 0 are the oracle's ranking of that
        layer's first sequence (2048 rows) of the engine's own h_gate / h_up;
      - every MLP ran FlashFFN v3 and saved exactly the closed form."""
    from compact_amd import e2e
    from compact_amd.kernels import _V3_COUNTERS, v3_reset_counters
    from compact_amd.model_patch import apply_flash_ffn_v3, inject_lora
    _, L, G = _mods()
    cfg = e2e.CONFIGS[name]
    model = e2e.build_llama(cfg, device, seed=0)
    if cfg.get("lora"):
        inject_lora(model, cfg["lora"], cfg["lora_r"], cfg["lora_alpha"], b_std=0.01)
    model.train()
    ids = e2e.random_batch(cfg, device)
    mlps = [layer.mlp for layer in model.model.layers]
    int4 = cfg["cache_mode"] == "int4"

    def floor(k):
        return (0.99 if k == "grad_x" else 0.98) if int4 else 0.999

    # the unpatched step: reference gradients of every MLP trainable
    with e2e.fused_attention_only():
        model(input_ids=ids, labels=ids).loss.backward()
    ref_whole = [{k: p.grad.detach().clone() for k, p in _mlp_trainables(m).items()}
                 for m in mlps]
    model.zero_grad(set_to_none=True)

    def whole_cos(li, m):
        return {kk: R.tensor_cos(p.grad.float(), ref_whole[li][kk].float())
                for kk, p in _mlp_trainables(m).items()}

    if int4:
        # the same patched model with the lossless bf16 cache
        assert apply_flash_ffn_v3(model, "bf16", cfg["group"]) == cfg["layers"]
        with e2e.fused_attention_only():
            model(input_ids=ids, labels=ids).loss.backward()
        lossless = min(min(whole_cos(li, m).values()) for li, m in enumerate(mlps))
        print(name, "bf16 cache, whole-model min cos", round(lossless, 6))
        assert lossless >= 0.995, lossless
        model.zero_grad(set_to_none=True)

    assert apply_flash_ffn_v3(model, cfg["cache_mode"], cfg["group"],
                              outlier_ratio=cfg["outlier_ratio"]) == cfg["layers"]

    rec = [dict() for _ in mlps]
    inside = [-1]
    params = {p.data_ptr() for p in model.parameters()}
    seen, total, saved0 = set(), [0], []

    def pack(t):
        if inside[0] >= 0:
            key = (t.data_ptr(), t.nbytes)
            if t.data_ptr() not in params and key not in seen:
                seen.add(key)
                total[0] += t.nbytes
            if inside[0] == 0:
                saved0.append(t)
        return t

    def pre(li):
        def f(mod, args):
            inside[0] = li
            x = args[0]
            rec[li]["x"] = x.detach()
            x.register_hook(lambda g: rec[li].__setitem__("gx", g.detach()))
        return f

    def post(li):
        def f(mod, args, out):
            inside[0] = -1
            rec[li]["y"] = out.detach()
            out.register_hook(lambda g: rec[li].__setitem__("gy", g.detach()))
        return f
    hooks = []
    for li, m in enumerate(mlps):
        hooks.append(m.register_forward_pre_hook(pre(li)))
        hooks.append(m.register_forward_hook(post(li)))
    v3_reset_counters()
    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t), e2e.fused_attention_only():
        loss = model(input_ids=ids, labels=ids).loss
    loss.backward()
    for hk in hooks:
        hk.remove()
    assert _V3_COUNTERS["forward"] == cfg["layers"] and _V3_COUNTERS["backward"] == cfg["layers"]
    assert np.isfinite(float(loss.detach()))

    n_tok, h, d = cfg["batch"] * cfg["seq"], cfg["hidden"], cfg["inter"]
    bits = 4 if int4 else 8
    k = int(d * cfg["outlier_ratio"])
    lora_mlp = cfg.get("lora") and "gate_proj" in cfg["lora"]
    per_layer = R.saved_bytes_closed_form(n_tok, h, d, bits, cfg["group"],
                                          n_thin=3 if lora_mlp else 0,
                                          rank=cfg.get("lora_r", 0), n_outlier=k)
    per_layer += 2 * d * 2 if k else 0                     # the int16 slot maps
    assert total[0] == per_layer * cfg["layers"], (total[0], per_layer * cfg["layers"])
    trainable = [p for p in model.parameters() if p.requires_grad]
    assert trainable and all(p.grad is not None and torch.isfinite(p.grad).all()
                             for p in trainable)

    # every layer against float32 autograd of the stock MLP on its own inputs,
    # and against the unpatched model's gradients
    worst = {}
    for li, m in enumerate(mlps):
        r = rec[li]
        x2, y2 = r["x"].reshape(n_tok, h), r["y"].reshape(n_tok, h)
        ps = _mlp_params(m)
        ref, y_ref = _fp32_ref(ps, x2, r["gy"].reshape(n_tok, h))
        got = {"grad_x": r["gx"].reshape(n_tok, h)}
        got.update({kk: p.grad for kk, p in _mlp_trainables(m).items()})
        assert set(got) == set(ref), (li, set(got), set(ref))
        checks = {"y_rel": R.rel_frob(y2, y_ref)}
        for kk, g in got.items():
            checks[kk] = R.tensor_cos(g.float(), ref[kk])
        wc = whole_cos(li, m)
        if li in (0, len(mlps) // 2, len(mlps) - 1):
            print(name, "layer", li, "whole-model cos",
                  {kk: round(v, 6) for kk, v in wc.items()})
        last = li == len(mlps) - 1
        for kk, v in wc.items():
            assert v >= (floor(kk) if (last or not int4) else 0.9), (li, kk, v)
        for kk, v in checks.items():
            worst[kk] = max(worst.get(kk, v), v) if kk == "y_rel" else min(worst.get(kk, v), v)
        del ref, y_ref
    print(name, "per-layer worst", {kk: round(v, 6) for kk, v in worst.items()})
    assert worst["y_rel"] < 1e-2, worst
    for kk, v in worst.items():
        if kk != "y_rel":
            assert v >= floor(kk), (kk, v)

    if k:
        # layer 0's outlier channels: the oracle's ranking of its first sequence
        slots = _of(saved0, torch.int16, (d,))
        assert len(slots) == 2
        ps = _mlp_params(mlps[0])
        # the Function's own x A^T terms, then the first sequence's rows
        x0 = rec[0]["x"].reshape(n_tok, h)
        s1 = cfg["seq"]
        xa_g = G.mm(x0, ps["a_gate"].t())[:s1].contiguous()
        xa_u = G.mm(x0, ps["a_up"].t())[:s1].contiguous()
        _, hg, hu, *_ = G.ffn_gate_up(x0[:s1].contiguous(), ps["w_gate"], ps["w_up"],
                                      L.CACHE_BF16, cfg["group"], want_h_mid=False,
                                      lora_gate=(xa_g, ps["b_gate"], ps["s_gate"]),
                                      lora_up=(xa_u, ps["b_up"], ps["s_up"]))
        for hh, slot in ((hg, slots[0]), (hu, slots[1])):
            ref_idx = np.asarray(R.outlier_select(hh.cpu(), cfg["outlier_ratio"], cfg["seq"]))
            got_idx = torch.nonzero(slot >= 0).flatten().cpu().numpy()
            assert np.array_equal(np.sort(ref_idx), got_idx)
            assert np.array_equal(slot[slot >= 0].cpu().numpy(), np.arange(k))
