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
C4 / C5 run the whole-model training step at full size and check properties:
every MLP ran FlashFFN v3, the MLPs saved exactly the closed form per layer,
the loss is finite and within 1e-2 of the unpatched model's on the same
weights and tokens, and every trainable gradient is finite.

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


def test_c3_token_reductions_repeated_block(device):
    """The adapter gradients reduce over all 8192 tokens: with the input one
    512-row block repeated 16 times they equal 16 x the oracle's on the
    block.  The first sequence (1024 rows) is two copies of the block, so it
    ranks the outlier channels as the block alone does."""
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

@pytest.mark.parametrize("name", ["c4", "c5"])
def test_model_step_full_size(device, name):
    from compact_amd import e2e
    from compact_amd.kernels import _V3_COUNTERS, v3_reset_counters
    from compact_amd.model_patch import apply_flash_ffn_v3, inject_lora
    cfg = e2e.CONFIGS[name]
    model = e2e.build_llama(cfg, device, seed=0)
    if cfg.get("lora"):
        inject_lora(model, cfg["lora"], cfg["lora_r"], cfg["lora_alpha"], b_std=0.01)
    model.train()
    ids = e2e.random_batch(cfg, device)
    with torch.no_grad(), e2e.fused_attention_only():
        loss_ref = float(model(input_ids=ids, labels=ids).loss)
    assert apply_flash_ffn_v3(model, cfg["cache_mode"], cfg["group"],
                              outlier_ratio=cfg["outlier_ratio"]) == cfg["layers"]

    mlps = [layer.mlp for layer in model.model.layers]
    inside = [False]
    params = {p.data_ptr() for p in model.parameters()}
    seen, total = set(), [0]

    def pack(t):
        if inside[0]:
            key = (t.data_ptr(), t.nbytes)
            if t.data_ptr() not in params and key not in seen:
                seen.add(key)
                total[0] += t.nbytes
        return t
    hooks = []
    for m in mlps:
        hooks.append(m.register_forward_pre_hook(lambda mod, a: inside.__setitem__(0, True)))
        hooks.append(m.register_forward_hook(lambda mod, a, o: inside.__setitem__(0, False)))
    v3_reset_counters()
    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t), e2e.fused_attention_only():
        loss = model(input_ids=ids, labels=ids).loss
    for hk in hooks:
        hk.remove()
    loss.backward()
    assert _V3_COUNTERS["forward"] == cfg["layers"] and _V3_COUNTERS["backward"] == cfg["layers"]
    loss = float(loss.detach())
    assert np.isfinite(loss) and abs(loss - loss_ref) / abs(loss_ref) < 1e-2, (loss, loss_ref)

    n_tok, h, d = cfg["batch"] * cfg["seq"], cfg["hidden"], cfg["inter"]
    bits = 4 if cfg["cache_mode"] == "int4" else 8
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
