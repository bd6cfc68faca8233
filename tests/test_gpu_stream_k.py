"""The stream-K schedule of the 16x16x32 loop (cpt_gemm_stream_k_workspace).

Products with a K-major A whose 256 x 256 tile count is above the CU count
and not a multiple of it share the k-iterations of their last (T mod S) + S
tiles over S blocks (an MN-major A keeps one tile per block).
Checked here, for every operand layout, two K-concatenated pairs and adapter
terms:
  - the result against float32 (the GEMM tolerance of the other tests);
  - against the same product with stream-K off: the outputs differ only by
    the fp32 summation order of the shared tiles (one bf16 rounding, or a
    cancellation far below the output's scale), and they do differ, so the
    shared schedule ran;
  - determinism: two calls give the same bits;
  - the workspace is left as the kernels need it: flags zero, no wait that
    ran out of polls."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _cpt():
    from compact_amd import gemm as G
    return G


def rnd(shape, seed, device, scale=1.0):
    g = torch.Generator(device=device).manual_seed(seed)
    return (torch.randn(*shape, device=device, generator=g) * scale).to(torch.bfloat16)


def _close_orders(on, off, acc=None):
    """Two summation orders of one product: different bits somewhere, every
    difference a rounding-sized one.  `acc`: the product before an adapter
    term was added, whose bf16 rounding then carries the difference."""
    diff = (on.float() - off.float()).abs()
    rms = off.float().pow(2).mean().sqrt()
    # one bf16 ulp of the value (2^-7 relative bounds it), or a cancellation
    # far below the output's scale
    mag = off.float().abs() if acc is None else off.float().abs() + 2 * acc.float().abs()
    bound = mag * 2.0 ** -7 + 1e-3 * rms
    return bool((diff <= bound).all().item()), int((diff > 0).sum().item())


def _flags_clear(G, device):
    ws = G._sk_attached[device.index if device.index is not None else torch.cuda.current_device()]
    from compact_amd import _lib
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    flags = ws[cus * 256 * 256 * 4:].view(torch.int32)
    return int(flags[:cus].abs().sum().item()) == 0 and int(flags[cus].item()) == 0


@pytest.mark.parametrize("layout", ["nt", "nn", "tn", "tt"])
def test_stream_k_layouts(device, layout):
    G = _cpt()
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    # 1376 tiles at CU count 256 (the C2 down-projection dgrad shape, fewer rows)
    m, n, k = 256 * 12, 11008, 1024
    tiles = (m // 256) * ((n + 255) // 256)
    assert tiles > cus and tiles % cus
    a = rnd((m, k), 1, device) if layout[0] == "n" else rnd((k, m), 1, device).t()
    b = rnd((k, n), 2, device, 0.05) if layout[1] == "n" else rnd((n, k), 2, device, 0.05).t()
    G.set_stream_k(False)
    off = G.mm(a, b)
    G.set_stream_k(True)
    on = G.mm(a, b)
    again = G.mm(a, b)
    torch.cuda.synchronize()
    ref = a.float() @ b.float()
    rel = ((on.float() - ref).norm() / ref.norm()).item()
    assert rel < 5e-3, rel
    assert torch.equal(on.view(torch.int16), again.view(torch.int16))
    if layout[0] == "n":
        ok, ndiff = _close_orders(on, off)
        assert ok and ndiff > 0, ndiff
    else:
        # an MN-major A (the weight gradients) keeps one tile per block
        assert torch.equal(on.view(torch.int16), off.view(torch.int16))
    assert _flags_clear(G, device)
    assert G.stream_k_errors(device) == 0


def test_stream_k_two_pairs_and_lora(device):
    G = _cpt()
    m, n = 8192, 4096 + 256 * 3          # 32 x 19 = 608 tiles
    k1, k2 = 512, 768
    a, b = rnd((m, k1), 3, device), rnd((k1, n), 4, device, 0.05)
    a2, b2 = rnd((m, k2), 5, device), rnd((k2, n), 6, device, 0.05)
    p, q = rnd((m, 16), 7, device), rnd((16, n), 8, device, 0.05)
    G.set_stream_k(False)
    off2 = G.mm2(a, b, a2, b2)
    offl = G.mm2(a, b, lora=[(p, q, 2.0)])
    off1 = G.mm2(a, b)
    G.set_stream_k(True)
    on2 = G.mm2(a, b, a2, b2)
    onl = G.mm2(a, b, lora=[(p, q, 2.0)])
    torch.cuda.synchronize()
    ref2 = a.float() @ b.float() + a2.float() @ b2.float()
    assert ((on2.float() - ref2).norm() / ref2.norm()).item() < 5e-3
    ok, ndiff = _close_orders(on2, off2)
    assert ok and ndiff > 0, ndiff
    # the adapter term is added after the shared tiles' partials: PEFT's order
    # on the same fp32 sum
    ok, ndiff = _close_orders(onl, offl, off1)
    assert ok and ndiff > 0, ndiff
    assert _flags_clear(G, device) and G.stream_k_errors(device) == 0


def test_stream_k_not_used_below_a_wave(device):
    """A product of at most one wave, or of whole waves, keeps one tile per
    block: bit-identical with stream-K on or off."""
    G = _cpt()
    for m, n in ((512, 768), (256 * 16, 256 * 16), (256 * 32, 256 * 16)):
        a, b = rnd((m, 1024), 9, device), rnd((1024, n), 10, device, 0.05)
        G.set_stream_k(False)
        off = G.mm(a, b)
        G.set_stream_k(True)
        on = G.mm(a, b)
        assert torch.equal(on.view(torch.int16), off.view(torch.int16)), (m, n)
