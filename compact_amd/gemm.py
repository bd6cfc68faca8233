"""torch-facing wrappers of the MFMA GEMMs (libcompact_amd.so): the 16x16x32
direct-to-LDS loop for products whose K is a multiple of 64, the 32x32x16
engine otherwise.

mm(a, b)        a @ b for 2-D bf16 tensors; each operand may be row-major or
                a transposed view (K-major / MN-major on the device side).
mm2(a, b, a2, b2)  a @ b + a2 @ b2 in one fp32 accumulation.
mm_engine(a, b) a @ b on the 32x32x16 engine whatever the shape (the fused
                kernels' summation order).
linear(x, w)    x @ w.T (F.linear without bias).
ffn_gate_up     fused dual GEMM + GLU + codec (forward of gate/up + K1).
ffn_down_dgrad  fused grad_y @ w_down + dequantise + SwiGLU backward (+ K2).

LoRA adapter terms (`lora=` / `lora_gate=`, `lora_up=`): PEFT's
`h + s * B(A(x))` applied in the GEMM epilogue, each step rounded to bf16 as
the reference does (src/flashffn.py:1414,1420,1439,1529,1558-1566), for every
rank from 1 to 16, and from 17 to 32 where the product runs on the 16x16x32
loop (`lora_fusable`; a rank that is not a multiple of 8 is zero-padded to the
next multiple of 8).

mm_any          any dtype and any strides (cpt_gemm_any, fp32 MFMA): float32
                (config C1), float16, unaligned bf16 views, rank-1 factors.

These replace the cuBLAS GEMMs the reference issues through F.linear / @
(src/flashffn.py:1410-1439,1503-1587).
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import check
from .kernels import _require_device, _stream, _timed


def _layout_a(a: torch.Tensor):
    """(tensor, ld, kmajor) for a logical [M, K] operand: rows 16-byte aligned
    in place, otherwise a contiguous copy."""
    if a.data_ptr() % 16 == 0:
        if a.stride(1) == 1 and a.stride(0) % 8 == 0 and a.stride(0) >= a.shape[1]:
            return a, a.stride(0), 1
        if a.stride(0) == 1 and a.stride(1) % 8 == 0 and a.stride(1) >= a.shape[0]:
            return a, a.stride(1), 0
    a = a.contiguous()
    return a, a.stride(0), 1


def _layout_b(b: torch.Tensor):
    """(tensor, ld, kmajor) for a logical [K, N] operand (kmajor: stored [N][ld]):
    rows 16-byte aligned in place, otherwise a contiguous copy."""
    if b.data_ptr() % 16 == 0:
        if b.stride(0) == 1 and b.stride(1) % 8 == 0 and b.stride(1) >= b.shape[0]:
            return b, b.stride(1), 1
        if b.stride(1) == 1 and b.stride(0) % 8 == 0 and b.stride(0) >= b.shape[1]:
            return b, b.stride(0), 0
    b = b.contiguous()
    return b, b.stride(0), 0


def _with_ld(t: torch.Tensor, ld: int, rows_dim: int) -> torch.Tensor:
    """Copy of 2-D `t` whose storage rows (along `rows_dim`) are `ld` apart."""
    if rows_dim == 0:
        buf = torch.zeros((t.shape[0], ld), dtype=t.dtype, device=t.device)
        buf[:, :t.shape[1]] = t
        return buf[:, :t.shape[1]]
    buf = torch.zeros((t.shape[1], ld), dtype=t.dtype, device=t.device)
    buf[:, :t.shape[0]] = t.t()
    return buf[:, :t.shape[0]].t()


def _common_ld(x, x2, kmajor: int, is_b: bool):
    """The two pairs of mm2 share per-thread offsets, so their operands need
    one leading dimension: re-lay both with the larger one."""
    # storage row axis: A K-major [M][ld] -> dim 0; A MN-major [K][ld] -> dim 1;
    # B K-major [N][ld] -> dim 1; B MN-major [K][ld] -> dim 0
    rows_dim = (0 if kmajor else 1) if not is_b else (1 if kmajor else 0)
    extent = lambda t: t.shape[1 - rows_dim]
    ld = max((extent(x) + 7) // 8 * 8, (extent(x2) + 7) // 8 * 8)
    return _with_ld(x, ld, rows_dim), _with_ld(x2, ld, rows_dim), ld


def _check_bf16(*ts):
    for t in ts:
        assert t.dtype == torch.bfloat16, f"MFMA GEMM path is bf16-only, got {t.dtype}"
        assert t.dim() == 2


LORA_MAX_RANK = 32


def lora_fusable(rank: int, *dims) -> bool:
    """Adapter terms of this rank ride in the epilogue of a GEMM whose summed
    products have the (k, n) `dims` (inner dim, output columns).  One MFMA per
    output block and term over k = 16 (v_mfma_f32_16x16x16_bf16 per 16 x 16
    block on the 16x16x32 loop, v_mfma_f32_32x32x16_bf16 per 32 x 32 block on
    the engine) covers ranks up to 16 on either loop.  Ranks 17 to 32 take a
    second MFMA accumulated onto the first, carried by the 16x16x32 loop's
    kernels only (not the engine's, nor stream-K's): every k a positive
    multiple of 64 and n a multiple of 8."""
    if not 1 <= rank <= LORA_MAX_RANK:
        return False
    return rank <= 16 or (len(dims) > 0 and all(k > 0 and k % 64 == 0 and n % 8 == 0
                                                for k, n in dims))


def _lora_args(terms, n_q, dims):
    """(rank, ldp, q_kmajor, ldq, [(p, q, alpha) x 2], keep) for up to two
    terms (p [M, r], q the logical [r, N] factor, alpha) of a GEMM with the
    (k, n) `dims` (lora_fusable); `keep` holds any
    re-laid copies alive until the launch.  The kernels fetch P and K-major Q
    in 16-byte chunks of 8 k, so a rank that is not a multiple of 8 is
    zero-padded to the next one (8, 16, 24 or 32): the padded k add exact zeros to
    each fp32 dot product."""
    terms = [t for t in terms if t is not None]
    assert 1 <= len(terms) <= 2
    r = terms[0][0].shape[1]
    assert lora_fusable(r, *dims), \
        f"adapter rank {r} not carried by a GEMM of (k, n) {tuple(dims)} (lora_fusable)"
    if r % 8:
        rp = (r + 7) // 8 * 8
        pad = torch.nn.functional.pad
        padded = []
        for pm, q, al in terms:
            # a factor given as [r, N] rows (an A weight) gains zero rows; one
            # stored [N, r] (a B weight, q its transposed view) zero columns
            if q.stride(1) == 1 and q.stride(0) != 1:
                q = pad(q, (0, 0, 0, rp - r))
            else:
                q = pad(q.t(), (0, rp - r)).t()
            padded.append((pad(pm, (0, rp - r)), q, al))
        terms, r = padded, rp
    keep, ps, qs = [], [], []
    for pm, q, _ in terms:
        _check_bf16(pm, q)
        assert pm.shape[1] == r and q.shape[0] == r and q.shape[1] == n_q
        if pm.stride(1) != 1 or pm.stride(0) % 8 or pm.data_ptr() % 16:
            pm = pm.contiguous()
        ps.append(pm)
        qs.append(q)
    ldp = ps[0].stride(0)
    if any(x.stride(0) != ldp for x in ps):
        ps = [x.contiguous() for x in ps]
        ldp = r
    # Q: K-major when the [N, r] storage is contiguous, else MN-major rows
    if all(q.stride(0) == 1 and q.stride(1) == r and q.data_ptr() % 16 == 0 for q in qs):
        q_kmajor, ldq = 1, r
    elif all(q.stride(1) == 1 for q in qs) and len({q.stride(0) for q in qs}) == 1:
        q_kmajor, ldq = 0, qs[0].stride(0)
    else:
        qs = [q.t().contiguous().t() for q in qs]
        q_kmajor, ldq = 1, r
    keep += ps + qs
    out = [(ps[i].data_ptr(), qs[i].data_ptr(), float(terms[i][2])) for i in range(len(terms))]
    while len(out) < 2:
        out.append((None, None, 0.0))
    return r, ldp, q_kmajor, ldq, out, keep


SKINNY_MAX_RANK = 32
# blocks of 128 rows x one K range the skinny projection aims for.  In the C3
# step on MI355X (M = 8192: 4 K ranges) h_mid A_d^T took 44.5 us and
# x [A_g; A_u]^T 21.5 us, against 52.0 and 23.6 at 512 blocks (8 ranges) and
# 52.4 / 24.6 at 384, including their reductions.
SKINNY_BLOCKS = 256

# Buffer offsets are 32-bit.  Every kernel's resource starts where a block's
# reads start (a tile's first row, a split's first token or k row), so an
# operand of any size works as long as one block's range spans less than this.
_SPAN_BYTES = 1 << 31


def skinny(a: torch.Tensor, q: torch.Tensor, alpha: float = 1.0,
           name: str = "gemm_skinny", out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(alpha * a [M, K] @ q[R, K].T) for a rank R <= 32: the tall-skinny
    adapter products (x A^T, grad_y B, ...), streamed once through HBM with K
    split across blocks (fp32 partials summed in a fixed order).  Each output
    column's sum runs in the same order whatever R is, so stacked factors
    give the columns of separate products bit for bit.  out: a bf16 [M, R]
    view with unit column stride and 16-byte aligned rows (e.g. the column
    half of a wider buffer) to write into."""
    _require_device(a, q)
    _check_bf16(a, q)
    M, K = a.shape
    R = q.shape[0]
    assert q.shape[1] == K and R <= SKINNY_MAX_RANK
    if a.stride(1) != 1 or a.stride(0) % 8 or a.stride(0) < K or a.data_ptr() % 16:
        a = a.contiguous()
    if q.stride(1) != 1 or q.stride(0) % 8 or q.stride(0) < K or q.data_ptr() % 16:
        q = q.contiguous()
    # K ranges for ~SKINNY_BLOCKS blocks of 128 rows (each range >= 256 of
    # K): more ranges cost more partials than they gain in parallelism
    blocks = (M + 127) // 128
    splits = max(1, min(K // 256, (SKINNY_BLOCKS + blocks - 1) // blocks))
    if out is None:
        c = torch.empty((M, R), dtype=torch.bfloat16, device=a.device)
    else:
        c = out
        assert (tuple(c.shape) == (M, R) and c.dtype == torch.bfloat16 and c.stride(1) == 1
                and c.stride(0) % 8 == 0 and c.data_ptr() % 16 == 0), "skinny out layout"
    ws = (torch.empty((splits * M * R,), dtype=torch.float32, device=a.device)
          if splits > 1 else None)
    with _timed(name):
        rc = _lib.lib().cpt_gemm_bf16_skinny(a.data_ptr(), a.stride(0), q.data_ptr(),
                                             q.stride(0), c.data_ptr(), c.stride(0), M, R, K,
                                             float(alpha),
                                             splits, None if ws is None else ws.data_ptr(),
                                             _stream(a))
    check(rc, name)
    return c


def _row_major(t: torch.Tensor) -> bool:
    return t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0


def skinny_t(x: torch.Tensor, p: torch.Tensor, alpha: float = 1.0, trans: bool = False,
             name: str = "gemm_skinny_t") -> torch.Tensor:
    """bf16(alpha * x[T, N].T @ p[T, R]) -> [N, R] (or its transpose [R, N]
    with trans) for R <= 32: the adapter-factor gradients that reduce over
    the tokens, x and p token-major."""
    _require_device(x, p)
    _check_bf16(x, p)
    T, N = x.shape
    R = p.shape[1]
    assert p.shape[0] == T and R <= SKINNY_MAX_RANK
    if not _row_major(x) or x.stride(0) < N:
        x = x.contiguous()
    if not _row_major(p) or p.stride(0) < R:
        p = p.contiguous()
    splits = skinny_t_splits(T, N)
    # each split reads its tokens (plus 128 of prefetch) within 32-bit offsets
    per = (_SPAN_BYTES // (2 * max(x.stride(0), p.stride(0))) - 129) // 64 * 64
    assert per >= 64, "operand rows too long for 32-bit buffer offsets"
    splits = max(splits, (T + per - 1) // per)
    out = torch.empty((R, N) if trans else (N, R), dtype=torch.bfloat16, device=x.device)
    ws = torch.empty((splits * N * R,), dtype=torch.float32, device=x.device)
    with _timed(name):
        rc = _lib.lib().cpt_gemm_bf16_skinny_t(x.data_ptr(), x.stride(0), p.data_ptr(),
                                               p.stride(0), out.data_ptr(), out.stride(0),
                                               1 if trans else 0, T, N, R, float(alpha), splits,
                                               ws.data_ptr(), _stream(x))
    check(rc, name)
    return out


# Blocks of a skinny_dual launch (column blocks x token splits).  In the C3
# step on MI355X, 176 (8 token splits over d_ff 11008, 22 over d_model 4096)
# against 256: 64.6 / 62.7 / 37.1 us against 66.6 / 68.8 / 44.5 us for the
# gate, up and down passes including their reductions (128, 352, 512 and 704
# blocks were no better).  Fewer, longer token splits also cut the Z partials
# by a third.
SKINNY_DUAL_BLOCKS = 176


def transpose_ok(x: torch.Tensor) -> bool:
    """transpose takes a bf16 row-major [rows, cols] device tensor with rows,
    cols and the row stride multiples of 8 and a 16-byte aligned base."""
    return (x.dtype == torch.bfloat16 and x.is_cuda and x.dim() == 2 and x.stride(1) == 1
            and x.shape[0] % 8 == 0 and x.shape[1] % 8 == 0 and x.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0)


def transpose(x: torch.Tensor, name: str = "transpose") -> torch.Tensor:
    """x^T as a new row-major [cols, rows] bf16 tensor (cpt_transpose_bf16)."""
    _require_device(x)
    assert transpose_ok(x), "transpose operand"
    rows, cols = x.shape
    out = torch.empty((cols, rows), dtype=x.dtype, device=x.device)
    with _timed(name):
        rc = _lib.lib().cpt_transpose_bf16(x.data_ptr(), x.stride(0), rows, cols, out.data_ptr(),
                                           out.stride(0), _stream(x))
    check(rc, name)
    return out


def skinny_dual_ok(x: torch.Tensor, q: torch.Tensor, p: torch.Tensor) -> bool:
    """skinny_dual takes bf16 x [T, N] with N a multiple of 8 and a rank
    (q [R, N], p [T, R]) that is a multiple of 8 up to 32."""
    T, N = x.shape
    R = q.shape[0]
    return (x.dtype == q.dtype == p.dtype == torch.bfloat16 and x.is_cuda and N % 8 == 0
            and R % 8 == 0 and 0 < R <= SKINNY_MAX_RANK and q.shape[1] == N
            and tuple(p.shape) == (T, R))


def skinny_dual(x: torch.Tensor, q: torch.Tensor, p: torch.Tensor, alpha_c: float = 1.0,
                alpha_z: float = 1.0, out_c: torch.Tensor | None = None,
                name: str = "gemm_skinny_dual"):
    """(bf16(alpha_c * x @ q.T) [T, R], bf16(alpha_z * x.T @ p) [N, R]) in one
    pass over x [T, N] (cpt_gemm_bf16_skinny_dual): the projection and the
    token reduction a LoRA backward takes of one tensor (grad_h B and
    s grad_h^T (x A^T)).  out_c: a bf16 [T, R] view with unit column stride
    and 16-byte aligned rows to write C into."""
    _require_device(x, q, p)
    assert skinny_dual_ok(x, q, p), "skinny_dual operands"
    T, N = x.shape
    R = q.shape[0]
    if not _row_major(x) or x.stride(0) < N:
        x = x.contiguous()
    # Q as rank rows [R][ld], or its transpose B [N][ld] as stored (no copy)
    if q.stride(1) == 1 and q.stride(0) % 8 == 0 and q.stride(0) >= N and q.data_ptr() % 16 == 0:
        q_nr, ldq = 0, q.stride(0)
    elif q.stride(0) == 1 and q.stride(1) >= R and q.data_ptr() % 16 == 0:
        q_nr, ldq = 1, q.stride(1)
    else:
        q = q.contiguous()
        q_nr, ldq = 0, q.stride(0)
    if not _row_major(p) or p.stride(0) < R:
        p = p.contiguous()
    # blocks of 512 columns x T / splits tokens: ~SKINNY_DUAL_BLOCKS of them
    csplits = (N + 511) // 512
    splits = max(1, min(max(T // 256, 1), (SKINNY_DUAL_BLOCKS + csplits - 1) // csplits))
    per = (_SPAN_BYTES // (2 * max(x.stride(0), p.stride(0))) - 129) // 64 * 64
    assert per >= 64, "operand rows too long for 32-bit buffer offsets"
    splits = max(splits, (T + per - 1) // per)
    if out_c is None:
        c = torch.empty((T, R), dtype=torch.bfloat16, device=x.device)
    else:
        c = out_c
        assert (tuple(c.shape) == (T, R) and c.dtype == torch.bfloat16 and c.stride(1) == 1
                and c.stride(0) % 8 == 0 and c.data_ptr() % 16 == 0), "skinny_dual out layout"
    z = torch.empty((N, R), dtype=torch.bfloat16, device=x.device)
    nbytes = int(_lib.lib().cpt_gemm_bf16_skinny_dual_workspace_bytes(T, N, R, splits))
    ws = torch.empty((max(nbytes, 4) // 4,), dtype=torch.float32, device=x.device)
    with _timed(name):
        rc = _lib.lib().cpt_gemm_bf16_skinny_dual(
            x.data_ptr(), x.stride(0), q.data_ptr(), ldq, q_nr, p.data_ptr(), p.stride(0),
            c.data_ptr(), c.stride(0), float(alpha_c), z.data_ptr(), z.stride(0), 0,
            float(alpha_z), T, N, R, splits, ws.data_ptr(), _stream(x))
    check(rc, name)
    return c, z


def skinny_t_splits(T: int, N: int) -> int:
    """Token splits of the token-reduction kernel: ~768 blocks of 64 columns."""
    blocks = (N + 63) // 64
    return max(1, min(max(T // 256, 1), (768 + blocks - 1) // blocks))


def skinny_t_noalloc(x: torch.Tensor, p: torch.Tensor, out: torch.Tensor, alpha: float = 1.0,
                     trans: bool = False, splits: int | None = None,
                     name: str = "gemm_skinny_t_noalloc") -> torch.Tensor:
    """skinny_t into a caller-provided `out` through the allocation-free entry
    point: the split partials use the library's fixed per-GPU scratch, so the
    call allocates nothing (x, p token-major rows 16-byte aligned; out [N, R],
    or [R, N] with trans, rows `out.stride(0)` apart)."""
    _require_device(x, p, out)
    _check_bf16(x, p)
    T, N = x.shape
    R = p.shape[1]
    assert p.shape[0] == T and out.dtype == torch.bfloat16 and out.stride(1) == 1
    assert tuple(out.shape) == ((R, N) if trans else (N, R))
    assert _row_major(x) and _row_major(p), "x and p must have 16-byte aligned rows"
    if splits is None:
        splits = skinny_t_splits(T, N)
    with _timed(name):
        rc = _lib.lib().cpt_gemm_bf16_skinny_t_noalloc(
            x.data_ptr(), x.stride(0), p.data_ptr(), p.stride(0), out.data_ptr(), out.stride(0),
            1 if trans else 0, T, N, R, float(alpha), splits, _stream(x))
    check(rc, f"{name} (split partials beyond the {_lib.NOALLOC_SCRATCH_BYTES >> 20} MiB "
              "scratch?)" if rc == _lib.ERR_TOO_LARGE else name)
    return out


def _max_k_rows(ld: int) -> int:
    """k rows one block may read from an MN-major operand with rows ld apart
    (prefetch overhang of 256 rows included)."""
    return _SPAN_BYTES // (2 * ld) - 257


def _min_splits(K: int, lda: int, ak: int, ldb: int, bk: int) -> int:
    """Fewest k ranges that keep every block of a product within 32-bit
    offsets, given its operand layouts (1 for everything but products over
    very long k, e.g. the weight gradients of ~100k+ tokens whose operands
    exceed 2 GiB)."""
    lim = K
    if not ak:
        lim = min(lim, _max_k_rows(lda))       # A MN-major: [K][lda]
    if not bk:
        lim = min(lim, _max_k_rows(ldb))       # B MN-major: [K][ldb]
    if lim >= K:
        return 1
    assert lim >= 64, "operand rows too long for 32-bit buffer offsets"
    nk, per = (K + 63) // 64, lim // 64
    return (nk + per - 1) // per


def mm(a: torch.Tensor, b: torch.Tensor, name: str = "gemm") -> torch.Tensor:
    """a [M, K] @ b [K, N] -> bf16 [M, N] on the MFMA GEMM loops (16x16x32 when
    K is a multiple of 64 and N of 8, else the 32x32x16 engine).  Tall products
    with N <= 32 (the adapter terms' x A^T, grad_y B, ...) go to the skinny
    kernel; other products with too few 256x256 output tiles to fill the chip
    (N or M = rank) split K across blocks instead, as do products whose
    transposed operands are too long for one block's 32-bit offsets."""
    M, K = a.shape
    N = b.shape[1]
    if (N <= SKINNY_MAX_RANK and K >= 256 and K % 8 == 0 and M >= 256
            and a.stride(1) == 1):
        return skinny(a, b.t(), 1.0, name)
    tiles = ((M + 255) // 256) * ((N + 255) // 256)
    if tiles < 128 and K >= 1024:
        return mm_splitk(a, b, 1.0, name=name)
    a, lda, ak = _layout_a(a)
    b, ldb, bk = _layout_b(b)
    if _min_splits(K, lda, ak, ldb, bk) > 1:
        return mm_splitk(a, b, 1.0, name=name)
    return mm2(a, b, None, None, name)


# Stream-K workspace per device (cpt_gemm_stream_k_workspace): attached at
# the first product on a device while stream-K is on.
_STREAM_K = {"on": True}
_sk_attached: dict = {}      # device index -> workspace tensor, or None if detached


def set_stream_k(on: bool) -> None:
    """Turn the stream-K schedule of the 16x16x32 loop on or off for later
    products on every device (on by default).  Results are deterministic
    either way; the two summation orders differ in the last bits of the
    tiles the schedule shares."""
    _STREAM_K["on"] = bool(on)
    for idx in list(_sk_attached):
        with torch.cuda.device(idx):
            check(_lib.lib().cpt_gemm_stream_k_workspace(None, 0), "stream_k_workspace")
        del _sk_attached[idx]


def _stream_k(dev: torch.device) -> None:
    """Attach a zero-filled stream-K workspace to `dev` once (the kernels
    leave it zero-filled)."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx in _sk_attached or not _STREAM_K["on"]:
        return
    with torch.cuda.device(idx):
        nbytes = int(_lib.lib().cpt_gemm_stream_k_bytes())
        assert nbytes > 0, "stream-K workspace size"
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        torch.cuda.synchronize(idx)
        check(_lib.lib().cpt_gemm_stream_k_workspace(ws.data_ptr(), nbytes), "stream_k_workspace")
    _sk_attached[idx] = ws


def stream_k_errors(dev: torch.device) -> int:
    """Waits for a partial that ran out of polls on `dev` since its workspace
    was attached (the word after the flags); 0 unless the schedule broke."""
    ws = _sk_attached.get(dev.index if dev.index is not None else torch.cuda.current_device())
    if ws is None:
        return 0
    return int(ws[-4:].view(torch.int32).item())


def mm2(a, b, a2=None, b2=None, name: str = "gemm", lora=None) -> torch.Tensor:
    """a @ b (+ a2 @ b2) in one fp32 accumulation -> bf16 [M, N], then the
    adapter terms `lora` = [(p [M, r], q [r, N], alpha), ...] (at most two),
    each `out = bf16(out + bf16(alpha * bf16(p @ q)))`."""
    _require_device(a, b)
    _check_bf16(a, b)
    M, K = a.shape
    K_, N = b.shape
    assert K == K_, f"inner dims differ: {tuple(a.shape)} @ {tuple(b.shape)}"
    a, lda, ak = _layout_a(a)
    b, ldb, bk = _layout_b(b)
    p_a2 = p_b2 = None
    lda2 = ldb2 = K2 = 0
    if a2 is not None:
        _check_bf16(a2, b2)
        assert a2.shape[0] == M and b2.shape[1] == N and a2.shape[1] == b2.shape[0]
        K2 = a2.shape[1]
        a2, lda2, ak2 = _layout_a(a2)
        b2, ldb2, bk2 = _layout_b(b2)
        if ak2 != ak:
            a2 = a2.t().contiguous().t() if ak == 0 else a2.contiguous()
            a2, lda2, ak2 = _layout_a(a2)
        if bk2 != bk:
            b2 = b2.t().contiguous().t() if bk == 1 else b2.contiguous()
            b2, ldb2, bk2 = _layout_b(b2)
        assert ak2 == ak and bk2 == bk
        if lda2 != lda:
            a, a2, lda = _common_ld(a, a2, ak, is_b=False)
            lda2 = lda
        if ldb2 != ldb:
            b, b2, ldb = _common_ld(b, b2, bk, is_b=True)
            ldb2 = ldb
        p_a2, p_b2 = a2.data_ptr(), b2.data_ptr()
    ldc = (N + 7) // 8 * 8
    c = torch.empty((M, ldc), dtype=torch.bfloat16, device=a.device)
    _stream_k(a.device)
    if lora:
        if ak != 1:
            a = a.contiguous()
            a, lda, ak = _layout_a(a)
            assert a2 is None, "adapter terms with a K-concatenated MN-major A"
        dims = ((K, N),) if a2 is None else ((K, N), (K2, N))
        r, ldp, qk, ldq, t, keep = _lora_args(lora, N, dims)
        with _timed(name):
            rc = _lib.lib().cpt_gemm_bf16_lora(
                a.data_ptr(), lda, ak, b.data_ptr(), ldb, bk, p_a2, lda2, p_b2, ldb2, K2,
                c.data_ptr(), ldc, M, N, K, r, ldp, qk, ldq, t[0][0], t[0][1], t[0][2],
                t[1][0], t[1][1], t[1][2], _stream(a))
        del keep
    else:
        with _timed(name):
            rc = _lib.lib().cpt_gemm_bf16(a.data_ptr(), lda, ak, b.data_ptr(), ldb, bk, p_a2,
                                          lda2, p_b2, ldb2, K2, c.data_ptr(), ldc, M, N, K,
                                          _stream(a))
    check(rc, name)
    return c if ldc == N else c[:, :N]


def mm_engine(a: torch.Tensor, b: torch.Tensor, name: str = "gemm_engine") -> torch.Tensor:
    """a [M, K] @ b [K, N] -> bf16 [M, N] on the 32x32x16 engine loop for
    every shape: the fp32 summation order of the fused FFN kernels, so a
    fused kernel equals its unfused composition through this product bit for
    bit.  mm runs every layout on the 16x16x32 loop instead whenever K is a
    multiple of 64 and N of 8 (same bf16 rounding of the fp32 sum, another
    summation order)."""
    _require_device(a, b)
    _check_bf16(a, b)
    M, K = a.shape
    K_, N = b.shape
    assert K == K_, f"inner dims differ: {tuple(a.shape)} @ {tuple(b.shape)}"
    a, lda, ak = _layout_a(a)
    b, ldb, bk = _layout_b(b)
    ldc = (N + 7) // 8 * 8
    c = torch.empty((M, ldc), dtype=torch.bfloat16, device=a.device)
    with _timed(name):
        rc = _lib.lib().cpt_gemm_bf16_ex(a.data_ptr(), lda, ak, b.data_ptr(), ldb, bk, c.data_ptr(),
                                         ldc, M, N, K, 1.0, 0, 1, None, _stream(a))
    check(rc, name)
    return c if ldc == N else c[:, :N]


def linear(x: torch.Tensor, w: torch.Tensor, name: str = "gemm") -> torch.Tensor:
    """x [M, K] @ w[N, K].T -> [M, N] (F.linear without bias)."""
    return mm(x, w.t(), name)


def linear_lora(x: torch.Tensor, w: torch.Tensor, xa: torch.Tensor, b: torch.Tensor,
                alpha: float, name: str = "gemm") -> torch.Tensor:
    """PEFT's LoRA Linear without dropout: bf16(bf16(x W^T) + bf16(alpha *
    bf16(xa B^T))) with xa = x A^T [M, r] and B [N, r]."""
    return mm2(x, w.t(), None, None, name, lora=[(xa, b.t(), alpha)])


def ffn_gate_up(x, w_gate, w_up, cache: int, group_size: int, want_h_mid: bool = True,
                lora_gate=None, lora_up=None):
    """Fused dual GEMM + GLU + codec.  Returns (h_mid | None, h_gate | None,
    h_up | None, q_gate | None, s_gate | None, q_up | None, s_up | None).
    lora_gate / lora_up = (xa [n, r], B [inter, r], s): the projection's LoRA
    term, added to h_gate / h_up before the GLU and the codec."""
    _require_device(x, w_gate, w_up)
    _check_bf16(x, w_gate, w_up)
    n, hdim = x.shape
    d = w_gate.shape[0]
    assert w_gate.shape == (d, hdim) and w_up.shape == (d, hdim)
    x, w_gate, w_up = x.contiguous(), w_gate.contiguous(), w_up.contiguous()
    dev = x.device
    h_mid = torch.empty((n, d), dtype=torch.bfloat16, device=dev) if want_h_mid else None
    hg = hu = qg = sg = qu = su = None
    if cache == _lib.CACHE_BF16:
        hg = torch.empty((n, d), dtype=torch.bfloat16, device=dev)
        hu = torch.empty((n, d), dtype=torch.bfloat16, device=dev)
    elif cache in (_lib.CACHE_INT4, _lib.CACHE_INT8):
        g = d // group_size
        shape = (n, d // 2) if cache == _lib.CACHE_INT4 else (n, d)
        qdt = torch.uint8 if cache == _lib.CACHE_INT4 else torch.int8
        qg = torch.empty(shape, dtype=qdt, device=dev)
        qu = torch.empty(shape, dtype=qdt, device=dev)
        sg = torch.empty((n, g), dtype=torch.float16, device=dev)
        su = torch.empty((n, g), dtype=torch.float16, device=dev)

    def p(t):
        return None if t is None else t.data_ptr()

    if lora_gate is not None or lora_up is not None:
        # term 0 on the gate columns, term 1 on the up columns (absent: no-op)
        present = [t for t in (lora_gate, lora_up) if t is not None]
        r, ldp, qk, _, t, keep = _lora_args([(xa, bw.t(), s) for xa, bw, s in present], d,
                                            ((hdim, d),))
        assert qk == 1, "the gate/up adapter B factors go K-major"
        if lora_gate is None:
            t = [(None, None, 0.0), t[0]]
        with _timed("ffn_gate_up"):
            rc = _lib.lib().cpt_ffn_gate_up_lora(
                x.data_ptr(), w_gate.data_ptr(), w_up.data_ptr(), n, hdim, d, cache, group_size,
                p(h_mid), p(hg), p(hu), p(qg), p(sg), p(qu), p(su), r, ldp, t[0][0], t[0][1],
                t[0][2], t[1][0], t[1][1], t[1][2], _stream(x))
        del keep
    else:
        with _timed("ffn_gate_up"):
            rc = _lib.lib().cpt_ffn_gate_up(x.data_ptr(), w_gate.data_ptr(), w_up.data_ptr(), n,
                                            hdim, d, cache, group_size, p(h_mid), p(hg), p(hu),
                                            p(qg), p(sg), p(qu), p(su), _stream(x))
    check(rc, "ffn_gate_up")
    return h_mid, hg, hu, qg, sg, qu, su


def ffn_gate_up_outlier_fits(hidden: int) -> bool:
    """The outlier-codec epilogue runs on the 16x16x32 loop: d_model a
    multiple of 64."""
    return hidden > 0 and hidden % 64 == 0


def ffn_gate_up_outlier(x, w_gate, w_up, cache: int, group_size: int, slot_gate, slot_up,
                        k: int, out, lora_gate=None, lora_up=None):
    """Fused dual GEMM + GLU + int codec with config C3's outlier channels
    (cpt_ffn_gate_up_outlier): writes into `out` = (h_mid, q_gate, s_gate,
    o_gate, q_up, s_up, o_up), preallocated (row slices of the Function's
    buffers are fine); the slot maps come from an outlier selection."""
    _require_device(x, w_gate, w_up, slot_gate, slot_up)
    _check_bf16(x, w_gate, w_up)
    n, hdim = x.shape
    d = w_gate.shape[0]
    assert w_gate.shape == (d, hdim) and w_up.shape == (d, hdim)
    assert cache in (_lib.CACHE_INT4, _lib.CACHE_INT8) and k > 0
    x, w_gate, w_up = x.contiguous(), w_gate.contiguous(), w_up.contiguous()
    h_mid, qg, sg, og, qu, su, ou = out
    for t, shape in ((h_mid, (n, d)), (sg, (n, d // group_size)), (su, (n, d // group_size)),
                     (og, (n, k)), (ou, (n, k)),
                     (qg, (n, d // 2) if cache == _lib.CACHE_INT4 else (n, d)),
                     (qu, (n, d // 2) if cache == _lib.CACHE_INT4 else (n, d))):
        assert tuple(t.shape) == shape and t.is_contiguous(), (tuple(t.shape), shape)
    assert slot_gate.dtype == torch.int16 and slot_gate.shape == (d,) and slot_up.shape == (d,)
    rank = ldp = 0
    t = [(None, None, 0.0), (None, None, 0.0)]
    keep = None
    if lora_gate is not None or lora_up is not None:
        present = [tt for tt in (lora_gate, lora_up) if tt is not None]
        rank, ldp, qk, _, t, keep = _lora_args([(xa, bw.t(), sc) for xa, bw, sc in present], d,
                                               ((hdim, d),))
        assert qk == 1, "the gate/up adapter B factors go K-major"
        if lora_gate is None:
            t = [(None, None, 0.0), t[0]]
        elif lora_up is None:
            t = [t[0], (None, None, 0.0)]
    with _timed("ffn_gate_up"):
        rc = _lib.lib().cpt_ffn_gate_up_outlier(
            x.data_ptr(), w_gate.data_ptr(), w_up.data_ptr(), n, hdim, d, cache, group_size,
            h_mid.data_ptr(), qg.data_ptr(), sg.data_ptr(), qu.data_ptr(), su.data_ptr(),
            slot_gate.data_ptr(), og.data_ptr(), slot_up.data_ptr(), ou.data_ptr(), k, rank, ldp,
            t[0][0], t[0][1], t[0][2], t[1][0], t[1][1], t[1][2], _stream(x))
    del keep
    check(rc, "ffn_gate_up_outlier")
    return out


def ffn_down_dgrad(grad_y, w_down, cache: int, group_size: int, c_gate, s_gate, c_up, s_up,
                   want_h_mid: bool, lora=None, outliers=None, inplace: bool = False):
    """Fused grad_y @ w_down + dequantise + SwiGLU backward.
    Returns (grad_h_gate, grad_h_up, h_mid_hat | None).  lora = (gy B_d
    [n, r], A_d [r, inter], s): the down projection's LoRA term of
    grad_h_mid.  outliers = (slot_gate, o_gate, slot_up, o_up): the C3
    outlier channels (int16 slot maps [inter], bf16 blocks [n, k]) that
    replace their dequantised columns.  `inplace=True` (bf16 cache only)
    writes grad_h_gate / grad_h_up over c_gate / c_up, which must be
    contiguous and private to the caller (the in-place GLU backward,
    src/flashffn.py:129-198)."""
    _require_device(grad_y, w_down)
    _check_bf16(grad_y, w_down)
    n, hdim = grad_y.shape
    d = w_down.shape[1]
    assert w_down.shape == (hdim, d)
    grad_y, w_down = grad_y.contiguous(), w_down.contiguous()
    dev = grad_y.device
    if inplace:
        assert cache == _lib.CACHE_BF16 and c_gate.is_contiguous() and c_up.is_contiguous()
        assert tuple(c_gate.shape) == (n, d) and tuple(c_up.shape) == (n, d)
        dg, du = c_gate, c_up
    else:
        dg = torch.empty((n, d), dtype=torch.bfloat16, device=dev)
        du = torch.empty((n, d), dtype=torch.bfloat16, device=dev)
    hm = torch.empty((n, d), dtype=torch.bfloat16, device=dev) if want_h_mid else None

    keep_in = [None if t is None else t.contiguous() for t in (c_gate, s_gate, c_up, s_up)]
    c_gate, s_gate, c_up, s_up = keep_in

    def p(t):
        return None if t is None else t.data_ptr()

    if outliers is not None:
        slot_g, o_g, slot_u, o_u = [t.contiguous() for t in outliers]
        k = o_g.shape[1]
        assert o_u.shape[1] == k and slot_g.numel() == d and slot_u.numel() == d
        rank, ldp, pp, qq, alpha, keep = 0, 0, None, None, 0.0, []
        if lora is not None:
            gyb, a_down, s = lora
            a_down = a_down.contiguous()
            rank, ldp, qk, ldq, t, keep = _lora_args([(gyb, a_down, s)], d, ((hdim, d),))
            assert qk == 0 and ldq == d
            pp, qq, alpha = t[0]
        with _timed("ffn_down_dgrad"):
            rc = _lib.lib().cpt_ffn_down_dgrad_outlier(
                grad_y.data_ptr(), w_down.data_ptr(), n, hdim, d, cache, group_size, p(c_gate),
                p(s_gate), slot_g.data_ptr(), o_g.data_ptr(), p(c_up), p(s_up),
                slot_u.data_ptr(), o_u.data_ptr(), k, dg.data_ptr(), du.data_ptr(), p(hm),
                rank, ldp, pp, qq, alpha, _stream(grad_y))
        del keep
    elif lora is not None:
        gyb, a_down, s = lora
        a_down = a_down.contiguous()          # [r, inter] rows: the MN-major factor
        r, ldp, qk, ldq, t, keep = _lora_args([(gyb, a_down, s)], d, ((hdim, d),))
        assert qk == 0 and ldq == d
        with _timed("ffn_down_dgrad"):
            rc = _lib.lib().cpt_ffn_down_dgrad_lora(
                grad_y.data_ptr(), w_down.data_ptr(), n, hdim, d, cache, group_size, p(c_gate),
                p(s_gate), p(c_up), p(s_up), dg.data_ptr(), du.data_ptr(), p(hm), r, ldp,
                t[0][0], t[0][1], t[0][2], _stream(grad_y))
        del keep
    else:
        with _timed("ffn_down_dgrad"):
            rc = _lib.lib().cpt_ffn_down_dgrad(grad_y.data_ptr(), w_down.data_ptr(), n, hdim, d,
                                               cache, group_size, p(c_gate), p(s_gate), p(c_up),
                                               p(s_up), dg.data_ptr(), du.data_ptr(), p(hm),
                                               _stream(grad_y))
    check(rc, "ffn_down_dgrad")
    return dg, du, hm


def wgrad_glu(grad_y: torch.Tensor, cache: int, group_size: int, q_gate, s_gate, q_up, s_up,
              name: str = "gemm_wgrad_down_glu") -> torch.Tensor:
    """grad_y^T @ h^ -> bf16 [hidden, inter], h^ = bf16(SiLU(hg^) * hu^) formed
    from the int4/int8 cache inside the GEMM's operand staging: the weight
    gradient of the down projection without K2's h_mid^ (bit-equal to
    mm(grad_y.t(), h_mid_hat), src/flashffn.py:1538-1543)."""
    _require_device(grad_y, q_gate, s_gate, q_up, s_up)
    _check_bf16(grad_y)
    n, hdim = grad_y.shape
    assert cache in (_lib.CACHE_INT4, _lib.CACHE_INT8), f"int4/int8 cache expected, got {cache}"
    d = q_gate.shape[1] * (2 if cache == _lib.CACHE_INT4 else 1)
    assert tuple(q_up.shape) == tuple(q_gate.shape) and q_gate.shape[0] == n
    assert group_size > 0 and d % group_size == 0, \
        f"D={d} not divisible by group_size={group_size}"
    assert tuple(s_gate.shape) == (n, d // group_size) == tuple(s_up.shape), \
        f"scales {tuple(s_gate.shape)} / {tuple(s_up.shape)} != {(n, d // group_size)}"
    q_gate, s_gate, q_up, s_up = (t.contiguous() for t in (q_gate, s_gate, q_up, s_up))
    if grad_y.stride(1) != 1 or grad_y.stride(0) % 8 or grad_y.data_ptr() % 16:
        grad_y = grad_y.contiguous()
    c = torch.empty((hdim, d), dtype=torch.bfloat16, device=grad_y.device)
    with _timed(name):
        rc = _lib.lib().cpt_gemm_wgrad_glu(grad_y.data_ptr(), grad_y.stride(0), cache, group_size,
                                           q_gate.data_ptr(), s_gate.data_ptr(), q_up.data_ptr(),
                                           s_up.data_ptr(), c.data_ptr(), c.stride(0), hdim, d, n,
                                           _stream(grad_y))
    check(rc, name)
    return c


def addmm_(c: torch.Tensor, a: torch.Tensor, b: torch.Tensor, alpha: float,
           name: str = "gemm_lora_add") -> torch.Tensor:
    """In place: c = bf16(c + bf16(alpha * bf16(a @ b))), PEFT's
    `h + s * B(A(x))` in bf16 (src/flashffn.py:1414,1420,1439,1529)."""
    _require_device(c, a, b)
    _check_bf16(c, a, b)
    M, K = a.shape
    K_, N = b.shape
    assert K == K_ and tuple(c.shape) == (M, N) and c.stride(1) == 1
    a, lda, ak = _layout_a(a)
    b, ldb, bk = _layout_b(b)
    with _timed(name):
        rc = _lib.lib().cpt_gemm_bf16_ex(a.data_ptr(), lda, ak, b.data_ptr(), ldb, bk, c.data_ptr(),
                                         c.stride(0), M, N, K, float(alpha), 1, 1, None, _stream(a))
    check(rc, name)
    return c


def mm_splitk(a: torch.Tensor, b: torch.Tensor, alpha: float = 1.0, splits: int | None = None,
              name: str = "gemm_splitk") -> torch.Tensor:
    """bf16(alpha * (a @ b)) with the K reduction split across blocks (fp32
    partials, fixed-order sum): for the thin adapter gradients that reduce
    over all tokens.  With a token-major operand on each side and M or N <=
    32 (the rank: grad_A = s (grad B)^T x, grad_B = s grad_y^T (x A^T)) the
    token-reduction kernel runs instead of 256 x 256 tiles."""
    _require_device(a, b)
    _check_bf16(a, b)
    M, K = a.shape
    K_, N = b.shape
    assert K == K_
    at = a.t()
    if splits is None and _row_major(at) and _row_major(b) and K >= 256:
        if M <= SKINNY_MAX_RANK and M % 8 == 0 and N % 8 == 0:
            return skinny_t(b, at, alpha, trans=True, name=name)
        if N <= SKINNY_MAX_RANK and N % 8 == 0 and M % 8 == 0:
            return skinny_t(at, b, alpha, trans=False, name=name)
    a, lda, ak = _layout_a(a)
    b, ldb, bk = _layout_b(b)
    if splits is None:
        tiles = ((M + 255) // 256) * ((N + 255) // 256)
        splits = max(1, min((K + 63) // 64, (512 + tiles - 1) // tiles))
    splits = max(splits, _min_splits(K, lda, ak, ldb, bk))
    ldc = (N + 7) // 8 * 8
    c = torch.empty((M, ldc), dtype=torch.bfloat16, device=a.device)
    ws = torch.empty((splits * M * N,), dtype=torch.float32, device=a.device)
    with _timed(name):
        rc = _lib.lib().cpt_gemm_bf16_ex(a.data_ptr(), lda, ak, b.data_ptr(), ldb, bk, c.data_ptr(),
                                         ldc, M, N, K, float(alpha), 2, splits, ws.data_ptr(),
                                         _stream(a))
    check(rc, name)
    return c if ldc == N else c[:, :N]


# epilogues of the general-layout GEMM (cpt_gemm_any)
ANY_STORE, ANY_ADD, ANY_SCALE = 0, 1, 2
_ANY_DT = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


def mm_any(a: torch.Tensor, b: torch.Tensor, alpha: float = 1.0, mode: int = ANY_STORE,
           out: torch.Tensor | None = None, name: str = "gemm_any") -> torch.Tensor:
    """a [M, K] @ b [K, N] for float32 / float16 / bfloat16 operands of any
    strides, on the fp32 MFMA (cpt_gemm_any): the products the bf16 engine
    does not take (config C1's float32, unaligned views, rank-1 factors).
    mode ANY_STORE: rd(a @ b); ANY_SCALE: rd(alpha * rd(a @ b)); ANY_ADD: in
    place, out = rd(out + rd(alpha * rd(a @ b))), with rd the rounding to the
    operands' dtype (the reference's eager op order)."""
    _require_device(a, b)
    assert a.dim() == 2 and b.dim() == 2, "2-D operands expected"
    assert a.dtype == b.dtype and a.dtype in _ANY_DT, f"unsupported dtypes {a.dtype}, {b.dtype}"
    M, K = a.shape
    K_, N = b.shape
    assert K == K_, f"inner dims differ: {tuple(a.shape)} @ {tuple(b.shape)}"
    if mode == ANY_ADD:
        assert out is not None and tuple(out.shape) == (M, N) and out.dtype == a.dtype
    else:
        out = torch.empty((M, N), dtype=a.dtype, device=a.device)
    with _timed(name):
        rc = _lib.lib().cpt_gemm_any(_ANY_DT[a.dtype], a.data_ptr(), a.stride(0), a.stride(1),
                                     b.data_ptr(), b.stride(0), b.stride(1), out.data_ptr(),
                                     out.stride(0), out.stride(1), M, N, K, float(alpha), mode,
                                     _stream(a))
    check(rc, name)
    return out
