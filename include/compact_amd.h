/*
 * compact_amd.h -- C ABI of libcompact_amd.so, the gfx950 (MI355X) kernels of
 * the FlashFFN v3 hot path (SwiGLU FFN with a compressed GLU cache).
 *
 * Every entry point takes device pointers, sizes and a HIP stream (passed as
 * void*; NULL is the legacy default stream), launches asynchronously on that
 * stream, allocates nothing and returns a status code (0 = success, see
 * CPT_* below; cpt_status_string() gives the text).  Tensors are row-major and
 * contiguous.  dtype codes: 0 = float32, 1 = float16, 2 = bfloat16.
 * References are file:line in the reference repository SDMuhsin/CompAct.
 */
#ifndef COMPACT_AMD_H
#define COMPACT_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  CPT_OK = 0,
  CPT_ERR_BITS = 1,        /* bits not in {4, 8} */
  CPT_ERR_RAGGED = 2,      /* D % group_size != 0 (ragged last group) */
  CPT_ERR_GROUP_POW2 = 3,  /* group_size not a power of two (fused kernels) */
  CPT_ERR_SHAPE = 4,       /* negative / inconsistent size, null pointer */
  CPT_ERR_DTYPE = 5,       /* dtype code not supported by this entry point */
  CPT_ERR_LAUNCH = 6,      /* the HIP launch failed */
  CPT_ERR_ALIGN = 7,       /* a pointer misses the alignment the kernel needs */
  CPT_ERR_TOO_LARGE = 8    /* size beyond what the kernel indexes (GEMM: a transposed
                              operand whose k range in one block spans >= 2 GiB; the
                              Python host splits k before that) */
};

enum { CPT_F32 = 0, CPT_F16 = 1, CPT_BF16 = 2 };

const char* cpt_status_string(int status);
int cpt_abi_version(void);

/* ---------------- per-group absmax codec ---------------- */

/* Replaces v3_quantize_group_absmax (src/flashffn.py:1055-1088).
 * t: [n, d] of `dtype`; payload: uint8 [n, d/2] (bits=4, code+8 nibbles, even
 * column low) or int8 [n, d] (bits=8); scales: fp16 [n, d/group_size].
 * scale = fp16(absmax/qmax); code = clamp(rint(v/safe), +-qmax).  Any
 * group_size dividing d (the eager codec has no power-of-two requirement). */
int cpt_v3_quantize_group_absmax(const void* t, int dtype, int64_t n, int64_t d, int bits,
                                 int64_t group_size, void* payload, void* scales, void* stream);

/* Replaces v3_dequantize_group_absmax (src/flashffn.py:1091-1110):
 * out[n, d] (out_dtype) = out_dtype(fp32(code) * fp32(scale)). */
int cpt_v3_dequantize_group_absmax(const void* payload, const void* scales, int64_t n, int64_t d,
                                   int bits, int64_t group_size, void* out, int out_dtype,
                                   void* stream);

/* ---------------- GLU elementwise kernels ---------------- */

/* Replaces triton_silu_mul / _silu_mul_fwd_kernel (src/flashffn.py:50-82,205-220):
 * out = (g * sigmoid(g)) * u in float32, stored in `dtype`. */
int cpt_silu_mul(const void* h_gate, const void* h_up, void* out, int64_t n_elements, int dtype,
                 void* stream);

/* Replaces triton_swiglu_backward / _swiglu_bwd_kernel (src/flashffn.py:85-126,223-239). */
int cpt_swiglu_backward(const void* grad_h_mid, const void* h_gate, const void* h_up,
                        void* grad_h_gate, void* grad_h_up, int64_t n_elements, int dtype,
                        void* stream);

/* Replaces triton_swiglu_backward_glu / _swiglu_bwd_glu_kernel
 * (src/flashffn.py:129-198,259-293): the backward plus h_mid (NULL to skip);
 * outputs may alias inputs (in-place mode). */
int cpt_swiglu_backward_glu(const void* grad_h_mid, const void* h_gate, const void* h_up,
                            void* grad_h_gate, void* grad_h_up, void* h_mid, int64_t n_elements,
                            int dtype, void* stream);

/* ---------------- fused codec kernels (bf16 only) ---------------- */

/* Replaces triton_silu_mul_quant / K1 _v3_silu_mul_quant_fwd_kernel
 * (src/flashffn.py:1188-1225,1314-1340): h_mid = SiLU(g)*u (bf16 [n,d]) and
 * the codec of both g and u.  group_size must be a power of two. */
int cpt_silu_mul_quant(const void* h_gate, const void* h_up, int64_t n, int64_t d, int bits,
                       int64_t group_size, void* h_mid, void* q_gate, void* s_gate, void* q_up,
                       void* s_up, void* stream);

/* Replaces triton_dequant_swiglu_backward / K2 _v3_dequant_swiglu_bwd_kernel
 * (src/flashffn.py:1256-1300,1343-1373): dequantise both caches through bf16,
 * SwiGLU backward, and h_mid^ when h_mid_hat is not NULL.  grad_h_gate may
 * be the same buffer as grad_h_mid (written over it); no other output may
 * alias an input. */
int cpt_dequant_swiglu_backward(const void* grad_h_mid, const void* q_gate, const void* s_gate,
                                const void* q_up, const void* s_up, int64_t n, int64_t d,
                                int bits, int64_t group_size, void* grad_h_gate,
                                void* grad_h_up, void* h_mid_hat, void* stream);

/* ---------------- outlier channels (config C3) ---------------- */
/* The reference has no per-group codec with outlier channels; this is the
 * build's specification after HyC-LoRA (hyclora/operators/compress_function.py):
 * the k columns with the largest L2 norm over all rows are kept in bf16
 * (:80-88), zeroed before quantisation (:111-143) and written back after
 * dequantisation (:147-174).  slot: int16 [d], -1 or the column's position
 * among the selected columns in ascending column order; outliers: bf16 [n, k].
 * The outlier kernels need group_size in 8..512, d % 8 == 0 and 16-byte
 * aligned rows. */

/* Select the k outlier columns of t [n, d]: fp64 column sums of squares in a
 * fixed order (partial: fp64 [ceil(n/64), d]; sumsq: fp64 [d]), rank with
 * ties to the lower column, write slot [d] and idx int32 [k] (ascending).
 * n is the number of leading rows that rank the channels: HyC-LoRA ranks on
 * the first sample, x_[0] of a [B, S, d] tensor (S rows). */
int cpt_outlier_select(const void* t, int dtype, int64_t n, int64_t d, int64_t k,
                       void* partial, void* sumsq, void* slot, void* idx, void* stream);

/* cpt_outlier_select on two tensors of one shape, t0 and t1 (the gate and up
 * activations), in the same three launches, so the two single-block ranking
 * passes run side by side.  Each tensor's results equal a cpt_outlier_select
 * call on it.  Workspace: partial fp64 [2, ceil(n/64), d] and sumsq fp64
 * [2, d], tensor i using block i.  No counterpart in the reference, which
 * ranks each tensor on its own (compress_function.py:80-88); for callers that
 * select the gate and up channels of one forward together. */
int cpt_outlier_select_pair(const void* t0, const void* t1, int dtype, int64_t n, int64_t d,
                            int64_t k, void* partial, void* sumsq, void* slot0, void* idx0,
                            void* slot1, void* idx1, void* stream);

/* v3_quantize_group_absmax with the slot columns extracted (copied to
 * outliers, zeroed) before quantisation. */
int cpt_v3_quantize_outlier(const void* t, int dtype, int64_t n, int64_t d, int bits,
                            int64_t group_size, const void* slot, int64_t k, void* outliers,
                            void* payload, void* scales, void* stream);

/* Dequantise to bf16 [n, d] and write the stored outlier columns back. */
int cpt_v3_dequantize_outlier(const void* payload, const void* scales, const void* slot, int64_t k,
                              const void* outliers, int64_t n, int64_t d, int bits,
                              int64_t group_size, void* out, void* stream);

/* K1 with outlier channels: h_mid from the full g, u; the codes of the
 * zeroed tensors; outliers of each (slot tables may differ). */
int cpt_silu_mul_quant_outlier(const void* h_gate, const void* h_up, int64_t n, int64_t d,
                               int bits, int64_t group_size, const void* slot_gate,
                               const void* slot_up, int64_t k, void* h_mid, void* q_gate,
                               void* s_gate, void* o_gate, void* q_up, void* s_up, void* o_up,
                               void* stream);

/* K2 with the outlier columns restored after the bf16 dequantisation
 * (grad_h_gate may be written over grad_h_mid, as in K2). */
int cpt_dequant_swiglu_backward_outlier(const void* grad_h_mid, const void* q_gate,
                                        const void* s_gate, const void* slot_gate,
                                        const void* o_gate, const void* q_up, const void* s_up,
                                        const void* slot_up, const void* o_up, int64_t k,
                                        int64_t n, int64_t d, int bits, int64_t group_size,
                                        void* grad_h_gate, void* grad_h_up, void* h_mid_hat,
                                        void* stream);

/* ---------------- MFMA bf16 GEMMs (gfx950) ---------------- */

/* Replaces the cuBLAS GEMMs the reference issues through F.linear / @
 * (src/flashffn.py:1410-1439,1503-1587):  C[M, N] = A[M, K] . B[K, N]
 * (+ A2[M, K2] . B2[K2, N] when a2 != NULL, same layouts), fp32 accumulate,
 * bf16 in and out.  a_kmajor: A stored [M][lda] (1) or [K][lda] (0);
 * b_kmajor: B stored [N][ldb] (1, the nn.Linear weight) or [K][ldb] (0).
 * Pointers 16-byte aligned, leading dims multiples of 8, the contiguous
 * extent of each operand a multiple of 8, N and ldc multiples of 4.
 * A product whose K (and K2, for a second pair) is a multiple of 64, with N
 * and ldc multiples of 8 and C 16-byte aligned, runs on the 16x16x32 MFMA
 * loop: any M, every operand layout, one pair or two.  Every other product
 * runs on the 32x32x16 loop of the fused FFN kernels.  Both round the fp32
 * sum to bf16 once; their summation orders differ (cpt_gemm_bf16_ex mode 0
 * always uses the 32x32x16 loop). */
int cpt_gemm_bf16(const void* a, int64_t lda, int a_kmajor, const void* b, int64_t ldb,
                  int b_kmajor, const void* a2, int64_t lda2, const void* b2, int64_t ldb2,
                  int64_t K2, void* c, int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream);

/* Stream-K workspace of the 16x16x32 loop.  The reference's GEMMs come from
 * cuBLAS, which picks its own split of K (src/flashffn.py:1410-1439,
 * 1503-1587); this is the same choice made explicit, in the manner of
 * cublasSetWorkspace.  A product of cpt_gemm_bf16 or cpt_gemm_bf16_lora on
 * the 16x16x32 loop whose tile count T (256 x 256 tiles) is above the CU
 * count S and not a multiple of it, with at least 4 k-tiles of 64, leaves
 * its last wave part-empty; with a workspace attached to the device it runs
 * T - (T mod S) - S tiles one per block and shares the k-iterations of the
 * other (T mod S) + S tiles evenly over S more blocks, which finish shared
 * tiles in a fixed order: the result is deterministic for a given shape and
 * CU count, and differs from the unshared summation order in the last bits.
 * cpt_gemm_stream_k_bytes() is the size the current device needs (-1 without
 * a device).  cpt_gemm_stream_k_workspace(ws, bytes) attaches caller-owned
 * device memory of at least that size, 256-byte aligned and zero-filled, to
 * the current device for every later call on it (the kernels leave it
 * zero-filled again); NULL detaches it (one tile per block).  The memory
 * must stay valid while attached, and products that run at the same time on
 * one device (several streams) must not share it. */
int64_t cpt_gemm_stream_k_bytes(void);
int cpt_gemm_stream_k_workspace(void* workspace, int64_t bytes);

/* Skinny product of the adapter terms: C[M, R] = bf16(alpha * A[M, K] . Q^T)
 * with A [M][lda] and Q [R][ldq] both K-contiguous, R <= 32 (the rank), bf16
 * in and out, fp32 accumulate.  Replaces the thin F.linear / @ of the LoRA
 * terms (src/flashffn.py:1414,1420,1439: x A^T, h_mid A_d^T; :1521,1556-1557:
 * grad_y B_d, grad_h_gate B_g, grad_h_up B_u).  HBM-bound: A is streamed once.
 * K is split `splits` ways; with splits > 1 `workspace` holds splits * M * R
 * floats and the partials are summed in split order (deterministic).
 * Pointers 16-byte aligned, lda, ldq and K multiples of 8. */
int cpt_gemm_bf16_skinny(const void* a, int64_t lda, const void* q, int64_t ldq, void* c,
                         int64_t ldc, int64_t M, int64_t R, int64_t K, float alpha, int splits,
                         void* workspace, void* stream);

/* Token reduction of the adapter gradients: Z[N, R] = bf16(alpha * X^T . P)
 * with X [T][ldx] and P [T][ldp] token-major, R <= 32, written to
 * out[n * ldo + r] or, with out_trans, out[r * ldo + n] (Z^T).  Replaces the
 * thin gradient GEMMs of the LoRA factors (src/flashffn.py:1538-1545,
 * 1575-1582: grad_B = s grad_y^T (x A^T), grad_A = s (grad B)^T x).  The
 * tokens are split `splits` ways; `workspace` holds splits * N * R floats and
 * the partials are summed in split order (deterministic).  Pointers 16-byte
 * aligned, ldx, ldp, N and R multiples of 8. */
int cpt_gemm_bf16_skinny_t(const void* x, int64_t ldx, const void* p, int64_t ldp, void* out,
                           int64_t ldo, int out_trans, int64_t T, int64_t N, int64_t R,
                           float alpha, int splits, void* workspace, void* stream);

/* Both adapter products of one token-major operand X [T, N] in one pass over
 * it: C[T, R] = bf16(alpha_c * X . Q^T) (Q [R, N] rows ldq apart, or with
 * q_nr the B factor itself, [N, R] rows ldq apart: the projection of
 * cpt_gemm_bf16_skinny) and Z = bf16(alpha_z * X^T . P) (P
 * [T, R]: the token reduction of cpt_gemm_bf16_skinny_t, written [N, R] or,
 * with z_trans, [R, N]).  Replaces the pairs the reference issues on one
 * tensor in the LoRA backward (src/flashffn.py:1556-1557 with :1575-1582:
 * grad_h_gate B_g and s grad_h_gate^T (x A_g^T), likewise grad_h_up; :1521
 * with :1545: grad_y B_d and s grad_y^T (h_mid A_d^T)), which read X twice.
 * Blocks take 512 columns and T / `splits` tokens; the fp32 partials (C per
 * column block, Z per token split) are summed in split order
 * (deterministic).  workspace: cpt_gemm_bf16_skinny_dual_workspace_bytes
 * bytes.  R <= 32 and a multiple of 8, N a multiple of 8, pointers 16-byte
 * aligned. */
int64_t cpt_gemm_bf16_skinny_dual_workspace_bytes(int64_t T, int64_t N, int64_t R, int splits);
int cpt_gemm_bf16_skinny_dual(const void* x, int64_t ldx, const void* q, int64_t ldq, int q_nr,
                              const void* p, int64_t ldp, void* c, int64_t ldc, float alpha_c,
                              void* z, int64_t ldz, int z_trans, float alpha_z, int64_t T,
                              int64_t N, int64_t R, int splits, void* workspace, void* stream);

/* dst [cols][ld_dst] = src [rows][ld_src] transposed (bf16).  No reference
 * counterpart: a layout helper for the weight gradients dg^T x and du^T x
 * (src/flashffn.py:1585,1587), which then read x^T as a K-major operand with
 * bit-identical results.  rows, cols and both strides multiples of 8,
 * pointers 16-byte aligned. */
int cpt_transpose_bf16(const void* src, int64_t ld_src, int64_t rows, int64_t cols, void* dst,
                       int64_t ld_dst, void* stream);

/* No counterpart in the reference.  cpt_gemm_bf16_skinny_t for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the same kernels and result, with the
 * split partials in a fixed device array of CPT_NOALLOC_SCRATCH_BYTES per GPU
 * inside the library instead of a caller workspace.  The caller passes the
 * inputs and the output.  splits * N * R * 4 bytes (after the split count is
 * normalised as in cpt_gemm_bf16_skinny_t) must fit, else CPT_ERR_TOO_LARGE.
 * The array persists until the process ends and every call on a GPU shares
 * it: calls that overlap on one GPU (two streams, two threads) race. */
#define CPT_NOALLOC_SCRATCH_BYTES (16 << 20)
int cpt_gemm_bf16_skinny_t_noalloc(const void* x, int64_t ldx, const void* p, int64_t ldp,
                                   void* out, int64_t ldo, int out_trans, int64_t T, int64_t N,
                                   int64_t R, float alpha, int splits, void* stream);

/* Extended GEMM for the adapter (LoRA) terms, one operand pair:
 *   mode 0: C = bf16(A.B) on the 32x32x16 loop for every shape: the
 *           summation order of the fused FFN kernels' GEMMs
 *   mode 1: C = bf16(C + bf16(alpha * bf16(A.B)))   (PEFT's h + s * B(A(x)),
 *           src/flashffn.py:1414,1420,1439,1529; C read and written in place)
 *   mode 2: C = bf16(alpha * sum of `splits` fp32 partials of A.B over K
 *           chunks); `workspace` holds splits * M * N floats (16-byte aligned).
 *           For the thin adapter gradients that reduce over tokens
 *           (src/flashffn.py:1538-1545,1575-1582). */
int cpt_gemm_bf16_ex(const void* a, int64_t lda, int a_kmajor, const void* b, int64_t ldb,
                     int b_kmajor, void* c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                     float alpha, int mode, int splits, void* workspace, void* stream);

/* General-layout GEMM for every product the bf16 engine above does not take:
 * float32 (config C1) and float16 operands, bf16 views whose rows are not
 * 16-byte aligned, ranks and widths that are not multiples of 8.  Replaces
 * the library GEMMs the reference calls through F.linear / @ for those
 * operands (src/flashffn.py:1410-1439,1503-1587).
 *   A(m, k) = a[m*sam + k*sak], B(k, n) = b[k*sbk + n*sbn],
 *   C(m, n) = c[m*scm + n*scn]; a, b, c all of `dtype`.
 * fp32 accumulation on the fp32 MFMA (bf16 / fp16 products exact); with rd()
 * the rounding to dtype:
 *   mode 0: C = rd(A.B)
 *   mode 1: C = rd(C + rd(alpha * rd(A.B)))   (h + s * F.linear(xa, b))
 *   mode 2: C = rd(alpha * rd(A.B))           (s * (a @ b))
 * Any strides (elements, not bytes); pointers aligned to the element size. */
int cpt_gemm_any(int dtype, const void* a, int64_t sam, int64_t sak, const void* b, int64_t sbk,
                 int64_t sbn, void* c, int64_t scm, int64_t scn, int64_t M, int64_t N,
                 int64_t K, float alpha, int mode, void* stream);

/* Low-rank adapter terms folded into a GEMM's output ahead of its epilogue,
 * in PEFT's op order `h + s * B(A(x))` (src/flashffn.py:1414,1420,1439,1529,
 * 1558-1566):
 *   out = bf16(bf16(out) + bf16(alpha_t * bf16(P_t . Q_t)))   t = 0, then 1
 * rank in {8, 16}, or {24, 32} where the product runs on the 16x16x32 loop
 * (every K a multiple of 64, N of 8; otherwise CPT_ERR_SHAPE); a rank that is
 * not a multiple of 8 is passed zero-padded to the next one, P's extra
 * columns and Q's extra k zero;
 * P_t [M, rank] (tokens x rank, e.g. x A^T or grad_y B) with
 * rows ldp apart (ldp % 8 == 0, 16-byte aligned); Q_t the [rank, N] factor,
 * given as [N, rank] contiguous (q_kmajor = 1: an nn.Linear B weight) or as
 * [rank, N] with rows ldq apart (q_kmajor = 0: an A weight).  A term whose P
 * is NULL is skipped.  Replaces the separate `F.linear(xa, b)`, scale and add
 * of the reference; the result equals cpt_gemm_bf16 followed by
 * cpt_gemm_bf16_ex mode 1 up to the fp32 summation order of the rank-sized
 * dot products. */
int cpt_gemm_bf16_lora(const void* a, int64_t lda, int a_kmajor, const void* b, int64_t ldb,
                       int b_kmajor, const void* a2, int64_t lda2, const void* b2, int64_t ldb2,
                       int64_t K2, void* c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                       int64_t rank, int64_t ldp, int q_kmajor, int64_t ldq, const void* p0,
                       const void* q0, float alpha0, const void* p1, const void* q1,
                       float alpha1, void* stream);

/* Cache kinds of the fused FFN kernels. */
enum { CPT_CACHE_NONE = 0, CPT_CACHE_BF16 = 1, CPT_CACHE_INT4 = 4, CPT_CACHE_INT8 = 8 };

/* Fused forward of the gate/up projections (replaces F.linear(x, w_gate),
 * F.linear(x, w_up) and K1, src/flashffn.py:1410-1433): one dual MFMA GEMM
 * over x [n_tok, hidden] and w_gate, w_up [inter, hidden] whose epilogue
 * rounds h_gate/h_up to bf16 and writes h_mid = SiLU(h_gate)*h_up (if
 * h_mid != NULL) plus, by `cache`: nothing (NONE), h_gate/h_up bf16 (BF16),
 * or the int4/int8 per-group absmax codes and fp16 scales of both (bit-equal
 * to cpt_silu_mul_quant on the same bf16 values).  group_size in {32,64,128}. */
int cpt_ffn_gate_up(const void* x, const void* w_gate, const void* w_up, int64_t n_tok,
                    int64_t hidden, int64_t inter, int cache, int64_t group_size, void* h_mid,
                    void* h_gate, void* h_up, void* q_gate, void* s_gate, void* q_up,
                    void* s_up, void* stream);

/* cpt_ffn_gate_up with LoRA adapters on the gate and/or up projection
 * (src/flashffn.py:1410-1420): h_gate = bf16(bf16(x W_g^T) + bf16(alpha_gate
 * * bf16(p_gate . b_gate^T))) with p_gate = x A_g^T [n_tok, rank] (rows ldp
 * apart) and b_gate the B weight [inter, rank]; likewise h_up.  The GLU and
 * the codec then see these h.  Either term may be absent (NULL p). */
int cpt_ffn_gate_up_lora(const void* x, const void* w_gate, const void* w_up, int64_t n_tok,
                         int64_t hidden, int64_t inter, int cache, int64_t group_size,
                         void* h_mid, void* h_gate, void* h_up, void* q_gate, void* s_gate,
                         void* q_up, void* s_up, int64_t rank, int64_t ldp, const void* p_gate,
                         const void* b_gate, float alpha_gate, const void* p_up,
                         const void* b_up, float alpha_up, void* stream);

/* cpt_ffn_gate_up (with LoRA terms when rank > 0, as cpt_ffn_gate_up_lora)
 * for an int4/int8 cache with config C3's outlier channels in the codec:
 * the forward half of K1 with outliers (cpt_silu_mul_quant_outlier, the
 * reference's HyC-LoRA extraction, hyclora/operators/compress_function.py:
 * 111-143) fused into the dual GEMM's epilogue, so only h_mid, codes, scales
 * and the [n_tok, k] bf16 outlier blocks reach HBM.  slot_gate / slot_up:
 * int16 [inter] slot maps (-1 for ordinary columns, 16-byte aligned) from
 * cpt_outlier_select; a column with slot s >= 0 is copied to o[m * k + s]
 * and zeroed before the group absmax.  Bit-equal to the dual GEMM with a bf16
 * output followed by cpt_silu_mul_quant_outlier.  d_model a multiple of 64
 * (the 16x16x32 loop), else CPT_ERR_SHAPE. */
int cpt_ffn_gate_up_outlier(const void* x, const void* w_gate, const void* w_up, int64_t n_tok,
                            int64_t hidden, int64_t inter, int cache, int64_t group_size,
                            void* h_mid, void* q_gate, void* s_gate, void* q_up, void* s_up,
                            const void* slot_gate, void* o_gate, const void* slot_up, void* o_up,
                            int64_t k, int64_t rank, int64_t ldp, const void* p_gate,
                            const void* b_gate, float alpha_gate, const void* p_up,
                            const void* b_up, float alpha_up, void* stream);

/* Weight gradient of the down projection with the GLU decompressed in the
 * GEMM's operand staging (replaces K2's h_mid^ output and gy^T @ h_mid_hat,
 * src/flashffn.py:1538-1543): C[hidden, inter] (bf16, rows ldc apart) =
 * grad_y^T . h^, grad_y [n_tok, hidden] rows ldg apart, h^ = bf16(SiLU(hg^) *
 * hu^) with hg^ / hu^ the int4/int8 cache (codes + fp16 scales of
 * group_size 32/64/128) dequantised through bf16, bit-equal to the h_mid^
 * of cpt_dequant_swiglu_backward, so C equals that GEMM bit for bit. */
int cpt_gemm_wgrad_glu(const void* grad_y, int64_t ldg, int cache, int64_t group_size,
                       const void* q_gate, const void* s_gate, const void* q_up,
                       const void* s_up, void* c, int64_t ldc, int64_t hidden, int64_t inter,
                       int64_t n_tok, void* stream);

/* Fused backward of the down projection into the GLU (replaces gy @ w_down
 * and K2, src/flashffn.py:1525-1533): grad_h_mid = bf16(grad_y @ w_down)
 * with grad_y [n_tok, hidden], w_down [hidden, inter]; the epilogue reads the
 * cache (BF16: c_gate/c_up are h_gate/h_up bf16; INT4/INT8: codes + fp16
 * scales, dequantised through bf16) and writes grad_h_gate, grad_h_up and,
 * if h_mid_hat != NULL, h_mid^ = SiLU(hg^)*hu^ (bit-equal to
 * cpt_dequant_swiglu_backward on the same bf16 grad_h_mid).  With a BF16
 * cache, grad_h_gate / grad_h_up may be written over c_gate / c_up (each
 * element is read before it is overwritten, by the same thread). */
int cpt_ffn_down_dgrad(const void* grad_y, const void* w_down, int64_t n_tok, int64_t hidden,
                       int64_t inter, int cache, int64_t group_size, const void* c_gate,
                       const void* s_gate, const void* c_up, const void* s_up, void* grad_h_gate,
                       void* grad_h_up, void* h_mid_hat, void* stream);

/* cpt_ffn_down_dgrad with a LoRA adapter on the down projection
 * (src/flashffn.py:1527-1529): grad_h_mid = bf16(bf16(grad_y W_d) +
 * bf16(alpha * bf16(p . a_down))) with p = grad_y B_d [n_tok, rank] (rows ldp
 * apart) and a_down the A weight [rank, inter]. */
int cpt_ffn_down_dgrad_lora(const void* grad_y, const void* w_down, int64_t n_tok,
                            int64_t hidden, int64_t inter, int cache, int64_t group_size,
                            const void* c_gate, const void* s_gate, const void* c_up,
                            const void* s_up, void* grad_h_gate, void* grad_h_up,
                            void* h_mid_hat, int64_t rank, int64_t ldp, const void* p,
                            const void* a_down, float alpha, void* stream);

/* cpt_ffn_down_dgrad (optionally with the LoRA term of cpt_ffn_down_dgrad_lora:
 * rank 0 = none) for an int4/int8 cache with outlier channels (config C3;
 * HyC-LoRA's zero-and-overwrite on the v3 codec, hyclora/operators/
 * compress_function.py:147-174): columns with slot_gate[d] >= 0 take
 * o_gate[m * k + slot] (bf16 [n_tok, k]) in place of their dequantised value,
 * likewise for up, before the SwiGLU backward.  Bit-equal to the dgrad GEMM
 * followed by cpt_dequant_swiglu_backward_outlier. */
int cpt_ffn_down_dgrad_outlier(const void* grad_y, const void* w_down, int64_t n_tok,
                               int64_t hidden, int64_t inter, int cache, int64_t group_size,
                               const void* c_gate, const void* s_gate, const void* slot_gate,
                               const void* o_gate, const void* c_up, const void* s_up,
                               const void* slot_up, const void* o_up, int64_t k,
                               void* grad_h_gate, void* grad_h_up, void* h_mid_hat,
                               int64_t rank, int64_t ldp, const void* p, const void* a_down,
                               float alpha, void* stream);

/* ---------------- adapter families (DoRA magnitude) ---------------- */
/* VeRA, AdaLoRA and DyLoRA reach the kernels above as composed or sliced thin
 * factors (src/flashffn.py:1850-1921); DoRA's per-output-channel magnitude
 * c = m / nu needs the three entry points below.  All tensors of one call
 * share `dtype`; rd() is round-to-nearest-even to that dtype. */

/* out[i, j] = rd(x[i, j] * rd(m[j] / nu[j])) for x, out [n, d] (out may
 * alias x).  Replaces `h * (m / nu).unsqueeze(0)` and the chain rule
 * `g * c` of FlashFFNv3AdapterFunction (src/flashffn.py:1967-1975,2054,
 * 2128-2130). */
int cpt_dora_scale(const void* x, const void* m, const void* nu, int64_t n, int64_t d, int dtype,
                   void* out, void* stream);

/* Bytes of fp32 workspace cpt_col_dot_div needs for [n, d] inputs. */
int64_t cpt_col_dot_workspace_bytes(int64_t n, int64_t d);

/* out[j] = rd((sum_i rd(a[i, j] * b[i, j])) / den[j]) with the sum in fp32:
 * the DoRA magnitude gradients `((g * raw).sum(0, dtype=float32) /
 * den.float()).to(dtype)` (src/flashffn.py:2086-2089,2112-2125).  The
 * summation order is fixed (128-row chunks, then the chunks in order), so the
 * result is deterministic. */
int cpt_col_dot_div(const void* a, const void* b, const void* den, int64_t n, int64_t d,
                    int dtype, void* workspace, void* out, void* stream);

/* Bytes of fp32 workspace cpt_dora_col_norm needs. */
int64_t cpt_dora_col_norm_workspace_bytes(int64_t rows, int64_t r);

/* Replaces _v3_dora_col_norm (src/flashffn.py:1824-1840): nu[j] =
 * ||W_j + s (B A)_j||_2 for W [rows, cols], A [r, cols], B [rows, r] through
 * the Gram identity, in fp32, without forming B A; nu written in nu_dtype. */
int cpt_dora_col_norm(const void* w, const void* a, const void* b, int64_t rows, int64_t cols,
                      int64_t r, double s, int dtype, void* workspace, void* nu, int nu_dtype,
                      void* stream);

/* ---------------- top-K activation compression (FlashFFN v1/v2 API) ---------------- */

/* Replaces `torch.topk(h_mid.abs(), k, dim=-1, sorted=False)` + gather + the
 * int16 index cast of FlashFFNFunction (src/flashffn.py:349-356): per row of
 * t [n, d], the k entries of largest magnitude -> values [n, k] (t's dtype)
 * and columns indices [n, k] int16, in ascending column order; of entries
 * tied at the k-th magnitude the lowest columns are kept.  d <= 32767. */
int cpt_topk_abs(const void* t, int dtype, int64_t n, int64_t d, int64_t k, void* values,
                 void* indices, void* stream);

/* Replaces `zeros(n, d).scatter_(-1, indices, values)` (src/flashffn.py:
 * 410-415): out [n, d] = values at their columns, zero elsewhere.
 * d <= 32767 and d * sizeof(dtype) <= 64 KiB (one row is assembled in LDS). */
int cpt_topk_scatter(const void* values, const void* indices, int dtype, int64_t n, int64_t d,
                     int64_t k, void* out, void* stream);

/* ---------------- measurement ---------------- */

/* No counterpart in the reference: a probe for the sustained bf16 MFMA rate
 * the part reaches under its power cap, the achievable peak that the GEMM
 * roofline figures are read against.  `blocks` blocks of 4 wavefronts each
 * issue iters * 16 independent MFMAs on register operands (no memory
 * traffic): shape 0 v_mfma_f32_32x32x16_bf16 (32768 FLOPs each), shape 1
 * v_mfma_f32_16x16x32_bf16 (16384).  out [blocks * 4] fp32 receives one
 * partial sum per wavefront.  FLOPs per launch = blocks * iters * 64 *
 * (FLOPs per MFMA). */
int cpt_probe_mfma_rate(int shape, int blocks, int iters, float seed, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* COMPACT_AMD_H */
