/*
 * moc_amd.h - C ABI of the MI355X (gfx950) MoC sparse SwiGLU FFN library.
 *
 * libmoc_amd.so exports exactly the functions declared here.  All of them
 * take raw device pointers, element counts and element strides; `stream` is
 * a hipStream_t passed as void* (NULL = the default stream).  Nothing here
 * allocates device memory: callers own every buffer (outputs and workspaces;
 * the one exception, moc_global_after_gate_noalloc_bf16, uses a fixed device
 * array of the library's own), so any sequence of calls may be recorded into
 * a HIP graph.  No function
 * throws; each returns MOC_OK or a negative status, and moc_last_error()
 * describes the last failure on the calling thread.
 *
 * Selection rule used everywhere: values ordered descending, ties broken
 * toward the lower channel index, -0.0 == +0.0, NaN ranks above +inf.
 *
 * Citations name the reference interface each entry point replaces
 * (paths relative to the xiaohuangji/MoC repository).
 */
#ifndef MOC_AMD_H_
#define MOC_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOC_ABI_VERSION 3

/* status codes */
#define MOC_OK 0
#define MOC_ERR_INVALID (-1) /* bad argument: shape, dtype, stride, alignment */
#define MOC_ERR_HIP (-2)     /* HIP runtime / launch failure */

/* element types */
#define MOC_BF16 0
#define MOC_F32 1

/* index types */
#define MOC_I16 0
#define MOC_I32 1
#define MOC_I64 2

/* moc_gemm_ws: bytes of arrival counters at the start of its workspace (zero
 * when a call starts; every call leaves them zero). */
#define MOC_GEMM_WS_COUNTER_BYTES 4096

/* W_down^T [inter, hidden] of the decode entry points comes with its row
 * pitch ldw_down (elements; >= hidden, a multiple of 8).  A pitch that is a
 * multiple of 4 KB makes every row's same column block fall on the same
 * memory channels; the decode kernels read one column block per workgroup
 * down all selected rows, so MOC_DOWN_T_PITCH_PAD extra elements per row
 * (128 bytes) spread them (1b decode layer at one token: 19.5 -> 18.3 us). */
#define MOC_DOWN_T_PITCH_PAD 64

/* ------------------------------------------------------------------ misc */
const char* moc_last_error(void);
int moc_abi_version(void);

/* Zero `bytes` bytes at 16-byte aligned `dst` with a fill kernel (graph-safe
 * replacement for the reference's `tensor.zero_()` before scatters,
 * moc/training/triton_sparse_aux.py:212-213,277-278,345-346,404-405). */
int moc_fill_zero(void* dst, int64_t bytes, void* stream);

/* dst[r, c] = src[r, c] for c < cols, 0 for cols <= c < dst_cols.  Builds the
 * padded, 16-byte aligned copies the MFMA GEMM reads (no reference
 * counterpart beyond the contiguous copy of moc/inference/inference_ffn.py:109). */
int moc_copy_pad_2d(int dtype, const void* src, int64_t rows, int64_t cols, int64_t src_ld,
                    void* dst, int64_t dst_ld, int64_t dst_cols, void* stream);

/* ------------------------------------------------------------- selection */
/* Row-wise Top-K of scores[rows, inter] (leading dimension ld).
 * Replaces torch.topk(g, k, dim=-1, largest=True, sorted=False) at
 * moc/ffn.py:144,392 and moc/inference/inference_ffn.py:147-153, and the CUB
 * kernels behind moc_native::optimized_global_topk_bf16
 * (moc/inference/cuda/optimized_global_moc_ext.cu:39-125,376-398;
 * optimized_global_moc_ext.cpp:25-33,89).
 * Writes idx_out[rows, k] (MOC_I16/I32/I64) in ascending channel order,
 * optionally vals_out[rows, k] (scores at idx, same dtype) and a bitmask
 * mask_out[rows, mask_ld] of uint32 words (bit c%32 of word c/32 = channel
 * c selected).  score_transform 1 ranks by |SiLU(score)| rounded to the
 * score dtype (moc/ffn.py:335-338) while vals keep the raw scores.
 * Limits: 1 <= k <= inter <= 16384. */
int moc_topk_rows(int dtype, const void* scores, int64_t rows, int64_t inter, int64_t ld,
                  int64_t k, int score_transform, void* vals_out, void* idx_out, int idx_dtype,
                  uint32_t* mask_out, int64_t mask_ld, void* stream);

/* Channel indices of a selection bit mask (mask[rows, ld_words] of uint32
 * words, bit c%32 of word c/32 = channel c): idx[r, :] = the first k set
 * bits of row r in ascending channel order (a moc_topk_rows mask has exactly
 * k; slots a shorter row leaves empty get channel 0).  The backward's side
 * of the compact saved-mask format (a bitmask of
 * I bits per token instead of K int16 indices, moc/ffn.py:147,395,417); no
 * counterpart in the reference. */
int moc_mask_to_idx(const void* mask, int64_t rows, int64_t inter, int64_t ld_words, int64_t k,
                    void* idx, int idx_dtype, void* stream);

/* K' of the 2:8 structure: 2*floor(inter/8) + min(2, inter%8)
 * (moc/ffn.py:62-65). */
int64_t moc_moc28_effective_k(int64_t inter);

/* Top-2 of each aligned group of 8 channels, top-min(2, tail) of a trailing
 * partial group (moc/ffn.py:68-108).  idx_out/vals_out are [rows, K'] with
 * (top-1, top-2) per group. */
int moc_select_2of8(int dtype, const void* scores, int64_t rows, int64_t inter, int64_t ld,
                    void* vals_out, void* idx_out, int idx_dtype, void* stream);

/* ------------------------------------------------------- training helpers */
/* u_s = U[r, idx], s_s = SiLU(vals), z_s = s_s * u_s, z_full[r, idx] = z_s
 * with z_full zero-filled first (moc/training/triton_sparse_aux.py:197-231,
 * kernel :17-49; bf16 rounds s, then z).  Any output may be NULL. */
int moc_sparse_forward_aux(int dtype, const void* topk_vals, const void* idx, int idx_dtype,
                           const void* u_full, int64_t u_ld, int64_t rows, int64_t k,
                           int64_t inter, void* u_sparse, void* s_sparse, void* z_sparse,
                           void* z_full, int64_t z_ld, void* stream);

/* dense (zero-filled) [rows, ld] <- sparse [rows, k] at idx
 * (moc/training/triton_sparse_aux.py:266-290, kernel :71-87). */
int moc_scatter_sparse_to_dense(int dtype, const void* sparse, const void* idx, int idx_dtype,
                                int64_t rows, int64_t k, int64_t inter, void* dense, int64_t ld,
                                void* stream);

/* sparse [rows, k] <- dense [rows, ld] at idx
 * (moc/training/triton_sparse_aux.py:234-263, kernel :52-68). */
int moc_gather_dense_to_sparse(int dtype, const void* dense, int64_t ld, const void* idx,
                               int idx_dtype, int64_t rows, int64_t k, void* sparse,
                               void* stream);

/* GCP recompute s = SiLU(g_s), z = s * u_s over n entries
 * (_MoCGCPFunction.backward, moc/ffn.py:435-436).  Outputs may be NULL. */
int moc_gcp_recompute(int dtype, const void* g_sparse, const void* u_sparse, int64_t n,
                      void* s_sparse, void* z_sparse, void* stream);

/* GCP recompute and the scatter of z in one pass: s_sparse = bf16(SiLU(g)),
 * z_full[r, idx[r,j]] = bf16(s * u), zeros elsewhere (incl. pad columns up
 * to ld) (moc/ffn.py:435-442).  bf16 only; z_full rows 16-byte aligned with
 * ld a multiple of 8 and <= 8192.  s_sparse may be NULL. */
int moc_gcp_recompute_scatter(int dtype, const void* g_sparse, const void* u_sparse,
                              const void* idx, int idx_dtype, int64_t rows, int64_t k,
                              int64_t inter, void* s_sparse, void* z_full, int64_t ld,
                              void* stream);

/* grad_g, grad_u dense [rows, inter] rows out_ld elements apart (each row
 * written whole: inter values plus zeros up to the next multiple of 8,
 * nothing beyond it, so out_ld may leave room for the other tensor's rows,
 * e.g. grad_u = grad_g + pitch with out_ld = 2 pitch) from grad_z_full at idx:
 * grad_u = s*gz, grad_g = u*gz*SiLU'(g) (moc/training/triton_sparse_aux.py:
 * 363-423; bf16 follows the materialised-bf16 chain at :376-400, f32 the fused
 * kernel :139-182).  s_sparse may be NULL: s is then recomputed from g
 * (GCP, moc/ffn.py:435).  gz_full may be grad_u itself (gz_ld == out_ld,
 * bf16 with 16-byte aligned rows, pitch a multiple of 8 and <= 8192): each
 * row's gZ is read whole before that row is written. */
int moc_sparse_backward_aux(int dtype, const void* idx, int idx_dtype, const void* g_sparse,
                            const void* u_sparse, const void* s_sparse, const void* gz_full,
                            int64_t gz_ld, int64_t rows, int64_t k, int64_t inter, void* grad_g,
                            void* grad_u, int64_t out_ld, void* stream);

/* ------------------------------------------------------------------ GEMM */
/* C[M,N] (row-major, ldc) = sum_k A(m,k) B(k,n) [+ sum_k A2(m,k) B2(k,n)],
 * A(m,k) = A[m*a_sm + k*a_sk], B(k,n) = B[k*b_sk + n*b_sn].  Each operand
 * needs a unit stride along K or along M/N; the second pair (K2 > 0, A2 set)
 * must share the first pair's layouts.  bf16 operands: 16-byte aligned, the
 * non-unit stride a multiple of 8; f32 accumulation; c_dtype bf16 or f32.
 * f32 operands: any strides, f32 output.
 * Replaces the torch GEMMs of the FFN (moc/ffn.py:141,146,163,203-254,389,394,
 * 414,447-494) and the dense gate/up/down projections of
 * moc/inference/inference_ffn.py:166,171-179. */
int moc_gemm(int dtype, int64_t M, int64_t N, int64_t K, const void* A, int64_t a_sm,
             int64_t a_sk, const void* B, int64_t b_sk, int64_t b_sn, int64_t K2, const void* A2,
             int64_t a2_sm, int64_t a2_sk, const void* B2, int64_t b2_sk, int64_t b2_sn, void* C,
             int64_t ldc, int c_dtype, void* stream);

/* moc_gemm with a caller-provided device workspace (256-byte aligned).  A
 * bf16 product with fewer 256x256 output tiles than CUs then splits its K
 * range over several workgroups per tile:
 *  - at most half the CUs (weight gradients of small models): each tile as
 *    `ks` workgroups writing f32 partial tiles, summed in a fixed order by a
 *    second kernel;
 *  - more than half (weight gradients at the 1b shape, 176 tiles on 256
 *    CUs): each tile as two workgroups over an uneven K split; the one that
 *    finishes second adds the other's f32 partial and writes C (a + b = b + a:
 *    the result does not depend on timing).
 * The first 4 KB of the workspace hold the arrival counters of the second
 * form: they must be zero when a call starts and every call leaves them
 * zero, so a workspace zeroed once can be reused; calls that share a
 * workspace must not run concurrently.  With a null or too small workspace
 * it is moc_gemm.  Same reference call sites as moc_gemm. */
int moc_gemm_ws(int dtype, int64_t M, int64_t N, int64_t K, const void* A, int64_t a_sm,
                int64_t a_sk, const void* B, int64_t b_sk, int64_t b_sn, int64_t K2, const void* A2,
                int64_t a2_sm, int64_t a2_sk, const void* B2, int64_t b2_sk, int64_t b2_sn,
                void* C, int64_t ldc, int c_dtype, void* workspace, int64_t workspace_bytes,
                void* stream);

/* C = bf16(bf16(A B) + R) for bf16 A, B, C: moc_gemm_ws (single product,
 * same strides, workspace rules and results) with the residual R [M, N]
 * (16-byte aligned rows, ldres a multiple of 8) added where C is written.
 * The decoder block's residual add around the FFN, x + ffn(ffn_norm(x))
 * (moc/model.py:85), in the Down projection's epilogue: D is rounded to
 * bf16 first, then added to R and rounded again, the rounding of the
 * reference's bf16 add of two bf16 tensors.  C may be R itself. */
int moc_gemm_residual_bf16(int64_t M, int64_t N, int64_t K, const void* A, int64_t a_sm, int64_t a_sk,
                           const void* B, int64_t b_sk, int64_t b_sn, void* C, int64_t ldc, const void* res,
                           int64_t ldres, void* workspace, int64_t workspace_bytes, void* stream);

/* C1[M,N1] = A W1^T and C2[M,N2] = A W2^T (bf16) in one launch: A [M,K]
 * row-major (lda), W1 [N1,K] and W2 [N2,K] nn.Linear weights (ldw1, ldw2),
 * C1/C2 row-major (ldc1, ldc2).  The gate and up projections of the MoC FFN
 * input, G = x W_gate^T and U = x W_up^T (moc/ffn.py:141,146 for `moc`,
 * :389,394 for `moc_gcp`), which the reference runs as two library GEMMs.
 * Results equal two moc_gemm_ws calls bit for bit; pairs too small to fill
 * the CUs run as exactly those two calls (with the given workspace). */
int moc_gemm_pair(int64_t M, int64_t K, const void* A, int64_t lda, const void* W1, int64_t ldw1,
                  int64_t N1, void* C1, int64_t ldc1, const void* W2, int64_t ldw2, int64_t N2,
                  void* C2, int64_t ldc2, void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes moc_gemm_ws uses for this shape on the current device (0:
 * the product does not split; otherwise 4 KB of counters plus the f32
 * partial tiles).  No counterpart in the reference (its GEMMs
 * are library calls). */
int64_t moc_gemm_workspace_size(int dtype, int64_t M, int64_t N, int64_t K, int64_t K2);

/* ----------------------------------------------------------------- layer */
/* GEMM workspace bytes of moc_ffn_forward_bf16 (0: none). */
int64_t moc_ffn_forward_workspace_size(int64_t rows, int64_t d, int64_t inter);

/* The MoC FFN forward for rows tokens, bf16, as one call
 * (_MoCFunction.forward, moc/ffn.py:130-173; the 2:8 and post-SiLU variants
 * :266-308, :322-367; _MoCGCPFunction.forward :378-421): G = x Wg^T and
 * U = x Wu^T, the selection (0: Top-K of G, 1: Top-K of |SiLU(G)|, 2: top-2
 * of every 8 channels, k its 2 floor(I/8) + min(2, I mod 8)), u_s = U[idx],
 * s_s = SiLU(vals), z_s = s_s u_s (s_s, z_s may be NULL), the dense Z
 * (written into g's buffer), out = Z W_down^T.  g, u [rows, ld_gu] are
 * scratch; wd is W_down [d, inter] with 16-byte aligned rows.  Same launches
 * and results as the per-kernel entry points in that order. */
int moc_ffn_forward_bf16(int64_t rows, int64_t d, int64_t inter, int64_t k, int selection, const void* x,
                         int64_t ldx, const void* wg, int64_t ldwg, const void* wu, int64_t ldwu,
                         const void* wd, int64_t ldwd, void* g, void* u, int64_t ld_gu, void* vals,
                         void* idx, int idx_dtype, void* u_s, void* s_s, void* z_s, void* out, int64_t ldo,
                         void* workspace, int64_t workspace_bytes, void* stream);

/* GEMM workspace bytes of moc_ffn_forward_f32 (0: none). */
int64_t moc_ffn_forward_f32_workspace_size(int64_t rows, int64_t d, int64_t inter);

/* moc_ffn_forward_bf16 with f32 operands and outputs (the reference's f32
 * path, _MoCFunction.forward, moc/ffn.py:130-173): the same steps and
 * arguments, every float pointer f32 with 16-byte aligned rows; G and U run
 * on the fp32 MFMA as one launch where the split plan allows. */
int moc_ffn_forward_f32(int64_t rows, int64_t d, int64_t inter, int64_t k, int selection, const void* x,
                        int64_t ldx, const void* wg, int64_t ldwg, const void* wu, int64_t ldwu,
                        const void* wd, int64_t ldwd, void* g, void* u, int64_t ld_gu, void* vals,
                        void* idx, int idx_dtype, void* u_s, void* s_s, void* z_s, void* out, int64_t ldo,
                        void* workspace, int64_t workspace_bytes, void* stream);

/* GEMM workspace bytes of moc_ffn_backward_bf16 (0: none). */
int64_t moc_ffn_backward_workspace_size(int64_t rows, int64_t d, int64_t inter, int64_t ld_ggu, int stacked);

/* The MoC FFN backward for rows tokens, bf16 operands, as one call
 * (_MoCFunction.backward, moc/ffn.py:175-259; _MoCGCPFunction.backward
 * :423-497): with s_s NULL (GCP) S and Z are recomputed from g_s, u_s and Z
 * scattered dense (S also into s_tmp when it is not NULL; the gradient step
 * recomputes S from g_s, the same bits), else Z is scattered from z_s; dWd =
 * go^T Z, gZ = go W_down (into zbuf after Z), gG and gU dense from gZ, dWg =
 * gG^T x, dWu = gU^T x (stacked: one GEMM over [gG | gU], gu = gg + ld_ggu/2
 * and dwu = dwg + ld_ggu/2 rows), dX = gG Wg + gU Wu.  Stacked with ld_ggu
 * and ldz at most 8192: gZ goes into gu's rows, one pass turns them into
 * gG | gU in place and writes Z into zbuf (no scatter launch; with s_tmp
 * set in GCP mode the scatter runs to fill it), and the weight gradients
 * run after it, dWd beside [dWg | dWu] as one grouped launch where both
 * split K (fewer K splits each, one reduction).  Weight gradients in
 * grad_dtype (MOC_BF16 or MOC_F32), dX in bf16. */
int moc_ffn_backward_bf16(int64_t rows, int64_t d, int64_t inter, int64_t k, const void* go, int64_t ldgo,
                          const void* x, int64_t ldx, const void* idx, int idx_dtype, const void* g_s,
                          const void* u_s, const void* s_s, const void* z_s, const void* wg, int64_t ldwg,
                          const void* wu, int64_t ldwu, const void* wd, int64_t ldwd, void* zbuf, int64_t ldz,
                          void* gg, void* gu, int64_t ld_ggu, int stacked, void* s_tmp, void* dx, int64_t lddx,
                          void* dwg, void* dwu, int64_t ld_dw, void* dwd, int64_t lddwd, int grad_dtype,
                          void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------- pre-norm and FFN block */
/* RMSNorm of rows of bf16 activations, the FFN's pre-norm (RMSNorm.forward,
 * moc/model.py:20-28): r = 1 / sqrt(mean(x^2) + eps) in f32 per row,
 * y = bf16(bf16(x * r) * w) with w bf16 [d]; rstd (f32 [rows], may be NULL)
 * receives r.  d a multiple of 8 up to 8192, rows 16-byte aligned. */
int moc_rmsnorm_rows_bf16(const void* x, int64_t ldx, int64_t rows, int64_t d, const void* w, float eps,
                          void* y, int64_t ldy, float* rstd, void* stream);

/* Workspace bytes of moc_rmsnorm_backward_bf16 (f32 partial rows of dw). */
int64_t moc_rmsnorm_backward_workspace_size(int64_t rows, int64_t d);

/* Backward of moc_rmsnorm_rows_bf16 (the autograd of moc/model.py:26-28)
 * with a second gradient dres reaching x around the norm (the block's
 * residual branch, moc/model.py:85; NULL: none):
 *   dx = dres + r (dy w) - (r^3 / d) x sum_j(dy_j w_j x_j)   (bf16 [rows, d])
 *   dw = sum over rows of dy bf16(x r)                        (dw_dtype [d])
 * in f32, each rounded once.  dw is summed in a fixed order (no atomics).
 * d a multiple of 8 up to 4096. */
int moc_rmsnorm_backward_bf16(const void* x, int64_t ldx, int64_t rows, int64_t d, const void* w,
                              const float* rstd, const void* dy, int64_t lddy, const void* dres, int64_t ldres,
                              void* dx, int64_t lddx, void* dw, int dw_dtype, void* workspace,
                              int64_t workspace_bytes, void* stream);

/* The FFN half of a pre-norm decoder block, out = h + FFN(RMSNorm(h))
 * (TransformerBlock.forward, moc/model.py:83-86, with the FFN of
 * moc/ffn.py:124-497), as one call: moc_rmsnorm_rows_bf16 into xn (the
 * FFN's input, [rows, d] scratch the caller may free afterwards) and rstd,
 * then moc_ffn_forward_bf16 on xn (same arguments and outputs) with h
 * added in the Down GEMM's epilogue.  Workspace: that of
 * moc_ffn_forward_bf16. */
int moc_ffn_block_forward_bf16(int64_t rows, int64_t d, int64_t inter, int64_t k, int selection, const void* h,
                               int64_t ldh, const void* norm_w, float eps, void* xn, int64_t ldxn, float* rstd,
                               const void* wg, int64_t ldwg, const void* wu, int64_t ldwu, const void* wd,
                               int64_t ldwd, void* g, void* u, int64_t ld_gu, void* vals, void* idx, int idx_dtype,
                               void* u_s, void* s_s, void* z_s, void* out, int64_t ldo, void* workspace,
                               int64_t workspace_bytes, void* stream);

/* Workspace bytes of moc_ffn_block_backward_bf16. */
int64_t moc_ffn_block_backward_workspace_size(int64_t rows, int64_t d, int64_t inter, int64_t ld_ggu, int stacked);

/* Backward of moc_ffn_block_forward_bf16 given dout: recomputes xn from h
 * (the forward's row pass, same bits) into xn, runs moc_ffn_backward_bf16
 * on it (same arguments; its dX lands in xn's buffer), then
 * moc_rmsnorm_backward_bf16 with dres = dout: dh (bf16 [rows, d]) and the
 * norm weight's gradient dnorm_w (dnorm_dtype [d]). */
int moc_ffn_block_backward_bf16(int64_t rows, int64_t d, int64_t inter, int64_t k, const void* dout, int64_t ldgo,
                                const void* h, int64_t ldh, const void* norm_w, float eps, const float* rstd,
                                void* xn, int64_t ldxn, const void* idx, int idx_dtype, const void* g_s,
                                const void* u_s, const void* s_s, const void* z_s, const void* wg, int64_t ldwg,
                                const void* wu, int64_t ldwu, const void* wd, int64_t ldwd, void* zbuf,
                                int64_t ldz, void* gg, void* gu, int64_t ld_ggu, int stacked, void* s_tmp, void* dh,
                                int64_t lddh, void* dwg, void* dwu, int64_t ld_dw, void* dwd, int64_t lddwd,
                                int grad_dtype, void* dnorm_w, int dnorm_dtype, void* workspace,
                                int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- decode */
/* y[b, r] = bf16(sum_h x[b,h] W[r,h]) for b < nb <= 16 tokens: the decode
 * gate projection (module.gate_proj(x) before
 * moc_native::optimized_global_after_gate_bf16,
 * moc/inference/inference_ffn.py:188, benchmark_ffn_latency.py:130).
 * bf16 only; x, W 16-byte aligned with ldx, ldw multiples of 8. */
int moc_gemv_bf16(const void* x, int64_t ldx, int64_t nb, const void* W, int64_t ldw,
                  int64_t rows, int64_t hidden, void* y, int64_t ldy, void* stream);

/* moc_gemv_bf16 of the RMSNorm'd tokens, for nb <= 4 and hidden <= 4096:
 * xn[b] = bf16(bf16(x[b] * r_b) * norm_w) with r_b = 1 / sqrt(mean(x[b]^2) +
 * eps) in f32 (the FFN's pre-norm, benchmark_decode.py:101-109,303:
 * ffn_norm fused into the gate projection), y[b] = bf16(W . xn[b]); xn is
 * also written out (the up projection's input).  bf16 only. */
int moc_gemv_rmsnorm_bf16(const void* x, int64_t ldx, int64_t nb, const void* norm_w, float eps,
                          void* xn, int64_t ldxn, const void* W, int64_t ldw, int64_t rows,
                          int64_t hidden, void* y, int64_t ldy, void* stream);

/* z[b,k] = bf16(bf16(SiLU(vals[b,k])) * bf16(x[b] . W_up[idx[b,k]]))
 * (moc_native::optimized_global_selected_up_silu_bf16,
 * optimized_global_moc_ext.cu:127-162,400-427; rounding points of
 * masked_reference, moc/inference/inference_ffn.py:171-175).  bf16 only. */
int moc_selected_up_silu_bf16(const void* x, int64_t nb, int64_t hidden, const void* topk_vals,
                              const void* idx, int idx_dtype, int64_t k, const void* w_up,
                              int64_t inter, void* z, void* stream);

/* Workspace bytes moc_selected_down_bf16 needs for (nb, k, hidden). */
int64_t moc_selected_down_workspace_size(int64_t nb, int64_t k, int64_t hidden);

/* y[b,h] = bf16(sum_k z[b,k] W_down_t[idx[b,k], h]), split over k with a
 * fixed-order f32 reduction (moc_native::optimized_global_selected_down_bf16,
 * optimized_global_moc_ext.cu:247-372,429-455; moc::selected_grouped_down,
 * moc/inference/triton_fused_ffn_kernels.py:228-267). */
int moc_selected_down_bf16(const void* z, const void* idx, int idx_dtype, int64_t nb, int64_t k,
                           const void* w_down_t, int64_t ldw_down, int64_t inter, int64_t hidden, void* y,
                           void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes moc_global_after_gate_bf16 needs. */
int64_t moc_global_after_gate_workspace_size(int64_t nb, int64_t inter, int64_t k,
                                             int64_t hidden);

/* Global-MoC decode after the gate: Top-K of gate_scores[nb, inter], selected
 * Up * SiLU, selected Down -> y[nb, hidden], in one kernel launch
 * (moc_native::optimized_global_after_gate_bf16, optimized_global_moc_ext.cu:
 * 457-540, optimized_global_moc_ext.cpp:61-76,92).
 * idx_out, if not NULL, receives the selection the kernel made: int32
 * [nb, k], ascending channel order (the reference keeps its int32 indices
 * internal, optimized_global_moc_ext.cu:468-483).
 * The workspace starts with 64 KB of arrival counters that must be zero
 * before the first call with that workspace (e.g. hipMemset once after
 * allocation); every call, of any shape, leaves them zero again.  Calls
 * sharing a workspace must not overlap. */
int moc_global_after_gate_bf16(const void* x, const void* gate_scores, int64_t nb, int64_t inter,
                               int64_t hidden, const void* w_up, const void* w_down_t, int64_t ldw_down,
                               int64_t k, void* y, void* idx_out, void* workspace, int64_t workspace_bytes,
                               void* stream);

/* moc_global_after_gate_bf16 with the layer's residual added in its last
 * step: y = bf16(residual + bf16(FFN)), the decoder's x + ffn(norm(x))
 * (benchmark_decode.py:303) without a separate add.  Same workspace rules. */
int moc_global_after_gate_residual_bf16(const void* x, const void* gate_scores, int64_t nb,
                                        int64_t inter, int64_t hidden, const void* w_up,
                                        const void* w_down_t, int64_t ldw_down, int64_t k,
                                        const void* residual, void* y, void* idx_out, void* workspace,
                                        int64_t workspace_bytes, void* stream);

/* Workspace bytes moc_global_decode_bf16 and
 * moc_global_decode_rmsnorm_residual_bf16 need (the after-gate workspace's
 * 64 KB of counters, then G and U, or the after-gate workspace and G). */
int64_t moc_global_decode_workspace_size(int64_t nb, int64_t inter, int64_t k, int64_t hidden);

/* The global-MoC decode layer from x (nb <= 16 tokens): module.gate_proj(x)
 * followed by moc_native::optimized_global_after_gate_bf16 (moc/inference/
 * inference_ffn.py:181-196, optimized_global_moc_ext.cu:457-540).  Where
 * hidden % 256 == 0, inter <= 8192 and k <= 4096: G = x W_gate^T and the
 * dense U = x W_up^T in one GEMV launch, then one launch in which each
 * workgroup ranks a token's G row and sums the token's selected channels
 * for a block of output columns; otherwise the gate GEMV (with the dense U
 * from 4 tokens) and moc_global_after_gate_bf16.  The selection (idx_out)
 * is the Top-K's bit for bit, z rounds as in moc_global_after_gate_bf16,
 * and y is the same sum in another f32 order.  Same workspace rules (64 KB
 * of counters at its start, zero before the first call, left zero). */
int moc_global_decode_bf16(const void* x, int64_t nb, int64_t hidden, const void* w_gate,
                           const void* w_up, int64_t inter, const void* w_down_t, int64_t ldw_down,
                           int64_t k, void* y, void* idx_out, void* workspace, int64_t workspace_bytes,
                           void* stream);

/* The decoder layer's FFN half y = bf16(x + bf16(FFN(RMSNorm(x)))) for nb <= 4
 * tokens (benchmark_decode.py:101-109,303): the norm (rounding as in
 * moc_gemv_rmsnorm_bf16) inside the gate/up GEMV pair, the residual added in
 * the last step of the after-gate kernel.  hidden % 256 == 0 and <= 4096,
 * inter <= 8192, k <= 4096; workspace of moc_global_decode_workspace_size;
 * y must not alias x. */
int moc_global_decode_rmsnorm_residual_bf16(const void* x, int64_t nb, int64_t hidden,
                                            const void* norm_w, float eps, const void* w_gate,
                                            const void* w_up, int64_t inter, const void* w_down_t,
                                            int64_t ldw_down, int64_t k, void* y, void* idx_out,
                                            void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of the library's own device scratch array (one per GPU, held until
 * the process ends) behind moc_global_after_gate_noalloc_bf16. */
#define MOC_NOALLOC_SCRATCH_BYTES (4 * 1024 * 1024)

/* moc_global_after_gate_residual_bf16 (residual may be NULL: plain
 * moc_global_after_gate_bf16) that allocates nothing and takes no workspace.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture without an allocator, tight
 * serving loops).  The workspace is the library's fixed device scratch array
 * of MOC_NOALLOC_SCRATCH_BYTES per GPU; shapes that need more are rejected
 * (MOC_ERR_INVALID).  The stream must belong to the current device.  The
 * first call on a device clears the array's counters and waits for the clear
 * (so later calls on any stream find them zero); it must not be made under
 * HIP graph capture (MOC_ERR_INVALID), later calls may be captured and
 * replayed.  All calls on one GPU share its array: calls that overlap on one
 * GPU race. */
int moc_global_after_gate_noalloc_bf16(const void* x, const void* gate_scores, int64_t nb,
                                       int64_t inter, int64_t hidden, const void* w_up,
                                       const void* w_down_t, int64_t ldw_down, int64_t k,
                                       const void* residual, void* y, void* idx_out, void* stream);

/* ------------------------------------------------------------------- 2:8 */
/* Fused gate+up projection with top-2-of-8 selection for nb tokens:
 * idx[b, 2g+j] (int64), sz[b, 2g+j] = bf16(SiLU(g)*u) with g, u the bf16
 * projections of the selected channel (moc::fused_grouped_top2_up_silu,
 * moc/inference/triton_grouped_moc_ops.py:26-78; kernel
 * triton_fused_ffn_kernels.py:29-156).  inter % 8 == 0; bf16 only. */
int moc_grouped_top2_up_silu_bf16(const void* x, int64_t nb, int64_t hidden, const void* w_gate,
                                  const void* w_up, int64_t inter, void* idx, void* sz,
                                  void* stream);

/* Workspace bytes of moc_moc28_decode_bf16 (no zeroing needed). */
int64_t moc_moc28_decode_workspace_size(int64_t nb, int64_t inter, int64_t hidden);

/* The MoC 2:8 decode layer, nb <= 16 tokens: moc::fused_grouped_top2_up_silu
 * followed by moc::selected_grouped_down (moc/inference/
 * triton_grouped_moc_ops.py:26-131; inference_ffn.py:281-297) in two
 * launches: G and U of every token in one GEMV launch, then one launch in
 * which each workgroup picks the top 2 of every 8 channels of a token's G
 * row (the selection, tie rule and z rounding of
 * moc_grouped_top2_up_silu_bf16) and sums the token's selected Down rows
 * for a block of output columns.  norm_w (optional, nb <= 4, hidden <= 4096):
 * of RMSNorm(x) (rounding as in moc_gemv_rmsnorm_bf16).  residual
 * (optional): y = bf16(residual + bf16(FFN)), the decoder's x + ffn(norm(x))
 * when residual = x (benchmark_decode.py:303).  idx_out (optional): the
 * selection, int64 [nb, inter / 4] as moc_grouped_top2_up_silu_bf16 writes
 * it.  inter % 8 == 0 and <= 8192, hidden % 256 == 0; y must not alias x or
 * the residual. */
int moc_moc28_decode_bf16(const void* x, int64_t nb, int64_t hidden, const void* norm_w, float eps,
                          const void* w_gate, const void* w_up, int64_t inter, const void* w_down_t,
                          int64_t ldw_down, const void* residual, void* y, void* idx_out, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* moc_grouped_top2_up_silu_bf16 of the RMSNorm'd tokens (rounding as in
 * moc_gemv_rmsnorm_bf16: the FFN's pre-norm fused into the gate/up
 * projection, benchmark_decode.py:101-109,303), nb <= 4, hidden <= 4096. */
int moc_grouped_top2_up_silu_rmsnorm_bf16(const void* x, int64_t nb, int64_t hidden,
                                          const void* norm_w, float eps, const void* w_gate,
                                          const void* w_up, int64_t inter, void* idx, void* sz,
                                          void* stream);

/* Workspace bytes moc_selected_grouped_down_bf16 needs. */
int64_t moc_selected_grouped_down_workspace_size(int64_t nb, int64_t k, int64_t inter,
                                                 int64_t hidden);

/* y[b,h] = bf16(sum_k sz[b,k] W_down_t[idx[b,k], h]) for the 2:8 layout
 * (moc::selected_grouped_down, triton_grouped_moc_ops.py:96-131; kernel
 * triton_fused_ffn_kernels.py:228-267). */
int moc_selected_grouped_down_bf16(const void* sz, const void* idx, int64_t nb, int64_t k,
                                   const void* w_down_t, int64_t ldw_down, int64_t inter, int64_t hidden,
                                   void* y, void* workspace, int64_t workspace_bytes, void* stream);

/* moc_selected_grouped_down_bf16 for nb <= 64 tokens with the layer's
 * residual added in its last step: y = bf16(residual + bf16(FFN)), the
 * decoder's x + ffn(norm(x)) (benchmark_decode.py:303).  Same workspace. */
int moc_selected_grouped_down_residual_bf16(const void* sz, const void* idx, int64_t nb, int64_t k,
                                            const void* w_down_t, int64_t ldw_down, int64_t inter,
                                            int64_t hidden, const void* residual, void* y, void* workspace,
                                            int64_t workspace_bytes, void* stream);

/* 2:4-packed form of a 2:8 selection (this library's operand format for the
 * structured-sparse MFMA, no reference counterpart; it carries exactly the
 * (idx, sz) of moc_grouped_top2_up_silu_bf16).  For nb rows and
 * nt = ceil(inter / 64) channel tiles:
 *   ap[nb, ld_ap] bf16, ld_ap >= 32 nt: 4-channel group q of a row keeps two
 *     stored values at columns 2q, 2q + 1 (its selected values in channel
 *     order, zeros for the rest; columns of groups past inter hold zeros);
 *   meta[nt][meta_rows][2] uint32 (meta_rows >= nb, a multiple of 64; 256
 *     for moc_sparse28_down_bf16): word h of row r for tile t holds the 2-bit
 *     position inside its 4-group of each stored value of channels
 *     64t + 16h .. +16 (bits 0-15, stored value v at bits 2v..2v+1) and of
 *     64t + 32 + 16h .. +16 (bits 16-31).
 * moc_pack28_bf16 builds it from (sz, idx) as moc_grouped_top2_up_silu_bf16
 * writes them (idx int64 [nb, inter/4]: top-1, top-2 of each 8-group).  An
 * index outside its own 8-group, or a repeated one, cannot be packed: that
 * group's values become NaN.  zero4k (optional, 16-byte aligned) gets 4096
 * zero bytes (the counter block of a moc_sparse28_down_bf16 workspace). */
int moc_pack28_bf16(const void* sz, const void* idx, int64_t nb, int64_t inter, void* ap, int64_t ld_ap,
                    uint32_t* meta, int64_t meta_rows, void* zero4k, void* stream);

/* moc_grouped_top2_up_silu_bf16 (same selection and sz values) writing the
 * 2:4-packed form above (ap, meta) instead of (idx, sz): the fused gate/up
 * kernel's epilogue packs directly, for moc_sparse28_down_bf16 to consume
 * (the prefill pair of kernel A and kernel B, triton_fused_ffn_kernels.py:
 * 29-156, 228-267, without the int64 indices in between).  Rows of meta past
 * nb are left as they are (the Down never reads them as data: its A rows
 * there are zero). */
int moc_grouped_top2_up_silu_packed_bf16(const void* x, int64_t nb, int64_t hidden, const void* w_gate,
                                         const void* w_up, int64_t inter, void* ap, int64_t ld_ap,
                                         uint32_t* meta, int64_t meta_rows, void* stream);

/* Workspace bytes of moc_sparse28_down_bf16 (its first MOC_GEMM_WS_COUNTER_BYTES
 * are arrival counters: zero when a call starts, left zero). */
int64_t moc_sparse28_down_workspace_size(int64_t nb, int64_t inter, int64_t hidden);

/* The MoC 2:8 compacted Down at prefill: y[nb, hidden] = bf16(A W^T) with A
 * the 2:4-packed activations (ap, meta above, meta_rows >= nb rounded up to
 * 256), on the structured-sparse MFMA (v_smfmac_f32_32x32x32_bf16: half the
 * MFMA work and half the activation bytes of the dense product, twice the
 * 2:8 product's own FLOP).  w: W_down [hidden, inter] (w_kc = 1) or W_down^T
 * [inter, hidden] (w_kc = 0), row pitch ldw.  Replaces the gathered down of
 * moc::selected_grouped_down (triton_grouped_moc_ops.py:96-131; kernel
 * triton_fused_ffn_kernels.py:228-267) for prefill batches. */
int moc_sparse28_down_bf16(const void* ap, int64_t ld_ap, const uint32_t* meta, int64_t meta_rows,
                           int64_t nb, int64_t inter, const void* w, int64_t ldw, int w_kc, int64_t hidden,
                           void* y, int64_t ldy, void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOC_AMD_H_ */
