// The MoC FFN layer's forward (bf16 or f32) and backward (bf16) as one C-ABI
// call each: the launches of the single-stream path (moc/ffn.py:124-259 for `moc`,
// :262-369 for the 2:8 and post-SiLU selections, :372-497 for `moc_gcp`)
// issued from here instead of one host call per kernel.  At the shapes
// whose GEMMs fill the CUs about once (the 130m and 350m layers) the layer
// is host-bound otherwise: every Python wrapper and ctypes call costs
// microseconds that the GPU spends idle.
//
// No kernels of its own: the steps are the library's entry points, in the
// order of the reference's autograd Functions, on the caller's stream.
#include <algorithm>

#include "abi.h"

namespace {

int64_t gemm_ws(int64_t M, int64_t N, int64_t K, int64_t K2, int dt = MOC_BF16) {
  const int64_t b = moc_gemm_workspace_size(dt, M, N, K, K2);
  return b > 0 ? b : 0;
}

int64_t effective_2of8(int64_t inter) { return (inter / 8) * 2 + std::min<int64_t>(2, inter % 8); }

// 16-byte aligned rows of at least `cols` elements of `esz` bytes
bool ld_ok(const void* p, int64_t ld, int64_t cols, int64_t esz = 2) {
  return p != nullptr && moc::aligned16(p) && (ld * esz) % 16 == 0 && ld >= cols;
}

// The forward of moc_ffn_forward_bf16 / moc_ffn_forward_f32 in element type
// dt: G and U (one launch), the selection, the sparse aux, D.
int ffn_forward(int dt, const char* name, int64_t rows, int64_t d, int64_t inter, int64_t k, int selection,
                const void* x, int64_t ldx, const void* wg, int64_t ldwg, const void* wu, int64_t ldwu,
                const void* wd, int64_t ldwd, void* g, void* u, int64_t ld_gu, void* vals, void* idx,
                int idx_dtype, void* u_s, void* s_s, void* z_s, void* out, int64_t ldo, void* workspace,
                int64_t workspace_bytes, void* stream, const void* res = nullptr, int64_t ldres = 0) {
  const int64_t esz = dt == MOC_BF16 ? 2 : 4;
  MOC_REQUIRE(rows >= 1 && d >= 1 && inter >= 1 && k >= 1 && k <= inter, "%s: bad shape", name);
  MOC_REQUIRE(selection >= 0 && selection <= 2, "%s: selection 0 (Top-K), 1 (Top-K of |SiLU(G)|) or 2 (top-2 of 8)",
              name);
  MOC_REQUIRE(selection != 2 || k == effective_2of8(inter), "%s: the 2:8 selection keeps %lld channels", name,
              (long long)effective_2of8(inter));
  MOC_REQUIRE(ld_ok(x, ldx, d, esz) && ld_ok(wg, ldwg, d, esz) && ld_ok(wu, ldwu, d, esz) &&
                  ld_ok(wd, ldwd, inter, esz) && ld_ok(g, ld_gu, inter, esz) && ld_ok(u, ld_gu, inter, esz) &&
                  ld_ok(out, ldo, d, esz),
              "%s: operands need 16-byte aligned rows (leading dimensions multiples of %lld)", name,
              (long long)(16 / esz));
  MOC_REQUIRE(vals && idx && u_s, "%s: null output", name);
  const int64_t need = dt == MOC_BF16 ? moc_ffn_forward_workspace_size(rows, d, inter)
                                      : moc_ffn_forward_f32_workspace_size(rows, d, inter);
  MOC_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr),
              "%s: workspace of %lld bytes required", name, (long long)need);
  // G = x Wg^T and U = x Wu^T (one launch)
  int rc;
  if (dt == MOC_BF16) {
    rc = moc_gemm_pair(rows, d, x, ldx, wg, ldwg, inter, g, ld_gu, wu, ldwu, inter, u, ld_gu, workspace,
                       workspace_bytes, stream);
  } else {
    rc = ldwg == ldwu ? moc::f32_gemm_pair(rows, inter, d, static_cast<const float*>(x), ldx,
                                           static_cast<const float*>(wg), static_cast<const float*>(wu), ldwg,
                                           static_cast<float*>(g), static_cast<float*>(u), ld_gu,
                                           moc::as_stream(stream))
                      : 1;
    if (rc == 1) {  // two launches
      rc = moc_gemm_ws(dt, rows, inter, d, x, ldx, 1, wg, 1, ldwg, 0, nullptr, 0, 0, nullptr, 0, 0, g, ld_gu, dt,
                       workspace, workspace_bytes, stream);
      if (rc == MOC_OK)
        rc = moc_gemm_ws(dt, rows, inter, d, x, ldx, 1, wu, 1, ldwu, 0, nullptr, 0, 0, nullptr, 0, 0, u, ld_gu,
                         dt, workspace, workspace_bytes, stream);
    }
  }
  if (rc != MOC_OK) return rc;
  // the selection (indices in ascending channel order) and its gate values
  if (selection == 2)
    rc = moc_select_2of8(dt, g, rows, inter, ld_gu, vals, idx, idx_dtype, stream);
  else
    rc = moc_topk_rows(dt, g, rows, inter, ld_gu, k, selection, vals, idx, idx_dtype, nullptr, 0, stream);
  if (rc != MOC_OK) return rc;
  // U at the selection, SiLU, Z; the dense zero-filled Z goes into G's
  // buffer, which nothing reads after the selection
  rc = moc_sparse_forward_aux(dt, vals, idx, idx_dtype, u, ld_gu, rows, k, inter, u_s, s_s, z_s, g, ld_gu,
                              stream);
  if (rc != MOC_OK) return rc;
  // D = Z W_down^T (with a residual: res + D from the same epilogue)
  if (res != nullptr)
    return moc_gemm_residual_bf16(rows, d, inter, g, ld_gu, 1, wd, 1, ldwd, out, ldo, res, ldres, workspace,
                                  workspace_bytes, stream);
  return moc_gemm_ws(dt, rows, d, inter, g, ld_gu, 1, wd, 1, ldwd, 0, nullptr, 0, 0, nullptr, 0, 0, out, ldo, dt,
                     workspace, workspace_bytes, stream);
}

}  // namespace

// GEMM workspace of moc_ffn_forward_bf16: the G,U pair and D = Z W_down^T.
extern "C" int64_t moc_ffn_forward_workspace_size(int64_t rows, int64_t d, int64_t inter) {
  if (rows <= 0 || d <= 0 || inter <= 0) return 0;
  return std::max(gemm_ws(rows, inter, d, 0), gemm_ws(rows, d, inter, 0));
}

// GEMM workspace of moc_ffn_forward_f32: G and U when they run as two
// launches, and D = Z W_down^T.
extern "C" int64_t moc_ffn_forward_f32_workspace_size(int64_t rows, int64_t d, int64_t inter) {
  if (rows <= 0 || d <= 0 || inter <= 0) return 0;
  return std::max(gemm_ws(rows, inter, d, 0, MOC_F32), gemm_ws(rows, d, inter, 0, MOC_F32));
}

extern "C" int moc_ffn_forward_bf16(int64_t rows, int64_t d, int64_t inter, int64_t k, int selection,
                                    const void* x, int64_t ldx, const void* wg, int64_t ldwg,
                                    const void* wu, int64_t ldwu, const void* wd, int64_t ldwd, void* g,
                                    void* u, int64_t ld_gu, void* vals, void* idx, int idx_dtype,
                                    void* u_s, void* s_s, void* z_s, void* out, int64_t ldo,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
  return ffn_forward(MOC_BF16, "moc_ffn_forward_bf16", rows, d, inter, k, selection, x, ldx, wg, ldwg, wu, ldwu,
                     wd, ldwd, g, u, ld_gu, vals, idx, idx_dtype, u_s, s_s, z_s, out, ldo, workspace,
                     workspace_bytes, stream);
}

extern "C" int moc_ffn_forward_f32(int64_t rows, int64_t d, int64_t inter, int64_t k, int selection,
                                   const void* x, int64_t ldx, const void* wg, int64_t ldwg, const void* wu,
                                   int64_t ldwu, const void* wd, int64_t ldwd, void* g, void* u, int64_t ld_gu,
                                   void* vals, void* idx, int idx_dtype, void* u_s, void* s_s, void* z_s,
                                   void* out, int64_t ldo, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  return ffn_forward(MOC_F32, "moc_ffn_forward_f32", rows, d, inter, k, selection, x, ldx, wg, ldwg, wu, ldwu,
                     wd, ldwd, g, u, ld_gu, vals, idx, idx_dtype, u_s, s_s, z_s, out, ldo, workspace,
                     workspace_bytes, stream);
}

// GEMM workspace of moc_ffn_backward_bf16 (stacked: dWg and dWu as one GEMM
// over [gG | gU] with rows ld_ggu / 2 apart).
extern "C" int64_t moc_ffn_backward_workspace_size(int64_t rows, int64_t d, int64_t inter, int64_t ld_ggu,
                                                   int stacked) {
  if (rows <= 0 || d <= 0 || inter <= 0) return 0;
  int64_t w = std::max(gemm_ws(d, inter, rows, 0), gemm_ws(rows, inter, d, 0));
  w = std::max(w, stacked ? gemm_ws(ld_ggu, d, rows, 0) : gemm_ws(inter, d, rows, 0));
  if (stacked) w = std::max(w, moc::gemm_split_pair_workspace(ld_ggu, d, rows, d, inter, rows));
  return std::max(w, gemm_ws(rows, d, inter, inter));
}

extern "C" int moc_ffn_backward_bf16(int64_t rows, int64_t d, int64_t inter, int64_t k, const void* go,
                                     int64_t ldgo, const void* x, int64_t ldx, const void* idx, int idx_dtype,
                                     const void* g_s, const void* u_s, const void* s_s, const void* z_s,
                                     const void* wg, int64_t ldwg, const void* wu, int64_t ldwu,
                                     const void* wd, int64_t ldwd, void* zbuf, int64_t ldz, void* gg, void* gu,
                                     int64_t ld_ggu, int stacked, void* s_tmp, void* dx, int64_t lddx,
                                     void* dwg, void* dwu, int64_t ld_dw, void* dwd, int64_t lddwd,
                                     int grad_dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(rows >= 1 && d >= 1 && inter >= 1 && k >= 1 && k <= inter, "moc_ffn_backward_bf16: bad shape");
  MOC_REQUIRE(grad_dtype == MOC_BF16 || grad_dtype == MOC_F32, "moc_ffn_backward_bf16: grad dtype bf16 or f32");
  MOC_REQUIRE(ld_ok(go, ldgo, d) && ld_ok(x, ldx, d) && ld_ok(wg, ldwg, d) && ld_ok(wu, ldwu, d) &&
                  ld_ok(wd, ldwd, inter) && ld_ok(zbuf, ldz, inter) && ld_ok(gg, ld_ggu, inter) &&
                  ld_ok(gu, ld_ggu, inter) && ld_ok(dx, lddx, d),
              "moc_ffn_backward_bf16: operands need 16-byte aligned rows (leading dimensions multiples of 8)");
  MOC_REQUIRE(idx && g_s && u_s && dwg && dwu && dwd && ld_dw >= d && lddwd >= inter,
              "moc_ffn_backward_bf16: null operand or bad leading dimension");
  MOC_REQUIRE(s_s == nullptr || z_s != nullptr, "moc_ffn_backward_bf16: saved S needs saved Z");
  const int64_t esz = grad_dtype == MOC_BF16 ? 2 : 4;
  const int64_t pitch = ld_ggu / 2;
  if (stacked) {
    MOC_REQUIRE(ld_ggu % 16 == 0 && pitch >= inter &&
                    static_cast<const char*>(gu) == static_cast<const char*>(gg) + pitch * 2 &&
                    static_cast<const char*>(dwu) == static_cast<const char*>(dwg) + pitch * ld_dw * esz,
                "moc_ffn_backward_bf16: stacked gG | gU and dWg | dWu must be one buffer each, pitch apart");
  }
  const int64_t need = moc_ffn_backward_workspace_size(rows, d, inter, ld_ggu, stacked);
  MOC_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr),
              "moc_ffn_backward_bf16: workspace of %lld bytes required", (long long)need);
  // Stacked layout within the row kernels' limits: gZ goes into gU's rows,
  // the gradient pass turns them into gG | gU in place and writes the dense
  // Z as well (no scatter launch), so Z outlives gZ and the weight gradients
  // run last, dWd beside [dWg | dWu] as one grouped split-K launch where
  // both split K.
  const bool late = stacked && ld_ggu <= 8192 && ldz <= 8192 && moc::aligned16(gu);
  hipStream_t st = moc::as_stream(stream);
  int rc;
  if (late) {
    // gZ = go W_down into gU's rows
    rc = moc_gemm_ws(MOC_BF16, rows, inter, d, go, ldgo, 1, wd, ldwd, 1, 0, nullptr, 0, 0, nullptr, 0, 0, gu,
                     ld_ggu, MOC_BF16, workspace, workspace_bytes, stream);
    if (rc != MOC_OK) return rc;
    // gG, gU dense (:455-480) and Z (GCP: S, Z recomputed, :435-437)
    rc = 1;
    if (s_s != nullptr || s_tmp == nullptr) {
      rc = moc::sparse_backward_aux_z(idx, idx_dtype, g_s, u_s, s_s, s_s != nullptr ? z_s : nullptr, gu, ld_ggu,
                                      rows, k, inter, gg, gu, ld_ggu, zbuf, ldz, st);
      if (rc < 0) return rc;
    }
    if (rc == 1) {  // S wanted in s_tmp, or no fused form: the scatter, then gG | gU in place
      rc = s_s == nullptr
               ? moc_gcp_recompute_scatter(MOC_BF16, g_s, u_s, idx, idx_dtype, rows, k, inter, s_tmp, zbuf, ldz,
                                           stream)
               : moc_scatter_sparse_to_dense(MOC_BF16, z_s, idx, idx_dtype, rows, k, inter, zbuf, ldz, stream);
      if (rc != MOC_OK) return rc;
      rc = moc_sparse_backward_aux(MOC_BF16, idx, idx_dtype, g_s, u_s, s_s, gu, ld_ggu, rows, k, inter, gg, gu,
                                   ld_ggu, stream);
    }
    if (rc != MOC_OK) return rc;
    // [dWg | dWu] = [gG | gU]^T x (:483-490) and dWd = go^T Z (:447): one
    // grouped launch where the plan takes them, else two
    const int64_t pair_ws = moc::gemm_split_pair_workspace(2 * pitch, d, rows, d, inter, rows);
    rc = 1;
    if (pair_ws > 0 && workspace_bytes >= pair_ws)
      rc = moc::gemm_split_pair(2 * pitch, d, rows, gg, 1, ld_ggu, x, ldx, 1, dwg, ld_dw, d, inter, rows, go, 1,
                                ldgo, zbuf, ldz, 1, dwd, lddwd, grad_dtype, workspace, workspace_bytes, st);
    if (rc == 1) {
      rc = moc_gemm_ws(MOC_BF16, 2 * pitch, d, rows, gg, 1, ld_ggu, x, ldx, 1, 0, nullptr, 0, 0, nullptr, 0, 0,
                       dwg, ld_dw, grad_dtype, workspace, workspace_bytes, stream);
      if (rc == MOC_OK)
        rc = moc_gemm_ws(MOC_BF16, d, inter, rows, go, 1, ldgo, zbuf, ldz, 1, 0, nullptr, 0, 0, nullptr, 0, 0,
                         dwd, lddwd, grad_dtype, workspace, workspace_bytes, stream);
    }
    if (rc != MOC_OK) return rc;
    // dX = gG Wg + gU Wu (:491-497)
    return moc_gemm_ws(MOC_BF16, rows, d, inter, gg, ld_ggu, 1, wg, ldwg, 1, inter, gu, ld_ggu, 1, wu, ldwu, 1,
                       dx, lddx, MOC_BF16, workspace, workspace_bytes, stream);
  }
  if (s_s == nullptr) {
    // GCP: S = SiLU(G M), Z = S U M recomputed, Z scattered dense (:435-442)
    rc = moc_gcp_recompute_scatter(MOC_BF16, g_s, u_s, idx, idx_dtype, rows, k, inter, s_tmp, zbuf, ldz, stream);
  } else {
    rc = moc_scatter_sparse_to_dense(MOC_BF16, z_s, idx, idx_dtype, rows, k, inter, zbuf, ldz, stream);
  }
  if (rc != MOC_OK) return rc;
  // dWd = go^T Z
  rc = moc_gemm_ws(MOC_BF16, d, inter, rows, go, 1, ldgo, zbuf, ldz, 1, 0, nullptr, 0, 0, nullptr, 0, 0, dwd,
                   lddwd, grad_dtype, workspace, workspace_bytes, stream);
  if (rc != MOC_OK) return rc;
  // gZ = go W_down, into Z's buffer (Z is consumed)
  rc = moc_gemm_ws(MOC_BF16, rows, inter, d, go, ldgo, 1, wd, ldwd, 1, 0, nullptr, 0, 0, nullptr, 0, 0, zbuf,
                   ldz, MOC_BF16, workspace, workspace_bytes, stream);
  if (rc != MOC_OK) return rc;
  // gG, gU dense (:455-480); GCP: the kernel recomputes S from g_s (the
  // same bits as the recompute above)
  rc = moc_sparse_backward_aux(MOC_BF16, idx, idx_dtype, g_s, u_s, s_s, zbuf, ldz, rows, k, inter, gg, gu,
                               ld_ggu, stream);
  if (rc != MOC_OK) return rc;
  // dWg = gG^T x, dWu = gU^T x (:483-490)
  if (stacked) {
    rc = moc_gemm_ws(MOC_BF16, 2 * pitch, d, rows, gg, 1, ld_ggu, x, ldx, 1, 0, nullptr, 0, 0, nullptr, 0, 0,
                     dwg, ld_dw, grad_dtype, workspace, workspace_bytes, stream);
  } else {
    rc = moc_gemm_ws(MOC_BF16, inter, d, rows, gg, 1, ld_ggu, x, ldx, 1, 0, nullptr, 0, 0, nullptr, 0, 0, dwg,
                     ld_dw, grad_dtype, workspace, workspace_bytes, stream);
    if (rc != MOC_OK) return rc;
    rc = moc_gemm_ws(MOC_BF16, inter, d, rows, gu, 1, ld_ggu, x, ldx, 1, 0, nullptr, 0, 0, nullptr, 0, 0, dwu,
                     ld_dw, grad_dtype, workspace, workspace_bytes, stream);
  }
  if (rc != MOC_OK) return rc;
  // dX = gG Wg + gU Wu (:491-497)
  return moc_gemm_ws(MOC_BF16, rows, d, inter, gg, ld_ggu, 1, wg, ldwg, 1, inter, gu, ld_ggu, 1, wu, ldwu, 1, dx,
                     lddx, MOC_BF16, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// The FFN half of a pre-norm decoder block, h + FFN(RMSNorm(h))
// (moc/model.py:20-28,83-86), as one call per pass: the norm as a row pass,
// the FFN's launches, the residual add in the Down GEMM's epilogue; the
// backward recomputes the norm's output (same kernel, same bits) instead of
// keeping it, runs the FFN backward and then the norm's backward with the
// residual branch's gradient added.

extern "C" int moc_ffn_block_forward_bf16(int64_t rows, int64_t d, int64_t inter, int64_t k, int selection,
                                          const void* h, int64_t ldh, const void* norm_w, float eps, void* xn,
                                          int64_t ldxn, float* rstd, const void* wg, int64_t ldwg, const void* wu,
                                          int64_t ldwu, const void* wd, int64_t ldwd, void* g, void* u,
                                          int64_t ld_gu, void* vals, void* idx, int idx_dtype, void* u_s,
                                          void* s_s, void* z_s, void* out, int64_t ldo, void* workspace,
                                          int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(rstd != nullptr, "moc_ffn_block_forward_bf16: null rstd");
  MOC_REQUIRE(ld_ok(h, ldh, d), "moc_ffn_block_forward_bf16: h needs 16-byte aligned rows");
  int rc = moc_rmsnorm_rows_bf16(h, ldh, rows, d, norm_w, eps, xn, ldxn, rstd, stream);
  if (rc != MOC_OK) return rc;
  return ffn_forward(MOC_BF16, "moc_ffn_block_forward_bf16", rows, d, inter, k, selection, xn, ldxn, wg, ldwg, wu,
                     ldwu, wd, ldwd, g, u, ld_gu, vals, idx, idx_dtype, u_s, s_s, z_s, out, ldo, workspace,
                     workspace_bytes, stream, h, ldh);
}

namespace {
// Where the norm backward's partial rows start in the block backward's
// workspace: after the FFN backward's GEMM workspace, and never inside the
// GEMM arrival counters at its start (which must stay zero between calls).
int64_t block_rms_offset(int64_t rows, int64_t d, int64_t inter, int64_t ld_ggu, int stacked) {
  const int64_t f = (moc_ffn_backward_workspace_size(rows, d, inter, ld_ggu, stacked) + 255) / 256 * 256;
  return std::max<int64_t>(f, MOC_GEMM_WS_COUNTER_BYTES);
}
}  // namespace

extern "C" int64_t moc_ffn_block_backward_workspace_size(int64_t rows, int64_t d, int64_t inter, int64_t ld_ggu,
                                                         int stacked) {
  if (rows <= 0 || d <= 0 || inter <= 0) return 0;
  return block_rms_offset(rows, d, inter, ld_ggu, stacked) + moc_rmsnorm_backward_workspace_size(rows, d);
}

extern "C" int moc_ffn_block_backward_bf16(int64_t rows, int64_t d, int64_t inter, int64_t k, const void* dout,
                                           int64_t ldgo, const void* h, int64_t ldh, const void* norm_w, float eps,
                                           const float* rstd, void* xn, int64_t ldxn, const void* idx,
                                           int idx_dtype, const void* g_s, const void* u_s, const void* s_s,
                                           const void* z_s, const void* wg, int64_t ldwg, const void* wu,
                                           int64_t ldwu, const void* wd, int64_t ldwd, void* zbuf, int64_t ldz,
                                           void* gg, void* gu, int64_t ld_ggu, int stacked, void* s_tmp,
                                           void* dh, int64_t lddh, void* dwg, void* dwu, int64_t ld_dw, void* dwd,
                                           int64_t lddwd, int grad_dtype, void* dnorm_w, int dnorm_dtype,
                                           void* workspace, int64_t workspace_bytes, void* stream) {
  MOC_REQUIRE(rows >= 1 && d >= 1, "moc_ffn_block_backward_bf16: bad shape");
  const int64_t need = moc_ffn_block_backward_workspace_size(rows, d, inter, ld_ggu, stacked);
  MOC_REQUIRE(workspace != nullptr && workspace_bytes >= need && moc::aligned16(workspace),
              "moc_ffn_block_backward_bf16: workspace of %lld bytes required", (long long)need);
  MOC_REQUIRE(ld_ok(h, ldh, d) && ld_ok(xn, ldxn, d) && ld_ok(dh, lddh, d) && rstd != nullptr,
              "moc_ffn_block_backward_bf16: h, xn and dh need 16-byte aligned rows");
  const int64_t f = block_rms_offset(rows, d, inter, ld_ggu, stacked);
  // the FFN's input again (the forward's row pass: same bits)
  int rc = moc_rmsnorm_rows_bf16(h, ldh, rows, d, norm_w, eps, xn, ldxn, nullptr, stream);
  if (rc != MOC_OK) return rc;
  // FFN backward; its dX (the norm output's gradient) goes into xn's buffer:
  // xn is last read by the weight-gradient GEMMs, which run before dX
  rc = moc_ffn_backward_bf16(rows, d, inter, k, dout, ldgo, xn, ldxn, idx, idx_dtype, g_s, u_s, s_s, z_s, wg,
                             ldwg, wu, ldwu, wd, ldwd, zbuf, ldz, gg, gu, ld_ggu, stacked, s_tmp, xn, ldxn, dwg,
                             dwu, ld_dw, dwd, lddwd, grad_dtype, workspace, f, stream);
  if (rc != MOC_OK) return rc;
  // dh = dout (the residual branch) + the norm's backward of dX
  return moc_rmsnorm_backward_bf16(h, ldh, rows, d, norm_w, rstd, xn, ldxn, dout, ldgo, dh, lddh, dnorm_w,
                                   dnorm_dtype, static_cast<char*>(workspace) + f, workspace_bytes - f, stream);
}
