// Internal helpers shared by the C-ABI entry points: argument checks that
// record a message instead of throwing, and the launch check.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>

#include "../../include/moc_amd.h"

namespace moc {

// Records a printf-style message retrievable through moc_last_error().
void set_error(const char* fmt, ...);

// After a launch: turns a pending HIP error into MOC_ERR_HIP with a message.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Compute units of the current device (cached per device; abi.hip).
int cu_count();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// moc_selected_down_bf16 with an optional residual added in the last step
// (y = bf16(res + bf16(sum)); res may be null) (decode.hip).
int selected_down_impl(const void* z, const void* idx, int idx_dtype, int64_t nb, int64_t k,
                       const void* w_down_t, int64_t ldw_down, int64_t inter, int64_t hidden, const void* res,
                       void* y, void* workspace, int64_t workspace_bytes, void* stream);

// Bytes of arrival counters at the start of an after-gate workspace.
constexpr int64_t kAfterGateCounterBytes = 64 * 1024;

// moc_global_after_gate_bf16 / _residual_bf16 (res may be null, idx_out may
// be null) on a caller workspace (decode.hip).  up_ready: the dense U that
// the workspace holds from 4 tokens on was already written by the caller.
int global_after_gate(const void* x, const void* gate_scores, int64_t nb, int64_t inter,
                      int64_t hidden, const void* w_up, const void* w_down_t, int64_t ldw_down, int64_t k,
                      const void* res, void* y, void* idx_out, void* workspace,
                      int64_t workspace_bytes, void* stream, bool up_ready = false);

// MoC 2:8 gate/up + top-2-of-8 for nb tokens on the MFMA GEMM kernel
// (gemm.hip); 1: shape not supported there (nothing launched).
int launch_gate_up_2of8(const void* x, int64_t nb, int64_t hidden, const void* wg, const void* wu,
                        int64_t inter, int64_t* idx, uint16_t* sz, hipStream_t st, uint16_t* ap = nullptr,
                        int64_t ld_ap = 0, uint32_t* meta = nullptr, int64_t meta_rows = 0);

// f32 pair C1 = A W1^T, C2 = A W2^T as one launch (gemm.hip); 1: shapes not
// taken (nothing launched).
int f32_gemm_pair(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* W1,
                  const float* W2, int64_t ldw, float* C1, float* C2, int64_t ldc, hipStream_t st);

// Two bf16 GEMMs of split-K size (C1 [M1, N1] = A1 B1, C2 [M2, N2] = A2 B2,
// strides as in moc_gemm_ws, output dtype c_dtype for both) as one grouped
// split-K launch plus one reduction launch (gemm.hip).  Returns 1 without
// launching when the grouped plan does not beat the two products apart or
// the operands do not suit it; the caller then issues two GEMMs.
// gemm_split_pair_workspace: its workspace bytes, 0 where it does not apply.
int64_t gemm_split_pair_workspace(int64_t M1, int64_t N1, int64_t K1, int64_t M2, int64_t N2, int64_t K2);
int gemm_split_pair(int64_t M1, int64_t N1, int64_t K1, const void* A1, int64_t a1_sm, int64_t a1_sk,
                    const void* B1, int64_t b1_sk, int64_t b1_sn, void* C1, int64_t ldc1, int64_t M2, int64_t N2,
                    int64_t K2, const void* A2, int64_t a2_sm, int64_t a2_sk, const void* B2, int64_t b2_sk,
                    int64_t b2_sn, void* C2, int64_t ldc2, int c_dtype, void* workspace, int64_t workspace_bytes,
                    hipStream_t st);

// moc_sparse_backward_aux in its bf16 row form that also writes the dense Z
// rows (z_full, pitch z_ld): z = bf16(S u) from the recomputed S when
// z_sparse is NULL (GCP), else the saved z_sparse scattered (sparse_aux.hip).
// Returns 1 without launching where the row form does not apply.
int sparse_backward_aux_z(const void* idx, int idx_dtype, const void* g_sparse, const void* u_sparse,
                          const void* s_sparse, const void* z_sparse, const void* gz_full, int64_t gz_ld,
                          int64_t rows, int64_t k, int64_t inter, void* grad_g, void* grad_u, int64_t out_ld,
                          void* z_full, int64_t z_ld, hipStream_t st);

}  // namespace moc

#define MOC_REQUIRE(cond, ...)        \
  do {                                \
    if (!(cond)) {                    \
      ::moc::set_error(__VA_ARGS__);  \
      return MOC_ERR_INVALID;         \
    }                                 \
  } while (0)
