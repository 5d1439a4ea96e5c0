// rt_kernels.hpp -- host-side launchers for the rich-triplet HIP kernels.
// Shapes are validated by the C ABI layer before any of these is called.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace rt {

hipError_t launch_q4k_dequant(const void *blocks, size_t n_blocks, void *out, bool bf16, hipStream_t s);
hipError_t launch_q4k_gemv(const void *W, const float *x, float *y, int N, int K, hipStream_t s);
// Up to kGemvMaxMats Q4_K matrices sharing the activation x in one launch.
constexpr int kGemvMaxMats = 4;
hipError_t launch_q4k_gemv_multi(const void *const *w, float *const *y, const int *n, int count, const float *x,
                                 int K, hipStream_t s);
hipError_t launch_q4k_gemv_generic(const void *W, const float *x, float *y, int N, int K, hipStream_t s);
int q4k_gemv_rows_per_wg(int N, int K);
hipError_t launch_bf16_gemv(const uint16_t *W, const float *x, float *y, int N, int K, hipStream_t s);
// Q6_K / Q8_0 in the planar device layout of kquant.hip.
void q6k_repack_host(const uint8_t *src, size_t n_blocks, uint8_t *dst);
void q8_0_repack_host(const uint8_t *src, size_t n_blocks, uint8_t *dst);
hipError_t launch_q6k_dequant(const void *w, size_t n_blocks, float *out, hipStream_t s);
hipError_t launch_q8_0_dequant(const void *w, size_t n_elem, float *out, hipStream_t s);
hipError_t launch_q6k_gemv(const void *W, const float *x, float *y, int N, int K, hipStream_t s);
hipError_t launch_q8_0_gemv(const void *W, const float *x, float *y, int N, int K, hipStream_t s);
// c[i] = sum over s < ksplit of part[s*mn + i], in split order.
hipError_t launch_gemm_splitk_sum(const float *part, float *c, size_t mn, int ksplit, hipStream_t s);
// A (f32 [M][K]) -> f16 with a per-row power-of-two exponent (the GEMMs' A prep).
hipError_t launch_gemm_prep_a(const float *a, int M, int K, _Float16 *a16, int *ea, hipStream_t s);
// C[M,N] = A[M,K] . W[N,K]^T for a projection stored as RT_LINEAR_Q6K, _Q8_0
// or _BF16 (planar layouts of kquant.hip): its rows are widened to f16 with a
// per-row power-of-two scale and multiplied on the matrix cores in f32.
size_t proj_gemm_workspace_bytes(int M, int N, int K);
// c[m][n] = a[m][k] . W[n][k] (+ bias[n]) on f32 weights, rows of A in groups
// of 8 (each weight row read once per group); k % 4 == 0, w and a 16-byte aligned.
hipError_t launch_f32_gemv_rows(const float *w, const float *a, const float *bias, float *c, int M, int N, int K,
                                hipStream_t s);
// the same on BF16 weights; k % 8 == 0
hipError_t launch_bf16_gemv_rows(const uint16_t *w, const float *a, const float *bias, float *c, int M, int N, int K,
                                 hipStream_t s);
// y = gelu_tanh(x), elementwise (the decode step's and prefill's activation)
hipError_t launch_gelu_tanh(const float *x, float *y, size_t n, hipStream_t s);
// c[m][n] += bias[n]
hipError_t launch_add_bias_rows(float *c, const float *bias, int M, int N, hipStream_t s);
hipError_t launch_proj_gemm(const float *a, int fmt, const void *w, float *c, int M, int N, int K, void *ws,
                            hipStream_t s);
// The same two GEMMs on an A prepared once (launch_gemm_prep_a) for several
// matrices; ws needs the respective workspace bytes minus the A part
// (M*K*2 and M*4 bytes, each rounded up to 256).
hipError_t launch_proj_gemm_prepped(const _Float16 *a16, const int *ea, int fmt, const void *w, float *c, int M,
                                    int N, int K, void *ws, hipStream_t s);
// With `left`, a Q4_K GEMM that splits K leaves its partial tiles in ws
// (left->part = [left->ks][M][N], summed by the consumer in split order)
// instead of summing them into c; left->ks = 1 means the result is in c.
struct GemmLeft {
  const float *part;
  int ks;
};
// ew_pre: the weight's row exponents from launch_q4k_row_exponents, kept
// with the weight (null: computed into ws by this call).
hipError_t launch_q4k_gemm_prepped(const _Float16 *a16, const int *ea, const void *w, float *c, int M, int N, int K,
                                   void *ws, hipStream_t s, GemmLeft *left = nullptr, const int *ew_pre = nullptr);
// Up to three Q4_K matrices sharing a prepared A (q|k|v, gate|up) in one
// matrix-core launch, for M > 1024 or at least 512 output tiles of 128x256
// (q4k_gemm_multi_ok); ws[i] holds at least n[i]*4 bytes (matrix i's row
// exponents, unless ew_pre[i] gives them); no K split.
bool q4k_gemm_multi_ok(int M, int count, const int *n);
hipError_t launch_q4k_gemm_multi_prepped(const _Float16 *a16, const int *ea, int count, const void *const *w,
                                         float *const *c, const int *n, void *const *ws, int M, int K,
                                         hipStream_t s, const int *const *ew_pre = nullptr);
// An FFN's gate and up Q4_K matrices (N rows each) on a prepared A in one
// launch that stores h = gelu_tanh(A.Wg^T) * (A.Wu^T) [M][N] instead of the
// two products, as the next GEMM's A operand: f16 rows h16 with exponents
// eh (|h| <= 2 a_nrm2[m] gu_bound sets them).  a_nrm2[m] = |A row m|^2 in f32,
// gu_bound >= max_n |Wg row n| |Wu row n| (launch_q4k_row_norms); for the
// shapes q4k_gemm_multi_ok takes as a set; needs both weights' row
// exponents (launch_q4k_row_exponents).
bool q4k_gemm_gelu_ok(int M, int N);
hipError_t launch_q4k_gemm_gelu_prepped(const _Float16 *a16, const int *ea, const float *a_nrm2, const void *w_gate,
                                        const void *w_up, const int *ew_gate, const int *ew_up, float gu_bound,
                                        _Float16 *h16, int *eh, int M, int N, int K, hipStream_t s);
// The q, k and v Q4_K matrices of an attention layer (QD, KVD, KVD rows,
// head_dim 256) on a prepared A in one launch that applies the per-head
// RMSNorm (gammas g_q, g_k) and NeoX RoPE (row m's cos | sin at
// cs + m*cs_stride, 128 each) to q and k before storing: q_out [M][QD],
// k_rows and v_rows [M][KVD] (the KV cache rows of positions p0 .. p0+M-1).
bool q4k_gemm_qkv_ok(int M, int QD, int KVD, int head_dim);
hipError_t launch_q4k_gemm_qkv_prepped(const _Float16 *a16, const int *ea, const void *const *w, const int *const *ew,
                                       float *q_out, float *k_rows, float *v_rows, int M, int QD, int KVD, int K,
                                       const float *cs, int cs_stride, const float *g_q, const float *g_k, float eps,
                                       hipStream_t s);
// |W row n|_2 of a Q4_K weight [N][K] (dequantised values) into nrm[N].
hipError_t launch_q4k_row_norms(const void *w, int N, int K, float *nrm, hipStream_t s);
// The GEMM's power-of-two row exponents of a Q4_K weight [N][K] (from its
// block headers) into ew[N]: they depend on the weight alone, so a caller
// that keeps the weight can compute them once.
hipError_t launch_q4k_row_exponents(const void *w, int N, int K, int *ew, hipStream_t s);
// Workspace bytes of the two prepped calls.
size_t q4k_gemm_prepped_ws_bytes(int M, int N, int K);
size_t proj_gemm_prepped_ws_bytes(int M, int N, int K);
// Q4_K GEMM C[M,N] = A[M,K] . W[N,K]^T; A bf16 bits (a_bf16) or f32; ws holds
// q4k_gemm_workspace_bytes(M, N, K) bytes of device scratch.
size_t q4k_gemm_workspace_bytes(int M, int N, int K);
hipError_t launch_q4k_gemm(const void *a, bool a_bf16, const void *w, float *c, int M, int N, int K, void *ws,
                           hipStream_t s);

}  // namespace rt
