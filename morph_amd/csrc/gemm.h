// Library-internal entry of the batched bf16 GEMM (gemm.hip).
#pragma once

#include <stdint.h>

namespace morph {

// morph_gemm_nt_bf16 with an optional per-matrix factor: when bscale is not
// null, matrix b of the batch uses alpha * bscale[b] and beta * bscale[b]
// (bscale: device array of batch floats, read by the epilogue); and, for a
// symmetric product, a constant added to every diagonal element: C[i][i] =
// fp32(alpha * acc + beta * D) + diag, then the one rounding to bf16 (diag =
// 0 adds nothing; off-diagonal elements never take the add).
__attribute__((visibility("hidden"))) int gemm_nt_bf16_scaled(
    const uint16_t* P, const uint16_t* Q, const uint16_t* D, uint16_t* C, uint16_t* Ct,
    int64_t M, int64_t N, int64_t K, int64_t batch, int64_t ldp, int64_t ldq, int64_t ldd,
    int64_t ldc, int64_t ldct, int64_t stride_p, int64_t stride_q, int64_t stride_d,
    int64_t stride_c, int64_t stride_ct, float alpha, float beta, const float* bscale,
    float diag, int flags, void* stream);

// The Muon master update carried by the last Newton-Schulz product X' = B' X
// (gemm_kn_apply): instead of storing X', the epilogue rounds each element to
// bf16 as the store would and updates matrix b's FP32 parameter in place,
// p = fma(bf16(X') * scale[b], neg_lr, p * decay), with X' in p's layout.  X
// is [m, n] with no padding (m, n multiples of the 256 tile); p[b] is [m, n]
// (row length n), or [n, m] (row length m) when transposed[b], 16-byte aligned.
constexpr int kGemmMaxApply = 64;
struct GemmApply {
  float* p[kGemmMaxApply];
  int32_t transposed[kGemmMaxApply];
  float scale[kGemmMaxApply];
  int64_t m, n;
  float decay, neg_lr;
};

// C[b] = alpha * bscale[b] * P[b] . Q[b] with Q stored [K, N] (the
// MORPH_GEMM_Q_KN form) and the update above in place of the store of C.
// P [M, K] = B' (M = m, K = m), Q [K, N] = X (N = n); batch <= 64.
__attribute__((visibility("hidden"))) int gemm_kn_apply(
    const uint16_t* P, const uint16_t* Q, int64_t M, int64_t N, int64_t K, int64_t batch,
    int64_t ldp, int64_t ldq, int64_t stride_p, int64_t stride_q, const float* bscale,
    const GemmApply& ap, void* stream);

}  // namespace morph
