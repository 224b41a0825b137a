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

}  // namespace morph
