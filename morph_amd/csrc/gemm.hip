// Batched bf16 "NT" GEMM on gfx950 MFMA, the building block of the Muon
// Newton-Schulz iteration (streamtrain/optimizer.py:19-21):
//
//   C[b] = alpha * P[b] . Q[b]^T + beta * D[b]      (bf16 in, fp32 accumulate, bf16 out)
//   Ct[b] = C[b]^T                                   (optional second output)
//
// P is [M, K] and Q is [N, K], both row-major with K contiguous, so every MFMA
// operand fragment is 16 contiguous bytes of one row.  One NS iteration is three
// such products: A = X X^T; B = b A + c A A^T (A is symmetric); X' = a X + B Xt^T
// (B is symmetric, Xt = X^T), which is why only this one layout is needed.
//
// Tiling.  A workgroup (256 lanes, 4 wave64) owns a 128 x 128 tile of C; wave w
// owns the 64 x 64 quarter (w / 2, w % 2) as 2 x 2 tiles of
// v_mfma_f32_32x32x16_bf16.  K advances 64 per iteration: the P and Q tiles
// (128 x 64 bf16 each) are staged global -> registers -> LDS, the next
// iteration's global loads are issued before this iteration's MFMAs so their
// latency hides behind the math.  LDS rows are padded to 72 bf16 (144 bytes)
// so the 128-bit fragment reads of 16 consecutive rows hit distinct banks.
//
// MFMA 32x32x16 lane layout (checked on the device): lane l holds
// A[l % 32][8 (l / 32) + i] and B[8 (l / 32) + i][l % 32] for i < 8; output
// register r of lane l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
//
// Dimensions must be multiples of the tile (M, N of 128, K of 64): callers pad
// with zeros, which is exact for Newton-Schulz (zero rows stay zero).
#include "common.h"

namespace morph {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = MORPH_GEMM_TILE_M;
constexpr int BN = MORPH_GEMM_TILE_N;
constexpr int BK = MORPH_GEMM_TILE_K;
constexpr int LDK = BK + 8;  // padded LDS row (bf16 elements)
constexpr int kThreads = 256;
constexpr int kChunks = BM * BK / 8 / kThreads;  // 16-byte chunks per lane per tile (4)

struct GemmArgs {
  const uint16_t* P;
  const uint16_t* Q;
  const uint16_t* D;
  uint16_t* C;
  uint16_t* Ct;
  int64_t M, N, K;
  int64_t ldp, ldq, ldd, ldc, ldct;
  int64_t sp, sq, sd, sc, sct;
  float alpha, beta;
};

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return float_to_bf16_bits(lo) | (float_to_bf16_bits(hi) << 16);
}

__global__ __launch_bounds__(kThreads) void gemm_nt_kernel(const GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t sP[BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t sQ[BN * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t b = blockIdx.z;
  const int64_t row0 = (int64_t)blockIdx.y * BM;
  const int64_t col0 = (int64_t)blockIdx.x * BN;
  const uint16_t* P = g.P + b * g.sp + row0 * g.ldp;
  const uint16_t* Q = g.Q + b * g.sq + col0 * g.ldq;

  // Global -> register staging: chunk c of a tile is row c / 8, 16-byte column c % 8.
  u32x4 rp[kChunks], rq[kChunks];
  auto load_tiles = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = tid + i * kThreads;
      const int r = c >> 3, kc = (c & 7) * 8;
      rp[i] = *reinterpret_cast<const u32x4*>(P + r * g.ldp + k0 + kc);
      rq[i] = *reinterpret_cast<const u32x4*>(Q + r * g.ldq + k0 + kc);
    }
  };
  auto store_tiles = [&]() {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = tid + i * kThreads;
      const int r = c >> 3, kc = (c & 7) * 8;
      *reinterpret_cast<u32x4*>(sP + r * LDK + kc) = rp[i];
      *reinterpret_cast<u32x4*>(sQ + r * LDK + kc) = rq[i];
    }
  };

  const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
  const int fr = lane & 31, fk = (lane >> 5) * 8;
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int64_t KT = g.K / BK;
  load_tiles(0);
  for (int64_t kt = 0; kt < KT; ++kt) {
    __syncthreads();  // every wave finished reading the previous tile
    store_tiles();
    __syncthreads();
    if (kt + 1 < KT) load_tiles((kt + 1) * BK);  // in flight during the MFMAs below
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 a[2], q[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[i] = *reinterpret_cast<const bf16x8*>(sP + (wr + i * 32 + fr) * LDK + kk + fk);
        q[i] = *reinterpret_cast<const bf16x8*>(sQ + (wc + i * 32 + fr) * LDK + kk + fk);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], q[j], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue: out = alpha * acc + beta * D, rounded once to bf16.
  const uint16_t* D = g.D ? g.D + b * g.sd : nullptr;
  uint16_t* C = g.C + b * g.sc;
  uint16_t* Ct = g.Ct ? g.Ct + b * g.sct : nullptr;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = col0 + wc + j * 32 + fr;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int64_t rbase = row0 + wr + i * 32 + q4 * 8 + (lane >> 5) * 4;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = g.alpha * acc[i][j][q4 * 4 + r];
          if (D) x = __fmaf_rn(g.beta, bf16_bits_to_float(D[(rbase + r) * g.ldd + col]), x);
          v[r] = x;
          C[(rbase + r) * g.ldc + col] = (uint16_t)float_to_bf16_bits(x);
        }
        if (Ct) {
          u32x2 t;
          t.x = pack_bf16x2(v[0], v[1]);
          t.y = pack_bf16x2(v[2], v[3]);
          *reinterpret_cast<u32x2*>(Ct + col * g.ldct + rbase) = t;
        }
      }
    }
  }
}

}  // namespace
}  // namespace morph

using namespace morph;

extern "C" int morph_gemm_nt_bf16(const uint16_t* P, const uint16_t* Q, const uint16_t* D,
                                  uint16_t* C, uint16_t* Ct, int64_t M, int64_t N, int64_t K,
                                  int64_t batch, int64_t ldp, int64_t ldq, int64_t ldd,
                                  int64_t ldc, int64_t ldct, int64_t stride_p, int64_t stride_q,
                                  int64_t stride_d, int64_t stride_c, int64_t stride_ct,
                                  float alpha, float beta, void* stream) {
  if (P == nullptr || Q == nullptr || C == nullptr || M < 0 || N < 0 || K <= 0 || batch < 0)
    return MORPH_EINVAL;
  auto misaligned = [](const void* p, uintptr_t a) {
    return p != nullptr && (reinterpret_cast<uintptr_t>(p) % a) != 0;
  };
  if (misaligned(P, 16) || misaligned(Q, 16) || misaligned(Ct, 8) || misaligned(C, 2) ||
      misaligned(D, 2))
    return MORPH_EINVAL;
  if (M % BM || N % BN || K % BK) return MORPH_ERANGE;
  if (ldp < K || ldq < K || ldc < N || (D && ldd < N) || (Ct && ldct < M)) return MORPH_EINVAL;
  if (ldp % 8 || ldq % 8 || stride_p % 8 || stride_q % 8 || (Ct && (ldct % 4 || stride_ct % 4)))
    return MORPH_EINVAL;  // 16-byte operand loads, 8-byte transposed stores
  if (M == 0 || N == 0 || batch == 0) return MORPH_OK;
  if (M / BM > 65535 || batch > 65535 || N / BN > (1 << 30)) return MORPH_ERANGE;
  GemmArgs g{P, Q, D, C, Ct, M, N, K, ldp, ldq, ldd, ldc, ldct,
             stride_p, stride_q, stride_d, stride_c, stride_ct, alpha, beta};
  hipLaunchKernelGGL(gemm_nt_kernel, dim3((unsigned)(N / BN), (unsigned)(M / BM), (unsigned)batch),
                     dim3(kThreads), 0, as_stream(stream), g);
  return launch_status();
}
