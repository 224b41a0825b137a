// Block-scaled FP8 (E4M3FN) transport encoding for gfx950:
//   pack:   per 256-element block, scale = max(amax(|x|) / 448, 1e-30);
//           byte = e4m3fn(clamp(x / scale, -448, 448))
//   unpack: y = dtype(float(byte) * scale)
// following streamtrain/precision.py:24-37 (pack_fp8 / unpack_fp8, used for
// the opt-in FP8 weight transfer of disk.py:330-345).  The reference computes
// with torch ops in FP32 (IEEE division, one rounding each); the bytes and
// scales here are identical.  The scale is the same IEEE division; each
// element's quotient is the IEEE division for FP32 inputs, and for FP16/BF16
// inputs Markstein's correction of the product with the block's reciprocal
// (pack_kernel), checked exhaustively against the division.
//
// E4M3FN: 1 sign, 4 exponent (bias 7), 3 mantissa bits; no infinities, NaN =
// S.1111.111, largest finite 448, smallest subnormal 2^-9.  The conversion is
// round to nearest even; e4m3fn_from_float writes it from the format
// definition: normal results round the FP32 bit pattern at mantissa bit 20 (a
// carry moves into the exponent), subnormal results are rint(|x| * 2^9); NaN
// stays NaN.  The pack encodes with gfx950's v_cvt_pk_fp8_f32, which gives the
// same bytes for every non-NaN input in range (all FP32 bit patterns compared
// on the device), and uses e4m3fn_from_float for NaN.  Inputs here are already
// clamped to +-448, so the out-of-range case only arises for NaN.  Torch
// propagates NaN through amax, clamp_min and clamp, so a block with a NaN has
// a NaN scale and all-NaN bytes; that is reproduced too.
//
// One wave per 4 blocks (64 lanes x 16 elements); each block is held by 32
// lanes (8 elements each), and its amax is a reduction over those lanes
// (half_wave_max_bits).  A workgroup holds 4 waves / 16 blocks.
#include <type_traits>

#include "common.h"

namespace morph {
namespace {

constexpr int kBlockElems = MORPH_FP8_BLOCK;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBlocksPerWave = 4;  // 64 lanes x 16 elements
static_assert(kBlockElems == 256, "32 lanes x 8 elements per block");

__device__ __forceinline__ bool is_nan(float x) { return x != x; }

// torch.amax of |x| over a block held by 32 lanes (lanes 0-31 or 32-63 of the
// wave): the bit patterns of non-negative floats order like the values, and
// every NaN pattern (above 0x7F800000) above +inf, so an unsigned maximum of
// |x|'s bits is the amax, NaN if any element is NaN.  Within each row of 16
// lanes by DPP (quad swaps, half-row and row mirrors), then across the two rows
// of each half with gfx950's v_permlane16_swap; no LDS round trips.
__device__ __forceinline__ uint32_t half_wave_max_bits(uint32_t x) {
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xF, 0xF, false));  // row_half_mirror
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x140, 0xF, 0xF, false));  // row_mirror
  const auto r16 = __builtin_amdgcn_permlane16_swap(x, x, false, false);  // rows 0 <-> 1, 2 <-> 3
  return max((uint32_t)r16[0], (uint32_t)r16[1]);
}

__device__ __forceinline__ uint32_t e4m3fn_from_float(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;  // NaN
  uint32_t r;
  if (a < 0x3C800000u) {  // below 2^-6: subnormal (or zero) result, step 2^-9
    r = (uint32_t)__builtin_rintf(__builtin_bit_cast(float, a) * 512.0f);
  } else {
    r = ((a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20) - (120u << 3);  // rebias 127 -> 7
    if (r > 0x7Eu) r = 0x7Fu;  // beyond 448 after rounding: NaN (no infinities)
  }
  return sign | r;
}

__device__ __forceinline__ float float_from_e4m3fn(uint32_t b) {
  const uint32_t e = (b >> 3) & 0xFu, m = b & 7u;
  float v;
  if (e == 0)
    v = (float)m * 0.001953125f;  // m * 2^-9, exact
  else if (e == 0xFu && m == 7u)
    v = __builtin_nanf("");
  else
    v = __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  return (b & 0x80u) ? -v : v;
}

// Elements i .. i + 7 of the input as floats (zeros past n: the reference pads
// the last block with zeros); one 16-byte load (two for FP32) when they are all
// inside and aligned.
template <typename IT>
__device__ __forceinline__ void load8(const void* src, int64_t i, int64_t n, float (&x)[8]) {
  constexpr int kBytes = Fmt<IT>::bytes;
  if (i + 8 <= n && (reinterpret_cast<uintptr_t>(src) + i * kBytes) % 16 == 0) {
    if constexpr (std::is_same_v<IT, F32>) {
      const f32x4 v0 = *reinterpret_cast<const f32x4*>(static_cast<const float*>(src) + i);
      const f32x4 v1 = *reinterpret_cast<const f32x4*>(static_cast<const float*>(src) + i + 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) x[k] = v0[k], x[4 + k] = v1[k];
    } else {
      const u32x4 v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(src) + i);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        x[2 * k] = to_float<IT>(v[k] & 0xFFFFu);
        x[2 * k + 1] = to_float<IT>(v[k] >> 16);
      }
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int64_t j = i + k;
    if (j < n) {
      if constexpr (std::is_same_v<IT, F32>)
        x[k] = static_cast<const float*>(src)[j];
      else
        x[k] = to_float<IT>(static_cast<const uint16_t*>(src)[j]);
    } else {
      x[k] = 0.0f;
    }
  }
}

// One wave per kBlocksPerWave consecutive blocks: in half h (0, 1) of the
// wave's span, lane l holds the 8 elements at 512 h + 8 l, so lanes 0-31 and
// 32-63 each hold one whole block per half, every access is a contiguous 512 B
// (16-bit input) per instruction, and the amax needs no cross-half exchange.
template <typename IT>
__global__ __launch_bounds__(kThreads) void pack_kernel(const void* __restrict__ src, int64_t n,
                                                        uint8_t* __restrict__ bytes,
                                                        float* __restrict__ scales,
                                                        int64_t blocks) {
  const int64_t wave = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int64_t first = wave * kBlocksPerWave;
  if (first >= blocks) return;  // whole waves exit together
  const int lane = threadIdx.x & 63;
  auto mag = [](float v) { return __builtin_bit_cast(uint32_t, v) & 0x7FFFFFFFu; };
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t blk = first + 2 * h + (lane >> 5);
    const int64_t i = first * kBlockElems + 512 * h + 8 * lane;
    float x[8];
    load8<IT>(src, i, n, x);  // zeros past n, so blocks past the end reduce harmlessly
    uint32_t mb = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) mb = max(mb, mag(x[k]));
    const float m = __builtin_bit_cast(float, half_wave_max_bits(mb));
    float s = m / 448.0f;
    s = (s < 1e-30f) ? 1e-30f : s;  // clamp_min keeps NaN
    if ((lane & 31) == 0 && blk < blocks) scales[blk] = s;
    float q[8];
    // FP32 inputs, and blocks holding an infinity (s = inf: x / s is 0, or NaN for the
    // infinities themselves), take the IEEE division.
    if (std::is_same_v<IT, F32> || __builtin_isinf(s)) {
#pragma unroll
      for (int k = 0; k < 8; ++k) q[k] = x[k] / s;
    } else {
      // 16-bit inputs, finite scale (NaN propagates either way): x / s by
      // Markstein's correction of |x| * (1 / s) -- one IEEE division per block
      // instead of one per element -- with x's sign put back (so -0 stays -0, as
      // in the division).  q = RN(|x| y), r = |x| - q s (exact by the fma), q' =
      // RN(q + r y).  Checked against the IEEE quotient for every finite FP16 and
      // BF16 block maximum and every element up to it: FP16 quotients are
      // identical; BF16 ones differ only for subnormal elements, whose quotients
      // (below 2^-13) encode as zero either way.
      const float y = 1.0f / s;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float ax = __builtin_fabsf(x[k]);
        const float t = ax * y;
        const float r = __fmaf_rn(-t, s, ax);
        q[k] = __builtin_copysignf(__fmaf_rn(r, y, t), x[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
      q[k] = is_nan(q[k]) ? q[k] : (q[k] < -448.0f ? -448.0f : (q[k] > 448.0f ? 448.0f : q[k]));
    // v_cvt_pk_fp8_f32 is gfx950's OCP E4M3 conversion, round to nearest even:
    // equal to e4m3fn_from_float for every non-NaN FP32 input in [-448, 448] (all
    // 2^32 bit patterns were compared on the device); NaN keeps the format rule's
    // encoding.
    u32x2 w;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      uint32_t word = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[4 * k], q[4 * k + 1], 0, false);
      word = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[4 * k + 2], q[4 * k + 3], (int)word, true);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (is_nan(q[4 * k + e]))
          word = (word & ~(0xFFu << (8 * e))) | (e4m3fn_from_float(q[4 * k + e]) << (8 * e));
      w[k] = word;
    }
    if (i + 8 <= n && ((reinterpret_cast<uintptr_t>(bytes) + i) & 7) == 0) {
      *reinterpret_cast<u32x2*>(bytes + i) = w;
    } else {
      for (int k = 0; k < 8; ++k)
        if (i + k < n) bytes[i + k] = (uint8_t)(w[k >> 2] >> (8 * (k & 3)));
    }
  }
}

// The same layout as pack_kernel: in half h of the wave's span, lane l turns
// the 8 bytes at 512 h + 8 l into 8 outputs with its block's scale.
template <typename OT>
__global__ __launch_bounds__(kThreads) void unpack_kernel(const uint8_t* __restrict__ bytes,
                                                          const float* __restrict__ scales,
                                                          int64_t n, void* __restrict__ dst,
                                                          int64_t blocks) {
  const int64_t wave = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int64_t first = wave * kBlocksPerWave;
  if (first >= blocks) return;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t i = first * kBlockElems + 512 * h + 8 * lane;
    if (i >= n) continue;  // no cross-lane work here: lanes may leave on their own
    const float s = scales[first + 2 * h + (lane >> 5)];
    u32x2 w = u32x2{0u, 0u};
    if (i + 8 <= n && ((reinterpret_cast<uintptr_t>(bytes) + i) & 7) == 0) {
      w = *reinterpret_cast<const u32x2*>(bytes + i);
    } else {
      for (int k = 0; k < 8; ++k)
        if (i + k < n) w[k >> 2] |= (uint32_t)bytes[i + k] << (8 * (k & 3));
    }
    float y[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = float_from_e4m3fn((w[k >> 2] >> (8 * (k & 3))) & 0xFFu) * s;
    constexpr int kBytes = Fmt<OT>::bytes;
    if (i + 8 <= n && (reinterpret_cast<uintptr_t>(dst) + i * kBytes) % 16 == 0) {
      if constexpr (std::is_same_v<OT, F32>) {
        float* d = static_cast<float*>(dst) + i;
        *reinterpret_cast<f32x4*>(d) = f32x4{y[0], y[1], y[2], y[3]};
        *reinterpret_cast<f32x4*>(d + 4) = f32x4{y[4], y[5], y[6], y[7]};
      } else {
        u32x4 v;
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = from_float<OT>(y[2 * k]) | (from_float<OT>(y[2 * k + 1]) << 16);
        *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(dst) + i) = v;
      }
      continue;
    }
    for (int k = 0; k < 8; ++k) {
      if (i + k >= n) break;
      if constexpr (std::is_same_v<OT, F32>)
        static_cast<float*>(dst)[i + k] = y[k];
      else
        static_cast<uint16_t*>(dst)[i + k] = (uint16_t)from_float<OT>(y[k]);
    }
  }
}

int64_t nblocks(int64_t n) { return (n + kBlockElems - 1) / kBlockElems; }

}  // namespace
}  // namespace morph

using namespace morph;

extern "C" int morph_fp8_pack(const void* src, int src_dtype, int64_t n, uint8_t* bytes,
                              float* scales, void* stream) {
  if (n < 0 || (n > 0 && (src == nullptr || bytes == nullptr || scales == nullptr)))
    return MORPH_EINVAL;
  if (n == 0) return MORPH_OK;
  const int64_t blocks = nblocks(n);
  const int64_t per_group = (int64_t)kWaves * kBlocksPerWave;
  const int64_t groups = (blocks + per_group - 1) / per_group;
  if (groups > 0x7FFFFFFF) return MORPH_ERANGE;
  hipStream_t s = as_stream(stream);
  switch (src_dtype) {
    case MORPH_DTYPE_F32:
      hipLaunchKernelGGL(pack_kernel<F32>, dim3((unsigned)groups), dim3(kThreads), 0, s, src, n, bytes, scales, blocks);
      break;
    case MORPH_DTYPE_F16:
      hipLaunchKernelGGL(pack_kernel<F16>, dim3((unsigned)groups), dim3(kThreads), 0, s, src, n, bytes, scales, blocks);
      break;
    case MORPH_DTYPE_BF16:
      hipLaunchKernelGGL(pack_kernel<BF16>, dim3((unsigned)groups), dim3(kThreads), 0, s, src, n, bytes, scales, blocks);
      break;
    default:
      return MORPH_EDTYPE;
  }
  return launch_status();
}

extern "C" int morph_fp8_unpack(const uint8_t* bytes, const float* scales, int64_t n, void* dst,
                                int dst_dtype, void* stream) {
  if (n < 0 || (n > 0 && (bytes == nullptr || scales == nullptr || dst == nullptr)))
    return MORPH_EINVAL;
  if (n == 0) return MORPH_OK;
  const int64_t blocks = nblocks(n);
  const int64_t per_group = (int64_t)kWaves * kBlocksPerWave;
  const int64_t groups = (blocks + per_group - 1) / per_group;
  if (groups > 0x7FFFFFFF) return MORPH_ERANGE;
  hipStream_t s = as_stream(stream);
  switch (dst_dtype) {
    case MORPH_DTYPE_F32:
      hipLaunchKernelGGL(unpack_kernel<F32>, dim3((unsigned)groups), dim3(kThreads), 0, s, bytes, scales, n, dst, blocks);
      break;
    case MORPH_DTYPE_F16:
      hipLaunchKernelGGL(unpack_kernel<F16>, dim3((unsigned)groups), dim3(kThreads), 0, s, bytes, scales, n, dst, blocks);
      break;
    case MORPH_DTYPE_BF16:
      hipLaunchKernelGGL(unpack_kernel<BF16>, dim3((unsigned)groups), dim3(kThreads), 0, s, bytes, scales, n, dst, blocks);
      break;
    default:
      return MORPH_EDTYPE;
  }
  return launch_status();
}
