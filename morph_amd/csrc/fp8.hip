// Block-scaled FP8 (E4M3FN) transport encoding for gfx950:
//   pack:   per 256-element block, scale = max(amax(|x|) / 448, 1e-30);
//           byte = e4m3fn(clamp(x / scale, -448, 448))
//   unpack: y = dtype(float(byte) * scale)
// following streamtrain/precision.py:24-37 (pack_fp8 / unpack_fp8, used for
// the opt-in FP8 weight transfer of disk.py:330-345).  The reference computes
// with torch ops in FP32 (IEEE division, one rounding each); the bytes and
// the finite scales here are identical.  The scale is the same IEEE division; each
// element's quotient is the IEEE division for FP32 inputs, and for FP16/BF16
// inputs Markstein's correction of the product with the block's reciprocal
// (pack_kernel), checked exhaustively against the division.
//
// E4M3FN: 1 sign, 4 exponent (bias 7), 3 mantissa bits; no infinities, NaN =
// S.1111.111, largest finite 448, smallest subnormal 2^-9.  The pack encodes
// the quotients, clamped to +-448, with gfx950's v_cvt_pk_fp8_f32 (round to
// nearest even), which equals torch's conversion for every FP32 value in
// [-448, 448] (all compared on the device); the unpack decodes with
// v_cvt_pk_f32_fp8, exact for every code.  Torch propagates NaN through amax,
// clamp_min and clamp, so a block with a NaN has a NaN scale and NaN bytes, and
// a block with an infinity an infinite scale; their bytes follow the x86 NaN
// rules the reference's CPU ops run under (nonfinite_block_bytes8).
//
// One wave per 4 blocks (64 lanes x 16 elements).  Pack: each block is held
// by a row of 16 lanes (16 contiguous elements each), its amax a reduction
// within the row (row_max_bits).  Unpack: each block by 32 lanes, 8 bytes
// each per half of the wave's span.  A workgroup holds 4 waves / 16 blocks.
#include <type_traits>

#include "common.h"

namespace morph {
namespace {

constexpr int kBlockElems = MORPH_FP8_BLOCK;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBlocksPerWave = 4;  // 64 lanes x 16 elements
constexpr int kParts = 2;          // unpack: 512-element parts per wave, 8 elements per lane
static_assert(kBlockElems == 256, "16 lanes x 16 elements per block (pack), 32 x 8 (unpack)");

__device__ __forceinline__ bool is_nan(float x) { return x != x; }

// torch.amax of |x| over a block held by a row of 16 lanes: the bit patterns
// of non-negative floats order like the values, and every NaN pattern (above
// 0x7F800000) above +inf, so an unsigned maximum of |x|'s bits is the amax,
// NaN if any element is NaN.  By DPP within the row (quad swaps, half-row and
// row mirrors); every lane of the row ends with the maximum.
__device__ __forceinline__ uint32_t row_max_bits(uint32_t x) {
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xF, 0xF, false));  // row_half_mirror
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x140, 0xF, 0xF, false));  // row_mirror
  return x;
}

// Eight consecutive input elements as loaded: one 16-byte load of 16-bit
// values, two of FP32.
template <typename IT>
struct Raw8 {
  u32x4 v;
};
template <>
struct Raw8<F32> {
  f32x4 lo, hi;
};

// Elements i .. i + 7, all inside the input and 16-byte aligned.
template <typename IT>
__device__ __forceinline__ Raw8<IT> load_raw8(const void* src, int64_t i) {
  Raw8<IT> r;
  if constexpr (std::is_same_v<IT, F32>) {
    r.lo = *reinterpret_cast<const f32x4*>(static_cast<const float*>(src) + i);
    r.hi = *reinterpret_cast<const f32x4*>(static_cast<const float*>(src) + i + 4);
  } else {
    r.v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(src) + i);
  }
  return r;
}

template <typename IT>
__device__ __forceinline__ void raw8_to_float(const Raw8<IT>& r, float (&x)[8]) {
  if constexpr (std::is_same_v<IT, F32>) {
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] = r.lo[k], x[4 + k] = r.hi[k];
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = to_float<IT>(r.v[k] & 0xFFFFu);
      x[2 * k + 1] = to_float<IT>(r.v[k] >> 16);
    }
  }
}

// Elements i .. i + 7 of the input as floats (zeros past n: the reference pads
// the last block with zeros); one 16-byte load (two for FP32) when they are all
// inside and aligned.
template <typename IT>
__device__ __forceinline__ void load8(const void* src, int64_t i, int64_t n, float (&x)[8]) {
  constexpr int kBytes = Fmt<IT>::bytes;
  if (i + 8 <= n && (reinterpret_cast<uintptr_t>(src) + i * kBytes) % 16 == 0) {
    raw8_to_float<IT>(load_raw8<IT>(src, i), x);
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

// Eight quotients clamp(x / s, -448, 448) encoded as E4M3FN bytes (two words),
// for a finite scale s: x and the quotients are then finite too (|x| <= 448 s).
// For 16-bit inputs x / s is Markstein's correction of |x| * y with y = 1 / s --
// one IEEE division per block instead of one per element -- with x's sign put
// back (so -0 stays -0, as in the division): q = RN(|x| y), r = |x| - q s (exact
// by the fma), q' = RN(q + r y).  Checked against the IEEE quotient for every
// finite FP16 and BF16 block maximum and every element up to it: FP16 quotients
// are identical; BF16 ones differ only for subnormal elements, whose quotients
// (below 2^-13) encode as zero either way.  FP32 inputs take the IEEE division.
// v_cvt_pk_fp8_f32 is gfx950's OCP E4M3 conversion, round to nearest even:
// equal to torch's E4M3FN conversion for every FP32 value in [-448, 448] (all
// compared on the device).
template <typename IT>
__device__ __forceinline__ u32x2 quantize8(const float (&x)[8], float s, float y) {
  float q[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if constexpr (std::is_same_v<IT, F32>) {
      q[k] = x[k] / s;
    } else {
      const float ax = __builtin_fabsf(x[k]);
      const float t = ax * y;
      const float r = __fmaf_rn(-t, s, ax);
      q[k] = __builtin_copysignf(__fmaf_rn(r, y, t), x[k]);
    }
    q[k] = __builtin_amdgcn_fmed3f(q[k], -448.0f, 448.0f);
  }
  u32x2 w;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const uint32_t word = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[4 * k], q[4 * k + 1], 0, false);
    w[k] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[4 * k + 2], q[4 * k + 3], (int)word, true);
  }
  return w;
}

// The bytes of a block whose scale is NaN (it holds a NaN) or +inf (an
// infinity, no NaN), as the reference's CPU ops give them: x86 division
// returns its first NaN operand, and an invalid one (inf / inf) the negative
// default NaN; clamp keeps a NaN as it is and the E4M3FN conversion keeps its
// sign (NaN = S.1111.111).  s is a positive NaN (the amax of |x|), so
//   s = NaN: x's own NaN code for a NaN x, 0x7F for every other element;
//   s = inf: +-0 (x's sign) for finite x, 0xFF for x = +-inf.
__device__ __forceinline__ u32x2 nonfinite_block_bytes8(const float (&x)[8], float s) {
  u32x2 w = u32x2{0u, 0u};
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t sign = (__builtin_bit_cast(uint32_t, x[k]) >> 24) & 0x80u;
    uint32_t b;
    if (is_nan(x[k]))
      b = sign | 0x7Fu;
    else if (is_nan(s))
      b = 0x7Fu;
    else if (__builtin_isinf(x[k]))
      b = 0xFFu;
    else
      b = sign;
    w[k >> 2] |= b << (8 * (k & 3));
  }
  return w;
}

// One wave per kBlocksPerWave consecutive blocks: lane l holds the 16 elements
// at 16 l of the wave's span, so a row of 16 lanes holds one block, its amax is
// a reduction within the row, and each lane stores 16 contiguous bytes.  A wave
// whose span lies inside an aligned input issues all of its loads before the
// first is used.
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
  const int64_t i = first * kBlockElems + 16 * lane;
  const int64_t blk = first + (lane >> 4);
  float xa[8], xb[8];
  if ((first + kBlocksPerWave) * kBlockElems <= n &&
      reinterpret_cast<uintptr_t>(src) % 16 == 0) {  // wave-uniform
    const Raw8<IT> ra = load_raw8<IT>(src, i), rb = load_raw8<IT>(src, i + 8);
    raw8_to_float<IT>(ra, xa);
    raw8_to_float<IT>(rb, xb);
  } else {
    load8<IT>(src, i, n, xa);  // zeros past n, so blocks past the end reduce harmlessly
    load8<IT>(src, i + 8, n, xb);
  }
  uint32_t mb = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) mb = max(mb, max(mag(xa[k]), mag(xb[k])));
  const float m = __builtin_bit_cast(float, row_max_bits(mb));
  float s = m / 448.0f;
  s = (s < 1e-30f) ? 1e-30f : s;  // clamp_min keeps NaN
  if ((lane & 15) == 0 && blk < blocks) scales[blk] = s;
  u32x2 wa, wb;
  if (__builtin_isfinite(s)) {
    const float y = std::is_same_v<IT, F32> ? 0.0f : 1.0f / s;
    wa = quantize8<IT>(xa, s, y);
    wb = quantize8<IT>(xb, s, y);
  } else {
    wa = nonfinite_block_bytes8(xa, s);
    wb = nonfinite_block_bytes8(xb, s);
  }
  if (i + 16 <= n && ((reinterpret_cast<uintptr_t>(bytes) + i) & 15) == 0) {
    *reinterpret_cast<u32x4*>(bytes + i) = u32x4{wa[0], wa[1], wb[0], wb[1]};
  } else {
    for (int k = 0; k < 16; ++k)
      if (i + k < n) bytes[i + k] = (uint8_t)((k < 8 ? wa[k >> 2] : wb[(k - 8) >> 2]) >> (8 * (k & 3)));
  }
}

// The same layout as pack_kernel: in part h of the wave's span, lane l turns
// the 8 bytes at 512 h + 8 l into 8 outputs with its block's scale; a wave
// whose span lies inside aligned bytes loads all of its bytes and scales first.
template <typename OT>
__global__ __launch_bounds__(kThreads) void unpack_kernel(const uint8_t* __restrict__ bytes,
                                                          const float* __restrict__ scales,
                                                          int64_t n, void* __restrict__ dst,
                                                          int64_t blocks) {
  const int64_t wave = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int64_t first = wave * kBlocksPerWave;
  if (first >= blocks) return;
  const int lane = threadIdx.x & 63;
  const int64_t base = first * kBlockElems + 8 * lane;
  const bool whole = (first + kBlocksPerWave) * kBlockElems <= n &&
                     (reinterpret_cast<uintptr_t>(bytes) & 7) == 0;  // wave-uniform
  u32x2 wv[kParts];
  float sv[kParts];
  if (whole) {
#pragma unroll
    for (int h = 0; h < kParts; ++h) {
      wv[h] = *reinterpret_cast<const u32x2*>(bytes + base + 512 * h);
      sv[h] = scales[first + 2 * h + (lane >> 5)];
    }
  }
#pragma unroll
  for (int h = 0; h < kParts; ++h) {
    const int64_t i = base + 512 * h;
    float s;
    u32x2 w = u32x2{0u, 0u};
    if (whole) {
      s = sv[h];
      w = wv[h];
    } else {
      if (i >= n) continue;  // no cross-lane work here: lanes may leave on their own
      s = scales[first + 2 * h + (lane >> 5)];
      if (i + 8 <= n && ((reinterpret_cast<uintptr_t>(bytes) + i) & 7) == 0) {
        w = *reinterpret_cast<const u32x2*>(bytes + i);
      } else {
        for (int k = 0; k < 8; ++k)
          if (i + k < n) w[k >> 2] |= (uint32_t)bytes[i + k] << (8 * (k & 3));
      }
    }
    // gfx950's v_cvt_pk_f32_fp8 decodes two OCP E4M3 bytes (word_sel: the high
    // pair) exactly; every finite code is an FP32 value, and the NaN codes give NaN.
    float y[8];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[k], false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[k], true);
      y[4 * k] = lo[0] * s;
      y[4 * k + 1] = lo[1] * s;
      y[4 * k + 2] = hi[0] * s;
      y[4 * k + 3] = hi[1] * s;
    }
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
