// FP32 -> FP16 / BF16 / FP32 conversion of master weights for gfx950.
//
// Two callers in the reference do this on the CPU: the stage load casts each
// parameter's FP32 row of the [3, N] state file into the compute dtype before
// the H2D copy (streamtrain/disk.py:316-327, `destination.copy_(work)`), and
// the FP16 export encodes the same row with numpy (`value.astype('<f2')`)
// after checking that it is finite and within +-65504 (export.py:32-34).
// Here the row is already in HBM and one pass writes the compute copy (or the
// export bytes), optionally OR-ing a flag when some value is non-finite or,
// for FP16 output, beyond the FP16 range -- the export's check, made in the
// same pass.
//
// Rounding: FP16 by the hardware conversion (round to nearest even, overflow
// to inf, as numpy and torch); BF16 by round to nearest even with NaN ->
// 0x7FC0 (torch's c10::BFloat16).  Each lane converts 4 consecutive values of
// each half of its workgroup's 2048 (a 128-bit non-temporal load, a 64-bit
// store), so every access instruction covers whole lines: 2.5% faster than 8
// consecutive values per lane with temporal loads.  The FP32 -> FP32
// copy has a kernel of its own (copy_kernel): 64-lane workgroups, one 16-byte
// non-temporal load and store per lane, nothing rereads a copy soon.  Of the
// plain copies measured on 1.585 GB (64, 128 or 256 lanes, 1-4 accesses per
// lane, temporal or not, with or without a residency cap) this shape was the
// fastest, 6.58 TB/s against 6.40-6.48 for 128 or 256 lanes and 5.9-6.0 for
// two temporal or non-temporal accesses per lane of 256.
#include "common.h"

namespace morph {
namespace {

constexpr int kBlock = 256;
constexpr int kPerLane = 8;
constexpr int kPerBlock = kBlock * kPerLane;
constexpr float kF16Max = 65504.0f;
constexpr int kCopyLanes = 64;
constexpr int kCopyPerBlock = kCopyLanes * 4;

template <typename OT>
__device__ __forceinline__ bool out_of_range(float x) {
  const uint32_t b = __builtin_bit_cast(uint32_t, x);
  if (nonfinite_f32_bits(b)) return true;
  if constexpr (std::is_same_v<OT, F16>) return __builtin_fabsf(x) > kF16Max;
  return false;
}

template <typename OT, bool kCheck>
__global__ __launch_bounds__(kBlock) void convert_kernel(const float* __restrict__ src,
                                                         void* __restrict__ dst, int64_t n,
                                                         int vector_ok, uint32_t* flag) {
  static_assert(!std::is_same_v<OT, F32>, "the FP32 copy is copy_kernel");
  const int64_t base = (int64_t)blockIdx.x * kPerBlock;
  bool bad = false;
  if (vector_ok && base + kPerBlock <= n) {
#pragma unroll
    for (int h = 0; h < kPerLane / 4; ++h) {
      const int64_t e = base + ((int64_t)h * kBlock + threadIdx.x) * 4;
      const f32x4 a = load_stream<true>(reinterpret_cast<const f32x4*>(src + e));
      const float x[4] = {a.x, a.y, a.z, a.w};
      if constexpr (kCheck) {
#pragma unroll
        for (int k = 0; k < 4; ++k) bad |= out_of_range<OT>(x[k]);
      }
      const u32x2 w = u32x2{from_float<OT>(x[0]) | (from_float<OT>(x[1]) << 16),
                            from_float<OT>(x[2]) | (from_float<OT>(x[3]) << 16)};
      *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(dst) + e) = w;
    }
  } else {
    const int64_t end = base + kPerBlock < n ? base + kPerBlock : n;
    for (int64_t i = base + threadIdx.x; i < end; i += kBlock) {
      const float x = src[i];
      if constexpr (kCheck) bad |= out_of_range<OT>(x);
      static_cast<uint16_t*>(dst)[i] = (uint16_t)from_float<OT>(x);
    }
  }
  if constexpr (kCheck) {
    if (__builtin_amdgcn_ballot_w64(bad) != 0 && (threadIdx.x & 63) == 0) {
      volatile uint32_t* f = flag;
      *f = 1u;
    }
  }
}

// dst = src (FP32), flag as for FP32 output: some value is inf or NaN.
template <bool kCheck>
__global__ __launch_bounds__(kCopyLanes) void copy_kernel(const float* __restrict__ src,
                                                          float* __restrict__ dst, int64_t n,
                                                          int vector_ok, uint32_t* flag) {
  const int64_t base = (int64_t)blockIdx.x * kCopyPerBlock;
  bool bad = false;
  if (vector_ok && base + kCopyPerBlock <= n) {
    const int64_t i = base + (int64_t)threadIdx.x * 4;
    const f32x4 v = load_stream<true>(reinterpret_cast<const f32x4*>(src + i));
    if constexpr (kCheck) {
      const u32x4 u = __builtin_bit_cast(u32x4, v);
      bad = nonfinite_f32_bits(u.x) | nonfinite_f32_bits(u.y) | nonfinite_f32_bits(u.z) |
            nonfinite_f32_bits(u.w);
    }
    store_stream<true>(reinterpret_cast<f32x4*>(dst + i), v);
  } else {
    const int64_t end = base + kCopyPerBlock < n ? base + kCopyPerBlock : n;
    for (int64_t i = base + threadIdx.x; i < end; i += kCopyLanes) {
      const float x = src[i];
      if constexpr (kCheck) bad |= nonfinite_f32_bits(__builtin_bit_cast(uint32_t, x));
      dst[i] = x;
    }
  }
  if constexpr (kCheck) {
    if (__builtin_amdgcn_ballot_w64(bad) != 0 && threadIdx.x == 0) {
      volatile uint32_t* f = flag;
      *f = 1u;
    }
  }
}

int launch_copy(const float* src, float* dst, int64_t n, int vector_ok, uint32_t* flag,
                hipStream_t s) {
  const int64_t blocks = (n + kCopyPerBlock - 1) / kCopyPerBlock;
  if (blocks > 0x7FFFFFFF) return MORPH_ERANGE;
  if (flag)
    hipLaunchKernelGGL(copy_kernel<true>, dim3((unsigned)blocks), dim3(kCopyLanes), 0, s, src,
                       dst, n, vector_ok, flag);
  else
    hipLaunchKernelGGL(copy_kernel<false>, dim3((unsigned)blocks), dim3(kCopyLanes), 0, s, src,
                       dst, n, vector_ok, flag);
  return launch_status();
}

template <typename OT>
int launch(const float* src, void* dst, int64_t n, int vector_ok, uint32_t* flag, hipStream_t s) {
  const int64_t blocks = (n + kPerBlock - 1) / kPerBlock;
  if (flag)
    hipLaunchKernelGGL((convert_kernel<OT, true>), dim3((unsigned)blocks), dim3(kBlock), 0, s, src,
                       dst, n, vector_ok, flag);
  else
    hipLaunchKernelGGL((convert_kernel<OT, false>), dim3((unsigned)blocks), dim3(kBlock), 0, s,
                       src, dst, n, vector_ok, flag);
  return launch_status();
}

}  // namespace
}  // namespace morph

using namespace morph;

extern "C" int morph_convert_f32(const float* src, void* dst, int dst_dtype, int64_t n,
                                 uint32_t* d_range_flag, void* stream) {
  if (n < 0 || (n > 0 && (src == nullptr || dst == nullptr))) return MORPH_EINVAL;
  if (dst_dtype != MORPH_DTYPE_F32 && dst_dtype != MORPH_DTYPE_F16 && dst_dtype != MORPH_DTYPE_BF16)
    return MORPH_EDTYPE;
  if (n == 0) return MORPH_OK;
  if ((n + kPerBlock - 1) / kPerBlock > 0x7FFFFFFF) return MORPH_ERANGE;
  const int vector_ok = reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(dst) % 16 == 0;
  hipStream_t s = as_stream(stream);
  switch (dst_dtype) {
    case MORPH_DTYPE_F16: return launch<F16>(src, dst, n, vector_ok, d_range_flag, s);
    case MORPH_DTYPE_BF16: return launch<BF16>(src, dst, n, vector_ok, d_range_flag, s);
    default: return launch_copy(src, static_cast<float*>(dst), n, vector_ok, d_range_flag, s);
  }
}
