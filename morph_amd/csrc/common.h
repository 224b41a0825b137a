// Shared device helpers for the gfx950 optimizer kernels.
//
// All arithmetic here must round exactly like torch's CPU kernels do, so the
// library is compiled with -ffp-contract=off and every fused multiply-add is
// written out with __fmaf_rn.  Division (`/`) and square root
// (__builtin_sqrtf) lower to the correctly rounded IEEE sequences under
// -fhip-fp32-correctly-rounded-divide-sqrt.  (__fsqrt_rn is NOT used: without
// OCML_BASIC_ROUNDED_OPERATIONS clang maps it to the 1-ulp hardware sqrt.)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/morph_optim.h"

namespace morph {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Streaming loads/stores: the optimizer touches every byte exactly once, so
// non-temporal hints keep the L2 / MALL from retaining dead lines.
template <bool NT, typename V>
__device__ __forceinline__ V load_stream(const V* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

template <bool NT, typename V>
__device__ __forceinline__ void store_stream(V* p, V x) {
  if constexpr (NT) __builtin_nontemporal_store(x, p);
  else *p = x;
}

// ---- 16-bit formats --------------------------------------------------------
__device__ __forceinline__ float half_bits_to_float(uint32_t h16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}
__device__ __forceinline__ float bf16_bits_to_float(uint32_t b16) {
  return __builtin_bit_cast(float, b16 << 16);
}
// Round to nearest even (IEEE conversion; overflow -> inf).  The empty asm
// pins f as a finished FP32 value: without it the compiler may fold a
// preceding multiply and this conversion into v_fma_mixlo_f16 (a * b + 0),
// which turns a -0 product into +0 -- torch and numpy convert the rounded
// FP32 product, sign of zero included.
__device__ __forceinline__ uint32_t float_to_half_bits(float f) {
  asm volatile("" : "+v"(f));
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}
// Round to nearest even; NaN -> 0x7FC0 like torch's c10::BFloat16.
__device__ __forceinline__ uint32_t float_to_bf16_bits(float f) {
  uint32_t x = __builtin_bit_cast(uint32_t, f);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (x + 0x7FFFu + ((x >> 16) & 1u)) >> 16;
}

// The Muon master update of one element (streamtrain/optimizer.py:60-61):
// update = U * scale with U the bf16 Newton-Schulz result, then
// p.mul_(1 - lr * wd).add_(update, alpha=-lr), which torch's CPU kernels round
// as fma(update, -lr, p * decay).  Shared by the finish pass and the epilogue
// of the last Newton-Schulz product, so both give the same bits.
__device__ __forceinline__ float muon_update_element(float p, uint32_t u16, float scale,
                                                     float decay, float neg_lr) {
  const float upd = bf16_bits_to_float(u16) * scale;
  return __fmaf_rn(upd, neg_lr, p * decay);
}

// Tag types for the element formats of gradients and export copies.
struct F32 {};
struct F16 {};
struct BF16 {};
struct NoOut {};

template <typename T> struct Fmt;
template <> struct Fmt<F32> { static constexpr int bytes = 4; };
template <> struct Fmt<F16> { static constexpr int bytes = 2; };
template <> struct Fmt<BF16> { static constexpr int bytes = 2; };
template <> struct Fmt<NoOut> { static constexpr int bytes = 0; };

template <typename T>
__device__ __forceinline__ float to_float(uint32_t bits16);
template <> __device__ __forceinline__ float to_float<F16>(uint32_t b) { return half_bits_to_float(b); }
template <> __device__ __forceinline__ float to_float<BF16>(uint32_t b) { return bf16_bits_to_float(b); }

template <typename T>
__device__ __forceinline__ uint32_t from_float(float f);
template <> __device__ __forceinline__ uint32_t from_float<F16>(float f) { return float_to_half_bits(f); }
template <> __device__ __forceinline__ uint32_t from_float<BF16>(float f) { return float_to_bf16_bits(f); }

// Non-finite test on raw bits: exponent field all ones.
__device__ __forceinline__ bool nonfinite_f32_bits(uint32_t x) { return (x & 0x7F800000u) == 0x7F800000u; }
// Two packed 16-bit values per word.
__device__ __forceinline__ bool nonfinite_f16x2(uint32_t x) {
  return ((x & 0x7C00u) == 0x7C00u) | ((x & 0x7C000000u) == 0x7C000000u);
}
__device__ __forceinline__ bool nonfinite_bf16x2(uint32_t x) {
  return ((x & 0x7F80u) == 0x7F80u) | ((x & 0x7F800000u) == 0x7F800000u);
}

// Multi-tensor launches: segment i owns blocks [t[i].first_block,
// t[i + 1].first_block).  The segment of block b, by binary search over the
// kernel-argument table (first_block ascending, t[0].first_block == 0).
template <typename Seg>
__device__ __forceinline__ int segment_of(const Seg* t, int count, int b) {
  int lo = 0, hi = count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (t[mid].first_block <= b) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Kernel arguments travel in the 4 KiB kernel-argument segment.
constexpr size_t kMaxKernargBytes = 4096;

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MORPH_OK : MORPH_ELAUNCH;
}

}  // namespace morph
