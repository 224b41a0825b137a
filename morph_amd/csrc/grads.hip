// Stage-gradient accumulation for gfx950: unscale + accumulate into the FP32
// stage window, and on the last micro-batch the non-finite flag and the FP64
// sum of squares in the same pass.
//
// The reference does this with torch ops per micro-batch and parameter,
//   destination.add_(g.detach().float() / loss_scale)
// into a zeroed FP32 window (streamtrain/sparse_disk.py:82-87, 104-108;
// disk.py:446-448 on the CPU), then a separate pass
//   norm_squared += piece.double().square().sum().item()   (1M-element pieces)
// whose finiteness decides skip / retry and whose value sets the clip
// (disk.py:466-468, 485-489; sparse_disk.py:136).  Here each micro-batch is
// one pass over the window (10 B/param for 16-bit gradients: read g, read and
// write the FP32 sum) and the final pass also produces the flag and one FP64
// partial per workgroup, so the norm costs no extra read.
//
// Rounding: fp32(g) * 2^-k (or / scale when the scale is not a power of two,
// IEEE division as torch's CPU kernel), then one fp32 add -- the reference's
// two roundings.  The first micro-batch (MORPH_ACCUM_OVERWRITE) computes
// 0 + x rather than loading the buffer, which is what zero_() followed by
// add_() produces (including +0 for a -0 gradient), so no zeroing pass runs.
// Squares are exact in FP64 (24-bit mantissas); each workgroup sums its
// squares in a fixed order and a one-workgroup pass adds the partials in index
// order, so the result is deterministic for a given layout.  Its last bits can
// differ from the reference's chunked torch sum, whose order is different.
//
// Access layout: a workgroup owns 2048 consecutive elements; lane l moves
// elements 4 l .. 4 l + 3 of each 1024-element half, so every access
// instruction of a wave covers whole lines (1 KiB of the window, 512 B of a
// 16-bit gradient).  The gradient is read once, non-temporally; the window is
// read again by the next micro-batch and keeps ordinary accesses.  Against 8
// consecutive elements per lane with temporal loads: 92.8 -> 83.6 us per plain
// pass on the config-2 window (6.77 TB/s, 85% of 8 TB/s), same bits; with the
// window non-temporal too, 91.9 us; 128 or 64 lanes per workgroup, 84.2 and
// 85.8 us.
#include <mutex>

#include "common.h"

// FP64 partials of morph_grad_accumulate_final_noalloc: a library-owned array
// instead of a caller workspace (8 MiB per GPU, held until the process ends).
// Host code never uses this name as an address: the per-device address comes
// from hipGetSymbolAddress (noalloc_partials below).
static __device__ __align__(256) double scratch[MORPH_NOALLOC_MAX_PARTIALS];

namespace morph {
namespace {

constexpr int kBlock = 256;
constexpr int kPerLane = 8;
constexpr int kPerBlock = kBlock * kPerLane;
static_assert(kPerBlock == MORPH_ACCUM_ELEMS_PER_BLOCK, "header and kernel disagree");
constexpr int kMaxTensors = 32;
constexpr int64_t kMaxSegment = int64_t(1) << 30;

struct TensorArg {
  const void* g;  // nullptr: no gradient in this micro-batch
  float* dst;
  int64_t n;
  int32_t first_block;
  int32_t vector_ok;
};

struct LaunchArgs {
  TensorArg t[kMaxTensors];
  int32_t count;
  uint32_t divide;  // scale is not a power of two
  float scale, inv_scale;
  int64_t partial_base;  // index of this launch's first partial
};
static_assert(sizeof(LaunchArgs) + 64 <= kMaxKernargBytes, "launch table fits the kernel arguments");

// Four consecutive gradient elements, read once: non-temporal.
template <typename GT>
__device__ __forceinline__ void load4(const void* g, int64_t e, float (&x)[4]) {
  if constexpr (std::is_same_v<GT, F32>) {
    const f32x4 t =
        load_stream<true>(reinterpret_cast<const f32x4*>(static_cast<const float*>(g) + e));
    x[0] = t.x; x[1] = t.y; x[2] = t.z; x[3] = t.w;
  } else {
    const u32x2 t =
        load_stream<true>(reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(g) + e));
    x[0] = to_float<GT>(t.x & 0xFFFFu); x[1] = to_float<GT>(t.x >> 16);
    x[2] = to_float<GT>(t.y & 0xFFFFu); x[3] = to_float<GT>(t.y >> 16);
  }
}

template <typename GT>
__device__ __forceinline__ float load1(const void* g, int64_t i) {
  if constexpr (std::is_same_v<GT, F32>) return static_cast<const float*>(g)[i];
  else return to_float<GT>(static_cast<const uint16_t*>(g)[i]);
}

__device__ __forceinline__ float unscale(float x, const LaunchArgs& a) {
  return a.divide ? x / a.scale : x * a.inv_scale;
}

// Fixed-order FP64 sum over the workgroup (butterfly in each wave, then the
// four wave totals in wave order); the result is valid in thread 0.
__device__ __forceinline__ double block_sum(double x, double* lds) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = x;
  __syncthreads();
  double s = 0.0;
  if (threadIdx.x == 0)
    for (int w = 0; w < kBlock / 64; ++w) s += lds[w];
  return s;
}

template <typename GT, bool kOverwrite, bool kFinal>
__global__ __launch_bounds__(kBlock) void accumulate_kernel(const LaunchArgs a,
                                                            uint32_t* __restrict__ found_inf,
                                                            double* __restrict__ partials) {
  __shared__ double lds[kBlock / 64];
  const int b = blockIdx.x;
  const TensorArg& T = a.t[segment_of(a.t, a.count, b)];
  const int64_t base = (int64_t)(b - T.first_block) * kPerBlock;
  const int tid = threadIdx.x;
  bool bad = false;
  double ss = 0.0;
  if (T.vector_ok && base + kPerBlock <= T.n) {
#pragma unroll
    for (int half = 0; half < kPerLane / 4; ++half) {
      const int64_t e = base + ((int64_t)half * kBlock + tid) * 4;
      float d[4];
      if (T.g != nullptr) {
        float x[4];
        load4<GT>(T.g, e, x);
        if constexpr (kOverwrite) {
#pragma unroll
          for (int k = 0; k < 4; ++k) d[k] = 0.0f + unscale(x[k], a);
        } else {
          const f32x4 p = *reinterpret_cast<const f32x4*>(T.dst + e);
          const float old[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
          for (int k = 0; k < 4; ++k) d[k] = old[k] + unscale(x[k], a);
        }
        *reinterpret_cast<f32x4*>(T.dst + e) = f32x4{d[0], d[1], d[2], d[3]};
      } else if constexpr (kOverwrite) {
#pragma unroll
        for (int k = 0; k < 4; ++k) d[k] = 0.0f;
        *reinterpret_cast<f32x4*>(T.dst + e) = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      } else {
        const f32x4 p = *reinterpret_cast<const f32x4*>(T.dst + e);
        d[0] = p.x; d[1] = p.y; d[2] = p.z; d[3] = p.w;
      }
      if constexpr (kFinal) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          bad |= nonfinite_f32_bits(__builtin_bit_cast(uint32_t, d[k]));
          ss += (double)d[k] * (double)d[k];
        }
      }
    }
  } else {
    // ragged tail or unaligned tensor: lane-strided, same per-lane order
    const int64_t end = base + kPerBlock < T.n ? base + kPerBlock : T.n;
    for (int64_t i = base + tid; i < end; i += kBlock) {
      float d;
      if (T.g != nullptr) {
        d = (kOverwrite ? 0.0f : T.dst[i]) + unscale(load1<GT>(T.g, i), a);
        T.dst[i] = d;
      } else if (kOverwrite) {
        d = 0.0f;
        T.dst[i] = d;
      } else {
        d = kFinal ? T.dst[i] : 0.0f;
      }
      if constexpr (kFinal) {
        bad |= nonfinite_f32_bits(__builtin_bit_cast(uint32_t, d));
        ss += (double)d * (double)d;
      }
    }
  }
  if constexpr (kFinal) {
    if (__builtin_amdgcn_ballot_w64(bad) != 0 && (tid & 63) == 0) {
      volatile uint32_t* f = found_inf;
      *f = 1u;  // every writer stores the same value
    }
    const double s = block_sum(ss, lds);
    if (tid == 0) partials[a.partial_base + b] = s;
  }
}

// out = (accumulate ? *out : 0) + sum of partials[0..n) in index order per
// lane, lanes combined by a fixed tree: deterministic for a given n.
__global__ __launch_bounds__(1024) void partial_sum_kernel(const double* __restrict__ partials,
                                                           int64_t n, double* out,
                                                           int accumulate) {
  __shared__ double lds[1024 / 64];
  double s = 0.0;
  // 8 loads in flight per lane, added in index order (the order does not change)
  int64_t i = threadIdx.x;
  for (; i + 7 * 1024 < n; i += 8 * 1024) {
    double v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = partials[i + k * 1024];
#pragma unroll
    for (int k = 0; k < 8; ++k) s += v[k];
  }
  for (; i < n; i += 1024) s += partials[i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < 1024 / 64; ++w) t += lds[w];
    *out = accumulate ? *out + t : t;
  }
}

template <typename GT>
int launch(int flags, const LaunchArgs& a, int blocks, uint32_t* flag, double* partials,
           hipStream_t s) {
  const bool ow = (flags & MORPH_ACCUM_OVERWRITE) != 0, fin = (flags & MORPH_ACCUM_FINAL) != 0;
  const dim3 grid(blocks), block(kBlock);
  if (ow && fin)
    hipLaunchKernelGGL((accumulate_kernel<GT, true, true>), grid, block, 0, s, a, flag, partials);
  else if (ow)
    hipLaunchKernelGGL((accumulate_kernel<GT, true, false>), grid, block, 0, s, a, flag, partials);
  else if (fin)
    hipLaunchKernelGGL((accumulate_kernel<GT, false, true>), grid, block, 0, s, a, flag, partials);
  else
    hipLaunchKernelGGL((accumulate_kernel<GT, false, false>), grid, block, 0, s, a, flag, partials);
  return launch_status();
}

int gbytes(int dtype) {
  switch (dtype) {
    case MORPH_DTYPE_F32: return 4;
    case MORPH_DTYPE_F16:
    case MORPH_DTYPE_BF16: return 2;
    default: return 0;
  }
}

bool pow2(double x) {
  const uint64_t b = __builtin_bit_cast(uint64_t, x);
  const uint32_t e = (uint32_t)(b >> 52) & 0x7FFu;
  return (b >> 63) == 0 && e != 0 && e != 0x7FFu && (b & 0x000FFFFFFFFFFFFFull) == 0;
}

int64_t blocks_of(int64_t n) { return (n + kPerBlock - 1) / kPerBlock; }

}  // namespace
}  // namespace morph

using namespace morph;

extern "C" int64_t morph_grad_partials(const morph_accum_tensor* tensors, int count) {
  if (count < 0 || (count > 0 && tensors == nullptr)) return MORPH_EINVAL;
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    if (tensors[i].numel < 0) return MORPH_EINVAL;
    for (int64_t off = 0; off < tensors[i].numel; off += kMaxSegment)
      total += blocks_of(tensors[i].numel - off < kMaxSegment ? tensors[i].numel - off : kMaxSegment);
  }
  return total;
}

extern "C" int morph_grad_accumulate(const morph_accum_tensor* tensors, int count, int grad_dtype,
                                     double loss_scale, int flags, uint32_t* d_found_inf,
                                     double* d_partials, int64_t partials_len, void* stream) {
  const int gb = gbytes(grad_dtype);
  if (gb == 0) return MORPH_EDTYPE;
  if (flags & ~(MORPH_ACCUM_OVERWRITE | MORPH_ACCUM_FINAL)) return MORPH_EINVAL;
  if (!(loss_scale > 0.0) || !(loss_scale < 1e300)) return MORPH_EINVAL;  // also rejects NaN
  const int64_t need = morph_grad_partials(tensors, count);
  if (need < 0) return (int)need;
  for (int i = 0; i < count; ++i)
    if (tensors[i].numel > 0 && tensors[i].dst == nullptr) return MORPH_EINVAL;
  const bool fin = (flags & MORPH_ACCUM_FINAL) != 0;
  if (fin && (d_found_inf == nullptr || d_partials == nullptr)) return MORPH_EINVAL;
  if (fin && partials_len < need) return MORPH_EWORKSPACE;
  hipStream_t s = as_stream(stream);
  LaunchArgs a;
  a.divide = pow2(loss_scale) ? 0u : 1u;
  a.scale = (float)loss_scale;
  a.inv_scale = (float)(1.0 / loss_scale);
  a.count = 0;
  a.partial_base = 0;
  int blocks = 0;
  int64_t done = 0;
  auto flush = [&]() -> int {
    if (a.count == 0) return MORPH_OK;
    int rc;
    switch (grad_dtype) {
      case MORPH_DTYPE_F32: rc = launch<F32>(flags, a, blocks, d_found_inf, d_partials, s); break;
      case MORPH_DTYPE_F16: rc = launch<F16>(flags, a, blocks, d_found_inf, d_partials, s); break;
      default: rc = launch<BF16>(flags, a, blocks, d_found_inf, d_partials, s); break;
    }
    done += blocks;
    a.partial_base = done;
    a.count = 0;
    blocks = 0;
    return rc;
  };
  for (int i = 0; i < count; ++i) {
    const morph_accum_tensor& t = tensors[i];
    for (int64_t off = 0; off < t.numel; off += kMaxSegment) {
      const int64_t n = t.numel - off < kMaxSegment ? t.numel - off : kMaxSegment;
      if (a.count == kMaxTensors) {
        const int rc = flush();
        if (rc != MORPH_OK) return rc;
      }
      TensorArg& d = a.t[a.count++];
      d.g = t.grad ? static_cast<const char*>(t.grad) + off * gb : nullptr;
      d.dst = t.dst + off;
      d.n = n;
      d.first_block = blocks;
      // 16-byte accesses: two of the FP32 window per lane, one of 8 16-bit gradients
      // (two for FP32 gradients)
      d.vector_ok = (reinterpret_cast<uintptr_t>(d.dst) % 16 == 0) &&
                    (d.g == nullptr || reinterpret_cast<uintptr_t>(d.g) % 16 == 0);
      blocks += (int)blocks_of(n);
    }
  }
  return flush();
}

extern "C" int morph_sumsq_total(const double* d_partials, int64_t n, double* d_out, int accumulate,
                                 void* stream) {
  if (d_out == nullptr || n < 0 || (n > 0 && d_partials == nullptr)) return MORPH_EINVAL;
  hipLaunchKernelGGL(partial_sum_kernel, dim3(1), dim3(1024), 0, as_stream(stream), d_partials, n,
                     d_out, accumulate != 0 ? 1 : 0);
  return launch_status();
}

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
double* g_scratch[kMaxDevices];  // device address of `scratch` per GPU, set on first use

// The address of `scratch` on the GPU that `stream` belongs to (the current GPU
// for the legacy default stream), looked up once per GPU with that GPU current.
int noalloc_partials(hipStream_t stream, double** out) {
  int current = 0;
  if (hipGetDevice(&current) != hipSuccess) return MORPH_ELAUNCH;
  int dev = current;
  if (stream != nullptr) {
    hipDevice_t d = 0;
    if (hipStreamGetDevice(stream, &d) != hipSuccess) return MORPH_EINVAL;
    dev = d;
  }
  if (dev < 0 || dev >= kMaxDevices) return MORPH_ERANGE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    if (dev != current && hipSetDevice(dev) != hipSuccess) return MORPH_ELAUNCH;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != current) (void)hipSetDevice(current);
    if (e != hipSuccess || p == nullptr) return MORPH_ELAUNCH;
    g_scratch[dev] = static_cast<double*>(p);
  }
  *out = g_scratch[dev];
  return MORPH_OK;
}

}  // namespace

extern "C" int morph_grad_accumulate_final_noalloc(const morph_accum_tensor* tensors, int count,
                                                   int grad_dtype, double loss_scale, int flags,
                                                   uint32_t* d_found_inf, double* d_sumsq,
                                                   void* stream) {
  if (flags & ~MORPH_ACCUM_OVERWRITE) return MORPH_EINVAL;
  if (d_found_inf == nullptr || d_sumsq == nullptr) return MORPH_EINVAL;
  if (gbytes(grad_dtype) == 0) return MORPH_EDTYPE;
  const int64_t need = morph_grad_partials(tensors, count);
  if (need < 0) return (int)need;
  if (need > MORPH_NOALLOC_MAX_PARTIALS) return MORPH_ERANGE;
  double* partials = nullptr;
  int rc = noalloc_partials(as_stream(stream), &partials);
  if (rc != MORPH_OK) return rc;
  // every partial the sum reads is written by this call's pass: nothing to clear
  rc = morph_grad_accumulate(tensors, count, grad_dtype, loss_scale, flags | MORPH_ACCUM_FINAL,
                             d_found_inf, partials, MORPH_NOALLOC_MAX_PARTIALS, stream);
  if (rc != MORPH_OK) return rc;
  return morph_sumsq_total(partials, need, d_sumsq, 0, stream);
}
