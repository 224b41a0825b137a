// Non-finite / overflow detector for gfx950.
//
// Reads each gradient once (2 bytes/parameter for fp16/bf16) and sets a
// device flag when any element is +-inf or NaN.  The decision is a pure
// function of the exponent bits, so it is exact, and equals the reference's
// tests: torch.isfinite(p.grad).all() (streamtrain/optimizer.py:49-51) and
// math.isfinite(sqrt(sum(g.double()**2))) (streamtrain/disk.py:466-468, 485),
// which is non-finite exactly when some element is.
//
// Each lane loads 16 bytes per access (8 fp16/bf16 or 4 fp32), kUnroll
// accesses before testing, with temporal loads (see MORPH_NONFINITE_NT); a wave reduces its lanes with a ballot and one lane
// writes 1 to the flag with a plain vector store (every writer writes the
// same value, so the race is benign).  Nothing is ever written on a clean
// pass, so detector calls over several tensors OR into one flag.
//
// morph_nonfinite_or_close adds one workgroup (the first) that closes the
// previous optimizer step (close_step), which saves that close its own launch.  It reads and clears only the other step's flag word, so the
// detector workgroups and the close may run in any order.
#include "common.h"
#include "step_close.h"

#ifndef MORPH_NONFINITE_UNROLL
#define MORPH_NONFINITE_UNROLL 4
#endif
// Temporal loads on purpose: the fused AdamW pass re-reads these gradients
// right after, and leaving them in the Infinity Cache (MALL) takes that
// re-read off HBM, so detector + AdamW move 28 bytes/parameter of HBM traffic.
#ifndef MORPH_NONFINITE_NT
#define MORPH_NONFINITE_NT 0
#endif

namespace morph {
namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = MORPH_NONFINITE_UNROLL;
constexpr int kBytesPerBlock = kBlock * 16 * kUnroll;
constexpr int kMaxTensors = 160;
constexpr int64_t kMaxSegmentBytes = int64_t(1) << 32;

struct TensorArg {
  const void* g;
  int64_t n;  // elements
  int32_t first_block;
  int32_t vector_ok;
};

struct LaunchArgs {
  TensorArg t[kMaxTensors];
  int32_t count;
};
static_assert(sizeof(LaunchArgs) + 64 <= kMaxKernargBytes, "launch table fits the kernel arguments");

template <typename GT>
__device__ __forceinline__ bool word_nonfinite(uint32_t x) {
  if constexpr (std::is_same_v<GT, F32>) return nonfinite_f32_bits(x);
  else if constexpr (std::is_same_v<GT, F16>) return nonfinite_f16x2(x);
  else return nonfinite_bf16x2(x);
}

template <typename GT>
__device__ __forceinline__ bool elem_nonfinite(const void* g, int64_t i) {
  if constexpr (std::is_same_v<GT, F32>)
    return nonfinite_f32_bits(static_cast<const uint32_t*>(g)[i]);
  else
    return word_nonfinite<GT>(static_cast<const uint16_t*>(g)[i]);
}

// The previous step's close, carried by the detector launch of the next one.
struct CloseArgs {
  morph_step_state* state;
  int64_t* clocks;
  const int32_t* list;
  int32_t n;
  int32_t slot;
};

template <typename GT, bool kClose>
__global__ __launch_bounds__(kBlock) void nonfinite_kernel(const LaunchArgs a,
                                                           uint32_t* __restrict__ flag,
                                                           const CloseArgs c) {
  constexpr int kElemBytes = Fmt<GT>::bytes;
  constexpr int kPerBlock = kBytesPerBlock / kElemBytes;
  int b = blockIdx.x;
  if constexpr (kClose) {
    // Workgroup 0 closes the previous step: dispatched first, its chain of
    // dependent accesses runs under the scan instead of after it.
    if (b == 0) {
      close_step(c.state, c.clocks, c.list, c.n, c.slot, kBlock);
      return;
    }
    b -= 1;
  }
  const TensorArg& T = a.t[segment_of(a.t, a.count, b)];
  const int64_t base = (int64_t)(b - T.first_block) * kPerBlock;
  bool bad = false;
  if (T.vector_ok && base + kPerBlock <= T.n) {
    const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const char*>(T.g) +
                                                    base * kElemBytes);
    u32x4 w[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      w[u] = load_stream<MORPH_NONFINITE_NT != 0>(p + u * kBlock + threadIdx.x);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      bad |= word_nonfinite<GT>(w[u].x) | word_nonfinite<GT>(w[u].y) |
             word_nonfinite<GT>(w[u].z) | word_nonfinite<GT>(w[u].w);
  } else {
    const int64_t end = base + kPerBlock < T.n ? base + kPerBlock : T.n;
    for (int64_t i = base + threadIdx.x; i < end; i += kBlock) bad |= elem_nonfinite<GT>(T.g, i);
  }
  if (__any(bad) && (threadIdx.x & 63) == 0) *reinterpret_cast<volatile uint32_t*>(flag) = 1u;
}

template <typename GT>
int launch(const LaunchArgs& a, int blocks, uint32_t* flag, const CloseArgs* close,
           hipStream_t s) {
  if (close != nullptr)
    hipLaunchKernelGGL((nonfinite_kernel<GT, true>), dim3(blocks + 1), dim3(kBlock), 0, s, a,
                       flag, *close);
  else
    hipLaunchKernelGGL((nonfinite_kernel<GT, false>), dim3(blocks), dim3(kBlock), 0, s, a, flag,
                       CloseArgs{});
  return launch_status();
}

// `close` (nullable) rides in this launch as one extra workgroup.
int dispatch(int dtype, const LaunchArgs& a, int blocks, uint32_t* flag, const CloseArgs* close,
             hipStream_t s) {
  switch (dtype) {
    case MORPH_DTYPE_F32: return launch<F32>(a, blocks, flag, close, s);
    case MORPH_DTYPE_F16: return launch<F16>(a, blocks, flag, close, s);
    case MORPH_DTYPE_BF16: return launch<BF16>(a, blocks, flag, close, s);
    default: return MORPH_EDTYPE;
  }
}

__global__ void flag_clear_kernel(uint32_t* flag) {
  if (threadIdx.x == 0) *reinterpret_cast<volatile uint32_t*>(flag) = 0u;
}

}  // namespace
}  // namespace morph

using namespace morph;

extern "C" int morph_flag_clear(uint32_t* d_flag, void* stream) {
  if (d_flag == nullptr) return MORPH_EINVAL;
  hipLaunchKernelGGL(flag_clear_kernel, dim3(1), dim3(64), 0, as_stream(stream), d_flag);
  return launch_status();
}

namespace {

// Detector over `count` tensors into d_flag; `close` (nullable) rides in the
// first launch (or in a launch of its own when there is nothing to scan).
int nonfinite_impl(const void* const* grads, const int64_t* numels, int count, int dtype,
                   uint32_t* d_flag, const CloseArgs* close, hipStream_t s) {
  int eb;
  switch (dtype) {
    case MORPH_DTYPE_F32: eb = 4; break;
    case MORPH_DTYPE_F16:
    case MORPH_DTYPE_BF16: eb = 2; break;
    default: return MORPH_EDTYPE;
  }
  for (int i = 0; i < count; ++i)
    if (numels[i] < 0 || (numels[i] > 0 && grads[i] == nullptr)) return MORPH_EINVAL;
  const int per_block = kBytesPerBlock / eb;
  const int64_t max_seg = kMaxSegmentBytes / eb;
  LaunchArgs a;
  a.count = 0;
  int blocks = 0;
  for (int i = 0; i < count; ++i) {
    for (int64_t off = 0; off < numels[i]; off += max_seg) {
      if (a.count == kMaxTensors) {
        const int rc = dispatch(dtype, a, blocks, d_flag, close, s);
        if (rc != MORPH_OK) return rc;
        close = nullptr;
        a.count = 0;
        blocks = 0;
      }
      const int64_t n = numels[i] - off < max_seg ? numels[i] - off : max_seg;
      TensorArg& d = a.t[a.count++];
      d.g = static_cast<const char*>(grads[i]) + off * eb;
      d.n = n;
      d.first_block = blocks;
      d.vector_ok = (reinterpret_cast<uintptr_t>(d.g) % 16) == 0;
      blocks += (int)((n + per_block - 1) / per_block);
    }
  }
  if (a.count == 0 && close == nullptr) return MORPH_OK;
  return dispatch(dtype, a, blocks, d_flag, close, s);
}

}  // namespace

extern "C" int morph_nonfinite_or_multi(const void* const* grads, const int64_t* numels, int count,
                                        int dtype, uint32_t* d_flag, void* stream) {
  if (d_flag == nullptr || count < 0 || (count > 0 && (grads == nullptr || numels == nullptr)))
    return MORPH_EINVAL;
  return nonfinite_impl(grads, numels, count, dtype, d_flag, nullptr, as_stream(stream));
}

extern "C" int morph_nonfinite_or_close(const void* const* grads, const int64_t* numels, int count,
                                        int dtype, morph_step_state* d_state, int slot,
                                        int64_t* d_clocks, const int32_t* d_prev_clock_list,
                                        int n_prev, void* stream) {
  if (d_state == nullptr || count < 0 || (count > 0 && (grads == nullptr || numels == nullptr)) ||
      (slot != 0 && slot != 1) || n_prev < 0 ||
      (n_prev > 0 && (d_clocks == nullptr || d_prev_clock_list == nullptr)))
    return MORPH_EINVAL;
  const CloseArgs close{d_state, d_clocks, d_prev_clock_list, n_prev, slot ^ 1};
  return nonfinite_impl(grads, numels, count, dtype, &d_state->found_inf[slot], &close,
                        as_stream(stream));
}

extern "C" int morph_nonfinite_or(const void* grad, int dtype, int64_t n, uint32_t* d_flag,
                                  void* stream) {
  return morph_nonfinite_or_multi(&grad, &n, 1, dtype, d_flag, stream);
}
