// Fused mixed-precision AdamW step for gfx950 (MI355X).
//
// One pass over HBM per parameter: read grad (fp16/bf16/fp32), master, m, v;
// write master, m, v and the optional fp16/bf16 export copy.  That is 28 bytes
// per parameter for an fp16 grad with fp16 export, the algorithmic minimum.
//
// Arithmetic follows torch's _single_tensor_adam (torch/optim/adam.py:414-419,
// 457, 476, 528-547) and DiskState.update (streamtrain/disk.py:209-215) op for
// op; the host supplies each fp32 constant already rounded (morph_adamw_hp).
//
// Layout and launch shape.  A launch covers up to kMaxTensors tensors.  Each
// workgroup (kBlock lanes) owns one contiguous chunk of kPerBlock elements of
// one tensor; lane i moves 4 consecutive elements per access (one 128-bit load
// of each FP32 stream, one 64-bit load of a 16-bit grad), and consecutive
// lanes cover consecutive 16-byte pieces, so every wave-wide access is one
// contiguous 1 KiB (FP32) or 512 B (16-bit) segment.  All loads of a lane are
// issued before any arithmetic.  Measured on MI355X (config 2 window), small
// workgroups with one access per lane stream best: many short-lived
// workgroups keep every CU's memory pipeline full, while longer per-lane
// chains (unroll 2/4/8) or 1024-lane groups lose 3-7%; and fewer of them per
// CU at a time (16 waves, set by the launch's LDS reservation), with each
// lane's stream loads issued before the step's control words are read, are
// 0-6% faster than the hardware's own limit.  One-wave workgroups (64 x 1, 16
// per CU) beat two-wave ones (128 x 1, 8 per CU) by 1.5% (234.4-235.9 against
// 237.2-238.4 us, one variant per process, alternated on one box); 64 x 1 at
// 11, 13 or 20 per CU, 64 x 2 and 128 x 1 at 16 per CU were slower, uncapped
// 64 x 1 by 3%.  Chunks map to workgroups
// in address order; the dispatcher spreads consecutive workgroups round-robin
// over the 8 XCDs, which is what a pure stream with no reuse wants; a launch
// whose gradients do not fit the Infinity Cache runs its chunks in descending
// order (kReverseAboveBytes).
//
// Two launch forms share the kernel: host constants (morph_adamw_multi), and
// device-resident control (morph_adamw_multi_dev) where the loss scale, the
// skip decision and each tensor's step clock are read from HBM, so a training
// loop can enqueue steps without waiting for the previous outcome.
#include <hip/hip_ext.h>

#include "common.h"

#ifndef MORPH_ADAMW_UNROLL
#define MORPH_ADAMW_UNROLL 1
#endif
// The gradient is read with ordinary (temporal) loads: the detector that runs
// just before this kernel reads the same bytes with temporal loads too, which
// leaves them in the 256 MB Infinity Cache (MALL), so this kernel's gradient
// reads are served from there instead of HBM (measured: 261 -> 247 us on the
// config-2 window, whose 113 MB of FP16 gradients fit).
#ifndef MORPH_ADAMW_GRAD_NT
#define MORPH_ADAMW_GRAD_NT 0
#endif
#ifndef MORPH_ADAMW_BLOCK
#define MORPH_ADAMW_BLOCK 64
#endif
#ifndef MORPH_ADAMW_NT
#define MORPH_ADAMW_NT 1
#endif

namespace morph {
namespace {

constexpr int kBlock = MORPH_ADAMW_BLOCK;
constexpr int kUnroll = MORPH_ADAMW_UNROLL;
constexpr bool kNT = MORPH_ADAMW_NT != 0;
constexpr bool kGradNT = MORPH_ADAMW_GRAD_NT != 0;
// Chunk order.  The non-finite detector (or the final stage-gradient pass) that
// precedes this kernel walks the gradients in ascending address order and leaves
// what it touched last in the 256 MB Infinity Cache.  When a launch's gradients
// fit there, every gradient read hits it in either order and ascending order is
// the faster (config-2 window, 113 MB: 236.4 against 238.9 us median); when they
// do not, only the most recently scanned part is still cached, so the launch runs
// its chunks in descending order and reads that part before its own streams evict
// it (config-3 embedding, 402 MB of BF16 gradients: 902.5 -> 853.8 us median,
// round-robin in one process, identical bits).
constexpr int64_t kReverseAboveBytes = int64_t(256) << 20;
constexpr int kPerBlock = kBlock * 4 * kUnroll;
constexpr int kMaxTensors = 48;
constexpr int kMaxHp = 8;
// Residency cap: every workgroup reserves this much LDS, which it does not
// use, so at most 160 KiB / 10 KiB = 16 one-wave workgroups share a CU.  The
// stream runs faster with fewer waves in flight per CU, by an amount that
// depends on where the buffers sit in physical memory (measured with two-wave
// workgroups, config-2 window, round-robin against the uncapped kernel in one
// process: 0-15 us faster in most placements and up to 3 us slower in a few;
// 14 waves as fast, 12 slower and 10 far slower, 277 us).  The cap pays off
// with the loads issued before the control words (adamw_multi_kernel).
constexpr unsigned kOccupancyLds = 10 * 1024;
// A tensor is cut into segments of at most this many elements so block
// counts stay far inside the 32-bit grid limits.
constexpr int64_t kMaxSegment = int64_t(1) << 30;

struct TensorArg {
  const void* grad;
  float* p;
  float* m;
  float* v;
  void* out;
  int64_t n;
  int32_t hp;
  int32_t first_block;
  int32_t vector_ok;
  int32_t clock;
};

struct LaunchArgs {
  TensorArg t[kMaxTensors];
  morph_adamw_hp hp[kMaxHp];
  morph_adamw_sched sched[kMaxHp];  // device form only
  const int64_t* clocks;            // device form only
  const morph_step_state* state;    // device form only
  int32_t count;
  int32_t reverse;                  // chunks in descending order (see kReverseAboveBytes)
};
static_assert(sizeof(LaunchArgs) + 64 <= kMaxKernargBytes, "launch table fits the kernel arguments");

// Power of two (normal double): zero fraction field, finite, positive.
__device__ __forceinline__ bool pow2_double(double x) {
  const uint64_t b = __builtin_bit_cast(uint64_t, x);
  const uint32_t e = (uint32_t)(b >> 52) & 0x7FFu;
  return (b >> 63) == 0 && e != 0 && e != 0x7FFu && (b & 0x000FFFFFFFFFFFFFull) == 0;
}

__device__ __forceinline__ void adamw_update(float g, float& p, float& m, float& v,
                                             const morph_adamw_hp& hp) {
  const uint32_t fl = hp.flags;
  // Unscale: g / scale.  For scale = 2^k the product with 2^-k is the same
  // correctly rounded real number, so the cheaper multiply is bit-identical.
  g = (fl & MORPH_HP_DIVIDE_SCALE) ? g / hp.scale : g * hp.inv_scale;
  if (fl & MORPH_HP_APPLY_CLIP) g = g * hp.clip;
  if (fl & MORPH_HP_APPLY_DECAY) p = p * hp.decay;
  if (fl & MORPH_HP_LERP_LARGE)
    m = __fmaf_rn(hp.lerp_weight - 1.0f, g - m, g);
  else
    m = __fmaf_rn(hp.lerp_weight, g - m, m);
  v = __fmaf_rn(hp.one_minus_beta2 * g, g, v * hp.beta2);
  const float d = __builtin_sqrtf(v) / hp.bias_correction2_sqrt + hp.eps;
  p = p + (hp.neg_step_size * m) / d;
}

// ---- grad loads: 4 consecutive elements -----------------------------------
template <typename GT>
__device__ __forceinline__ void load_grad4(const void* g, int64_t e, float (&x)[4]);

template <>
__device__ __forceinline__ void load_grad4<F32>(const void* g, int64_t e, float (&x)[4]) {
  const f32x4 t = load_stream<kGradNT>(reinterpret_cast<const f32x4*>(static_cast<const float*>(g) + e));
  x[0] = t.x; x[1] = t.y; x[2] = t.z; x[3] = t.w;
}
template <typename H>
__device__ __forceinline__ void load_half4(const void* g, int64_t e, float (&x)[4]) {
  const u32x2 t = load_stream<kGradNT>(reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(g) + e));
  x[0] = to_float<H>(t.x & 0xFFFFu);
  x[1] = to_float<H>(t.x >> 16);
  x[2] = to_float<H>(t.y & 0xFFFFu);
  x[3] = to_float<H>(t.y >> 16);
}
template <>
__device__ __forceinline__ void load_grad4<F16>(const void* g, int64_t e, float (&x)[4]) { load_half4<F16>(g, e, x); }
template <>
__device__ __forceinline__ void load_grad4<BF16>(const void* g, int64_t e, float (&x)[4]) { load_half4<BF16>(g, e, x); }

template <typename GT>
__device__ __forceinline__ float load_grad1(const void* g, int64_t i) {
  if constexpr (std::is_same_v<GT, F32>) return static_cast<const float*>(g)[i];
  else return to_float<GT>(static_cast<const uint16_t*>(g)[i]);
}

// ---- export stores ----------------------------------------------------------
template <typename OT>
__device__ __forceinline__ void store_out4(void* out, int64_t e, const f32x4& p) {
  if constexpr (std::is_same_v<OT, NoOut>) {
    return;
  } else if constexpr (std::is_same_v<OT, F32>) {
    store_stream<kNT>(reinterpret_cast<f32x4*>(static_cast<float*>(out) + e), p);
  } else {
    u32x2 t;
    t.x = from_float<OT>(p.x) | (from_float<OT>(p.y) << 16);
    t.y = from_float<OT>(p.z) | (from_float<OT>(p.w) << 16);
    store_stream<kNT>(reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + e), t);
  }
}

template <typename OT>
__device__ __forceinline__ void store_out1(void* out, int64_t i, float p) {
  if constexpr (std::is_same_v<OT, NoOut>) {
    return;
  } else if constexpr (std::is_same_v<OT, F32>) {
    static_cast<float*>(out)[i] = p;
  } else {
    static_cast<uint16_t*>(out)[i] = (uint16_t)from_float<OT>(p);
  }
}

// One lane's share of a vector chunk, held between the loads and the update.
struct VecRegs {
  f32x4 P[kUnroll], M[kUnroll], V[kUnroll];
  float G[kUnroll][4];
};

template <typename GT>
__device__ __forceinline__ void load_vector(const TensorArg& T, int64_t base, VecRegs& r) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t e = base + (int64_t)(u * kBlock + tid) * 4;
    load_grad4<GT>(T.grad, e, r.G[u]);
    r.P[u] = load_stream<kNT>(reinterpret_cast<const f32x4*>(T.p + e));
    r.M[u] = load_stream<kNT>(reinterpret_cast<const f32x4*>(T.m + e));
    r.V[u] = load_stream<kNT>(reinterpret_cast<const f32x4*>(T.v + e));
  }
}

template <typename OT>
__device__ __forceinline__ void update_vector(const TensorArg& T, const morph_adamw_hp& hp,
                                              int64_t base, VecRegs& r) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float p = r.P[u][k], m = r.M[u][k], v = r.V[u][k];
      adamw_update(r.G[u][k], p, m, v, hp);
      r.P[u][k] = p; r.M[u][k] = m; r.V[u][k] = v;
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t e = base + (int64_t)(u * kBlock + tid) * 4;
    store_stream<kNT>(reinterpret_cast<f32x4*>(T.p + e), r.P[u]);
    store_stream<kNT>(reinterpret_cast<f32x4*>(T.m + e), r.M[u]);
    store_stream<kNT>(reinterpret_cast<f32x4*>(T.v + e), r.V[u]);
    if (T.out != nullptr) store_out4<OT>(T.out, e, r.P[u]);
  }
}

template <typename GT, typename OT>
__device__ __forceinline__ void chunk_scalar(const TensorArg& T, const morph_adamw_hp& hp,
                                             int64_t begin, int64_t end) {
  for (int64_t i = begin + threadIdx.x; i < end; i += kBlock) {
    float p = T.p[i], m = T.m[i], v = T.v[i];
    adamw_update(load_grad1<GT>(T.grad, i), p, m, v, hp);
    T.p[i] = p;
    T.m[i] = m;
    T.v[i] = v;
    if (T.out != nullptr) store_out1<OT>(T.out, i, p);
  }
}

// The step's constants for this workgroup's tensor, or false when the step
// must leave memory untouched (overflow flagged, fatal state, or a clock
// outside the tables).
template <bool kDev>
__device__ __forceinline__ bool control(const LaunchArgs& a, const TensorArg& T,
                                        const uint32_t* skip, morph_adamw_hp& hp) {
  hp = a.hp[T.hp];
  if constexpr (kDev) {
    // skip = &state->found_inf[slot], this step's flag word
    if ((*skip | a.state->fatal) != 0u) return false;
    // Step-dependent constants from device state, in the host's double arithmetic.
    const morph_adamw_sched& S = a.sched[T.hp];
    const int64_t t = a.clocks[T.clock] + 1;
    if (t < 1 || t > S.table_len) return false;  // host keeps clocks inside the tables
    const double scale = a.state->scale;
    hp.scale = (float)scale;
    hp.inv_scale = (float)(1.0 / scale);
    hp.flags = (hp.flags & ~MORPH_HP_DIVIDE_SCALE) | (pow2_double(scale) ? 0u : MORPH_HP_DIVIDE_SCALE);
    hp.bias_correction2_sqrt = S.bias_correction2_sqrt[t - 1];
    hp.neg_step_size = (float)(-(S.lr / S.bias_correction1[t - 1]));
  } else {
    if (skip != nullptr && *skip != 0u) return false;
  }
  return true;
}

template <typename GT, typename OT, bool kDev>
__global__ __launch_bounds__(kBlock) void adamw_multi_kernel(const LaunchArgs a,
                                                             const uint32_t* __restrict__ skip) {
  const int b = a.reverse ? (int)gridDim.x - 1 - (int)blockIdx.x : (int)blockIdx.x;
  const TensorArg& T = a.t[segment_of(a.t, a.count, b)];
  const int64_t base = (int64_t)(b - T.first_block) * kPerBlock;
  morph_adamw_hp hp;
  if (T.vector_ok && base + kPerBlock <= T.n) {
    // The streams are requested before the control words, so their latency
    // overlaps; a skipped step (control false) still writes nothing.
    VecRegs r;
    load_vector<GT>(T, base, r);
    if (!control<kDev>(a, T, skip, hp)) return;
    update_vector<OT>(T, hp, base, r);
  } else {
    if (!control<kDev>(a, T, skip, hp)) return;
    chunk_scalar<GT, OT>(T, hp, base, base + kPerBlock < T.n ? base + kPerBlock : T.n);
  }
}

// Events (nullable) are stamped by the dispatch itself (hipExtLaunchKernel):
// e0 with the kernel's start, e1 with its end, with no marker packets between
// this launch and its neighbours in the queue.
struct Stamps {
  hipEvent_t e0, e1;
};

template <typename K>
void launch_kernel(K kernel, int blocks, const LaunchArgs& a, const uint32_t* skip, hipStream_t s,
                   Stamps ev) {
  if (ev.e0 == nullptr && ev.e1 == nullptr)
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kBlock), kOccupancyLds, s, a, skip);
  else
    hipExtLaunchKernelGGL(kernel, dim3(blocks), dim3(kBlock), kOccupancyLds, s, ev.e0, ev.e1, 0u,
                          a, skip);
}

template <typename GT, typename OT>
int launch(bool dev, const LaunchArgs& a, int blocks, const uint32_t* skip, hipStream_t s,
           Stamps ev) {
  if (dev)
    launch_kernel(adamw_multi_kernel<GT, OT, true>, blocks, a, skip, s, ev);
  else
    launch_kernel(adamw_multi_kernel<GT, OT, false>, blocks, a, skip, s, ev);
  return launch_status();
}

template <typename GT>
int launch_out(bool dev, int out_dtype, const LaunchArgs& a, int blocks, const uint32_t* skip,
               hipStream_t s, Stamps ev) {
  switch (out_dtype) {
    case MORPH_DTYPE_NONE: return launch<GT, NoOut>(dev, a, blocks, skip, s, ev);
    case MORPH_DTYPE_F32: return launch<GT, F32>(dev, a, blocks, skip, s, ev);
    case MORPH_DTYPE_F16: return launch<GT, F16>(dev, a, blocks, skip, s, ev);
    case MORPH_DTYPE_BF16: return launch<GT, BF16>(dev, a, blocks, skip, s, ev);
    default: return MORPH_EDTYPE;
  }
}

int dispatch(bool dev, int grad_dtype, int out_dtype, const LaunchArgs& a, int blocks,
             const uint32_t* skip, hipStream_t s, Stamps ev) {
  switch (grad_dtype) {
    case MORPH_DTYPE_F32: return launch_out<F32>(dev, out_dtype, a, blocks, skip, s, ev);
    case MORPH_DTYPE_F16: return launch_out<F16>(dev, out_dtype, a, blocks, skip, s, ev);
    case MORPH_DTYPE_BF16: return launch_out<BF16>(dev, out_dtype, a, blocks, skip, s, ev);
    default: return MORPH_EDTYPE;
  }
}

int dtype_bytes(int dtype) {
  switch (dtype) {
    case MORPH_DTYPE_F32: return 4;
    case MORPH_DTYPE_F16:
    case MORPH_DTYPE_BF16: return 2;
    default: return 0;
  }
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Validates everything, then splits the tensor list into launches of at most
// kMaxTensors segments and kMaxHp constant sets.  `scheds`, `clocks` and
// `state` are non-null exactly for the device-resident form.  `stamps`: the
// first launch stamps e0 with its start, the last stamps e1 with its end.
int enqueue(const morph_adamw_tensor* tensors, int count, int grad_dtype, int out_dtype,
            const morph_adamw_hp* hps, const morph_adamw_sched* scheds, int n_hp,
            const int64_t* clocks, const morph_step_state* state, const uint32_t* d_skip,
            void* stream, Stamps stamps = Stamps{nullptr, nullptr}) {
  const bool dev = state != nullptr;
  if (count < 0 || (count > 0 && (tensors == nullptr || hps == nullptr)) || n_hp < 0)
    return MORPH_EINVAL;
  if (dev && (scheds == nullptr || clocks == nullptr)) return MORPH_EINVAL;
  const int gb = dtype_bytes(grad_dtype);
  if (gb == 0) return MORPH_EDTYPE;
  if (out_dtype != MORPH_DTYPE_NONE && dtype_bytes(out_dtype) == 0) return MORPH_EDTYPE;
  const int ob = out_dtype == MORPH_DTYPE_NONE ? 0 : dtype_bytes(out_dtype);
  for (int i = 0; i < count; ++i) {
    const morph_adamw_tensor& t = tensors[i];
    if (t.numel < 0 || t.hp_index < 0 || t.hp_index >= n_hp) return MORPH_EINVAL;
    if (t.numel > 0 && (t.grad == nullptr || t.param == nullptr || t.exp_avg == nullptr ||
                        t.exp_avg_sq == nullptr))
      return MORPH_EINVAL;
    if (dev && t.clock_index < 0) return MORPH_EINVAL;
  }
  if (dev)
    for (int k = 0; k < n_hp; ++k)
      if (scheds[k].table_len < 1 || scheds[k].bias_correction1 == nullptr ||
          scheds[k].bias_correction2_sqrt == nullptr)
        return MORPH_EINVAL;
  hipStream_t s = as_stream(stream);
  LaunchArgs a;
  a.clocks = clocks;
  a.state = state;
  int hp_src[kMaxHp];
  int blocks = 0;
  a.count = 0;
  int n_local_hp = 0;
  int64_t grad_bytes = 0;  // of the launch being filled
  bool first_launch = true;
  auto flush = [&](bool last) -> int {
    if (a.count == 0) return MORPH_OK;
    const Stamps ev{first_launch ? stamps.e0 : nullptr, last ? stamps.e1 : nullptr};
    first_launch = false;
    a.reverse = grad_bytes > kReverseAboveBytes ? 1 : 0;
    const int rc = dispatch(dev, grad_dtype, out_dtype, a, blocks, d_skip, s, ev);
    a.count = 0;
    n_local_hp = 0;
    blocks = 0;
    grad_bytes = 0;
    return rc;
  };
  for (int i = 0; i < count; ++i) {
    const morph_adamw_tensor& t = tensors[i];
    void* out = (out_dtype == MORPH_DTYPE_NONE) ? nullptr : t.out;
    for (int64_t off = 0; off < t.numel; off += kMaxSegment) {
      const int64_t n = t.numel - off < kMaxSegment ? t.numel - off : kMaxSegment;
      int local = -1;
      for (int k = 0; k < n_local_hp; ++k)
        if (hp_src[k] == t.hp_index) local = k;
      if (a.count == kMaxTensors || (local < 0 && n_local_hp == kMaxHp)) {
        const int rc = flush(false);
        if (rc != MORPH_OK) return rc;
        local = -1;
      }
      if (local < 0) {
        local = n_local_hp++;
        hp_src[local] = t.hp_index;
        a.hp[local] = hps[t.hp_index];
        if (dev) a.sched[local] = scheds[t.hp_index];
      }
      TensorArg& d = a.t[a.count++];
      d.grad = static_cast<const char*>(t.grad) + off * gb;
      d.p = t.param + off;
      d.m = t.exp_avg + off;
      d.v = t.exp_avg_sq + off;
      d.out = out ? static_cast<char*>(out) + off * ob : nullptr;
      d.n = n;
      d.hp = local;
      d.first_block = blocks;
      d.vector_ok = aligned(d.p, 16) && aligned(d.m, 16) && aligned(d.v, 16) &&
                    aligned(d.grad, 4 * gb) && (d.out == nullptr || aligned(d.out, 4 * ob));
      d.clock = dev ? t.clock_index : 0;
      blocks += (int)((n + kPerBlock - 1) / kPerBlock);
      grad_bytes += n * gb;
    }
  }
  return flush(true);
}

}  // namespace
}  // namespace morph

using namespace morph;

extern "C" int morph_adamw_multi(const morph_adamw_tensor* tensors, int count, int grad_dtype,
                                 int out_dtype, const morph_adamw_hp* hps, int n_hp,
                                 const uint32_t* d_skip, void* start_event, void* stop_event,
                                 void* stream) {
  return enqueue(tensors, count, grad_dtype, out_dtype, hps, nullptr, n_hp, nullptr, nullptr,
                 d_skip, stream,
                 Stamps{static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event)});
}

extern "C" int morph_adamw_multi_dev(const morph_adamw_tensor* tensors, int count, int grad_dtype,
                                     int out_dtype, const morph_adamw_hp* hps,
                                     const morph_adamw_sched* scheds, int n_hp,
                                     const int64_t* d_clocks, const morph_step_state* d_state,
                                     int slot, void* start_event, void* stop_event,
                                     void* stream) {
  if (d_state == nullptr || (slot != 0 && slot != 1)) return MORPH_EINVAL;
  return enqueue(tensors, count, grad_dtype, out_dtype, hps, scheds, n_hp, d_clocks, d_state,
                 &d_state->found_inf[slot], stream,
                 Stamps{static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event)});
}

extern "C" int morph_adamw_fused(const void* grad, int grad_dtype, float* param, float* exp_avg,
                                 float* exp_avg_sq, void* out, int out_dtype, int64_t n,
                                 const morph_adamw_hp* hp, const uint32_t* d_skip, void* stream) {
  if (hp == nullptr) return MORPH_EINVAL;
  morph_adamw_tensor t;
  t.grad = grad;
  t.param = param;
  t.exp_avg = exp_avg;
  t.exp_avg_sq = exp_avg_sq;
  t.out = out;
  t.numel = n;
  t.hp_index = 0;
  t.clock_index = 0;
  return morph_adamw_multi(&t, 1, grad_dtype, out_dtype, hp, 1, d_skip, nullptr, nullptr, stream);
}
