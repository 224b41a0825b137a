/*
 * morph_optim.h -- C ABI of the MI355X (gfx950) mixed-precision optimizer step.
 *
 * This is the boundary below MORPH's Python optimizer API.  The Python side
 * (morph_amd.optimizer / morph_amd.disk) keeps the reference signatures and
 * calls these entry points through ctypes; no torch type crosses the boundary.
 *
 * Conventions shared by every entry point:
 *   - Tensor pointers are device pointers owned by the caller (morph_host_copy
 *     alone takes host pointers).  The library allocates no device memory and
 *     keeps no state between calls, so calls are re-entrant from several host
 *     threads.  The exceptions are the library-owned partials array of
 *     morph_grad_accumulate_final_noalloc and the host thread pool of
 *     morph_host_copy (see there).
 *   - Work is enqueued asynchronously on `stream` (a hipStream_t passed as
 *     void*; NULL means the legacy default stream).  Ordering between calls
 *     comes only from the stream.
 *   - Return 0 (MORPH_OK) or a negative MORPH_E* code; morph_strerror()
 *     names it.  A negative return means nothing was enqueued.
 *
 * Reference interfaces replaced (paths relative to the MORPH repository):
 *   streamtrain/disk.py:203-223         DiskState.update chunk arithmetic
 *   streamtrain/state_cache.py:103-140  CachedDiskState.update (same arithmetic)
 *   streamtrain/optimizer.py:34-70      HybridMuonAdamW (Muon loop + AdamW group)
 *   streamtrain/optimizer.py:13-22      orthogonalize (Newton-Schulz quintic)
 *   streamtrain/optimizer.py:49-51      non-finite gradient gate
 *   streamtrain/disk.py:482-488         overflow detection that drives
 *                                       DynamicLossScale.overflow (precision.py:9-11)
 *   torch/optim/adam.py:347-547         _single_tensor_adam, the AdamW group's
 *                                       arithmetic (torch.optim.AdamW foreach=False)
 *   streamtrain/sparse_disk.py:82-108,  stage-gradient accumulation and the FP64
 *     136; disk.py:446-448, 466-468     norm pass
 *   streamtrain/disk.py:316-327         CPU cast of the weight row for the stage load
 *   streamtrain/export.py:32-34         FP16 encoding + range check of the export
 *   streamtrain/precision.py:24-37      block-scaled FP8 pack / unpack
 */
#ifndef MORPH_OPTIM_H
#define MORPH_OPTIM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MORPH_ABI_VERSION 9

/* Element types of gradient / export buffers. */
enum morph_dtype {
  MORPH_DTYPE_NONE = -1, /* no buffer (export disabled) */
  MORPH_DTYPE_F32 = 0,
  MORPH_DTYPE_F16 = 1,
  MORPH_DTYPE_BF16 = 2
};

enum morph_status {
  MORPH_OK = 0,
  MORPH_EINVAL = -1,    /* null pointer, negative size, bad count */
  MORPH_EDTYPE = -2,    /* unsupported dtype combination */
  MORPH_ELAUNCH = -3,   /* the HIP launch itself failed */
  MORPH_ERANGE = -4,    /* size exceeds what the entry point supports */
  MORPH_EWORKSPACE = -5 /* workspace missing or too small */
};

/*
 * Per-call AdamW constants.  Every field is computed on the host in double
 * precision exactly as the reference computes it and rounded once to fp32,
 * which is what torch's CPU kernels do with a Python scalar operand
 * (torch/optim/adam.py:416-419, 457, 476, 528-547; streamtrain/disk.py:210-214).
 *
 * Per element, in this order (matching torch CPU op by op):
 *   g  = grad / scale                 (or grad * inv_scale when scale is 2^k: identical bits)
 *   g  = g * clip                     if MORPH_HP_APPLY_CLIP            (disk.py:210)
 *   p  = p * decay                    if MORPH_HP_APPLY_DECAY           (adam.py:416-419)
 *   m  = fma(lerp_weight, g - m, m)   torch lerp, weight < 0.5          (adam.py:457)
 *      = fma(lerp_weight - 1, g - m, g)   if MORPH_HP_LERP_LARGE
 *   v  = v * beta2;  v = fma(one_minus_beta2 * g, g, v)   torch addcmul  (adam.py:476)
 *   d  = sqrt(v) / bias_correction2_sqrt + eps                           (adam.py:544)
 *   p  = p + (neg_step_size * m) / d  torch addcdiv                      (adam.py:547)
 *   out = round-to-nearest-even(p) to the export dtype (when out != NULL)
 */
typedef struct morph_adamw_hp {
  float scale;
  float inv_scale;
  float clip;
  float decay;
  float lerp_weight;
  float beta2;
  float one_minus_beta2;
  float bias_correction2_sqrt;
  float neg_step_size;
  float eps;
  uint32_t flags;
  uint32_t reserved;
} morph_adamw_hp;

#define MORPH_HP_DIVIDE_SCALE 1u /* scale is not a power of two: divide */
#define MORPH_HP_APPLY_CLIP 2u
#define MORPH_HP_APPLY_DECAY 4u /* weight_decay != 0 */
#define MORPH_HP_LERP_LARGE 8u  /* lerp_weight >= 0.5 */

/* One tensor of a multi-tensor AdamW launch. */
typedef struct morph_adamw_tensor {
  const void* grad;   /* grad_dtype elements */
  float* param;       /* FP32 master, updated in place */
  float* exp_avg;     /* FP32 first moment, in place */
  float* exp_avg_sq;  /* FP32 second moment, in place */
  void* out;          /* out_dtype export copy, or NULL */
  int64_t numel;
  int32_t hp_index;   /* index into the hps[] array of the call */
  int32_t clock_index; /* morph_adamw_multi_dev: index of this tensor's clock */
} morph_adamw_tensor;

/*
 * Device-resident step control, for steps enqueued without a host round trip.
 * Lives in device memory; the host initialises it once (a plain copy) and
 * reads it back only when it wants the outcome.
 *
 * scale/good_steps/growth_interval/scale_cap are DynamicLossScale's state
 * (streamtrain/precision.py:6-17) kept in double precision, so the device
 * sequence of scales is bit-identical to the host one.  found_inf[slot] is
 * the detector's output for a step in flight: steps alternate slots (the
 * host's step count & 1), so the close of step s can run inside step s+1's
 * detector launch (morph_nonfinite_or_close) while that launch ORs step
 * s+1's flag into the other word.  fatal is sticky: bit 0 = an overflow
 * happened at scale <= 1 (the reference raises FloatingPointError there).
 * While fatal is set every later step is a no-op, so the state the host
 * finds equals the reference's state at the point it would have raised.
 */
typedef struct morph_step_state {
  double scale;
  double scale_cap;
  int64_t good_steps;
  int64_t growth_interval;
  int64_t applied;        /* steps applied */
  int64_t skipped;        /* steps skipped on overflow */
  uint32_t found_inf[2];  /* per slot: written by the detector, consumed by the step's close */
  uint32_t fatal;
  uint32_t last_found_inf;
  uint32_t dynamic;       /* 1: DynamicLossScale state machine; 0: fixed scale */
  uint32_t reserved;
} morph_step_state;

#define MORPH_FATAL_MIN_SCALE 1u

/*
 * Per-constant-set schedule for morph_adamw_multi_dev.  The step-dependent
 * constants are looked up by the tensor's device clock t (1-based after the
 * increment):  neg_step_size = -(lr / bias_correction1[t-1]) in double, then
 * rounded to fp32 (adam.py:537-539 / disk.py:214); bias_correction2_sqrt =
 * bias_correction2_sqrt[t-1] (already fp32).  The tables are filled by the
 * host with the reference's own double expressions (1 - beta1 ** t, ...).
 * The host keeps every clock below table_len; a tensor whose clock is out of
 * range is left untouched by the kernel (no out-of-bounds table read).
 */
typedef struct morph_adamw_sched {
  double lr;
  const double* bias_correction1;      /* device, table_len entries */
  const float* bias_correction2_sqrt;  /* device, table_len entries */
  int64_t table_len;
} morph_adamw_sched;

int morph_abi_version(void);
const char* morph_strerror(int status);

/* Sets *d_flag = 0 with a one-thread kernel (safe inside stream capture). */
int morph_flag_clear(uint32_t* d_flag, void* stream);

/*
 * Non-finite detector.  Writes 1 to *d_flag if any of the n elements of
 * `grad` (dtype F32/F16/BF16) is +-inf or NaN; never writes 0, so several
 * calls OR into one flag.  Replaces the reference's non-finite decision:
 * optimizer.py:49-51 (torch.isfinite(p.grad).all()) and disk.py:466-468 +
 * 485 (math.isfinite of the FP64 gradient norm, which is non-finite exactly
 * when some gradient element is).
 */
int morph_nonfinite_or(const void* grad, int dtype, int64_t n, uint32_t* d_flag,
                       void* stream);
/* Same over `count` tensors of one dtype, in one launch. */
int morph_nonfinite_or_multi(const void* const* grads, const int64_t* numels, int count,
                             int dtype, uint32_t* d_flag, void* stream);

/*
 * Fused AdamW step over one tensor: unscale + clip + decoupled decay + m/v
 * update with bias correction + master update + optional FP16/BF16 export,
 * one pass over HBM (28 bytes/parameter for an FP16 grad with FP16 export).
 * If d_skip != NULL and *d_skip != 0 when the kernel runs, nothing is
 * written (the conditional skip of a step whose gradients overflowed).
 * Replaces disk.py:209-215 / state_cache.py:121-126 and the per-parameter
 * body of torch/optim/adam.py:347-547.
 */
int morph_adamw_fused(const void* grad, int grad_dtype, float* param, float* exp_avg,
                      float* exp_avg_sq, void* out, int out_dtype, int64_t n,
                      const morph_adamw_hp* hp, const uint32_t* d_skip, void* stream);

/*
 * Multi-tensor form: `count` tensors (any count; the library splits it
 * into launches of at most 48 tensors) sharing one grad and one export dtype.
 * Each tensor selects its constants by hp_index into hps[0..n_hp).  This is
 * the whole AdamW group of HybridMuonAdamW (optimizer.py:40, 62) or one
 * stage window in one launch.  start_event / stop_event: as for
 * morph_adamw_multi_dev (nullable; stamped by the dispatches themselves).
 */
int morph_adamw_multi(const morph_adamw_tensor* tensors, int count, int grad_dtype,
                      int out_dtype, const morph_adamw_hp* hps, int n_hp,
                      const uint32_t* d_skip, void* start_event, void* stop_event,
                      void* stream);

/*
 * Device-resident form of morph_adamw_multi.  Each tensor's step t is
 * d_clocks[clock_index] + 1; the unscale factor comes from d_state->scale; the
 * step is skipped when d_state->found_inf[slot] or d_state->fatal is set.  From
 * hps[] only the step-independent fields are used (clip, decay, lerp_weight,
 * beta2, one_minus_beta2, eps, flags minus MORPH_HP_DIVIDE_SCALE); scheds[]
 * parallels hps[].  Clocks are NOT advanced here: morph_step_end does that.
 * start_event / stop_event (nullable hipEvent_t, created by the caller): the
 * call's first kernel dispatch stamps start_event with its start and the last
 * stamps stop_event with its end (hipExtLaunchKernel), so a caller can time
 * the pass with no marker packets between it and its neighbours.
 */
int morph_adamw_multi_dev(const morph_adamw_tensor* tensors, int count, int grad_dtype,
                          int out_dtype, const morph_adamw_hp* hps,
                          const morph_adamw_sched* scheds, int n_hp, const int64_t* d_clocks,
                          const morph_step_state* d_state, int slot, void* start_event,
                          void* stop_event, void* stream);

/*
 * Closes a device-resident step (one workgroup): on overflow (found_inf[slot])
 * counts a skip and, when `dynamic`, applies DynamicLossScale.overflow (or sets
 * fatal bit 0 at scale <= 1); else counts the step, applies success() when
 * `dynamic`, and advances the clocks d_clocks[d_clock_list[0..n)] (indices must
 * be distinct).  Then records found_inf[slot] in last_found_inf and clears it.
 * No-op while fatal is set.  Must run after the step's AdamW launch and before
 * the next step's (stream order).  Replaces DynamicLossScale.overflow/success
 * (precision.py:6-17, called at disk.py:483-496) and the conditional clock
 * advance of sparse_disk.py:122-138.
 */
int morph_step_end(morph_step_state* d_state, int64_t* d_clocks, const int32_t* d_clock_list,
                   int n, int slot, void* stream);

/*
 * One launch that closes the previous step and runs this step's detector:
 * morph_nonfinite_or_multi over `grads` into d_state->found_inf[slot], and in
 * one extra workgroup morph_step_end(d_state, d_clocks, d_prev_clock_list,
 * n_prev, slot ^ 1).  The two touch disjoint words (the close reads and clears
 * only found_inf[slot ^ 1]), so their workgroups may run in any order.  This
 * saves the close's own launch on every step that runs the detector.
 * Replaces, per step, the reference's non-finite decision (optimizer.py:49-51;
 * disk.py:466-468, 485) and the previous step's DynamicLossScale update
 * (precision.py:6-17, called at disk.py:483-496) with its clock advance
 * (sparse_disk.py:122-138).
 */
int morph_nonfinite_or_close(const void* const* grads, const int64_t* numels, int count,
                             int dtype, morph_step_state* d_state, int slot, int64_t* d_clocks,
                             const int32_t* d_prev_clock_list, int n_prev, void* stream);

/* ---- Stage-gradient accumulation ------------------------------------------
 * Replaces the reference's per-micro-batch
 *   destination.add_(g.detach().float() / loss_scale)
 * into the zeroed FP32 stage window (streamtrain/sparse_disk.py:82-87,
 * 104-108; disk.py:446-448) and its norm pass
 *   norm_squared += piece.double().square().sum().item()
 * (disk.py:466-468; sparse_disk.py:136), whose finiteness is the skip / retry
 * decision (disk.py:485) and whose value sets the clip (disk.py:489).
 */
#define MORPH_ACCUM_ELEMS_PER_BLOCK 2048 /* elements per workgroup = per FP64 partial */
#define MORPH_ACCUM_OVERWRITE 1 /* first micro-batch: dst = 0 + x (zero_() then add_()) */
#define MORPH_ACCUM_FINAL 2     /* also OR the non-finite flag of dst and write FP64 partials */

typedef struct morph_accum_tensor {
  const void* grad; /* this micro-batch's gradient (grad_dtype), contiguous; NULL = none */
  float* dst;       /* FP32 accumulation window for the same parameter */
  int64_t numel;
} morph_accum_tensor;

/* Number of FP64 partials a MORPH_ACCUM_FINAL call over these tensors writes
 * (one per MORPH_ACCUM_ELEMS_PER_BLOCK elements of each tensor). */
int64_t morph_grad_partials(const morph_accum_tensor* tensors, int count);

/* dst = (OVERWRITE ? 0 : dst) + fp32(grad) / loss_scale, elementwise, for
 * every tensor (a NULL grad adds nothing).  The division is a multiply by
 * 2^-k when loss_scale = 2^k (the same bits) and an IEEE division otherwise.
 * With MORPH_ACCUM_FINAL the same pass ORs 1 into *d_found_inf when any
 * resulting dst element is inf or NaN, and writes sum((double)dst^2) per
 * workgroup into d_partials[0 .. morph_grad_partials()) for morph_sumsq_total. */
int morph_grad_accumulate(const morph_accum_tensor* tensors, int count, int grad_dtype,
                          double loss_scale, int flags, uint32_t* d_found_inf, double* d_partials,
                          int64_t partials_len, void* stream);

/* *d_out = (accumulate ? *d_out : 0) + sum of d_partials[0 .. n), in a fixed
 * order (deterministic for a given n). */
int morph_sumsq_total(const double* d_partials, int64_t n, double* d_out, int accumulate,
                      void* stream);

/*
 * Allocation-free final pass.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Equals
 * morph_grad_accumulate(..., flags | MORPH_ACCUM_FINAL, d_found_inf, partials,
 * ...) followed by morph_sumsq_total(partials, n, d_sumsq, 0, ...), with the
 * FP64 partials in a library-owned device array of MORPH_NOALLOC_MAX_PARTIALS
 * doubles (8 MiB on each GPU it runs on, held until the process ends) instead
 * of a caller workspace.  flags: 0 or MORPH_ACCUM_OVERWRITE.  *d_sumsq is
 * overwritten; d_found_inf is ORed into.  Calls needing more partials than
 * the maximum (morph_grad_partials > 2^20, i.e. more than 2^31 elements)
 * return MORPH_ERANGE.  Calls no allocating routine.  Every call on one GPU
 * uses that GPU's array and leaves its partials there: calls that can overlap
 * on one GPU (streams not ordered with each other) race, so the caller
 * serialises them.
 */
#define MORPH_NOALLOC_MAX_PARTIALS (1 << 20)
int morph_grad_accumulate_final_noalloc(const morph_accum_tensor* tensors, int count,
                                        int grad_dtype, double loss_scale, int flags,
                                        uint32_t* d_found_inf, double* d_sumsq, void* stream);

/* ---- Master-weight conversion --------------------------------------------
 * dst = dtype(src) elementwise (FP16: round to nearest even, overflow -> inf;
 * BF16: round to nearest even, NaN -> 0x7FC0; FP32: copy).  Replaces the CPU
 * cast of the FP32 weight row before the stage's H2D copy
 * (streamtrain/disk.py:316-327) and the FP16 encoding of the export
 * (streamtrain/export.py:32-34).  d_range_flag (nullable): OR 1 when some
 * source value is inf / NaN or, for FP16 output, |value| > 65504 -- the
 * export's "cannot be represented by finite FP16" condition. */
int morph_convert_f32(const float* src, void* dst, int dst_dtype, int64_t n,
                      uint32_t* d_range_flag, void* stream);

/* ---- Block-scaled FP8 (E4M3FN) transport ---------------------------------
 * streamtrain/precision.py:24-37 (pack_fp8 / unpack_fp8), the opt-in FP8
 * weight transfer of disk.py:330-345.  Blocks of MORPH_FP8_BLOCK elements,
 * the last one padded with zeros for the amax only. */
#define MORPH_FP8_BLOCK 256

/* scales[b] = max(amax(|src block b|) / 448, 1e-30) (NaN if the block holds a
 * NaN); bytes[i] = e4m3fn(clamp(src[i] / scale, -448, 448)), round to nearest
 * even.  bytes: n entries; scales: ceil(n / 256) entries.  A block with a NaN
 * or an infinity gets the bytes of the reference's x86 CPU ops: 0x7F for every
 * non-NaN element of a NaN block and a NaN element's own NaN code (sign kept);
 * in a block with an infinity +-0 for finite elements and 0xFF for +-inf. */
int morph_fp8_pack(const void* src, int src_dtype, int64_t n, uint8_t* bytes, float* scales,
                   void* stream);
/* dst[i] = dst_dtype(float(e4m3fn bytes[i]) * scales[i / 256]). */
int morph_fp8_unpack(const uint8_t* bytes, const float* scales, int64_t n, void* dst, int dst_dtype,
                     void* stream);

/* ---- Hybrid Muon: Newton-Schulz orthogonalisation on bf16 MFMA ---------- */

/* Tile of morph_gemm_nt_bf16: M and N must be multiples of 256, K of 64. */
#define MORPH_GEMM_TILE_M 256
#define MORPH_GEMM_TILE_N 256
#define MORPH_GEMM_TILE_K 64

/* Flags of morph_gemm_nt_bf16. */
#define MORPH_GEMM_SYMMETRIC 1 /* C symmetric: compute the upper triangle of tiles, mirror */
#define MORPH_GEMM_Q_KN 2      /* Q stored [K, N] (ldq >= N): C = alpha P Q + beta D */

/*
 * Batched bf16 GEMM, "NT" layout, fp32 accumulation:
 *   C[b] = alpha * P[b] . Q[b]^T + beta * D[b];   Ct[b] = C[b]^T if Ct != NULL
 * P [M, K], Q [N, K], D/C [M, N], Ct [N, M], all row-major bf16 (uint16 bits)
 * with leading dimensions ld* and batch strides stride_* in elements; b < batch.
 * D may be NULL (beta ignored) and may alias C.  Each output element is
 * rounded once (RNE) from fp32.  The three products of one Newton-Schulz
 * iteration of optimizer.py:19-21 are all of this form (see gemm.hip).
 * flags: MORPH_GEMM_SYMMETRIC (requires M == N, Ct == NULL, and D symmetric
 * if given): C is known to be symmetric, so only the upper triangle of tiles
 * is computed and each off-diagonal tile is mirrored.  MORPH_GEMM_Q_KN: Q is
 * stored [K, N] (ldq >= N) and the product is P . Q (not with SYMMETRIC).
 * C must not overlap P or Q.  Pointers 16-byte aligned, leading dimensions
 * and strides multiples of 8, at most 2^23; MORPH_ERANGE when a dimension is
 * not a tile multiple.
 */
int morph_gemm_nt_bf16(const uint16_t* P, const uint16_t* Q, const uint16_t* D, uint16_t* C,
                       uint16_t* Ct, int64_t M, int64_t N, int64_t K, int64_t batch,
                       int64_t ldp, int64_t ldq, int64_t ldd, int64_t ldc, int64_t ldct,
                       int64_t stride_p, int64_t stride_q, int64_t stride_d, int64_t stride_c,
                       int64_t stride_ct, float alpha, float beta, int flags, void* stream);

/*
 * One Muon matrix: FP32 row-major device buffers of shape [rows, cols], or
 * [cols, rows] when `transposed` is 1.  Both orientations have the same
 * Newton-Schulz operand (optimizer.py:15-17 transposes the taller one), so one
 * batch can hold both, e.g. a SwiGLU block's [6144, 3072] and [3072, 6144]
 * weights.
 */
typedef struct morph_muon_matrix {
  const float* grad;
  float* momentum; /* updated in place (unused by morph_muon_orthogonalize) */
  float* param;    /* FP32 master, updated in place (the output of morph_muon_orthogonalize) */
  int32_t transposed; /* 0 or 1 */
  int32_t reserved;   /* 0 */
  /* NULL, or a separate buffer of the momentum's shape: the updated momentum
   * is written there and `momentum` is only read (see morph_muon_prepare) */
  float* momentum_out;
} morph_muon_matrix;

/*
 * Constants of one Muon step (streamtrain/optimizer.py:52-61), fp32 values of
 * the reference's Python scalars: momentum_weight = .05 (lerp_(g, .05)),
 * nesterov_weight = .95 (g.lerp(m, .95)), a/b/c = 3.4445, -4.775, 2.0315,
 * update_scale = sqrt(max(1, rows/cols)) for matrices stored [rows, cols] and
 * update_scale_transposed = sqrt(max(1, cols/rows)) for those stored
 * [cols, rows], decay = 1 - lr * weight_decay, neg_lr = -lr; ns_steps = 5.
 */
typedef struct morph_muon_hp {
  float momentum_weight;
  float nesterov_weight;
  float a, b, c;
  float update_scale;
  float decay;
  float neg_lr;
  int32_t ns_steps;
  float update_scale_transposed;
} morph_muon_hp;

/* Workspace bytes morph_muon_step needs for `count` matrices of [rows, cols] (either orientation). */
size_t morph_muon_workspace_bytes(int64_t rows, int64_t cols, int count);

/*
 * One Muon step for `count` (<= 64) matrices of one shape (in either
 * orientation), batched: momentum and Nesterov blend (fp32, torch's rounding),
 * Frobenius normalisation, ns_steps Newton-Schulz iterations in bf16 on MFMA
 * (A = X X^T, B' = b A + c A A + a I, X = B' X, fp32 accumulation), and the fp32
 * master update p = p * decay + (U * scale) * neg_lr with U in p's layout
 * (transposed back when p has more rows than columns, optimizer.py:15-17, 22)
 * and scale = update_scale or update_scale_transposed by the matrix's
 * orientation.  The workspace must be
 * 256-byte aligned; its contents need no initialisation (every call writes
 * what it reads, zero padding included, so a call on non-finite values leaves
 * nothing behind).  Replaces optimizer.py:13-22 and 52-61.
 */
int morph_muon_step(const morph_muon_matrix* mats, int count, int64_t rows, int64_t cols,
                    const morph_muon_hp* hp, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * orthogonalize(grad) alone (optimizer.py:13-22): param <- NS(grad / (|grad| + 1e-7))
 * as fp32 values of the bf16 result; momentum, update_scale, decay and neg_lr unused.
 */
int morph_muon_orthogonalize(const morph_muon_matrix* mats, int count, int64_t rows,
                             int64_t cols, const morph_muon_hp* hp, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * The three phases morph_muon_step / morph_muon_orthogonalize run, for callers
 * that interleave other work or time the Newton-Schulz GEMM chain on its own:
 * prepare (momentum + Nesterov, or u = grad when orthogonalize_only; X0 =
 * bf16(u) in the Newton-Schulz orientation and den = |u|_F + 1e-7 into the
 * workspace), newton_schulz (hp->ns_steps iterations, 3 GEMMs each, on the
 * workspace only; the first iteration's products apply 1 / den), finish
 * (master update, or U into param when orthogonalize_only).  Same arguments
 * and workspace throughout (with hp->ns_steps == 0 prepare itself writes
 * X = bf16(X0 / den), so the phases must see the same hp).
 * prepare with d_found_inf != NULL also tests every gradient for +-inf/NaN
 * in the same pass and stores 1 there if one is found (the gate of
 * optimizer.py:49-51); with each matrix's momentum_out set it then mutates
 * nothing the caller keeps, so the caller can read the flag and drop the
 * step before newton_schulz and finish (the updated momentum is in
 * momentum_out: swap the buffers after finish).
 */
int morph_muon_prepare(const morph_muon_matrix* mats, int count, int64_t rows, int64_t cols,
                       const morph_muon_hp* hp, int orthogonalize_only, void* workspace,
                       size_t workspace_bytes, uint32_t* d_found_inf, void* stream);
int morph_muon_newton_schulz(int count, int64_t rows, int64_t cols, const morph_muon_hp* hp,
                             void* workspace, size_t workspace_bytes, void* stream);
int morph_muon_finish(const morph_muon_matrix* mats, int count, int64_t rows, int64_t cols,
                      const morph_muon_hp* hp, int orthogonalize_only, void* workspace,
                      size_t workspace_bytes, void* stream);
/*
 * finish for matrices first .. first + n - 1 of the batch only (mats and count
 * as given to prepare): a caller that stages the parameters in and out of
 * device memory can update each matrix as soon as it has arrived and send it
 * back while the next ones arrive.  Calls over disjoint ranges that together
 * cover the batch equal one morph_muon_finish.  0 <= first, 0 <= n,
 * first + n <= count.
 */
int morph_muon_finish_range(const morph_muon_matrix* mats, int count, int64_t rows, int64_t cols,
                            const morph_muon_hp* hp, int orthogonalize_only, int first, int n,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * morph_muon_newton_schulz followed by morph_muon_finish (the master update,
 * not orthogonalize_only), after morph_muon_prepare, with the same bits.  When
 * the batch's operand has no padding (min(rows, cols) and max(rows, cols)
 * multiples of 256) and every param is 16-byte aligned, the last product
 * X' = B' X updates the parameters in its epilogue instead of storing X' (the
 * update runs while other tiles still compute, and the finish pass's reads of
 * X and p become the epilogue's reads of p); the last iteration's X is then not
 * written to the workspace.  Otherwise the two phases run as they are.
 * morph_muon_step uses it.  Replaces optimizer.py:19-22 and 60-61 for a batch.
 */
int morph_muon_newton_schulz_finish(const morph_muon_matrix* mats, int count, int64_t rows,
                                    int64_t cols, const morph_muon_hp* hp, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* ---- Host staging copy ---------------------------------------------------
 * dst[0, bytes) <- src[0, bytes) on the host, split over up to `threads`
 * threads (1..64) of a pool the library keeps; the calling thread copies
 * pieces too and the call returns when the copy is complete.  Host memory
 * only, no GPU work: the staging of pageable host tensors (masters, gradients)
 * through pinned buffers.  Its workers sleep when idle, so unlike an
 * intra-op pool spinning on every core they leave cores to the HIP runtime
 * while DMAs are in flight.  No counterpart in the reference, whose
 * optimizer updates the CPU tensors in place (streamtrain/optimizer.py:47-62).
 * MORPH_EINVAL for null pointers with bytes > 0, threads < 1 or overlapping
 * ranges; MORPH_ERANGE for threads > 64.  Calls are serialized.
 */
int morph_host_copy(void* dst, const void* src, size_t bytes, int threads);

#ifdef __cplusplus
}
#endif

#endif /* MORPH_OPTIM_H */
