// The close of one device-resident optimizer step: DynamicLossScale's state
// machine (streamtrain/precision.py:6-17) and the per-tensor step clocks.
//
// Run by one whole workgroup (every lane calls it).  Every lane reads the
// step's found_inf[slot] and fatal before lane 0 changes the scalar state (a
// barrier separates the two); the clocks of the tensors stepped in this step
// advance only when the step was applied.  The arithmetic is the reference's,
// in double: overflow -> raise at scale <= 1 (here: set fatal bit 0, change
// nothing), else scale = max(1, scale / 2), good_steps = 0; success ->
// good_steps += 1, and at growth_interval scale = min(scale * 2, cap),
// good_steps = 0.  Halving and doubling are exact in double, so the device
// sequence equals the host one bit for bit.
//
// Only found_inf[slot] of the two flag words is read and cleared, so a
// detector of the next step may OR into found_inf[slot ^ 1] at the same time.
#pragma once

#include "common.h"

namespace morph {

__device__ __forceinline__ void close_step(morph_step_state* st, int64_t* clocks,
                                           const int32_t* list, int n, int slot, int lanes) {
  volatile morph_step_state* vs = st;
  const uint32_t fatal = vs->fatal;
  const uint32_t inf = vs->found_inf[slot];
  __syncthreads();
  if (fatal != 0u) return;  // sticky: nothing advances after a fatal overflow
  if (threadIdx.x == 0) {
    const bool dynamic = vs->dynamic != 0u;
    if (inf != 0u) {
      vs->skipped = vs->skipped + 1;
      const double scale = vs->scale;
      if (!dynamic) {
        // fixed scale: the step is skipped and nothing else changes
      } else if (scale <= 1.0) {
        vs->fatal = fatal | MORPH_FATAL_MIN_SCALE;
      } else {
        vs->scale = fmax(1.0, scale / 2.0);
        vs->good_steps = 0;
      }
    } else if (!dynamic) {
      vs->applied = vs->applied + 1;
    } else {
      vs->applied = vs->applied + 1;
      const int64_t good = vs->good_steps + 1;
      if (good >= vs->growth_interval) {
        vs->scale = fmin(vs->scale * 2.0, vs->scale_cap);
        vs->good_steps = 0;
      } else {
        vs->good_steps = good;
      }
    }
    vs->last_found_inf = inf;
    vs->found_inf[slot] = 0u;
  }
  if (inf == 0u)
    for (int i = threadIdx.x; i < n; i += lanes) clocks[list[i]] += 1;
}

}  // namespace morph
