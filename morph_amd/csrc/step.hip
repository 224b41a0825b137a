// Device-resident close of an optimizer step as a launch of its own (one
// workgroup), for steps whose close does not ride in the next step's
// detector launch (morph_nonfinite_or_close): the last step before the host
// reads the state, and steps whose non-finite flag came from the gradients'
// producer.  The state machine is close_step (step_close.h).
#include "common.h"
#include "step_close.h"

namespace morph {
namespace {

constexpr int kBlock = 256;

__global__ __launch_bounds__(kBlock) void step_end_kernel(morph_step_state* st, int64_t* clocks,
                                                          const int32_t* list, int n, int slot) {
  close_step(st, clocks, list, n, slot, kBlock);
}

}  // namespace
}  // namespace morph

using namespace morph;

extern "C" int morph_step_end(morph_step_state* d_state, int64_t* d_clocks,
                              const int32_t* d_clock_list, int n, int slot, void* stream) {
  if (d_state == nullptr || n < 0 || (n > 0 && (d_clocks == nullptr || d_clock_list == nullptr)) ||
      (slot != 0 && slot != 1))
    return MORPH_EINVAL;
  hipLaunchKernelGGL(step_end_kernel, dim3(1), dim3(kBlock), 0, as_stream(stream), d_state,
                     d_clocks, d_clock_list, n, slot);
  return launch_status();
}
