"""Device-resident step control: loss-scale state, step clocks, bias-correction tables.

With these in HBM the optimizer step needs no host round trip: the detector
writes found_inf[slot] into the state block, the AdamW kernel reads the scale,
the skip decision and each tensor's clock from it, and the step's close
advances the loss scale and the clocks.  Steps alternate between the two flag
slots, so a step's close can ride in the next step's detector launch.  The
host mirrors (DynamicLossScale, per-tensor step counts) are refreshed only
when the caller asks (resolve()).
"""
import ctypes
import math

import numpy as np
import torch

from ._lib import FATAL_MIN_SCALE, AdamwSched, StepState
from .hyper import to_f32
from .precision import DynamicLossScale

STATE_BYTES = ctypes.sizeof(StepState)
FOUND_INF_OFFSET = StepState.found_inf.offset  # two uint32 words, one per slot


class BiasTables:
    """bias_correction1[t-1] = 1 - beta1 ** t (double) and
    bias_correction2_sqrt[t-1] = fp32((1 - beta2 ** t) ** 0.5) for t = 1..len,
    evaluated with Python floats exactly as torch/optim/adam.py:528-539 does
    (step is a float there).  Grown by doubling.  A replaced table may still be
    read by kernels enqueued on any stream that used it: every stream a step ran
    on is recorded (used_on), and at replacement the old tensors are marked in
    use on those streams, so the caching allocator does not hand their memory
    out again before that work is done."""

    def __init__(self, beta1, beta2, device, length=4096):
        self.beta1, self.beta2, self.device = float(beta1), float(beta2), device
        self.length = 0
        self.bc1 = self.bc2s = None
        self._streams = set()
        self.ensure(length)

    def used_on(self, stream):
        """Note that work reading the current tables is enqueued on `stream`."""
        if stream != torch.cuda.current_stream(self.device):
            self._streams.add(stream)

    def ensure(self, t_max):
        if t_max <= self.length:
            return
        for old in (self.bc1, self.bc2s):
            if old is not None:
                for s in self._streams:
                    old.record_stream(s)
        self._streams = set()
        length = max(4096, self.length)
        while length < t_max:
            length *= 2
        b1, b2 = self.beta1, self.beta2
        bc1 = np.empty(length, np.float64)
        bc2s = np.empty(length, np.float32)
        for i in range(length):
            t = float(i + 1)
            bc1[i] = 1 - b1 ** t
            bc2s[i] = to_f32((1 - b2 ** t) ** 0.5)
        self.bc1 = torch.from_numpy(bc1).to(self.device)
        self.bc2s = torch.from_numpy(bc2s).to(self.device)
        self.length = length

    def sched(self, lr):
        return AdamwSched(float(lr), self.bc1.data_ptr(), self.bc2s.data_ptr(), self.length)


class StepControl:
    """The morph_step_state block and the clocks of one optimizer, on `device`."""

    def __init__(self, device, n_clocks, loss_scale=None):
        self.device = device
        self.state = torch.zeros(STATE_BYTES, dtype=torch.uint8, device=device)
        self.clocks = torch.zeros(max(n_clocks, 1), dtype=torch.int64, device=device)
        self._host = torch.empty(STATE_BYTES, dtype=torch.uint8, pin_memory=True)
        self.loss_scale = loss_scale
        self._initialized = False
        self.push_scale()

    def found_inf_ptr(self, slot):
        if slot not in (0, 1):
            raise ValueError("slot must be 0 or 1")
        return self.state.data_ptr() + FOUND_INF_OFFSET + 4 * slot

    def found_inf_view(self, slot):
        """found_inf[slot] as a 1-element int32 view of the state block."""
        if slot not in (0, 1):
            raise ValueError("slot must be 0 or 1")
        at = FOUND_INF_OFFSET + 4 * slot
        return self.state[at:at + 4].view(torch.int32)

    def _scale_fields(self):
        s = self.loss_scale
        if isinstance(s, DynamicLossScale):
            # the raw host copy: reading .scale would settle the owner's queued steps
            return float(s._scale), int(s._good_steps), int(s.growth_interval), 1
        if hasattr(s, "overflow") and hasattr(s, "success"):
            return float(s.scale), int(s.good_steps), int(s.growth_interval), 1
        scale = 1.0 if s is None else float(s)
        if not (scale > 0 and math.isfinite(scale)):
            raise ValueError(f"loss scale must be positive and finite, got {scale}")
        return scale, 0, 1 << 62, 0

    def push_scale(self):
        """Write the host scaler's state into the device block (keeps counters and
        the fatal bit)."""
        current = self.read() if self._initialized else StepState()
        self._initialized = True
        scale, good, interval, dynamic = self._scale_fields()
        current.scale, current.good_steps, current.growth_interval = scale, good, interval
        current.scale_cap = DynamicLossScale.CAP if dynamic else scale
        current.dynamic = dynamic
        blob = bytes(current)
        self.state.copy_(torch.frombuffer(bytearray(blob), dtype=torch.uint8))
        self._mirrored = (scale, good, interval)

    def scaler_changed(self):
        return self._scale_fields()[:3] != self._mirrored

    def host_fields(self):
        """The host scaler's (scale, good_steps) as the caller last set them."""
        return self._scale_fields()[:2]

    def restore_host_fields(self, fields):
        """Put back host scaler fields that a mirror() overwrote (dynamic scalers only)."""
        s = self.loss_scale
        scale, good = fields
        if isinstance(s, DynamicLossScale):
            s._scale, s._good_steps = scale, good
        elif hasattr(s, "overflow") and hasattr(s, "success"):
            s.scale, s.good_steps = scale, good

    def read(self):
        """Synchronously copy the state block to the host."""
        self._host.copy_(self.state)
        return StepState.from_buffer_copy(self._host.numpy().tobytes())

    def scale_view(self):
        """The device loss scale (the state block's `scale`) as a 0-d float64 view."""
        return self.state[:8].view(torch.float64)[0]

    def clear_fatal(self):
        """Zero the sticky fatal word (stream-ordered on the current stream)."""
        at = StepState.fatal.offset
        self.state[at:at + 4].zero_()

    def mirror(self, st):
        """Refresh the host DynamicLossScale from a state read back from the device."""
        s = self.loss_scale
        if st.dynamic:
            if isinstance(s, DynamicLossScale):
                s._scale, s._good_steps = st.scale, int(st.good_steps)
            else:
                s.scale = st.scale
                s.good_steps = int(st.good_steps)
        self._mirrored = (st.scale if st.dynamic else self._mirrored[0],
                          int(st.good_steps) if st.dynamic else self._mirrored[1],
                          self._mirrored[2])

    @staticmethod
    def fatal_error(st):
        if st.fatal & FATAL_MIN_SCALE:
            return FloatingPointError('FP16 overflow at minimum loss scale; state unchanged')
        return None
