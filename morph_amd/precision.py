"""Dynamic FP16 loss scale with the reference's state machine.

Same constructor, methods and state_dict keys as DynamicLossScale in
streamtrain/precision.py:6-17, so code that persists or restores the scaler
(streamtrain/disk.py:245, 496, 508-512) works unchanged:
  * overflow(): at scale <= 1 raise FloatingPointError (nothing changes);
    otherwise halve (floored at 1) and reset the good-step counter;
  * success(): count a good step; after `growth_interval` of them double the
    scale, capped at 65536, and reset the counter.
All arithmetic is Python double, as in the reference; halving and doubling
are exact there.

When a FusedAdamW drives the scaler, its steps advance the state on the GPU
(the same rule, in double) and the host copy here is a mirror.  Reading
`scale` or `good_steps` then first settles the optimizer's enqueued steps
(a wait for the device), so the host never sees a stale scale: a training
loop that multiplies its loss by `scaler.scale` (disk.py:483, 437) scales
by exactly the factor the next step unscales by.  A loop that wants no wait
per step scales with FusedAdamW.scale_loss() instead, which reads the
scale on the device.
"""
import weakref


class DynamicLossScale:
    CAP = 65536.

    def __init__(self, scale=128., growth_interval=2000):
        self._scale = float(scale)
        self._good_steps = 0
        self.growth_interval = growth_interval
        self._owner = None  # weakref to the optimizer whose queued steps may move the state

    # -- host view -------------------------------------------------------------
    def _settle(self):
        owner = self._owner() if self._owner is not None else None
        if owner is not None:
            owner._refresh_scaler()

    @property
    def scale(self):
        self._settle()
        return self._scale

    @scale.setter
    def scale(self, value):
        # the owner's queued steps come first in program order: settle them, then
        # the assignment wins (the owner pushes it to the device at its next step)
        self._settle()
        self._scale = value

    @property
    def good_steps(self):
        self._settle()
        return self._good_steps

    @good_steps.setter
    def good_steps(self, value):
        self._settle()
        self._good_steps = value

    def attach(self, owner):
        """Called by the optimizer that advances this scaler on the device."""
        current = self._owner() if self._owner is not None else None
        if current is not None and current is not owner:
            raise ValueError("a DynamicLossScale can drive only one optimizer")
        self._owner = weakref.ref(owner)

    # -- the reference's state machine -----------------------------------------
    def overflow(self):
        self._settle()
        if self._scale <= 1:
            raise FloatingPointError('FP16 overflow at minimum loss scale; state unchanged')
        self._good_steps = 0
        self._scale = max(1., self._scale / 2)

    def success(self):
        self._settle()
        self._good_steps += 1
        if self._good_steps < self.growth_interval:
            return
        self._good_steps = 0
        self._scale = min(self.CAP, self._scale * 2)

    def state_dict(self):
        return {'scale': self.scale, 'good_steps': self.good_steps,
                'growth_interval': self.growth_interval}

    def load_state_dict(self, state):
        self._settle()
        self._scale = state['scale']
        self._good_steps = state['good_steps']
        self.growth_interval = state['growth_interval']
