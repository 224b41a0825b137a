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
"""


class DynamicLossScale:
    CAP = 65536.

    def __init__(self, scale=128., growth_interval=2000):
        self.scale = float(scale)
        self.good_steps = 0
        self.growth_interval = growth_interval

    def overflow(self):
        if self.scale <= 1:
            raise FloatingPointError('FP16 overflow at minimum loss scale; state unchanged')
        self.good_steps = 0
        self.scale = max(1., self.scale / 2)

    def success(self):
        self.good_steps += 1
        if self.good_steps < self.growth_interval:
            return
        self.good_steps = 0
        self.scale = min(self.CAP, self.scale * 2)

    def state_dict(self):
        return {'scale': self.scale, 'good_steps': self.good_steps,
                'growth_interval': self.growth_interval}

    def load_state_dict(self, state):
        self.scale = state['scale']
        self.good_steps = state['good_steps']
        self.growth_interval = state['growth_interval']
