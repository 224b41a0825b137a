"""Optimizers over the gfx950 kernels, with the reference's Python API.

FusedAdamW is the mixed-precision AdamW of a GPU-resident stage window: FP32
masters and moments in HBM, FP16/BF16 (loss-scaled) or FP32 gradients, an
optional FP16/BF16 export copy written by the same pass.  Its arithmetic is
torch.optim.AdamW(foreach=False) -- the AdamW group of HybridMuonAdamW
(streamtrain/optimizer.py:40) -- preceded by the unscale of
streamtrain/disk.py:447 / sparse_disk.py:107, with the non-finite decision of
optimizer.py:49-51 driving a conditional skip and DynamicLossScale
(precision.py:6-17).  Parameters whose gradient is None are not touched and
their step clock does not advance (sparse_disk.py:1-5, torch's own rule).
"""
import torch

from . import kernels
from .hyper import adamw_constants
from .precision import DynamicLossScale

_OVERFLOW_POLICIES = ("skip", "raise")


def _groups(params, defaults):
    params = list(params)
    if not params:
        raise ValueError("optimizer got an empty parameter list")
    if not isinstance(params[0], dict):
        params = [{"params": params}]
    groups = []
    for g in params:
        group = dict(defaults)
        group.update(g)
        group["params"] = list(group["params"])
        groups.append(group)
    return groups


class FusedAdamW:
    """torch.optim.AdamW(foreach=False)-exact AdamW with fused unscale, skip and export.

    params: FP32 CUDA tensors (or torch-style param-group dicts).
    loss_scale: None (no scaling), a float, or a DynamicLossScale whose
      overflow()/success() this optimizer calls after each step.
    export_dtype: torch.float16 / torch.bfloat16 to keep an export copy of
      every master (self.exports), written in the same pass.
    on_overflow: "skip" -- a step with a non-finite gradient changes no
      master/moment/clock and step() returns False; "raise" -- additionally
      raise FloatingPointError like HybridMuonAdamW (optimizer.py:50-51).
    """

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2, *,
                 loss_scale=None, export_dtype=None, on_overflow="skip"):
        if on_overflow not in _OVERFLOW_POLICIES:
            raise ValueError(f"on_overflow must be one of {_OVERFLOW_POLICIES}")
        if not 0.0 <= lr:
            raise ValueError(f"invalid learning rate {lr}")
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0):
            raise ValueError(f"invalid betas {betas}")
        self.defaults = dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay)
        self.param_groups = _groups(params, self.defaults)
        self.on_overflow = on_overflow
        self.loss_scale = loss_scale
        self.export_dtype = export_dtype
        self.state = {}
        self.exports = []
        device = None
        for group in self.param_groups:
            for p in group["params"]:
                kernels.require_device_tensor(p, "param")
                if p.dtype != torch.float32:
                    raise TypeError("FusedAdamW keeps FP32 masters; got " + str(p.dtype))
                device = device or p.device
                self.state[p] = {"step": 0, "exp_avg": torch.zeros_like(p),
                                 "exp_avg_sq": torch.zeros_like(p)}
                if export_dtype is not None:
                    self.exports.append(p.detach().to(export_dtype))
        self._flag = kernels.new_flag(device)
        self._flag_host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self._batch_key = None
        self._batch = None
        self.skipped_steps = 0

    # -- helpers -----------------------------------------------------------
    def _flat(self):
        return [(gi, p) for gi, group in enumerate(self.param_groups) for p in group["params"]]

    def _scale(self):
        s = self.loss_scale
        if s is None:
            return 1.0
        return float(s.scale) if hasattr(s, "scale") else float(s)

    def zero_grad(self, set_to_none=True):
        for _, p in self._flat():
            if set_to_none:
                p.grad = None
            elif p.grad is not None:
                p.grad.zero_()

    def set_exports(self, outs):
        """Write the export copy into caller buffers (e.g. a slot's compute weights)."""
        outs = list(outs)
        if len(outs) != len(self._flat()):
            raise ValueError("one export buffer per parameter")
        for (_, p), o in zip(self._flat(), outs):
            kernels.require_device_tensor(o, "export")
            if o.numel() != p.numel() or o.dtype not in (torch.float16, torch.bfloat16):
                raise ValueError("export buffers must match params and be fp16/bf16")
        self.exports = outs
        self._batch_key = None

    # -- the step ----------------------------------------------------------
    def enqueue(self, grads=None, stream=None):
        """Enqueue detector + fused AdamW without waiting; returns the launch record.

        finish(record) must follow before the next enqueue (it reads the
        device flag and advances clocks and the loss scale).
        """
        flat = self._flat()
        if grads is None:
            grads = [p.grad for _, p in flat]
        grads = list(grads)
        if len(grads) != len(flat):
            raise ValueError(f"expected {len(flat)} gradients, got {len(grads)}")
        present = [i for i, g in enumerate(grads) if g is not None]
        if not present:
            return None
        scale = self._scale()
        flag = self._flag
        kernels.flag_clear(flag, stream)
        kernels.nonfinite_or([grads[i] for i in present], flag, stream)
        hps, hp_of = [], {}
        hp_index = []
        for i in present:
            gi, p = flat[i]
            group = self.param_groups[gi]
            key = (gi, self.state[p]["step"] + 1)
            if key not in hp_of:
                beta1, beta2 = group["betas"]
                hp_of[key] = len(hps)
                hps.append(adamw_constants(lr=group["lr"], beta1=beta1, beta2=beta2,
                                           eps=group["eps"], weight_decay=group["weight_decay"],
                                           step=key[1], loss_scale=scale))
            hp_index.append(hp_of[key])
        outs = [self.exports[i] if self.exports else None for i in present]
        key = (tuple(present), tuple(grads[i].data_ptr() for i in present), tuple(hp_index),
               tuple(o.data_ptr() if o is not None else 0 for o in outs))
        if key != self._batch_key:
            ps = [flat[i][1] for i in present]
            self._batch = kernels.AdamwBatch(
                ps, [self.state[p]["exp_avg"] for p in ps],
                [self.state[p]["exp_avg_sq"] for p in ps], [grads[i] for i in present],
                outs if self.exports else None, hp_index)
            self._batch_key = key
        self._batch.launch(hps, skip_flag=flag, stream=stream)
        self._flag_host.copy_(flag, non_blocking=True)
        event = torch.cuda.Event()
        event.record(stream)
        return (present, event)

    def finish(self, record):
        """Wait for an enqueued step; apply the skip decision on the host side."""
        if record is None:
            return True
        present, event = record
        event.synchronize()
        overflowed = bool(self._flag_host.item())
        flat = self._flat()
        if overflowed:
            self.skipped_steps += 1
            if isinstance(self.loss_scale, DynamicLossScale) or hasattr(self.loss_scale, "overflow"):
                self.loss_scale.overflow()
            if self.on_overflow == "raise":
                raise FloatingPointError("nonfinite gradient; optimizer not updated")
            return False
        for i in present:
            self.state[flat[i][1]]["step"] += 1
        if hasattr(self.loss_scale, "success"):
            self.loss_scale.success()
        return True

    @torch.no_grad()
    def step(self, grads=None, stream=None):
        """One optimizer step; True if applied, False if skipped on overflow."""
        return self.finish(self.enqueue(grads, stream))

    # -- persistence (torch.optim.Optimizer layout) ------------------------
    def state_dict(self):
        index = {}
        groups = []
        for group in self.param_groups:
            packed = {k: v for k, v in group.items() if k != "params"}
            packed["params"] = []
            for p in group["params"]:
                index[p] = len(index)
                packed["params"].append(index[p])
            groups.append(packed)
        state = {index[p]: {"step": torch.tensor(float(s["step"])), "exp_avg": s["exp_avg"],
                            "exp_avg_sq": s["exp_avg_sq"]} for p, s in self.state.items()}
        return {"state": state, "param_groups": groups}

    def load_state_dict(self, state_dict):
        flat = [p for _, p in self._flat()]
        if len(state_dict["param_groups"]) != len(self.param_groups):
            raise ValueError("loaded state dict has a different number of parameter groups")
        for group, saved in zip(self.param_groups, state_dict["param_groups"]):
            if len(saved["params"]) != len(group["params"]):
                raise ValueError("loaded state dict contains a group of a different size")
            for k, v in saved.items():
                if k != "params":
                    group[k] = tuple(v) if k == "betas" else v
        for i, p in enumerate(flat):
            saved = state_dict["state"].get(i)
            if saved is None:
                continue
            st = self.state[p]
            st["step"] = int(float(saved["step"]))
            st["exp_avg"].copy_(saved["exp_avg"])
            st["exp_avg_sq"].copy_(saved["exp_avg_sq"])
        self._batch_key = None
