"""The FP32 stage-gradient window of the streamed backward, filled on the GPU.

Reference: for every micro-batch and parameter of a stage the reference runs
    destination.add_(g.detach().float() / self.loss_scale)
into a zeroed FP32 window (streamtrain/sparse_disk.py:82-87, 104-108; the CPU
variant disk.py:446-448), then, in the norm pass,
    for piece in gradient.flatten().split(1048576):
        norm_squared += piece.double().square().sum().item()
(disk.py:466-468; sparse_disk.py:136).  A non-finite norm means skip / retry
(disk.py:485), and clip = min(1, max_norm / (norm + 1e-6)) (disk.py:489).

StageGradients does the same with one kernel pass per micro-batch
(morph_grad_accumulate); the last micro-batch's pass also ORs the non-finite
flag and writes FP64 partial sums, so the norm needs no second read of the
window.  The accumulated values are bit-identical to the reference's torch
ops; the FP64 norm is deterministic and equals the reference's wherever FP64
addition is exact in both orders (otherwise it differs in the last bits).
"""
import ctypes
import math

import torch

from . import _lib, kernels
from ._lib import AccumTensor, check, dtype_code, lib, require_device_tensor, stream_handle


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


class StageGradients:
    """One stage's FP32 gradient window: a flat buffer viewed per parameter.

    shapes: parameter shapes (or tensors / parameters, whose shapes are used).
    Typical use, mirroring sparse_disk.py:82-108:

        window = StageGradients([p.shape for p in stage_params], device)
        window.zero_()
        for k, micro in enumerate(micro_batches):
            grads = torch.autograd.grad(...)
            window.accumulate(grads, loss_scale, final=(k == len(micro_batches) - 1))
        if window.found_inf(): ...             # skip / retry, state untouched
        norm = window.norm_squared() ** 0.5    # FP64, across the whole window

    The window's `views[i]` are FP32 tensors shaped like parameter i; they are
    what the optimizer update consumes.
    """

    def __init__(self, shapes, device=None, buffer=None):
        shapes = [tuple(s.shape) if isinstance(s, torch.Tensor) else tuple(s) for s in shapes]
        self.device = torch.device(device) if device is not None else torch.device(
            "cuda", torch.cuda.current_device())
        sizes = [int(torch.Size(s).numel()) for s in shapes]
        total = sum(sizes)
        if buffer is None:
            buffer = torch.empty(total, dtype=torch.float32, device=self.device)
        if buffer.dtype != torch.float32 or buffer.numel() < total:
            raise ValueError("buffer must be a float32 tensor with room for every parameter")
        require_device_tensor(buffer, "gradient window")
        self.flat = buffer.reshape(-1)[:total]
        self.views, offset = [], 0
        for shape, n in zip(shapes, sizes):
            self.views.append(self.flat[offset:offset + n].view(shape))
            offset += n
        self.seen = [False] * len(shapes)
        self._fresh = True
        self._flag = kernels.new_flag(self.device)
        self._sumsq = torch.zeros((), dtype=torch.float64, device=self.device)
        self._partials = None
        self._finalized = False

    def zero_(self):
        """Start a new accumulation: the next accumulate() overwrites instead of adding
        (the same values as zero_() followed by add_(), without the zeroing pass)."""
        self._fresh = True
        self._finalized = False
        self.seen = [False] * len(self.views)
        return self

    def _tensors(self, grads):
        if len(grads) != len(self.views):
            raise ValueError(f"{len(grads)} gradients for {len(self.views)} parameters")
        arr = (AccumTensor * len(self.views))()
        dtype = None
        keep = []
        for i, (view, g) in enumerate(zip(self.views, grads)):
            arr[i].dst = view.data_ptr()
            arr[i].numel = view.numel()
            if g is None:
                arr[i].grad = None
                continue
            if g.shape != view.shape:
                raise ValueError(f"gradient {i} has shape {tuple(g.shape)}, expected {tuple(view.shape)}")
            require_device_tensor(g, "gradient")
            if dtype is None:
                dtype = g.dtype
            elif g.dtype != dtype:
                raise TypeError("all gradients of one accumulate() call must share a dtype")
            g = g.detach()
            keep.append(g)
            arr[i].grad = g.data_ptr()
            self.seen[i] = True
        return arr, dtype_code(dtype if dtype is not None else torch.float32), keep

    def accumulate(self, grads, loss_scale=1.0, final=False, stream=None, found_inf=None):
        """views[i] += float(grads[i]) / loss_scale for every non-None gradient.

        final=True also computes the window's non-finite flag and FP64 sum of
        squares (read with found_inf() / norm_squared()).  found_inf: a device
        int32 flag to receive that flag instead of the window's own, e.g. a
        FusedAdamW's `found_inf`, whose step(..., checked=True) then needs no
        detector pass.  A caller's flag is only ever ORed into (never cleared
        here), so several windows can feed one step; its owner clears it (the
        optimizer's step close does).  The window's own flag is cleared first.
        """
        if self._finalized:
            raise RuntimeError("window already finalized; call zero_() to start again")
        arr, code, keep = self._tensors(list(grads))
        flags = (_lib.ACCUM_OVERWRITE if self._fresh else 0) | (_lib.ACCUM_FINAL if final else 0)
        L = lib()
        n_part = L.morph_grad_partials(arr, len(self.views))
        check(n_part if n_part < 0 else 0)
        if final and (self._partials is None or self._partials.numel() < max(n_part, 1)):
            self._partials = torch.empty(max(n_part, 1), dtype=torch.float64, device=self.device)
        if final:
            if found_inf is not None:
                kernels.require_device_tensor(found_inf, "found_inf")
                if found_inf.dtype != torch.int32 or found_inf.numel() < 1:
                    raise TypeError("found_inf must be a device int32 flag")
                self._flag_target = found_inf
            else:
                self._flag_target = self._flag
                kernels.flag_clear(self._flag, stream)  # on the same stream as the pass
        sh = stream_handle(stream)
        flag = (self._flag_target if final else self._flag)
        check(L.morph_grad_accumulate(arr, len(self.views), code, float(loss_scale), flags,
                                      _ptr(flag), _ptr(self._partials),
                                      self._partials.numel() if self._partials is not None else 0, sh))
        if final:
            check(L.morph_sumsq_total(_ptr(self._partials), n_part, _ptr(self._sumsq), 0, sh))
            self._finalized = True
        self._fresh = False
        del keep

    def found_inf(self):
        """True when the finished window holds an inf or NaN (synchronizes)."""
        self._require_final()
        return bool(self._flag_target.item())

    def norm_squared(self):
        """FP64 sum of squares of the finished window (synchronizes)."""
        self._require_final()
        return float(self._sumsq.item())

    def norm_squared_tensor(self):
        """The same FP64 sum as a 0-d device tensor (no synchronization)."""
        self._require_final()
        return self._sumsq

    def _require_final(self):
        if not self._finalized:
            raise RuntimeError("call accumulate(..., final=True) first")


def clip_coefficient(norm_squared, max_norm=1.0):
    """disk.py:466-489: norm = math.sqrt(norm^2); min(1, max_norm / (norm + 1e-6)) in floats."""
    return min(1.0, max_norm / (math.sqrt(norm_squared) + 1e-6))
