"""Thin Python wrappers of the C ABI that take torch device tensors.

Every function enqueues work on the current torch stream (or `stream`) and
returns without synchronizing.  Shapes, devices, dtypes and contiguity are
checked here so that the library only ever sees buffers that match what its
kernels assume.
"""
import ctypes

import torch

from . import _lib
from ._lib import AdamwTensor, check, dtype_code, lib, require_device_tensor, stream_handle


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _event_handles(events):
    """hipEvent_t handles of a (start, stop) pair of torch events, or (None, None)."""
    if events is None:
        return None, None
    return ctypes.c_void_p(events[0].cuda_event), ctypes.c_void_p(events[1].cuda_event)


def new_flag(device=None):
    """A device uint32 flag (stored as int32; only 0/1 are written)."""
    return torch.zeros(1, dtype=torch.int32, device=device or torch.cuda.current_device())


def flag_clear(flag, stream=None):
    require_device_tensor(flag, "flag")
    check(lib().morph_flag_clear(_ptr(flag), stream_handle(stream)))


def nonfinite_or(grads, flag, stream=None):
    """OR into `flag` whether any element of any gradient is +-inf/NaN.

    flag: a device int32 tensor, or a raw device address (int) of a uint32.
    """
    if isinstance(flag, int):
        flag_ptr = ctypes.c_void_p(flag)
    else:
        require_device_tensor(flag, "flag")
        flag_ptr = _ptr(flag)
    by_dtype = {}
    for i, g in enumerate(grads):
        require_device_tensor(g, f"grads[{i}]")
        by_dtype.setdefault(g.dtype, []).append(g)
    for dtype, group in by_dtype.items():
        ptrs = (ctypes.c_void_p * len(group))(*[g.data_ptr() for g in group])
        sizes = (ctypes.c_int64 * len(group))(*[g.numel() for g in group])
        check(lib().morph_nonfinite_or_multi(ptrs, sizes, len(group), dtype_code(dtype),
                                             flag_ptr, stream_handle(stream)))


class AdamwBatch:
    """A reusable ctypes descriptor array for one multi-tensor AdamW launch.

    Building the descriptor array is the only per-call Python cost that grows
    with the tensor count, so callers that step the same tensors repeatedly
    keep one batch and only swap the constants.
    """

    def __init__(self, params, exp_avgs, exp_avg_sqs, grads, outs=None, hp_index=None,
                 clock_index=None):
        n = len(params)
        if not (len(exp_avgs) == len(exp_avg_sqs) == len(grads) == n):
            raise ValueError("params, exp_avgs, exp_avg_sqs and grads must have equal length")
        outs = list(outs) if outs is not None else [None] * n
        hp_index = list(hp_index) if hp_index is not None else [0] * n
        clock_index = list(clock_index) if clock_index is not None else list(range(n))
        grad_dtypes = {g.dtype for g in grads}
        if len(grad_dtypes) > 1:
            raise ValueError(f"one launch takes one gradient dtype, got {grad_dtypes}")
        out_dtypes = {o.dtype for o in outs if o is not None}
        if len(out_dtypes) > 1:
            raise ValueError(f"one launch takes one export dtype, got {out_dtypes}")
        self.grad_dtype = dtype_code(next(iter(grad_dtypes))) if n else _lib.DTYPE_F32
        self.out_dtype = dtype_code(next(iter(out_dtypes))) if out_dtypes else _lib.DTYPE_NONE
        self.array = (AdamwTensor * max(n, 1))()
        self.count = n
        self.n_hp = (max(hp_index) + 1) if n else 1
        keep = []
        for i in range(n):
            p, m, v, g, o = params[i], exp_avgs[i], exp_avg_sqs[i], grads[i], outs[i]
            for name, t in (("param", p), ("exp_avg", m), ("exp_avg_sq", v), ("grad", g)):
                require_device_tensor(t, f"{name}[{i}]")
            for name, t in (("param", p), ("exp_avg", m), ("exp_avg_sq", v)):
                if t.dtype != torch.float32:
                    raise TypeError(f"{name}[{i}] must be float32, got {t.dtype}")
            if not (m.numel() == v.numel() == g.numel() == p.numel()):
                raise ValueError(f"tensor {i}: param/exp_avg/exp_avg_sq/grad sizes differ")
            if not (p.device == m.device == v.device == g.device):
                raise ValueError(f"tensor {i}: tensors on different devices")
            if o is not None:
                require_device_tensor(o, f"out[{i}]")
                if o.numel() != p.numel() or o.device != p.device:
                    raise ValueError(f"tensor {i}: export copy does not match param")
            d = self.array[i]
            d.grad, d.param, d.exp_avg, d.exp_avg_sq = (g.data_ptr(), p.data_ptr(),
                                                        m.data_ptr(), v.data_ptr())
            d.out = o.data_ptr() if o is not None else None
            d.numel = p.numel()
            d.hp_index = hp_index[i]
            d.clock_index = clock_index[i]
            keep.append((p, m, v, g, o))
        self._keep = keep  # the tensors must outlive the descriptors
        self._grad_dtype = grads[0].dtype if n else None
        self._numels = [p.numel() for p in params]
        self._device = params[0].device if n else None

    def rebind_grads(self, grads):
        """Point the descriptors at new gradient tensors of the same sizes and dtype.

        A training loop hands a new gradient buffer every step (autograd with
        zero_grad(set_to_none=True), a rotating stage window); this swaps the
        pointers without rebuilding and re-validating the whole table.
        """
        grads = list(grads)
        if len(grads) != self.count:
            raise ValueError(f"expected {self.count} gradients, got {len(grads)}")
        for i, g in enumerate(grads):
            require_device_tensor(g, f"grad[{i}]")
            if g.dtype != self._grad_dtype or g.numel() != self._numels[i] or g.device != self._device:
                raise ValueError(f"grad[{i}] does not match the batch (dtype, size or device)")
        for i, g in enumerate(grads):
            self.array[i].grad = g.data_ptr()
            p, m, v, _, o = self._keep[i]
            self._keep[i] = (p, m, v, g, o)

    def launch(self, hps, skip_flag=None, stream=None, events=None):
        """Enqueue the step.  hps: sequence of AdamwHP, indexed by hp_index; events:
        optional (start, stop) pair from a DispatchTimer."""
        if self.count == 0:
            return
        if len(hps) < self.n_hp:
            raise ValueError(f"need {self.n_hp} constant sets, got {len(hps)}")
        arr = (_lib.AdamwHP * len(hps))(*hps)
        if skip_flag is not None:
            require_device_tensor(skip_flag, "skip_flag")
        e0, e1 = _event_handles(events)
        check(lib().morph_adamw_multi(self.array, self.count, self.grad_dtype, self.out_dtype,
                                      arr, len(hps), _ptr(skip_flag), e0, e1,
                                      stream_handle(stream)))


    def launch_dev(self, hps, scheds, clocks, state, slot=0, stream=None, events=None):
        """Enqueue the device-resident form (morph_adamw_multi_dev).

        scheds: AdamwSched per constant set; clocks: device int64 tensor;
        state: device tensor holding a morph_step_state; slot: the step's
        found_inf word (0 or 1); events: optional (start, stop) pair from a
        DispatchTimer, stamped by the launch's own dispatch.
        """
        if self.count == 0:
            return
        if len(hps) < self.n_hp or len(scheds) != len(hps):
            raise ValueError("need one constant set and one schedule per hp index")
        require_device_tensor(clocks, "clocks")
        require_device_tensor(state, "state")
        if clocks.dtype != torch.int64 or state.numel() * state.element_size() < 64:
            raise ValueError("clocks must be int64 and state must hold a morph_step_state")
        harr = (_lib.AdamwHP * len(hps))(*hps)
        sarr = (_lib.AdamwSched * len(scheds))(*scheds)
        e0, e1 = _event_handles(events)
        check(lib().morph_adamw_multi_dev(self.array, self.count, self.grad_dtype,
                                          self.out_dtype, harr, sarr, len(hps), _ptr(clocks),
                                          _ptr(state), slot, e0, e1, stream_handle(stream)))


class DispatchTimer:
    """Pairs of timing events that a launch's own dispatch stamps with its start and
    end (hipExtLaunchKernel), so kernels are timed with no marker packets between
    them and their neighbours in the queue.  The events are created (and recorded
    once, which creates them) here, before the region they will time."""

    def __init__(self, pairs, device=None):
        stream = torch.cuda.current_stream(device)
        self.pairs = []
        for _ in range(pairs):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            b.record(stream)
            self.pairs.append((a, b))
        stream.synchronize()
        self.used = 0

    def next(self):
        if self.used >= len(self.pairs):
            raise RuntimeError(f"DispatchTimer holds {len(self.pairs)} pairs, all used")
        pair = self.pairs[self.used]
        self.used += 1
        return pair

    def elapsed_ms(self):
        """Durations of the stamped launches (call after synchronizing)."""
        return [a.elapsed_time(b) for a, b in self.pairs[:self.used]]


def _check_close_args(state, clocks, clock_list):
    require_device_tensor(state, "state")
    require_device_tensor(clocks, "clocks")
    require_device_tensor(clock_list, "clock_list")
    if clock_list.dtype != torch.int32 or clocks.dtype != torch.int64:
        raise TypeError("clock_list must be int32 and clocks int64")


def step_end(state, clocks, clock_list, slot=0, stream=None):
    """Enqueue morph_step_end (clock_list: device int32 tensor of distinct indices)."""
    _check_close_args(state, clocks, clock_list)
    check(lib().morph_step_end(_ptr(state), _ptr(clocks), _ptr(clock_list), clock_list.numel(),
                               slot, stream_handle(stream)))


def nonfinite_or_close(grads, state, slot, clocks, prev_clock_list, stream=None):
    """One launch: the detector over `grads` into found_inf[slot] of `state`, and the
    close of the previous step (slot ^ 1, clocks prev_clock_list) in one extra workgroup
    (morph_nonfinite_or_close).  All gradients must share one dtype."""
    _check_close_args(state, clocks, prev_clock_list)
    dtypes = {g.dtype for g in grads}
    if len(dtypes) > 1:
        raise ValueError(f"one launch takes one gradient dtype, got {dtypes}")
    for i, g in enumerate(grads):
        require_device_tensor(g, f"grads[{i}]")
    n = len(grads)
    ptrs = (ctypes.c_void_p * max(n, 1))(*[g.data_ptr() for g in grads])
    sizes = (ctypes.c_int64 * max(n, 1))(*[g.numel() for g in grads])
    dtype = dtype_code(next(iter(dtypes))) if n else _lib.DTYPE_F32
    check(lib().morph_nonfinite_or_close(ptrs, sizes, n, dtype, _ptr(state), slot, _ptr(clocks),
                                         _ptr(prev_clock_list), prev_clock_list.numel(),
                                         stream_handle(stream)))


def adamw_step(param, exp_avg, exp_avg_sq, grad, hp, out=None, skip_flag=None, stream=None,
               events=None):
    """One fused AdamW step on one tensor (morph_adamw_fused; with `events`, a (start,
    stop) pair from a DispatchTimer, the one-tensor morph_adamw_multi that stamps them)."""
    for name, t in (("param", param), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq),
                    ("grad", grad)):
        require_device_tensor(t, name)
    for name, t in (("param", param), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq)):
        if t.dtype != torch.float32:
            raise TypeError(f"{name} must be float32")
    n = param.numel()
    if not (exp_avg.numel() == exp_avg_sq.numel() == grad.numel() == n):
        raise ValueError("param/exp_avg/exp_avg_sq/grad sizes differ")
    if out is not None:
        require_device_tensor(out, "out")
        if out.numel() != n:
            raise ValueError("export copy size differs from param")
    if skip_flag is not None:
        require_device_tensor(skip_flag, "skip_flag")
    if events is not None:
        AdamwBatch([param], [exp_avg], [exp_avg_sq], [grad], [out]).launch(
            [hp], skip_flag, stream, events)
        return
    check(lib().morph_adamw_fused(
        _ptr(grad), dtype_code(grad.dtype), _ptr(param), _ptr(exp_avg), _ptr(exp_avg_sq),
        _ptr(out), dtype_code(out.dtype) if out is not None else _lib.DTYPE_NONE, n,
        ctypes.byref(hp), _ptr(skip_flag), stream_handle(stream)))
