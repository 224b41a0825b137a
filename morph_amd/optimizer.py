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

A step is two launches on the caller's stream -- the detector (which also
closes the previous step: loss scale, clocks) and the fused AdamW pass --
driven by device-resident state (morph_amd.control), so no step waits for the
host.  The last step's close is enqueued when the host next needs the state
(resolve()) or when the next step has no detector pass of its own.  The host
copies of the clocks are refreshed by resolve(); the host DynamicLossScale
settles the queued steps itself when its scale is read, and scale_loss()
multiplies a loss by the device scale without waiting.  With sync=True (or
on_overflow="raise") every step resolves and reports its outcome like the
reference does.
"""
import torch

from . import kernels
from .control import BiasTables, StepControl
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

    params: FP32 tensors (or torch-style param-group dicts), all on one GPU, or
      all on the CPU -- the streamed engines' masters (runner.py:41-46).  With
      CPU masters the moments stay resident in HBM; each step uploads the
      gradients (CPU p.grad, or device tensors) through pinned staging, runs
      the gate, then streams the masters through the update chunk by chunk
      (morph_amd.staging.HostStaging.pipeline) and returns with the updated
      masters in the CPU tensors.
    loss_scale: None (no scaling), a float (fixed scale), or a DynamicLossScale
      whose state this optimizer advances (on the device) after every step.
    export_dtype: torch.float16 / torch.bfloat16 to keep an export copy of
      every master (self.exports), written in the same pass.
    on_overflow: "skip" -- a step with a non-finite gradient changes no
      master/moment/clock; "raise" -- additionally raise FloatingPointError
      from step() like HybridMuonAdamW (optimizer.py:50-51); implies sync.
    sync: resolve after every step; step() then returns True (applied) or
      False (skipped).  Otherwise step() returns None and enqueues only.
    arena: place every master, both moments and the export copy in one device
      allocation laid out for the fused pass (morph_amd.arena), the way a stage
      window holds its state; each parameter's `.data` is moved there (its
      values copied), so views of a parameter taken before construction stop
      aliasing it.  Parameters must be distinct, non-overlapping tensors.
    resident_masters: CPU masters only.  Keep each master's device mirror as
      the working copy between steps and upload a master again only when its
      host tensor may have changed since its last step: a new storage
      (`p.data` rebound) or a bumped version counter (an in-place op on the
      parameter itself, as optimizer steps and `model.load_state_dict` make).
      Writes the counter cannot see -- through `p.data`, a NumPy view or raw
      memory -- must be followed by invalidate_masters().  Each step then moves
      the masters one way (down) instead of both.
    """

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2, *,
                 loss_scale=None, export_dtype=None, on_overflow="skip", sync=False,
                 arena=False, resident_masters=False):
        if on_overflow not in _OVERFLOW_POLICIES:
            raise ValueError(f"on_overflow must be one of {_OVERFLOW_POLICIES}")
        if not 0.0 <= lr:
            raise ValueError(f"invalid learning rate {lr}")
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0):
            raise ValueError(f"invalid betas {betas}")
        self.defaults = dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay)
        self.param_groups = _groups(params, self.defaults)
        self.on_overflow = on_overflow
        self.sync = sync or on_overflow == "raise"
        self.export_dtype = export_dtype
        self.state = {}
        self.exports = []
        flat = self._flat()
        if len({id(p) for _, p in flat}) != len(flat):
            raise ValueError("a parameter appears more than once")
        device = None
        for _, p in flat:
            if not isinstance(p, torch.Tensor):
                raise TypeError("params must be tensors")
            if p.dtype != torch.float32:
                raise TypeError("FusedAdamW keeps FP32 masters; got " + str(p.dtype))
            if device is not None and p.device != device:
                raise ValueError("all parameters must be on one device")
            device = p.device
        self._staging = None   # HostStaging of CPU masters (None: masters on the GPU)
        self._grad_staging = None
        self.resident_masters = bool(resident_masters)
        self._host_marks = {}  # index -> (storage, version) of the host master its mirror holds
        self._chunk_cache = None  # per-chunk descriptor batches of the CPU-master pipeline
        if device.type == "cpu":
            for _, p in flat:
                if not p.is_contiguous():
                    raise ValueError("CPU masters must be contiguous")
            if arena:
                raise ValueError("arena=True lays out device-resident masters; these are on the CPU")
            from .staging import HostStaging
            device = torch.device("cuda", torch.cuda.current_device())
            self._staging = HostStaging([p.shape for _, p in flat], torch.float32, device)
            self._dev = self._staging.views
            self._staging.upload([p for _, p in flat])  # for the initial export copies
            self._mark_masters(range(len(flat)))
        else:
            for _, p in flat:
                kernels.require_device_tensor(p, "param")
            self._dev = [p for _, p in flat]
        self.arena = None
        if arena:
            self._place_in_arena([p for _, p in flat], device, export_dtype)
            self._dev = [p for _, p in flat]
        else:
            for (_, p), d in zip(flat, self._dev):
                self.state[p] = {"step": 0, "exp_avg": torch.zeros_like(d),
                                 "exp_avg_sq": torch.zeros_like(d)}
                if export_dtype is not None:
                    self.exports.append(d.detach().to(export_dtype))
        self.device = device
        self._ctl = StepControl(device, len(flat), loss_scale)
        if isinstance(loss_scale, DynamicLossScale):
            loss_scale.attach(self)
        self._dirty = False     # steps enqueued since the host last read the device state
        self._tables = {}
        self._bound = [0] * len(flat)  # upper bound of each device clock
        self._cache_key = None
        self._cache = None
        self._slot = 0          # found_inf word of the next step (steps alternate)
        self._pending = None    # (slot, clock_list, stream) of a step whose close is not enqueued
        self.kernel_timer = None  # optional list: (start, end) events around each AdamW launch
        self.dispatch_timer = None  # optional kernels.DispatchTimer: stamps each AdamW launch
        self.skipped_steps = 0
        self.applied_steps = 0

    @property
    def loss_scale(self):
        return self._ctl.loss_scale

    @property
    def found_inf(self):
        """The next step's non-finite flag in the device step state, as a 1-element
        int32 tensor.  A producer that already tests every gradient (the final pass of
        StageGradients.accumulate(..., found_inf=opt.found_inf)) ORs its result into it
        and the caller then calls step(..., checked=True), which skips the detector
        pass.  Several producers may OR into it for one step (e.g. one per stage
        window); the step's close clears it.  Steps alternate between two flag words:
        read this property anew before every step."""
        return self._ctl.found_inf_view(self._slot)

    def loss_scale_tensor(self):
        """The loss scale the next step unscales by, as a 0-d float64 device tensor (a
        view of the device step state), without waiting for the device.  The previous
        step's close (which may halve or double the scale) is enqueued first if it is
        still pending, ordered before the caller's current stream."""
        if self._pending is not None:
            s = self._pending[2]
            self._flush_close()
            cur = torch.cuda.current_stream(self.device)
            if s != cur:
                cur.wait_stream(s)
        return self._ctl.scale_view()

    def scale_loss(self, loss):
        """loss * (the loss scale of the next step), computed on the GPU: the
        reference's `loss * loss_scale` (disk.py:437) with no host round trip."""
        return loss * self.loss_scale_tensor().to(loss.dtype)

    # -- helpers -----------------------------------------------------------
    @torch.no_grad()
    def _place_in_arena(self, params, device, export_dtype):
        """Masters, moments and export copies in one Arena; p.data moves to its master view."""
        from .arena import Arena
        streams = [[(p.numel(), torch.float32)] * 3
                   + ([(p.numel(), export_dtype)] if export_dtype is not None else [])
                   for p in params]
        self.arena = Arena(streams, device)
        for p, views in zip(params, self.arena.views):
            w, m, v = (t.view(p.shape) for t in views[:3])
            w.copy_(p.detach())
            m.zero_()
            v.zero_()
            p.data = w
            self.state[p] = {"step": 0, "exp_avg": m, "exp_avg_sq": v}
            if export_dtype is not None:
                self.exports.append(views[3].view(p.shape).copy_(w))

    def _flat(self):
        return [(gi, p) for gi, group in enumerate(self.param_groups) for p in group["params"]]

    def zero_grad(self, set_to_none=True):
        for _, p in self._flat():
            if set_to_none:
                p.grad = None
            elif p.grad is not None:
                p.grad.zero_()

    def set_exports(self, outs):
        """Write the export copy into caller buffers (e.g. a slot's compute weights)."""
        outs = list(outs)
        flat = self._flat()
        if len(outs) != len(flat):
            raise ValueError("one export buffer per parameter")
        for (_, p), o in zip(flat, outs):
            kernels.require_device_tensor(o, "export")
            if o.numel() != p.numel() or o.dtype not in (torch.float16, torch.bfloat16):
                raise ValueError("export buffers must match params and be fp16/bf16")
        if len({o.dtype for o in outs}) != 1:
            raise ValueError("export buffers must share one dtype")
        self.exports = outs
        self._cache_key = None

    def _table(self, betas):
        key = (float(betas[0]), float(betas[1]))
        if key not in self._tables:
            self._tables[key] = BiasTables(key[0], key[1], self.device)
        return self._tables[key]

    def _prepare(self, grads, present):
        """Descriptor batch, per-group constants and clock list for this set of tensors."""
        flat = self._flat()
        groups = sorted({flat[i][0] for i in present})
        hp_of = {gi: k for k, gi in enumerate(groups)}
        key = (tuple(present), tuple(grads[i].dtype for i in present),
               tuple(e.data_ptr() for e in self.exports) if self.exports else None)
        ptrs = tuple(grads[i].data_ptr() for i in present)
        if key != self._cache_key:
            ps = [flat[i][1] for i in present]
            batch = kernels.AdamwBatch(
                [self._dev[i] for i in present], [self.state[p]["exp_avg"] for p in ps],
                [self.state[p]["exp_avg_sq"] for p in ps], [grads[i] for i in present],
                [self.exports[i] for i in present] if self.exports else None,
                hp_index=[hp_of[flat[i][0]] for i in present], clock_index=list(present))
            clock_list = torch.tensor(present, dtype=torch.int32).to(self.device)
            self._cache = [batch, clock_list, ptrs]
            self._cache_key = key
        elif ptrs != self._cache[2]:
            # same tensors, new gradient buffers: swap pointers only (no table rebuild,
            # no host-to-device copy that would wait for the queued steps)
            self._cache[0].rebind_grads([grads[i] for i in present])
            self._cache[2] = ptrs
        batch, clock_list, _ = self._cache
        hps, scheds = [], []
        for gi in groups:
            group = self.param_groups[gi]
            beta1, beta2 = group["betas"]
            hps.append(adamw_constants(lr=group["lr"], beta1=beta1, beta2=beta2, eps=group["eps"],
                                       weight_decay=group["weight_decay"], step=1))
            table = self._table(group["betas"])
            need = max(self._bound[i] for i in present if flat[i][0] == gi) + 1
            table.ensure(need)
            scheds.append(table.sched(group["lr"]))
        return batch, clock_list, hps, scheds

    # -- the step ----------------------------------------------------------
    @torch.no_grad()
    def step(self, grads=None, stream=None, checked=False):
        """Enqueue one optimizer step: the detector (carrying the previous step's
        close), then the fused AdamW pass.  This step's close follows with the next
        step's detector, or on its own at resolve() or before a checked step.

        grads: one tensor (or None) per parameter in param-group order; by
        default p.grad.  checked=True: every gradient's non-finite test is
        already in `found_inf` (set on this stream since the last step), so
        the detector pass is skipped.  Returns None, or with sync the
        applied/skipped outcome.  With CPU masters the step also uploads the
        gradients and masters and returns once the updated masters are back in
        the CPU tensors.
        """
        flat = self._flat()
        if grads is None:
            grads = [p.grad for _, p in flat]
        grads = list(grads)
        if len(grads) != len(flat):
            raise ValueError(f"expected {len(flat)} gradients, got {len(grads)}")
        present = [i for i, g in enumerate(grads) if g is not None]
        if not present:
            return True if self.sync else None
        if self._staging is None:
            return self._enqueue(grads, present, stream, checked)
        # CPU masters: the gradients go up first (the gate needs all of them), then
        # the masters stream through the update chunk by chunk, each chunk coming
        # back while the next goes up
        dev_grads = self._stage_in(grads, present, stream, masters=False)
        return self._enqueue(dev_grads, present, stream, checked, pipeline=True)

    def _mark_masters(self, which):
        """Record that the mirrors of `which` now hold their host masters' values."""
        flat = self._flat()
        for i in which:
            p = flat[i][1]
            self._host_marks[i] = (p.data_ptr(), p._version)

    def _current_masters(self, which):
        """resident_masters: the indices of `which` whose mirrors still hold their host
        masters' values (same storage, same version since the last step); their
        marks are dropped until the caller marks them again after its step."""
        flat = self._flat()
        current = set()
        for i in which:
            mark = self._host_marks.pop(i, None)
            p = flat[i][1]
            if self.resident_masters and mark == (p.data_ptr(), p._version):
                current.add(i)
        return current

    def invalidate_masters(self):
        """resident_masters: upload every master again at its next step (after host
        writes its version counter cannot see, e.g. through `p.data` or NumPy)."""
        self._host_marks.clear()

    def _stage_in(self, grads, present, stream=None, masters=True):
        """CPU masters: upload the host gradients (and with `masters` the listed
        masters); returns the per-parameter device gradients (None where absent)."""
        flat = self._flat()
        host = [i for i in present if grads[i].device.type == "cpu"]
        for i in present:
            g = grads[i]
            if g.shape != flat[i][1].shape:
                raise ValueError(f"gradient {i} has shape {tuple(g.shape)}, expected "
                                 f"{tuple(flat[i][1].shape)}")
            if g.device.type not in ("cpu", "cuda"):
                raise ValueError(f"gradient {i} is on {g.device}")
            if g.device.type == "cuda" and g.device != self.device:
                raise ValueError(f"gradient {i} is on {g.device}, the optimizer on "
                                 f"{self.device}")
        dev = list(grads)
        if host:
            dtypes = {grads[i].dtype for i in host}
            if len(dtypes) != 1:
                raise ValueError(f"host gradients must share one dtype, got {dtypes}")
            dtype = dtypes.pop()
            if self._grad_staging is None or self._grad_staging.dtype != dtype:
                from .staging import HostStaging
                self._grad_staging = HostStaging([p.shape for _, p in flat], dtype, self.device)
            self._grad_staging.upload([grads[i].contiguous() for i in host], host, stream)
            for i in host:
                dev[i] = self._grad_staging.views[i]
        if masters:
            self._staging.upload([flat[i][1] for i in present], present, stream,
                                 current=self._current_masters(present))
        return dev

    def _stage_out(self, present, stream=None):
        """CPU masters: copy the listed device masters back into the CPU tensors."""
        flat = self._flat()
        self._staging.download([flat[i][1].data for i in present], present, stream)
        self._mark_masters(present)

    def _chunk_batches(self, grads, present, hp_of):
        """One descriptor batch per staging chunk of the listed tensors (CPU masters):
        views of the mirrors, moments, gradients and exports over the chunk's
        elements, each with its tensor's constants and clock."""
        flat = self._flat()
        key = (tuple(present), tuple(grads[i].dtype for i in present),
               tuple(grads[i].data_ptr() for i in present),
               tuple(e.data_ptr() for e in self.exports) if self.exports else None)
        if self._chunk_cache is not None and self._chunk_cache[0] == key:
            return self._chunk_cache[1]
        batches = []
        for _, _, pieces in self._staging._chunks(present):
            ps, ms, vs, gs, outs, hpi, ci = [], [], [], [], [], [], []
            for i, a, b in pieces:
                p = flat[i][1]
                ps.append(self._dev[i].view(-1)[a:b])
                ms.append(self.state[p]["exp_avg"].view(-1)[a:b])
                vs.append(self.state[p]["exp_avg_sq"].view(-1)[a:b])
                gs.append(grads[i].reshape(-1)[a:b])
                outs.append(self.exports[i].view(-1)[a:b] if self.exports else None)
                hpi.append(hp_of[flat[i][0]])
                ci.append(i)
            batches.append(kernels.AdamwBatch(ps, ms, vs, gs, outs if self.exports else None,
                                              hp_index=hpi, clock_index=ci))
        self._chunk_cache = (key, batches)
        return batches

    def _enqueue(self, grads, present, stream, checked, pipeline=False):
        """The device step over device gradients (see step()).  pipeline: CPU
        masters, streamed through the update by HostStaging.pipeline (the launch
        timers do not apply)."""
        flat = self._flat()
        if self._ctl.scaler_changed():
            # the caller set the scaler (scale, good_steps, load_state_dict) since the last
            # step: wait for the queued steps, then the caller's values replace what they
            # left on the device (the wait's mirror() would otherwise overwrite them)
            fields = self._ctl.host_fields()
            try:
                self.resolve()
            finally:
                self._ctl.restore_host_fields(fields)
            self._ctl.push_scale()
        batch, clock_list, hps, scheds = self._prepare(grads, present)
        # everything that can fail is done before the first launch is enqueued
        events = self.dispatch_timer.next() if self.dispatch_timer is not None else None
        ctl = self._ctl
        slot = self._slot
        s = stream or torch.cuda.current_stream(self.device)
        for table in self._tables.values():
            table.used_on(s)
        if s != torch.cuda.current_stream(self.device):
            clock_list.record_stream(s)  # allocated on the current stream, read on `s`
        if self._pending is not None and self._pending[2] != s:
            # the previous step ran on another stream: close it there, and order
            # this step after that close
            prev = self._pending[2]
            self._flush_close()
            s.wait_stream(prev)
        if checked:
            self._flush_close()
        elif self._pending is not None:
            kernels.nonfinite_or_close([grads[i] for i in present], ctl.state, slot, ctl.clocks,
                                       self._pending[1], s)
            self._pending = None
        else:
            kernels.nonfinite_or([grads[i] for i in present], ctl.found_inf_ptr(slot), s)
        if pipeline:
            flat = self._flat()
            groups = sorted({flat[i][0] for i in present})
            chunk_batches = self._chunk_batches(grads, present, {g: k for k, g in enumerate(groups)})
            launches = iter(chunk_batches)
            self._staging.pipeline(
                [flat[i][1].data for i in present], present,
                lambda lo, hi, pieces, st: next(launches).launch_dev(hps, scheds, ctl.clocks,
                                                                     ctl.state, slot, st, None),
                s, current=self._current_masters(present))
            self._mark_masters(present)
        elif self.kernel_timer is not None:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            batch.launch_dev(hps, scheds, ctl.clocks, ctl.state, slot, s, events)
            e1.record(s)
            self.kernel_timer.append((e0, e1))
        else:
            batch.launch_dev(hps, scheds, ctl.clocks, ctl.state, slot, s, events)
        self._pending = (slot, clock_list, s)
        self._slot = slot ^ 1
        self._dirty = True
        for i in present:
            self._bound[i] += 1
        if not self.sync:
            return None
        st = self.resolve()
        if st.last_found_inf and self.on_overflow == "raise":
            raise FloatingPointError("nonfinite gradient; optimizer not updated")
        return not st.last_found_inf

    def _flush_close(self):
        """Enqueue the pending step's close on that step's stream, on its own."""
        if self._pending is None:
            return
        slot, clock_list, s = self._pending
        self._pending = None
        kernels.step_end(self._ctl.state, self._ctl.clocks, clock_list, slot, s)

    def resolve(self):
        """Wait for enqueued steps; refresh clocks, counters and the host loss scale.

        Raises FloatingPointError if a step overflowed at loss scale <= 1 (the
        reference raises there, precision.py:9-10; on the device that step and every
        step enqueued after it changed nothing).  The error is raised once: the
        optimizer then stands where the reference stands after the raise (scale 1,
        state untouched) and the next step runs normally.
        """
        st = self._sync_state()
        err = self._ctl.fatal_error(st)
        if err is not None:
            self._ctl.clear_fatal()
            torch.cuda.current_stream(self.device).synchronize()
            raise err
        return st

    def _refresh_scaler(self):
        """DynamicLossScale's host view asks for the current state."""
        if self._dirty or self._pending is not None:
            self._sync_state()

    def _sync_state(self):
        """resolve() without raising: wait, then refresh the host mirrors."""
        if self._pending is not None:
            s = self._pending[2]
            self._flush_close()
            if s != torch.cuda.current_stream(self.device):
                s.synchronize()
        st = self._ctl.read()
        clocks = self._ctl.clocks.cpu().tolist()
        for i, (_, p) in enumerate(self._flat()):
            self.state[p]["step"] = clocks[i]
            self._bound[i] = clocks[i]
        self.skipped_steps = int(st.skipped)
        self.applied_steps = int(st.applied)
        self._ctl.mirror(st)
        self._dirty = False
        return st

    synchronize = resolve

    # -- persistence (torch.optim.Optimizer layout) ------------------------
    def state_dict(self):
        self._sync_state()
        index = {}
        groups = []
        for group in self.param_groups:
            packed = {k: v for k, v in group.items() if k != "params"}
            packed["params"] = []
            for p in group["params"]:
                index[p] = len(index)
                packed["params"].append(index[p])
            groups.append(packed)
        # the moments live with the masters in torch.optim: CPU masters get CPU copies
        host = self._staging is not None
        state = {index[p]: {"step": torch.tensor(float(s["step"])),
                            "exp_avg": s["exp_avg"].cpu() if host else s["exp_avg"],
                            "exp_avg_sq": s["exp_avg_sq"].cpu() if host else s["exp_avg_sq"]}
                 for p, s in self.state.items()}
        return {"state": state, "param_groups": groups}

    def load_state_dict(self, state_dict):
        self._sync_state()
        self._ctl.clear_fatal()  # a loaded state is a consistent point to go on from
        flat = [p for _, p in self._flat()]
        if len(state_dict["param_groups"]) != len(self.param_groups):
            raise ValueError("loaded state dict has a different number of parameter groups")
        for group, saved in zip(self.param_groups, state_dict["param_groups"]):
            if len(saved["params"]) != len(group["params"]):
                raise ValueError("loaded state dict contains a group of a different size")
        for group, saved in zip(self.param_groups, state_dict["param_groups"]):
            for k, v in saved.items():
                if k != "params":
                    group[k] = tuple(v) if k == "betas" else v
        clocks = []
        for i, p in enumerate(flat):
            st = self.state[p]
            saved = state_dict["state"].get(i)
            if saved is not None:
                st["step"] = int(float(saved["step"]))
                st["exp_avg"].copy_(saved["exp_avg"])
                st["exp_avg_sq"].copy_(saved["exp_avg_sq"])
            clocks.append(st["step"])
            self._bound[i] = st["step"]
        self._ctl.clocks.copy_(torch.tensor(clocks, dtype=torch.int64))
        self._cache_key = None
