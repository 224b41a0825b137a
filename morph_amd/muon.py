"""Hybrid Muon on the gfx950 kernels (streamtrain/optimizer.py:13-70).

orthogonalize() and muon_step() drive morph_muon_* (momentum, Nesterov blend,
Frobenius normalisation, bf16 MFMA Newton-Schulz, fp32 master update);
gemm_nt() exposes the batched bf16 GEMM the iteration is built from.
HybridMuonAdamW keeps the reference class's constructor, partition rule,
step/zero_grad/state_dict/load_state_dict, with the AdamW group on FusedAdamW.
"""
import ctypes

import torch
from torch import nn

from . import _lib, kernels
from ._lib import MuonHP, MuonMatrix, check, lib, require_device_tensor, stream_handle
from .hyper import to_f32
from .optimizer import FusedAdamW

NS_COEFFS = (3.4445, -4.775, 2.0315)  # optimizer.py:21
NS_STEPS = 5  # optimizer.py:13


def _bf16_ptr(t):
    if t is None:
        return None
    if t.dtype != torch.bfloat16:
        raise TypeError("bf16 tensor expected")
    require_device_tensor(t, "gemm operand")
    return ctypes.c_void_p(t.data_ptr())


def gemm_nt(P, Q, D=None, alpha=1.0, beta=0.0, out=None, out_t=None, symmetric=False,
            stream=None, q_kn=False):
    """out = alpha * P @ Q^T + beta * D (bf16, fp32 accumulation); out_t = out^T if given.

    P [.., M, K], Q [.., N, K], D/out [.., M, N], out_t [.., N, M]; a leading batch
    dimension is optional.  M, N multiples of 256 and K of 64.  symmetric=True:
    the result is known to be symmetric (M == N, D symmetric): only the upper
    triangle of tiles is computed and mirrored.  q_kn=True: Q is [.., K, N] and
    the product is P @ Q (transposing LDS reads; out must not overlap Q).
    """
    batched = P.dim() == 3
    if not batched:
        P, Q = P.unsqueeze(0), Q.unsqueeze(0)
        D = D.unsqueeze(0) if D is not None else None
    b, M, K = P.shape
    N = Q.shape[2] if q_kn else Q.shape[1]
    if Q.shape != ((b, K, N) if q_kn else (b, N, K)) or (D is not None and D.shape != (b, M, N)):
        raise ValueError("gemm_nt: shapes do not match P [b,M,K], Q [b,N,K] (or [b,K,N]), "
                         "D [b,M,N]")
    if out is None:
        out = torch.empty((b, M, N), dtype=torch.bfloat16, device=P.device)
    elif not batched:
        out = out.unsqueeze(0)
    if out_t is not None and not batched:
        out_t = out_t.unsqueeze(0)
    if out.shape != (b, M, N) or (out_t is not None and out_t.shape != (b, N, M)):
        raise ValueError("gemm_nt: output shapes do not match")
    flags = (_lib.GEMM_SYMMETRIC if symmetric else 0) | (_lib.GEMM_Q_KN if q_kn else 0)
    check(lib().morph_gemm_nt_bf16(
        _bf16_ptr(P), _bf16_ptr(Q), _bf16_ptr(D), _bf16_ptr(out), _bf16_ptr(out_t),
        M, N, K, b, K, N if q_kn else K, N, N, M, M * K, N * K, M * N, M * N, N * M,
        float(alpha), float(beta), flags, stream_handle(stream)))
    return out if batched else out[0]


class Workspaces:
    """Device workspaces of the Muon batches, one per (shape, device, batch index), each
    sized for the largest matrix count it has served.

    A call needs no particular contents: morph_muon_prepare writes the Newton-Schulz
    operand with its zero padding every time and each product rewrites its whole
    output, so a call on non-finite values leaves nothing behind for the next.
    Streams that used a workspace are recorded, so that a workspace replaced by a
    larger one stays allocated until their queued work is done.
    """

    def __init__(self):
        self._ws = {}

    def get(self, rows, cols, count, device, index=0, stream=None):
        nbytes = lib().morph_muon_workspace_bytes(rows, cols, count)
        if nbytes == 0:
            raise ValueError(f"bad Muon shape {rows}x{cols} x{count}")
        key = (rows, cols, torch.device(device), index)
        stream = stream or torch.cuda.current_stream(device)
        entry = self._ws.get(key)
        if entry is None or entry["buf"].numel() < nbytes:
            if entry is not None:
                for s in entry["streams"]:
                    entry["buf"].record_stream(s)
            with torch.cuda.stream(stream):
                entry = dict(buf=torch.empty(nbytes, dtype=torch.uint8, device=device),
                             streams=set())
            self._ws[key] = entry
        entry["streams"].add(stream)
        return entry["buf"]

    def note_stream(self, stream):
        """Record that `stream` uses the workspaces too (kept alive for its queued work)."""
        for entry in self._ws.values():
            entry["streams"].add(stream)


_WORKSPACES = Workspaces()  # for the free functions; each HybridMuonAdamW owns its own


def _hp(momentum_weight=.05, nesterov_weight=.95, update_scale=1.0, decay=1.0, neg_lr=0.0,
        steps=NS_STEPS, coeffs=NS_COEFFS, update_scale_transposed=1.0):
    a, b, c = coeffs
    return MuonHP(to_f32(momentum_weight), to_f32(nesterov_weight), to_f32(a), to_f32(b),
                  to_f32(c), to_f32(update_scale), to_f32(decay), to_f32(neg_lr), steps,
                  to_f32(update_scale_transposed))


def _by_shape(items):
    """Batches by Newton-Schulz operand: {(m, n): [(item, transposed)]} with m <= n.

    A [rows, cols] and a [cols, rows] matrix share the operand (optimizer.py:15-17
    transposes the taller one), so a SwiGLU block's up/gate and down weights run
    as one batch; `transposed` marks the ones stored [n, m].
    """
    groups = {}
    for item in items:
        rows, cols = item[0].shape
        key = (min(rows, cols), max(rows, cols))
        groups.setdefault(key, []).append((item, int(rows != key[0])))
    return groups


def ns_flops(rows, cols, count, steps=NS_STEPS):
    """Dense FLOPs of the Newton-Schulz chain: (4 m^2 n + 2 m^3) per matrix and iteration."""
    m, n = min(rows, cols), max(rows, cols)
    return count * steps * (4 * m * m * n + 2 * m ** 3)


def ns_executed_flops(rows, cols, count, steps=NS_STEPS):
    """FLOPs the MFMAs execute: the symmetric products (A = X X^T, B' = c A A + b A + a I)
    compute only the upper triangle of their 256 x 256 tiles, X' = B' X all of them; the
    operands are zero-padded to tile multiples (Mp, Np)."""
    m, n = min(rows, cols), max(rows, cols)
    mp, np_ = -(-m // 256) * 256, -(-n // 256) * 256
    t, tn = mp // 256, np_ // 256
    macs = t * (t + 1) // 2 * 256 * 256 * (np_ + mp) + t * tn * 256 * 256 * mp
    return 2 * count * steps * macs


def _prepare(mats, rows, cols, hp, orth_only, stream, workspaces, found_inf=None, first=0):
    """Enqueue prepare for up to 64 matrices per batch; returns the batches for _complete.

    mats: [((param, grad, momentum, momentum_out), transposed)], each stored
    [rows, cols], or [cols, rows] when transposed.  found_inf: optional device
    flag that prepare sets when a gradient is non-finite.  first: index of the
    first batch (each batch of one step gets its own workspace).
    """
    L = lib()
    batches = []
    for k, start in enumerate(range(0, len(mats), 64)):
        chunk = mats[start:start + 64]
        ws = workspaces.get(rows, cols, len(chunk), chunk[0][0][0].device, first + k, stream)
        arr = (MuonMatrix * len(chunk))()
        for i, ((p, g, m, m_out), transposed) in enumerate(chunk):
            arr[i].grad, arr[i].param = g.data_ptr(), p.data_ptr()
            arr[i].momentum = m.data_ptr() if m is not None else None
            arr[i].momentum_out = m_out.data_ptr() if m_out is not None else None
            arr[i].transposed = transposed
        flag = ctypes.c_void_p(found_inf.data_ptr()) if found_inf is not None else None
        check(L.morph_muon_prepare(arr, len(chunk), rows, cols, ctypes.byref(hp), int(orth_only),
                                   ctypes.c_void_p(ws.data_ptr()), ws.numel(), flag,
                                   stream_handle(stream)))
        batches.append((arr, len(chunk), rows, cols, hp, orth_only, ws))
    return batches


def _finish_range(batch, first, n, stream):
    """The parameter update (or U into param) of matrices first .. first + n - 1 of a
    batch _prepare enqueued."""
    arr, count, rows, cols, hp, orth_only, ws = batch
    check(lib().morph_muon_finish_range(arr, count, rows, cols, ctypes.byref(hp), int(orth_only),
                                        first, n, ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                        stream_handle(stream)))


def _chains(batches, stream, timer=None, with_update=False):
    """The Newton-Schulz chain of every batch _prepare enqueued.

    timer: optional list; (start_event, end_event, dense flops, executed flops) around
    each NS chain.  with_update: the chain of a Muon-step batch also applies the
    parameter update (morph_muon_newton_schulz_finish: in its last product's epilogue
    where the shape allows), so no finish follows; orthogonalize batches are chains only.
    """
    L = lib()
    sh = stream_handle(stream)
    for arr, count, rows, cols, hp, orth_only, ws in batches:
        wsp, wsn = ctypes.c_void_p(ws.data_ptr()), ws.numel()
        if timer is not None:
            s = stream or torch.cuda.current_stream()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
        if with_update and not orth_only:
            check(L.morph_muon_newton_schulz_finish(arr, count, rows, cols, ctypes.byref(hp), wsp,
                                                    wsn, sh))
        else:
            check(L.morph_muon_newton_schulz(count, rows, cols, ctypes.byref(hp), wsp, wsn, sh))
        if timer is not None:
            e1.record(s)
            timer.append((e0, e1, ns_flops(rows, cols, count, hp.ns_steps),
                          ns_executed_flops(rows, cols, count, hp.ns_steps)))


def _complete(batches, stream, timer=None):
    """Newton-Schulz chains and the finish of every batch _prepare enqueued: a Muon
    step's update rides on its chain (morph_muon_newton_schulz_finish), orthogonalize's
    U goes into param by the finish pass."""
    _chains(batches, stream, timer, with_update=True)
    L = lib()
    sh = stream_handle(stream)
    for arr, count, rows, cols, hp, orth_only, ws in batches:
        if orth_only:
            check(L.morph_muon_finish(arr, count, rows, cols, ctypes.byref(hp), 1,
                                      ctypes.c_void_p(ws.data_ptr()), ws.numel(), sh))


def _check_matrix(t, name):
    require_device_tensor(t, name)
    if t.dim() != 2 or t.dtype != torch.float32:
        raise ValueError(f"{name} must be a 2-D float32 tensor")


def orthogonalize(gradients, steps=NS_STEPS, stream=None, workspaces=_WORKSPACES):
    """optimizer.py:13-22 on the GPU: NS(g / (|g|_F + 1e-7)), bf16 MFMA, returned as fp32.

    gradients: one 2-D tensor or a list; matrices with the same Newton-Schulz
    operand ([r, c] and [c, r] alike) run as one batch.
    """
    single = torch.is_tensor(gradients)
    gs = [gradients] if single else list(gradients)
    outs = []
    for g in gs:
        _check_matrix(g, "gradient")
        outs.append(torch.empty_like(g))
    items = [(o, g, None, None) for o, g in zip(outs, gs)]
    batches = []
    for (rows, cols), group in _by_shape(items).items():
        batches += _prepare(group, rows, cols, _hp(steps=steps), True, stream, workspaces,
                            first=len(batches))
    _complete(batches, stream)
    return outs[0] if single else outs


def _step_hp(rows, cols, lr, weight_decay, steps=NS_STEPS):
    """Constants of one Muon step for the [rows, cols] batch (optimizer.py:60-61): decay
    1 - lr * weight_decay, alpha -lr, update scale sqrt(max(1, rows / cols)) and, for the
    transposed members, sqrt(max(1, cols / rows))."""
    return _hp(update_scale=max(1, rows / cols) ** .5, decay=1 - lr * weight_decay,
               neg_lr=-lr, steps=steps, update_scale_transposed=max(1, cols / rows) ** .5)


def _check_items(params, grads, momenta, momenta_out):
    """(param, grad, momentum, momentum_out) tuples, validated."""
    items = []
    outs = momenta_out if momenta_out is not None else [None] * len(params)
    for p, g, m, mo in zip(params, grads, momenta, outs):
        for t, name in ((p, "param"), (g, "grad"), (m, "momentum")):
            _check_matrix(t, name)
        if not (p.shape == g.shape == m.shape):
            raise ValueError("param, grad and momentum shapes differ")
        if mo is not None:
            _check_matrix(mo, "momentum_out")
            if mo.shape != m.shape or mo.data_ptr() == m.data_ptr():
                raise ValueError("momentum_out must be a separate buffer of the momentum's shape")
        items.append((p, g, m, mo))
    return items


def muon_step(params, grads, momenta, lr, weight_decay, steps=NS_STEPS, stream=None,
              workspaces=_WORKSPACES, timer=None, momenta_out=None, found_inf=None, gate=None):
    """The Muon loop body of optimizer.py:55-61 for every (param, grad, momentum) triple.

    In place on params and momenta.  Scalars follow the reference: decay
    1 - lr * weight_decay, update scale sqrt(max(1, rows / cols)), alpha -lr.
    momenta_out: optional separate buffers that receive the updated momenta
    (momenta are then only read).  found_inf: optional device flag set when a
    gradient is non-finite, tested in the momentum pass.  gate: optional
    callable run after that pass and before anything the caller keeps is
    mutated (with momenta_out); it may raise to drop the step.
    """
    items = _check_items(params, grads, momenta, momenta_out)
    batches = []
    for (rows, cols), group in _by_shape(items).items():
        batches += _prepare(group, rows, cols, _step_hp(rows, cols, lr, weight_decay, steps),
                            False, stream, workspaces, found_inf, first=len(batches))
    if gate is not None:
        gate()
    _complete(batches, stream, timer)


def _muon_grad(g, p, device):
    """A Muon gradient of a CPU master: a float32 tensor of the parameter's shape, in CPU
    memory (uploaded through the staging) or on the optimizer's GPU (read in place)."""
    if g.dtype != torch.float32 or g.shape != p.shape:
        raise ValueError("with CPU masters the Muon gradients are float32 tensors of the "
                         "parameter's shape")
    if g.device.type == "cpu":
        return g.contiguous()
    if g.device != device:
        raise ValueError(f"a Muon gradient is on {g.device}; the optimizer works on {device}")
    _check_matrix(g, "gradient")
    return g


def partition(model):
    """optimizer.py:25-31: hidden nn.Linear weights (not lm_head) -> Muon; the rest -> AdamW."""
    hidden = {id(module.weight) for name, module in model.named_modules()
              if isinstance(module, nn.Linear) and name != 'lm_head'}
    muon, adam = [], []
    for param in model.parameters():
        (muon if id(param) in hidden else adam).append(param)
    return muon, adam


class HybridMuonAdamW:
    """streamtrain/optimizer.py:34-70 on the GPU.

    Same constructor and methods.  step() raises FloatingPointError before any
    mutation when a gradient is non-finite (optimizer.py:49-51), then runs the
    Muon update for the hidden matrices (batched by shape) and the AdamW group
    (betas .9/.95, FusedAdamW).  The Newton-Schulz iteration is bf16 on MFMA
    where the reference uses FP32 (optimizer.py:3-6).

    The model's parameters may all live on the GPU (engine='resident') or all on
    the CPU (engine='dls'/'async': FP32 masters in RAM, gradients left in CPU
    p.grad by the streaming engine; runner.py:41-46, engine.py:75-88).  With CPU
    masters the momenta and the AdamW moments stay resident in HBM; step()
    uploads the gradients and masters, runs the same kernels on device mirrors,
    and writes the updated masters back into the CPU tensors before returning,
    so the engine's next stage load (engine.py:109-115) reads the new weights.
    resident_masters=True (CPU masters only) keeps the masters' device mirrors
    between steps and uploads a master again only when its CPU tensor's storage
    or version counter changed since the step wrote it back; writes the counter
    cannot see (through `p.data`, a NumPy view, raw memory) must be followed by
    invalidate_masters().
    """

    def __init__(self, model, lr=1e-3, muon_lr=None, weight_decay=.01, *,
                 resident_masters=False):
        self.muon, adam = partition(model)
        kinds = {p.device.type for p in self.muon + adam}
        if len(kinds) > 1 or not kinds <= {"cpu", "cuda"}:
            raise ValueError("parameters must all be on the GPU or all on the CPU")
        self.host = kinds == {"cpu"}
        self._muon_masters = self._muon_grads = None
        if self.host and self.muon:
            from .staging import HostStaging
            for p in self.muon:
                if p.dim() != 2 or p.dtype != torch.float32 or not p.is_contiguous():
                    raise ValueError("Muon masters must be contiguous 2-D float32 tensors")
            dev = torch.device("cuda", torch.cuda.current_device())
            shapes = [p.shape for p in self.muon]
            sizes = {p.numel() for p in self.muon}
            # one matrix per staging chunk when they are all the same size, so each
            # can be updated as soon as it is on the device (_host_step)
            chunk = sizes.pop() if len(sizes) == 1 else 1 << 22
            self._muon_masters = HostStaging(shapes, torch.float32, dev, chunk_elements=chunk)
            self._muon_grads = HostStaging(shapes, torch.float32, dev)
            self._muon_dev = self._muon_masters.views
        else:
            self._muon_dev = list(self.muon)
        self.ns_timer = None  # optional list: HIP events around each Newton-Schulz chain
        # CPU masters: the Muon matrices go through the step in parts (uploads, momentum
        # pass and Newton-Schulz chain per part), so that the first parts' chains run while
        # later gradients cross PCIe and their updated masters come back while later
        # masters go up.  None: 2 parts when Muon gradients are uploaded (the gradient
        # upload bounds the step: 2, 6, 7, 10 or 14 parts measured within 3%), and one part
        # per 6 matrices when they are all on the GPU already, so the downloads of the first
        # parts overlap the later chains (config 5, pinned resident masters: 83.7 ms per
        # step with 2 parts, 68.9 with 7, 66.8 with 10, 67.7 with 14).  An int fixes it.
        self.stream_parts = None
        self._ns_stream = None
        self._workspaces = Workspaces()
        self.lr = lr if muon_lr is None else muon_lr
        self.weight_decay = weight_decay
        self.momentum = {}
        # the momentum pass writes into these and they swap with `momentum`
        # once the non-finite gate has passed, so a raise mutates nothing
        self._momentum_next = {}
        # The gate below has already seen every AdamW gradient finite when the group
        # steps (and it has no loss scale), so its step needs no host round trip of its
        # own: the one wait per step is the gate's.  Host mirrors of its step counts
        # refresh on resolve(), which state_dict() and load_state_dict() call.
        self.adam = FusedAdamW(adam, lr=lr, weight_decay=weight_decay, betas=(.9, .95),
                               sync=False, resident_masters=resident_masters) if adam else None
        # CPU masters: keep the Muon masters' device mirrors as the working copies
        # between steps (FusedAdamW's resident_masters, same rule)
        self.resident_masters = bool(resident_masters)
        self._host_marks = {}  # Muon index -> (storage, version) its mirror holds
        self._flag = None

    def invalidate_masters(self):
        """resident_masters: upload every master again at its next step (after host
        writes the parameters' version counters cannot see, e.g. through `p.data`)."""
        self._host_marks.clear()
        if self.adam is not None:
            self.adam.invalidate_masters()

    def _current_muon_masters(self, idx):
        """The Muon indices whose mirrors still hold their host masters' values; their
        marks are dropped until the step has written the masters back."""
        current = set()
        for i in idx:
            mark = self._host_marks.pop(i, None)
            p = self.muon[i]
            if self.resident_masters and mark == (p.data_ptr(), p._version):
                current.add(i)
        return current

    def zero_grad(self, set_to_none=True):
        for p in self.muon:
            p.grad = None if set_to_none else torch.zeros_like(p)
        if self.adam is not None:
            self.adam.zero_grad(set_to_none=set_to_none)

    @torch.no_grad()
    def step(self, grads=None):
        """The gate of optimizer.py:49-51 covers every gradient: the AdamW group's
        by the detector, the Muon matrices' inside their momentum pass (which
        writes only scratch buffers until the gate has passed).  With CPU masters
        every gradient is uploaded before the gate, and the masters go up and
        come back only after it has passed (_host_step).

        grads: optional {parameter: gradient} used instead of p.grad (a parameter
        missing from it has no gradient this step).  With CPU masters a gradient
        may be a float32 tensor on the GPU -- an engine's device stage buffer
        (Slot.grad_device, engine.py:67) before its flush to p.grad
        (engine.py:75-88) -- which the step reads where it is, with no upload."""
        if grads is None:
            grad_of = lambda p: p.grad  # noqa: E731
        else:
            grad_of = grads.get
        live = [(i, p) for i, p in enumerate(self.muon) if grad_of(p) is not None]
        adam_params = [p for g in (self.adam.param_groups if self.adam else []) for p in g["params"]]
        adam_grads = [grad_of(p) for p in adam_params]
        adam_present = [k for k, g in enumerate(adam_grads) if g is not None]
        if not live and not adam_present:
            return
        idx = [i for i, _ in live]
        if self.host and live:
            return self._host_step(live, idx, adam_params, adam_grads, adam_present, grad_of)
        if self.host:
            device = self.adam.device
            muon_grads = []
            adam_grads = self.adam._stage_in(adam_grads, adam_present)
        else:
            device = (live[0][1] if live else adam_params[adam_present[0]]).device
            muon_grads = [grad_of(p) for _, p in live]
        if self._flag is None:
            self._flag = kernels.new_flag(device)
        kernels.flag_clear(self._flag)
        if adam_present:
            kernels.nonfinite_or([adam_grads[k] for k in adam_present], self._flag)

        def gate():
            if self._flag.item():
                raise FloatingPointError('nonfinite gradient; optimizer not updated')

        if live:
            self._ensure_momenta(idx)
            muon_step([self._muon_dev[i] for i in idx], muon_grads,
                      [self.momentum[i] for i in idx], self.lr, self.weight_decay,
                      workspaces=self._workspaces, timer=self.ns_timer,
                      momenta_out=[self._momentum_next[i] for i in idx],
                      found_inf=self._flag, gate=gate)
            self._swap_momenta(idx)
        else:
            gate()
        self._adam_after_gate(adam_grads, adam_present)

    def _ensure_momenta(self, idx):
        for i in idx:
            if i not in self.momentum:
                self.momentum[i] = torch.zeros_like(self._muon_dev[i])
            if i not in self._momentum_next:
                self._momentum_next[i] = torch.empty_like(self._muon_dev[i])

    def _swap_momenta(self, idx):
        for i in idx:
            self.momentum[i], self._momentum_next[i] = self._momentum_next[i], self.momentum[i]

    def _adam_after_gate(self, adam_grads, adam_present):
        """The AdamW group's step.  The gate's detector has already seen every one of
        its gradients finite (the flag it read covers them), and the group has no loss
        scale, so the step's found_inf word stays clear: checked=True runs the fused
        pass without a second detector scan."""
        if not adam_present:
            return
        if self.host:
            self.adam._enqueue(adam_grads, adam_present, None, True)
            self.adam._stage_out(adam_present)
        else:
            self.adam.step(adam_grads, checked=True)

    def _host_step(self, live, idx, adam_params, adam_grads, adam_present, grad_of):
        """step() with CPU masters.  The Muon matrices go through in parts (see
        stream_parts): each part's gradients go up, then its momentum pass (which writes
        only scratch buffers and the non-finite flag) and its Newton-Schulz chain
        are enqueued while the next part's gradients go up; the chains run on a
        second stream, so that a part's updates wait only for its own chain.
        Once every gradient has passed the gate (optimizer.py:49-51), the masters
        stream through the updates: each matrix goes up, is updated as soon as it
        and its part's chain are done (morph_muon_finish_range) and comes back
        while the next ones go up.  Returns with the new masters in the CPU
        tensors."""
        device = self._muon_dev[0].device
        stream = torch.cuda.current_stream(device)
        masters = [p for _, p in live]
        grads = [_muon_grad(grad_of(p), p, device) for _, p in live]
        self._muon_masters._check(masters, idx)  # fail before anything is enqueued
        self._ensure_momenta(idx)
        if self._flag is None:
            self._flag = kernels.new_flag(device)
        if self._ns_stream is None:
            from .staging import shared_stream
            self._ns_stream = shared_stream(device, "side")
        ns = self._ns_stream
        kernels.flag_clear(self._flag, stream)
        parts = []
        try:
            # the chains may run on non-finite values before the gate raises; the next
            # step's prepare rewrites everything of the workspaces that its chains read
            self._host_step_on(live, idx, masters, grads, adam_grads, adam_present, stream, ns,
                               parts)
        finally:
            # later work on `stream` (the next step's momentum pass) follows the chains
            stream.wait_stream(ns)

    def _host_step_on(self, live, idx, masters, grads, adam_grads, adam_present, stream, ns,
                      parts):
        if self.stream_parts is not None:
            nparts = int(self.stream_parts)
        elif all(g.device.type != "cpu" for g in grads):
            nparts = -(-len(live) // 6)
        else:
            nparts = 2
        nparts = max(1, min(nparts, len(live)))
        bounds = [len(live) * k // nparts for k in range(nparts + 1)]
        ready, nbatch = [], 0
        for k in range(nparts):
            pos = range(bounds[k], bounds[k + 1])
            part = [idx[j] for j in pos]
            # CPU gradients go up (device ones are read in place).  wait=False: nothing
            # queued reads the gradient mirrors (the last step's momentum passes
            # finished before its masters came back)
            up = [j for j in pos if grads[j].device.type == "cpu"]
            if up:
                self._muon_grads.upload([grads[j] for j in up], [idx[j] for j in up], stream,
                                        wait=False)
            items = [(self._muon_dev[idx[j]],
                      self._muon_grads.views[idx[j]] if grads[j].device.type == "cpu" else grads[j],
                      self.momentum[idx[j]], self._momentum_next[idx[j]]) for j in pos]
            batches = []
            for (rows, cols), group in _by_shape(items).items():
                batches += _prepare(group, rows, cols,
                                    _step_hp(rows, cols, self.lr, self.weight_decay), False,
                                    stream, self._workspaces, self._flag,
                                    first=nbatch + len(batches))
            nbatch += len(batches)
            ns.wait_stream(stream)
            self._workspaces.note_stream(ns)
            parts.append(batches)
            _chains(batches, ns, self.ns_timer)
            done = torch.cuda.Event()
            done.record(ns)
            ready.append(done)
        adam_grads = self.adam._stage_in(adam_grads, adam_present) if adam_present else None
        if adam_present:
            kernels.nonfinite_or([adam_grads[k] for k in adam_present], self._flag)
        if self._flag.item():
            raise FloatingPointError('nonfinite gradient; optimizer not updated')
        where = {}
        for k, batches in enumerate(parts):
            for b, batch in enumerate(batches):
                arr, count = batch[0], batch[1]
                for j in range(count):
                    where[arr[j].param] = (k, b, j)
        staging = self._muon_masters
        waited = set()

        def after_chain(k, st):
            if k not in waited:
                st.wait_event(ready[k])
                waited.add(k)

        current = self._current_muon_masters(idx)
        if staging.whole_tensor_chunks(idx):
            def launch(lo, hi, pieces, st):
                for i, _, _ in pieces:
                    k, b, j = where[self._muon_dev[i].data_ptr()]
                    after_chain(k, st)
                    _finish_range(parts[k][b], j, 1, st)

            staging.pipeline(masters, idx, launch, stream, wait=False, current=current)
        else:
            staging.upload(masters, idx, stream, wait=False, current=current)
            for k, batches in enumerate(parts):
                after_chain(k, stream)
                for batch in batches:
                    _finish_range(batch, 0, batch[1], stream)
            staging.download([p.data for p in masters], idx, stream)
        for i in idx:
            p = self.muon[i]
            self._host_marks[i] = (p.data_ptr(), p._version)
        self._swap_momenta(idx)
        self._adam_after_gate(adam_grads, adam_present)

    def state_dict(self):
        """{momentum, adam, lr, weight_decay} as optimizer.py:64-65.  The momentum
        tensors are the current ones; a later step writes its update into a
        second buffer and swaps, so they are not updated in place afterwards.
        With CPU masters they are CPU copies, where the reference keeps them."""
        momentum = ({i: m.cpu() for i, m in self.momentum.items()} if self.host
                    else self.momentum)
        return dict(momentum=momentum,
                    adam=self.adam.state_dict() if self.adam else None,
                    lr=self.lr, weight_decay=self.weight_decay)

    def load_state_dict(self, state):
        self.momentum = {i: value.to(self._muon_dev[i].device)
                         for i, value in state['momentum'].items()}
        self._momentum_next = {}
        if self.adam is not None:
            self.adam.load_state_dict(state['adam'])
        self.lr, self.weight_decay = state['lr'], state['weight_decay']
