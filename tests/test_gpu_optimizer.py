"""GPU parity of FusedAdamW on the BASELINE configs, against the oracle and torch.

  config 1: 6 FP32 tensors, 10 steps, wd .1 on 2-D only (param groups);
  config 2: the 5B SwiGLU stage window, FP16 grads x 2^16, FP16 export;
  config 3: the tied 65536 x 3072 embedding, sparse Zipf rows, BF16 grads/export, wd 0;
  config 4: config 2 for 16 steps with inf/NaN injected at steps 3, 7, 12.
Bit-exact against the oracle everywhere; against torch.optim.AdamW the moments
are bit-exact and masters agree to max|dw|/max|w| <= 1e-6 (torch's CPU sqrt is
not correctly rounded; see tests/test_oracle_adamw.py).
"""
import json

import numpy as np
import pytest
import torch

import bench
from morph_amd import DynamicLossScale, FusedAdamW
from tests.golden.make_golden import CONFIG1, config1_inputs, sha
from tests.helpers import assert_same_bits, export_bits, to_oracle

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def oracle_adamw_threads(grad, w, m, v, hp, out_dtype, grad_dtype, parts=16):
    """The oracle's AdamW over `parts` slices on host threads.  Every element's arithmetic
    is its own, so the result is a single call's bit for bit; ctypes releases the GIL
    during the call, which brings a full-size config-3 step to about a second."""
    from concurrent.futures import ThreadPoolExecutor
    from oracle import reference as R
    n = w.size
    if n < (1 << 22):
        return R.adamw(grad, w, m, v, hp, out_dtype=out_dtype, grad_dtype=grad_dtype)
    cuts = [n * k // parts for k in range(parts + 1)]

    def one(k):
        lo, hi = cuts[k], cuts[k + 1]
        return R.adamw(grad[lo:hi], w[lo:hi], m[lo:hi], v[lo:hi], hp, out_dtype=out_dtype,
                       grad_dtype=grad_dtype)

    with ThreadPoolExecutor(parts) as pool:
        outs = list(pool.map(one, range(parts)))
    return None if outs[0] is None else np.concatenate(outs)


class OracleWindow:
    """The oracle's view of a window: one (w, m, v, clock) per tensor."""

    def __init__(self, masters):
        self.w = [to_oracle(t).copy() for t in masters]
        self.m = [np.zeros_like(w) for w in self.w]
        self.v = [np.zeros_like(w) for w in self.w]
        self.t = [0] * len(self.w)

    def step(self, grads, hps_for, out_dtype):
        from oracle import reference as R
        outs = []
        for i, g in enumerate(grads):
            self.t[i] += 1
            outs.append(oracle_adamw_threads(
                to_oracle(g), self.w[i], self.m[i], self.v[i], hps_for(i, self.t[i]), out_dtype,
                {torch.float16: R.DTYPE_F16, torch.bfloat16: R.DTYPE_BF16,
                 torch.float32: R.DTYPE_F32}[g.dtype]))
        return outs

    def check(self, opt, what):
        for i, p in enumerate(p for g in opt.param_groups for p in g["params"]):
            st = opt.state[p]
            assert_same_bits(p.detach().cpu().numpy().ravel(), self.w[i], f"{what} master[{i}]")
            assert_same_bits(st["exp_avg"].cpu().numpy().ravel(), self.m[i], f"{what} m[{i}]")
            assert_same_bits(st["exp_avg_sq"].cpu().numpy().ravel(), self.v[i], f"{what} v[{i}]")
            assert st["step"] == self.t[i]


def test_config1_bitexact_vs_oracle_and_torch_golden(golden_dir):
    from oracle import reference as R
    ref = json.loads((golden_dir / "config1.json").read_text())
    masters, grads = config1_inputs()
    dev = [m.to(DEV) for m in masters]
    groups = [dict(params=[p for p in dev if p.ndim == 2], weight_decay=CONFIG1["wd_2d"]),
              dict(params=[p for p in dev if p.ndim == 1], weight_decay=0.0)]
    opt = FusedAdamW(groups, lr=CONFIG1["lr"], betas=CONFIG1["betas"], eps=CONFIG1["eps"],
                     sync=True)
    order = [p for g in opt.param_groups for p in g["params"]]
    index = [next(i for i, q in enumerate(dev) if q is p) for p in order]
    ora = OracleWindow([masters[i] for i in index])
    for t in range(1, CONFIG1["steps"] + 1):
        gs = grads(t)
        assert opt.step([gs[i].to(DEV) for i in index]) is True
        ora.step([gs[i] for i in index],
                 lambda i, step: R.torch_adamw_hp(CONFIG1["lr"], *CONFIG1["betas"], CONFIG1["eps"],
                                                  CONFIG1["wd_2d"] if order[i].ndim == 2 else 0.,
                                                  step), R.DTYPE_NONE)
    ora.check(opt, "config1")
    for k, i in enumerate(index):  # torch.optim.AdamW golden: moments by SHA, masters sampled
        tref = ref["tensors"][i]
        st = opt.state[order[k]]
        assert sha(st["exp_avg"].cpu().numpy().ravel()) == tref["sha_m"]
        assert sha(st["exp_avg_sq"].cpu().numpy().ravel()) == tref["sha_v"]
        w = order[k].detach().cpu().numpy().ravel()
        idx = np.array(tref["sample_index"])
        assert np.abs(w[idx] - np.array(tref["sample_w"], np.float32)).max() <= 1e-6 * np.abs(w).max()


def test_config1_vs_live_torch_adamw_on_gpu_box():
    """torch.optim.AdamW(foreach=False) on this host's CPU, element by element."""
    masters, grads = config1_inputs()
    ref = [torch.nn.Parameter(m.clone()) for m in masters]
    tgroups = [dict(params=[p for p in ref if p.ndim == 2], weight_decay=.1),
               dict(params=[p for p in ref if p.ndim == 1], weight_decay=0.)]
    topt = torch.optim.AdamW(tgroups, lr=3e-4, betas=(.9, .95), eps=1e-8, foreach=False)
    dev = [m.to(DEV) for m in masters]
    groups = [dict(params=[p for p in dev if p.ndim == 2], weight_decay=.1),
              dict(params=[p for p in dev if p.ndim == 1], weight_decay=0.)]
    opt = FusedAdamW(groups, lr=3e-4, betas=(.9, .95), eps=1e-8)  # asynchronous steps
    for t in range(1, 11):
        gs = grads(t)
        for p, g in zip(ref, gs):
            p.grad = g.clone()
        topt.step()
        by_id = {id(p): g for p, g in zip(dev, gs)}
        opt.step([by_id[id(p)].to(DEV) for grp in opt.param_groups for p in grp["params"]])
    opt.resolve()
    for p, q in zip(ref, dev):
        st, qs = topt.state[p], opt.state[q]
        assert torch.equal(st["exp_avg"], qs["exp_avg"].cpu())
        assert torch.equal(st["exp_avg_sq"], qs["exp_avg_sq"].cpu())
        dw = (q.detach().cpu() - p.detach()).abs().max() / p.detach().abs().max()
        assert dw <= 1e-6
        assert int(qs["step"]) == int(st["step"]) == 10


def _config2_run(shapes, steps, seed, check_at=()):
    from oracle import reference as R
    masters = [m.cpu() for m in bench.config2_window("cpu", seed)] if shapes is None else [
        torch.randn(s, generator=torch.Generator().manual_seed(seed + i)) * .02
        for i, s in enumerate(shapes)]
    shapes = [tuple(m.shape) for m in masters]
    scaler = DynamicLossScale(65536., 2000)
    opt = FusedAdamW([m.to(DEV) for m in masters], lr=3e-4, betas=(.9, .95), eps=1e-8,
                     weight_decay=.1, loss_scale=scaler, export_dtype=torch.float16, sync=True)
    ora = OracleWindow(masters)
    outs = None
    for t in range(1, steps + 1):
        grads = bench.config2_grads("cpu", 1000 + t, shapes)
        assert opt.step([g.to(DEV) for g in grads]) is True
        outs = ora.step(grads, lambda i, step: R.torch_adamw_hp(3e-4, .9, .95, 1e-8, .1, step,
                                                                scale=65536.), R.DTYPE_F16)
        if t in check_at or t == steps:
            ora.check(opt, f"config2 step {t}")
            for i, o in enumerate(outs):
                assert_same_bits(export_bits(opt.exports[i]), o.view(np.uint16),
                                 f"step {t} export[{i}]")
            print(f"config 2 step {t}: masters, moments, export bit-exact", flush=True)
    assert scaler.scale == 65536. and scaler.good_steps == steps


def test_config2_window_reduced_20_steps():
    _config2_run([(768, 384), (768, 384), (384, 768)], steps=20, seed=3)


def test_config2_window_full_size_20_steps():
    """BASELINE config 2 as stated: N = 56,623,104 at the real shapes, 20 steps, bit-exact
    vs the oracle at step 10 and at the end (masters, moments, clocks, FP16 export)."""
    _config2_run(None, steps=20, seed=0, check_at=(10,))


def test_config3_tied_embedding_full_size_20_steps():
    """BASELINE config 3 as stated: [65536, 3072] BF16 sparse-row grads (a fresh Zipf draw
    per step), wd 0, BF16 export, 20 steps; every row decays/updates.  Bit-exact vs the
    oracle at step 10 and at the end."""
    from oracle import reference as R
    w0 = torch.randn(65536, 3072, generator=torch.Generator().manual_seed(4)) * .02
    opt = FusedAdamW([w0.to(DEV)], lr=3e-4, betas=(.9, .95), eps=1e-8, weight_decay=0.0,
                     export_dtype=torch.bfloat16, sync=True)
    ora = OracleWindow([w0])
    for t in range(1, 21):
        g, active = bench.config3_embedding_grad(7000 + t)
        assert 100 < active.numel() < 4096
        assert opt.step([g.to(DEV)]) is True
        outs = ora.step([g], lambda i, step: R.torch_adamw_hp(3e-4, .9, .95, 1e-8, 0.0, step),
                        R.DTYPE_BF16)
        del g
        if t in (10, 20):
            ora.check(opt, f"config3 step {t}")
            assert_same_bits(export_bits(opt.exports[0]), outs[0], f"step {t} export")
            print(f"config 3 step {t}: masters, moments, export bit-exact", flush=True)
    # property: a row that never had a gradient keeps m = v = 0 and w = w0 exactly
    p = opt.param_groups[0]["params"][0]
    st = opt.state[p]
    zero_rows = (st["exp_avg_sq"].abs().sum(1) == 0).nonzero().flatten()[:64].cpu()
    assert zero_rows.numel() > 0
    assert torch.equal(p.detach()[zero_rows.to(DEV)].cpu(), w0[zero_rows])


@pytest.mark.parametrize("shapes", [[(768, 384), (768, 384), (384, 768)], None],
                         ids=["reduced", "full"])
def test_config4_overflow_skip_sequence(golden_dir, shapes):
    """Skip decisions, untouched state on skipped steps and the scale sequence, bit-exact."""
    from oracle import reference as R
    cfg = json.loads((golden_dir / "loss_scale.json").read_text())["config4"]
    if shapes is None:
        masters = bench.config2_window("cpu", 0)
    else:
        masters = [torch.randn(s, generator=torch.Generator().manual_seed(20 + i)) * .02
                   for i, s in enumerate(shapes)]
    shapes = [tuple(m.shape) for m in masters]
    scaler = DynamicLossScale(cfg["initial"], cfg["growth_interval"])
    oscaler = R.LossScale(cfg["initial"], cfg["growth_interval"])
    opt = FusedAdamW([m.to(DEV) for m in masters], lr=3e-4, betas=(.9, .95), eps=1e-8,
                     weight_decay=.1, loss_scale=scaler, export_dtype=torch.float16, sync=True)
    ora = OracleWindow(masters)
    rng = np.random.RandomState(44)
    seen = []
    for t in range(1, cfg["steps"] + 1):
        seen.append(scaler.scale)
        assert scaler.scale == oscaler.scale
        grads = bench.config2_grads("cpu", 2000 + t, shapes, scale=scaler.scale)
        if t in cfg["overflow_steps"]:
            for _ in range(int(rng.randint(1, 9))):
                k = int(rng.randint(len(grads)))
                flat = grads[k].view(-1)
                flat[int(rng.randint(flat.numel()))] = float(rng.choice([np.inf, -np.inf, np.nan]))
        decision = any(R.nonfinite_any(to_oracle(g)) for g in grads)
        before = [p.detach().clone() for p in opt.param_groups[0]["params"]]
        before_exp = [e.clone() for e in opt.exports]
        applied = opt.step([g.to(DEV) for g in grads])
        assert applied is (not decision)
        if decision:
            oscaler.overflow()
            for p, b in zip(opt.param_groups[0]["params"], before):
                assert torch.equal(p, b)
            for e, b in zip(opt.exports, before_exp):
                assert torch.equal(e, b)
        else:
            oscaler.success()
            sc = seen[-1]
            ora.step(grads, lambda i, step: R.torch_adamw_hp(3e-4, .9, .95, 1e-8, .1, step,
                                                             scale=sc), R.DTYPE_F16)
    assert seen == cfg["scale_before_step"]
    assert scaler.state_dict() == oscaler.state_dict()
    assert opt.skipped_steps == len(cfg["overflow_steps"])
    ora.check(opt, "config4")


def test_none_grad_leaves_param_and_clock():
    """sparse_disk.py:1-5: no gradient -> no update, no clock advance."""
    a = torch.randn(1000, generator=torch.Generator().manual_seed(1)).to(DEV)
    b = torch.randn(1000, generator=torch.Generator().manual_seed(2)).to(DEV)
    b0 = b.clone()
    opt = FusedAdamW([a, b], lr=1e-3, sync=True)
    g = torch.randn(1000, device=DEV) * 1e-3
    assert opt.step([g, None])
    assert opt.step([g, None])
    assert opt.state[a]["step"] == 2 and opt.state[b]["step"] == 0
    assert torch.equal(b, b0)
    assert opt.step([None, g])
    assert opt.state[b]["step"] == 1


def test_state_dict_interchanges_with_torch_adamw():
    """A torch.optim.AdamW state dict loads into FusedAdamW and the runs continue identically."""
    gen = torch.Generator().manual_seed(6)
    w = torch.randn(5000, generator=gen) * .02
    grads = [torch.randn(5000, generator=gen) * 1e-3 for _ in range(4)]
    p = torch.nn.Parameter(w.clone())
    topt = torch.optim.AdamW([p], lr=1e-3, betas=(.9, .95), weight_decay=.1, foreach=False)
    for g in grads[:2]:
        p.grad = g.clone()
        topt.step()
    q = p.detach().clone().to(DEV)
    opt = FusedAdamW([q], lr=1e-3, betas=(.9, .95), weight_decay=.1)
    sd = topt.state_dict()
    opt.load_state_dict(sd)
    assert opt.state[q]["step"] == 2
    for g in grads[2:]:
        p.grad = g.clone()
        topt.step()
        opt.step([g.to(DEV)])
    opt.resolve()
    assert opt.state[q]["step"] == 4
    assert torch.equal(opt.state[q]["exp_avg"].cpu(), topt.state[p]["exp_avg"])
    assert torch.equal(opt.state[q]["exp_avg_sq"].cpu(), topt.state[p]["exp_avg_sq"])
    assert (q.cpu() - p.detach()).abs().max() <= 1e-6 * p.detach().abs().max()
    back = opt.state_dict()
    assert float(back["state"][0]["step"]) == 4.0



def test_arena_layout_gives_identical_steps():
    """arena=True moves masters, moments and exports into one allocation: the steps,
    the exports and the state dict are bit-identical to separate allocations, and each
    parameter object keeps its identity with its data in the arena."""
    shapes = [(1024, 1024), (3072,), (768, 384), (2048, 1024), (5,)]
    gen = torch.Generator().manual_seed(70)
    masters = [torch.randn(s, generator=gen) * .02 for s in shapes]
    grads = [[(torch.randn(s, generator=gen) * 1e-4 * 1024).half() for s in shapes]
             for _ in range(3)]
    runs = []
    for arena in (False, True):
        params = [torch.nn.Parameter(m.to(DEV)) for m in masters]
        groups = [{"params": params[:2], "weight_decay": .1}, {"params": params[2:]}]
        opt = FusedAdamW(groups, lr=3e-4, betas=(.9, .95), eps=1e-8, weight_decay=0.0,
                         loss_scale=1024.0, export_dtype=torch.float16, arena=arena)
        for p, m in zip(params, masters):
            assert torch.equal(p.detach().cpu(), m)
        if arena:
            base, end = opt.arena.storage.data_ptr(), opt.arena.storage.data_ptr() + opt.arena.nbytes
            for p in params:
                for t in (p, opt.state[p]["exp_avg"], opt.state[p]["exp_avg_sq"]):
                    assert base <= t.data_ptr() < end
        for gs in grads:
            opt.step([g.to(DEV) for g in gs])
        opt.resolve()
        runs.append((params, opt))
    (pa, a), (pb, b) = runs
    for p, q in zip(pa, pb):
        assert torch.equal(p, q)
        for k in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(a.state[p][k], b.state[q][k])
        assert a.state[p]["step"] == b.state[q]["step"] == 3
    for e, f in zip(a.exports, b.exports):
        assert torch.equal(e, f)
    sa, sb = a.state_dict(), b.state_dict()
    for i in sa["state"]:
        assert torch.equal(sa["state"][i]["exp_avg_sq"], sb["state"][i]["exp_avg_sq"])


def test_new_gradient_buffers_swap_pointers_only():
    """A new gradient buffer every step (autograd with set_to_none) reuses the launch
    table with swapped pointers and gives the same bytes as one reused buffer; a size
    mismatch is rejected before anything is enqueued."""
    shapes = [(300, 70), (4099,)]
    gen = torch.Generator().manual_seed(71)
    masters = [torch.randn(s, generator=gen) * .02 for s in shapes]
    grads = [[torch.randn(s, generator=gen).half() for s in shapes] for _ in range(4)]
    a = FusedAdamW([m.to(DEV) for m in masters], lr=1e-3, loss_scale=8.0)
    b = FusedAdamW([m.to(DEV) for m in masters], lr=1e-3, loss_scale=8.0)
    held = [g.to(DEV) for g in grads[0]]
    tables = set()
    for gs in grads:
        a.step([g.to(DEV) for g in gs])
        tables.add(id(a._cache[0]))
        for h, g in zip(held, gs):
            h.copy_(g.to(DEV))
        b.step(held)
    a.resolve()
    b.resolve()
    assert len(tables) == 1
    for p, q in zip(a.param_groups[0]["params"], b.param_groups[0]["params"]):
        assert torch.equal(p, q)
        assert torch.equal(a.state[p]["exp_avg_sq"], b.state[q]["exp_avg_sq"])
    with pytest.raises(ValueError):
        a._cache[0].rebind_grads([torch.zeros(10, dtype=torch.half, device=DEV), held[1]])


@pytest.mark.parametrize("prev_inf,now_inf,scale,count", [
    (0, 0, 1024.0, 2), (1, 0, 1024.0, 2), (0, 1, 1024.0, 2), (1, 1, 1024.0, 2),
    (1, 0, 1.0, 2), (0, 0, 2.0 ** 15, 0), (1, 0, 512.0, 0)],
    ids=["clean", "prev-overflow", "now-overflow", "both", "fatal", "close-only", "close-only-inf"])
def test_fused_detector_close_equals_separate_launches(prev_inf, now_inf, scale, count):
    """morph_nonfinite_or_close(slot) leaves the state block and the clocks byte-identical
    to morph_step_end(slot ^ 1) followed by the detector into found_inf[slot]."""
    from morph_amd import kernels
    from morph_amd.control import StepControl
    gen = torch.Generator().manual_seed(80)
    grads = [torch.randn(1000 + 37 * k, generator=gen).half() for k in range(count)]
    if now_inf:
        grads[0][17] = float("inf")
    grads = [g.to(DEV) for g in grads]
    blocks = []
    for fused in (False, True):
        ctl = StepControl(DEV, 4, DynamicLossScale(scale, growth_interval=3))
        st = ctl.read()
        st.good_steps = 2  # the next success grows the scale
        st.found_inf[1] = prev_inf
        ctl.state.copy_(torch.frombuffer(bytearray(bytes(st)), dtype=torch.uint8))
        ctl.clocks.copy_(torch.tensor([5, 6, 7, 8]))
        clock_list = torch.tensor([0, 2, 3], dtype=torch.int32, device=DEV)
        if fused:
            kernels.nonfinite_or_close(grads, ctl.state, 0, ctl.clocks, clock_list)
        else:
            kernels.step_end(ctl.state, ctl.clocks, clock_list, slot=1)
            kernels.nonfinite_or(grads, ctl.found_inf_ptr(0))
        torch.cuda.synchronize()
        blocks.append((ctl.state.cpu(), ctl.clocks.cpu(), ctl.read()))
    (sa, ca, a), (sb, cb, b) = blocks
    assert torch.equal(sa, sb) and torch.equal(ca, cb)
    assert b.found_inf[0] == now_inf and b.found_inf[1] == 0
    assert b.last_found_inf == prev_inf
    if prev_inf and scale <= 1.0:
        assert b.fatal == 1 and cb.tolist() == [5, 6, 7, 8]
    elif prev_inf:
        assert b.scale == scale / 2 and b.skipped == 1 and cb.tolist() == [5, 6, 7, 8]
    else:
        assert b.scale == min(2 * scale, 65536.0) and b.applied == 1
        assert cb.tolist() == [6, 6, 8, 9]


def test_steps_on_alternating_streams_equal_one_stream(golden_dir):
    """A pending step close is enqueued on the stream of its own step when the next step
    runs on another stream: 16 config-4 steps alternating between two streams (each
    waiting for the other) end where the step-by-step run ends."""
    cfg = json.loads((golden_dir / "loss_scale.json").read_text())["config4"]
    shapes = [(512, 256), (1000,)]
    masters = [torch.randn(s, generator=torch.Generator().manual_seed(90 + i)) * .02
               for i, s in enumerate(shapes)]
    streams = [torch.cuda.Stream(DEV), torch.cuda.Stream(DEV)]
    runs = []
    for alternate in (False, True):
        scaler = DynamicLossScale(cfg["initial"], cfg["growth_interval"])
        opt = FusedAdamW([m.to(DEV) for m in masters], lr=3e-4, betas=(.9, .95),
                         weight_decay=.1, loss_scale=scaler, export_dtype=torch.float16,
                         sync=not alternate)
        rng = np.random.RandomState(46)
        for t in range(1, cfg["steps"] + 1):
            grads = [g.to(DEV) for g in _config4_grads(shapes, rng, t, cfg["scale_before_step"][t - 1],
                                                       cfg["overflow_steps"])]
            if alternate:
                s = streams[t % 2]
                s.wait_stream(torch.cuda.current_stream(DEV))
                s.wait_stream(streams[(t + 1) % 2])
                opt.step(grads, stream=s)
                for g in grads:
                    g.record_stream(s)
            else:
                opt.step(grads)
        torch.cuda.current_stream(DEV).wait_stream(streams[0])
        torch.cuda.current_stream(DEV).wait_stream(streams[1])
        opt.resolve()
        runs.append((opt, scaler))
    (a, sa), (b, sb) = runs
    assert sa.state_dict() == sb.state_dict() and sb.scale == cfg["final_scale"]
    assert a.skipped_steps == b.skipped_steps == 3
    for p, q in zip(a.param_groups[0]["params"], b.param_groups[0]["params"]):
        assert torch.equal(p, q)
        assert torch.equal(a.state[p]["exp_avg_sq"], b.state[q]["exp_avg_sq"])
        assert a.state[p]["step"] == b.state[q]["step"] == 13


def test_checked_and_detector_steps_interleave(golden_dir):
    """Steps whose flag comes from the producer (checked=True, flag written into
    opt.found_inf) interleaved with steps that run the detector, overflows on both
    kinds: the same bytes, clocks and scale as the step-by-step run."""
    cfg = json.loads((golden_dir / "loss_scale.json").read_text())["config4"]
    shapes = [(384, 200), (777,)]
    masters = [torch.randn(s, generator=torch.Generator().manual_seed(95 + i)) * .02
               for i, s in enumerate(shapes)]
    runs = []
    for sync in (True, False):
        scaler = DynamicLossScale(cfg["initial"], cfg["growth_interval"])
        opt = FusedAdamW([m.to(DEV) for m in masters], lr=3e-4, betas=(.9, .95),
                         weight_decay=.1, loss_scale=scaler, export_dtype=torch.bfloat16, sync=sync)
        rng = np.random.RandomState(47)
        for t in range(1, cfg["steps"] + 1):
            grads = [g.to(DEV) for g in _config4_grads(shapes, rng, t, cfg["scale_before_step"][t - 1],
                                                       cfg["overflow_steps"])]
            if t % 3 == 0:  # the producer tested the gradients
                bad = any(not torch.isfinite(g).all() for g in grads)
                if bad:
                    opt.found_inf.fill_(1)
                opt.step(grads, checked=True)
            else:
                opt.step(grads)
        opt.resolve()
        runs.append((opt, scaler))
    (a, sa), (b, sb) = runs
    assert sa.state_dict() == sb.state_dict() and sb.scale == cfg["final_scale"]
    assert a.skipped_steps == b.skipped_steps == 3 and b.applied_steps == 13
    for p, q in zip(a.param_groups[0]["params"], b.param_groups[0]["params"]):
        assert torch.equal(p, q)
        assert torch.equal(a.state[p]["exp_avg"], b.state[q]["exp_avg"])
    for e, f in zip(a.exports, b.exports):
        assert torch.equal(e, f)


def test_fused_close_with_a_detector_over_several_launches():
    """400 tensors need three detector launches (160 tensors each) and nine AdamW
    launches; the previous step's close rides in exactly one of them.  Eight steps,
    two of them poisoned in the last launch's tensors, end where the step-by-step run ends."""
    gen = torch.Generator().manual_seed(97)
    sizes = [int(torch.randint(1, 3000, (1,), generator=gen)) for _ in range(400)]
    masters = [torch.randn(n, generator=gen) * .02 for n in sizes]
    steps = [[(torch.randn(n, generator=gen) * 1e-3 * 256).half() for n in sizes] for _ in range(8)]
    steps[2][395][0] = float("nan")
    steps[5][399][-1] = float("-inf")
    runs = []
    for sync in (True, False):
        scaler = DynamicLossScale(256.0, growth_interval=3)
        opt = FusedAdamW([m.to(DEV) for m in masters], lr=1e-3, betas=(.9, .95), weight_decay=.1,
                         loss_scale=scaler, sync=sync)
        for gs in steps:
            opt.step([g.to(DEV) for g in gs])
        opt.resolve()
        runs.append((opt, scaler))
    (a, sa), (b, sb) = runs
    assert sa.state_dict() == sb.state_dict()
    assert a.skipped_steps == b.skipped_steps == 2 and b.applied_steps == 6
    for p, q in zip(a.param_groups[0]["params"], b.param_groups[0]["params"]):
        assert torch.equal(p, q)
        assert a.state[p]["step"] == b.state[q]["step"] == 6


@pytest.mark.parametrize("count,size", [(1, 1 << 24), (200, 1 << 16)], ids=["one", "split"])
def test_dispatch_timer_stamps_the_adamw_launches(count, size):
    """Events stamped by the AdamW dispatch itself (hipExtLaunchKernel) time the pass: each
    interval lies inside the events recorded around the launch (which may also hold host
    delays) and is no shorter than the HBM traffic of the FP32 state at the 8 TB/s peak
    (24 B/param: master and moments read and written); a call split into several launches
    (200 tensors) runs from the first start to the last end."""
    from morph_amd.kernels import DispatchTimer
    gen = torch.Generator(device=DEV).manual_seed(98)
    ps = [torch.randn(size, generator=gen, device=DEV) * .02 for _ in range(count)]
    gs = [torch.randn(size, generator=gen, device=DEV).half() for _ in range(count)]
    opt = FusedAdamW(ps, lr=1e-3)
    opt.step(gs)
    opt.dispatch_timer = DispatchTimer(4, DEV)
    opt.kernel_timer = []
    for _ in range(4):
        opt.step(gs)
    torch.cuda.synchronize()
    stamped = opt.dispatch_timer.elapsed_ms()
    around = [a.elapsed_time(b) for a, b in opt.kernel_timer]
    assert len(stamped) == 4
    floor_ms = 24 * count * size / 8e12 * 1e3
    for x, y in zip(stamped, around):
        assert floor_ms <= x <= y + 0.002, (x, y, floor_ms)
    with pytest.raises(RuntimeError):
        opt.step(gs)  # the timer holds four pairs
    opt.dispatch_timer = None
    opt.resolve()
    assert opt.applied_steps == 5

def _config4_grads(shapes, rng, t, scale, overflow_steps):
    grads = bench.config2_grads("cpu", 2000 + t, shapes, scale=scale)
    if t in overflow_steps:
        for _ in range(int(rng.randint(1, 9))):
            k = int(rng.randint(len(grads)))
            flat = grads[k].view(-1)
            flat[int(rng.randint(flat.numel()))] = float(rng.choice([np.inf, -np.inf, np.nan]))
    return grads


def test_async_steps_equal_synchronous_steps(golden_dir):
    """16 steps enqueued back to back (no host round trip) end in the same bytes, clocks
    and loss scale as the step-by-step run, though the host learns the outcomes only at
    the end.  Gradients are pre-scaled with the scale sequence the skips imply."""
    cfg = json.loads((golden_dir / "loss_scale.json").read_text())["config4"]
    shapes = [(512, 256), (256, 512), (1000,)]
    masters = [torch.randn(s, generator=torch.Generator().manual_seed(60 + i)) * .02
               for i, s in enumerate(shapes)]
    runs = []
    for sync in (True, False):
        scaler = DynamicLossScale(cfg["initial"], cfg["growth_interval"])
        opt = FusedAdamW([m.to(DEV) for m in masters], lr=3e-4, betas=(.9, .95),
                         weight_decay=.1, loss_scale=scaler, export_dtype=torch.float16, sync=sync)
        rng = np.random.RandomState(45)
        for t in range(1, cfg["steps"] + 1):
            grads = _config4_grads(shapes, rng, t, cfg["scale_before_step"][t - 1],
                                   cfg["overflow_steps"])
            opt.step([g.to(DEV) for g in grads])
        opt.resolve()
        runs.append((opt, scaler))
    (a, sa), (b, sb) = runs
    assert sa.state_dict() == sb.state_dict() and sa.scale == cfg["final_scale"]
    assert a.skipped_steps == b.skipped_steps == 3 and a.applied_steps == b.applied_steps == 13
    for p, q in zip(a.param_groups[0]["params"], b.param_groups[0]["params"]):
        assert torch.equal(p, q)
        for k in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(a.state[p][k], b.state[q][k])
        assert a.state[p]["step"] == b.state[q]["step"] == 13
    for e, f in zip(a.exports, b.exports):
        assert torch.equal(e, f)


def test_overflow_at_minimum_scale_raises_and_freezes_state():
    """precision.py:9-10: overflow at scale <= 1 raises with the state unchanged; on the
    device every step after it is a no-op until the host sees the error."""
    w = torch.randn(4096, generator=torch.Generator().manual_seed(3)).to(DEV)
    scaler = DynamicLossScale(2., growth_interval=2000)
    opt = FusedAdamW([w], lr=1e-3, loss_scale=scaler)
    good = torch.randn(4096, device=DEV).half()
    bad = good.clone()
    bad[5] = float("inf")
    opt.step([good])
    opt.step([bad])   # scale 2 -> 1
    opt.step([bad])   # at scale 1: the reference raises here
    before = w.clone()
    opt.step([good])  # enqueued before the host knows: must change nothing
    with pytest.raises(FloatingPointError, match="minimum loss scale"):
        opt.resolve()
    assert torch.equal(w, before)
    assert scaler.scale == 1.0 and opt.state[w]["step"] == 1


def test_fixed_scale_and_raise_policy():
    """A float loss scale never changes; on_overflow='raise' raises before any mutation."""
    w = torch.randn(3000, generator=torch.Generator().manual_seed(4)).to(DEV)
    opt = FusedAdamW([w], lr=1e-3, loss_scale=1024.0, on_overflow="raise")
    g = (torch.randn(3000, device=DEV) * 1e-3 * 1024).half()
    assert opt.step([g]) is True
    before = w.clone()
    g[0] = float("nan")
    with pytest.raises(FloatingPointError, match="nonfinite gradient"):
        opt.step([g])
    assert torch.equal(w, before) and opt.state[w]["step"] == 1
    g[0] = 0.0
    assert opt.step([g]) is True and opt.state[w]["step"] == 2


def test_loss_scale_growth_on_device_matches_host_rule():
    """growth_interval 3: the scale doubles every 3 clean steps, capped at 65536."""
    from oracle import reference as R
    w = torch.randn(2048, generator=torch.Generator().manual_seed(5)).to(DEV)
    scaler = DynamicLossScale(16384., growth_interval=3)
    oscaler = R.LossScale(16384., 3)
    opt = FusedAdamW([w], lr=1e-3, loss_scale=scaler)
    for t in range(14):
        opt.step([(torch.randn(2048, device=DEV) * 1e-4).half()])
        oscaler.success()
    opt.resolve()
    assert scaler.state_dict() == oscaler.state_dict() and scaler.scale == 65536.


@pytest.mark.parametrize("mode", ["host_scale", "device_scale"])
def test_loss_scaled_by_the_exposed_scale_across_overflow_and_growth(mode):
    """A training loop scales each step's loss by the scale the API exposes -- the host
    DynamicLossScale's `scale` (which settles the queued steps when read) or the
    optimizer's device scale (scale_loss / loss_scale_tensor, no wait) -- and never
    calls resolve().  With growth every 3 clean steps and overflows at steps 4 and 9
    the scale moves 1024 -> 2048 -> 1024 -> 2048 -> 1024 ..., and every applied step
    must unscale by exactly the factor its gradient was scaled with: bit-exact
    against the oracle running the reference's loop (disk.py:483-496)."""
    from oracle import reference as R
    n = 5000
    w0 = torch.randn(n, generator=torch.Generator().manual_seed(31)) * .02
    scaler = DynamicLossScale(1024., growth_interval=3)
    w = w0.to(DEV)
    opt = FusedAdamW([w], lr=3e-4, betas=(.9, .95), weight_decay=.1, loss_scale=scaler)
    gen = torch.Generator().manual_seed(32)
    true_grads = [torch.randn(n, generator=gen) * 1e-4 for _ in range(12)]
    ow, om, ov = w0.numpy().copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    oscaler, ot, seen = R.LossScale(1024., 3), 0, []
    for k, g in enumerate(true_grads):
        if mode == "host_scale":
            scale = scaler.scale                     # the reference reads scaler.scale
            g16 = (g * scale).half().to(DEV)         # backward of loss * scale
        else:
            g16 = opt.scale_loss(g.to(DEV)).half()   # the same product on the GPU
        if k + 1 in (4, 9):
            g16[17] = float("inf")
        opt.step([g16])
        seen.append(oscaler.scale)
        o16 = (g * oscaler.scale).half()
        if k + 1 in (4, 9):
            oscaler.overflow()
            continue
        ot += 1
        R.adamw(o16.numpy(), ow, om, ov,
                R.torch_adamw_hp(3e-4, .9, .95, 1e-8, .1, ot, scale=oscaler.scale))
        oscaler.success()
    assert seen[:10] == [1024.] * 3 + [2048., 1024., 1024., 1024., 2048., 2048., 1024.]
    assert scaler.scale == oscaler.scale and scaler.good_steps == oscaler.good_steps
    assert_same_bits(w.cpu().numpy(), ow, "master")
    assert_same_bits(opt.state[w]["exp_avg"].cpu().numpy(), om, "exp_avg")
    assert opt.state[w]["step"] == ot == 10


@pytest.mark.parametrize("how", ["assign", "load_state_dict"])
def test_caller_edits_of_the_scaler_reach_the_device(how):
    """disk.py:245/509 and single_pass.py:183-184 restore the scaler on resume: a scale
    set on the host between steps (while earlier steps are still queued) is the scale
    the next step unscales by, bit-exact against the oracle, and the host keeps it."""
    from oracle import reference as R
    n = 3000
    w0 = torch.randn(n, generator=torch.Generator().manual_seed(36)) * .02
    w = w0.to(DEV)
    scaler = DynamicLossScale(65536., growth_interval=2000)
    opt = FusedAdamW([w], lr=3e-4, betas=(.9, .95), weight_decay=.1, loss_scale=scaler)
    gen = torch.Generator().manual_seed(37)
    grads = [torch.randn(n, generator=gen) * 1e-4 for _ in range(4)]
    ow, om, ov = w0.numpy().copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for t in (1, 2):  # queued, not resolved
        g16 = (grads[t - 1] * 65536.).half()
        opt.step([g16.to(DEV)])
        R.adamw(g16.numpy(), ow, om, ov, R.torch_adamw_hp(3e-4, .9, .95, 1e-8, .1, t, scale=65536.))
    if how == "assign":
        scaler.scale = 1024.
        expect_good = 2          # the queued steps' successes stand
    else:
        scaler.load_state_dict({"scale": 1024., "good_steps": 7, "growth_interval": 2000})
        expect_good = 7
    assert scaler.scale == 1024.
    for t in (3, 4):
        g16 = (grads[t - 1] * 1024.).half()
        opt.step([g16.to(DEV)])
        R.adamw(g16.numpy(), ow, om, ov, R.torch_adamw_hp(3e-4, .9, .95, 1e-8, .1, t, scale=1024.))
    opt.resolve()
    assert opt.loss_scale_tensor().item() == 1024.
    assert scaler.scale == 1024. and scaler.good_steps == expect_good + 2
    assert_same_bits(w.cpu().numpy(), ow, "master")
    assert_same_bits(opt.state[w]["exp_avg_sq"].cpu().numpy(), ov, "exp_avg_sq")


def test_after_the_minimum_scale_raise_the_optimizer_goes_on():
    """precision.py:9-11 raises and leaves the scaler usable: after the raise is reported
    (once), state_dict() works, load_state_dict() restores, and the next step applies."""
    w = torch.randn(4096, generator=torch.Generator().manual_seed(33)).to(DEV)
    scaler = DynamicLossScale(1., growth_interval=2000)
    opt = FusedAdamW([w], lr=1e-3, loss_scale=scaler)
    good = torch.randn(4096, device=DEV).half()
    bad = good.clone()
    bad[9] = float("nan")
    opt.step([good])
    saved = opt.state_dict()
    saved = {"state": {k: {kk: vv.clone() for kk, vv in v.items()} for k, v in saved["state"].items()},
             "param_groups": saved["param_groups"]}
    w_saved = w.clone()
    opt.step([bad])                      # overflow at scale 1: the reference raises here
    snapshot = opt.state_dict()          # reading the state does not raise
    assert snapshot["state"][0]["step"].item() == 1.0
    with pytest.raises(FloatingPointError, match="minimum loss scale"):
        opt.resolve()
    opt.resolve()                        # reported once
    opt.step([good])                     # and the optimizer goes on
    opt.resolve()
    assert opt.state[w]["step"] == 2 and scaler.scale == 1.0
    # fatal again, then restore a saved state: the restored optimizer steps normally
    opt.step([bad])
    w.copy_(w_saved)
    opt.load_state_dict(saved)
    opt.step([good])
    opt.resolve()
    assert opt.state[w]["step"] == 2


def test_bias_tables_grow_past_4096_steps_on_a_side_stream():
    """The bias-correction tables double at step 4097; the old ones stay valid for the
    side stream's queued launches.  Result bit-exact against the oracle."""
    from oracle import reference as R
    n = 1000
    w0 = torch.randn(n, generator=torch.Generator().manual_seed(34)) * .02
    w = w0.to(DEV)
    opt = FusedAdamW([w], lr=1e-4, betas=(.9, .95), weight_decay=.1)
    g = (torch.randn(n, generator=torch.Generator().manual_seed(35)) * 1e-3)
    gd = g.to(DEV)
    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    steps = 4100
    for _ in range(steps):
        opt.step([gd], stream=side)
    opt.resolve()
    torch.cuda.synchronize()
    ow, om, ov = w0.numpy().copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for t in range(1, steps + 1):
        R.adamw(g.numpy(), ow, om, ov, R.torch_adamw_hp(1e-4, .9, .95, 1e-8, .1, t))
    assert opt.state[w]["step"] == steps
    assert_same_bits(w.cpu().numpy(), ow, "master")
    assert_same_bits(opt.state[w]["exp_avg_sq"].cpu().numpy(), ov, "exp_avg_sq")
