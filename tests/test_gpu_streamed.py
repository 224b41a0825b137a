"""The streamed engines' optimizer path: FP32 masters on the CPU, gradients in CPU p.grad.

morph/training/runner.py builds the model on the CPU for engine='dls'/'async' (:41),
constructs HybridMuonAdamW(model, lr, muon_lr) or torch.optim.AdamW(model.parameters(),
lr, weight_decay=.01, foreach=False) on it (:44-46), and per step calls
zero_grad(set_to_none=True), lets StreamTrainEngine.backward leave the gradients in CPU
p.grad (Slot.flush, engine.py:75-88: p.grad = value.clone()), clips on the CPU (:100)
and calls step() (:101); checkpoints hold optimizer.state_dict() (:66-74).  Here the
same calls run with the state resident in HBM (morph_amd.staging):
  * FusedAdamW on CPU masters: bit-exact against the oracle and against the same
    optimizer on device-resident masters, config 1 for 10 steps;
  * HybridMuonAdamW on a CPU model through the runner's call sequence: the AdamW group
    bit-exact against the oracle, the Muon matrices bit-exact against the
    device-resident optimizer fed the same gradients, state_dict on the CPU and a
    save/restore that continues identically;
  * the non-finite gate: raise with CPU masters, momenta and moments untouched;
  * HostStaging round trips with small chunks, subsets and odd sizes, with pageable,
    pinned (direct DMA) and mixed host tensors; pinned masters (pin_host_tensors) give
    the same bits as pageable ones through both optimizers;
  * two optimizers interleaved over the shared per-device copy and side streams;
  * resident_masters=True: the masters' mirrors stay in HBM between steps and only
    changed host masters go up again (in-place ops, rebound storage, load_state_dict,
    and writes through .data with invalidate_masters()), bit-exact.
"""
import copy

import numpy as np
import pytest
import torch
from torch import nn

from morph_amd import FusedAdamW, pin_host_tensors
from morph_amd.muon import HybridMuonAdamW
from morph_amd.staging import HostStaging
from tests.golden.make_golden import CONFIG1, config1_inputs
from tests.helpers import assert_same_bits

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _pin(pin, tensors):
    """Pinned copies of all, every other or none of the tensors."""
    return [t.pin_memory() if pin == "all" or (pin == "some" and k % 2) else t
            for k, t in enumerate(tensors)]


@pytest.mark.parametrize("pin", ["none", "all", "some"])
def test_host_staging_round_trips(pin):
    gen = torch.Generator().manual_seed(1)
    shapes = [(7,), (1000, 3), (1,), (64, 65), (4099,)]
    st = HostStaging(shapes, torch.float32, DEV, chunk_elements=1000)
    host = _pin(pin, [torch.randn(s, generator=gen) for s in shapes])
    st.upload(host)
    for h, v in zip(host, st.views):
        assert torch.equal(v.cpu(), h)
    # a subset: only those mirrors change, chunks span tensor boundaries
    new = _pin(pin, [torch.randn(shapes[i], generator=gen) for i in (1, 3)])
    st.upload(new, [1, 3])
    for i, v in enumerate(st.views):
        expect = {1: new[0], 3: new[1]}.get(i, host[i])
        assert torch.equal(v.cpu(), expect), i
    out = _pin(pin, [torch.empty(s) for s in shapes])
    st.download(out)
    for o, v in zip(out, st.views):
        assert torch.equal(o, v.cpu())
    st.views[2].fill_(5.0)
    one = _pin(pin, [torch.zeros(1)])
    st.download(one, [2])
    assert float(one[0]) == 5.0
    assert st.bytes_h2d > 0 and st.bytes_d2h > 0


@pytest.mark.parametrize("pin", ["none", "all", "some"])
def test_host_staging_pipeline_updates_every_chunk(pin):
    """pipeline(): every listed tensor goes up, through the launch (x -> 2 x + 1 on the
    device, per chunk) and back into the same host tensor; unlisted mirrors untouched."""
    gen = torch.Generator().manual_seed(2)
    shapes = [(300,), (64, 65), (1,), (2000,), (77, 3)]
    st = HostStaging(shapes, torch.float32, DEV, chunk_elements=512)
    host = _pin(pin, [torch.randn(s, generator=gen) for s in shapes])
    before = [h.clone() for h in host]
    st.upload(host)
    st.views[2].fill_(9.0)
    which = [0, 1, 3, 4]
    seen = []

    def launch(lo, hi, pieces, stream):
        seen.extend(i for i, _, _ in pieces)
        with torch.cuda.stream(stream):
            for i, s, e in pieces:
                v = st.views[i].view(-1)[s:e]
                v.mul_(2.0).add_(1.0)

    st.pipeline([host[i] for i in which], which, launch)
    assert sorted(set(seen)) == which
    for i in which:
        assert torch.equal(host[i], before[i] * 2.0 + 1.0), i
        assert torch.equal(st.views[i].cpu(), host[i]), i
    assert torch.equal(host[2], before[2]) and float(st.views[2]) == 9.0


def test_pin_host_tensors_moves_data_in_place():
    gen = torch.Generator().manual_seed(3)
    lin = nn.Linear(16, 8)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(8, 16, generator=gen))
    w0, b0 = lin.weight.detach().clone(), lin.bias.detach().clone()
    moved = pin_host_tensors(lin.parameters())
    assert moved == (8 * 16 + 8) * 4
    assert lin.weight.is_pinned() and lin.bias.is_pinned()
    assert isinstance(lin.weight, nn.Parameter)
    assert torch.equal(lin.weight.detach(), w0) and torch.equal(lin.bias.detach(), b0)
    assert pin_host_tensors(lin.parameters()) == 0  # already pinned
    base = torch.zeros(10)
    with pytest.raises(ValueError, match="share host storage"):
        pin_host_tensors([base[:5], base[5:]])
    assert not base.is_pinned()


@pytest.mark.parametrize("chunk,pinned", [(None, False), (5000, False), (None, True),
                                          (5000, True)])
def test_fused_adamw_on_cpu_masters_config1(chunk, pinned):
    """BASELINE config 1 (param groups: wd .1 on 2-D only) with CPU masters and CPU FP32
    gradients: every step bit-exact against the oracle and against device masters.  With
    chunk=5000 the masters stream through the update in 60 chunks, most spanning two
    tensors at offsets that are not multiples of 64.  pinned: the masters live in
    page-locked memory (pin_host_tensors) and move by DMA alone."""
    from oracle import reference as R
    masters, grads = config1_inputs()
    cpu = [m.clone() for m in masters]
    if pinned:
        pin_host_tensors(cpu)
    dev = [m.to(DEV) for m in masters]
    groups = lambda ps: [dict(params=[p for p in ps if p.ndim == 2], weight_decay=CONFIG1["wd_2d"]),
                         dict(params=[p for p in ps if p.ndim == 1], weight_decay=0.0)]
    kw = dict(lr=CONFIG1["lr"], betas=CONFIG1["betas"], eps=CONFIG1["eps"])
    opt_c, opt_d = FusedAdamW(groups(cpu), **kw), FusedAdamW(groups(dev), **kw)
    if chunk is not None:
        opt_c._staging.chunk = chunk
    flat_c = [p for g in opt_c.param_groups for p in g["params"]]
    flat_d = [p for g in opt_d.param_groups for p in g["params"]]
    W = [p.numpy().ravel().copy() for p in flat_c]
    M = [np.zeros_like(w) for w in W]
    V = [np.zeros_like(w) for w in W]
    index = {id(p): i for i, p in enumerate(cpu)}
    for t in range(1, CONFIG1["steps"] + 1):
        gs = grads(t)
        for p in flat_c:
            p.grad = gs[index[id(p)]].clone()          # CPU p.grad, as Slot.flush leaves it
        for pc, pd in zip(flat_c, flat_d):
            pd.grad = pc.grad.to(DEV)
        opt_c.step()
        opt_d.step()
        for k, p in enumerate(flat_c):
            wd = CONFIG1["wd_2d"] if p.ndim == 2 else 0.0
            hp = R.torch_adamw_hp(CONFIG1["lr"], *CONFIG1["betas"], CONFIG1["eps"], wd, t)
            R.adamw(p.grad.numpy().ravel(), W[k], M[k], V[k], hp)
            assert p.device.type == "cpu"
            assert_same_bits(p.numpy().ravel(), W[k], f"master {k}, step {t}")
            assert torch.equal(p, flat_d[k].cpu())
    sd = opt_c.state_dict()
    for k in range(len(flat_c)):
        s = sd["state"][k]
        assert s["exp_avg"].device.type == "cpu" and float(s["step"]) == CONFIG1["steps"]
        assert_same_bits(s["exp_avg"].numpy().ravel(), M[k], "exp_avg")
        assert_same_bits(s["exp_avg_sq"].numpy().ravel(), V[k], "exp_avg_sq")


class Tiny(nn.Module):
    """Hidden Linear layers (Muon; both orientations), a LayerNorm and an lm_head (AdamW)."""

    def __init__(self):
        super().__init__()
        self.up = nn.Linear(64, 192, bias=True)
        self.down = nn.Linear(192, 64, bias=False)
        self.gate = nn.Linear(64, 192, bias=False)
        self.norm = nn.LayerNorm(64)
        self.lm_head = nn.Linear(64, 32, bias=False)


def _engine_grads(model, seed):
    """What StreamTrainEngine leaves behind: CPU FP32 p.grad (engine.py:82-84)."""
    gen = torch.Generator().manual_seed(seed)
    for p in model.parameters():
        p.grad = (torch.randn(p.shape, generator=gen) * 1e-3).to(p.device)


def test_hybrid_on_cpu_masters_through_the_runner_sequence():
    from oracle import reference as R
    torch.manual_seed(0)
    cpu_model = Tiny()
    dev_model = copy.deepcopy(cpu_model).to(DEV)
    opt_c = HybridMuonAdamW(cpu_model, lr=.003, muon_lr=.02)
    opt_d = HybridMuonAdamW(dev_model, lr=.003, muon_lr=.02)
    assert opt_c.host and not opt_d.host
    adam_names = [n for n, _ in cpu_model.named_parameters()
                  if n not in ("up.weight", "down.weight", "gate.weight")]
    ow = {n: p.detach().numpy().ravel().copy() for n, p in cpu_model.named_parameters()
          if n in adam_names}
    om = {n: np.zeros_like(w) for n, w in ow.items()}
    ov = {n: np.zeros_like(w) for n, w in ow.items()}
    for step in range(1, 4):
        opt_c.zero_grad(set_to_none=True)                  # runner.py:83
        opt_d.zero_grad(set_to_none=True)
        _engine_grads(cpu_model, step)                     # streaming.backward (:92)
        _engine_grads(dev_model, step)
        torch.nn.utils.clip_grad_norm_(cpu_model.parameters(), 1.0, error_if_nonfinite=True)
        torch.nn.utils.clip_grad_norm_(dev_model.parameters(), 1.0, error_if_nonfinite=True)
        for (n, pc), (_, pd) in zip(cpu_model.named_parameters(), dev_model.named_parameters()):
            pd.grad.copy_(pc.grad)  # identical clipped gradients on both sides
        opt_c.step()                                       # runner.py:101
        opt_d.step()
        for n, p in cpu_model.named_parameters():
            if n in adam_names:
                hp = R.torch_adamw_hp(.003, .9, .95, 1e-8, .01, step)
                R.adamw(p.grad.numpy().ravel(), ow[n], om[n], ov[n], hp)
    for (n, pc), (_, pd) in zip(cpu_model.named_parameters(), dev_model.named_parameters()):
        assert pc.device.type == "cpu"
        assert torch.equal(pc.detach(), pd.detach().cpu()), n
        if n in adam_names:
            assert_same_bits(pc.detach().numpy().ravel(), ow[n], n)
    sd = opt_c.state_dict()                                # runner.py:66-74 checkpoint
    assert set(sd) == {"momentum", "adam", "lr", "weight_decay"}
    assert all(m.device.type == "cpu" for m in sd["momentum"].values())
    for i, m in sd["momentum"].items():
        assert torch.equal(m, opt_d.momentum[i].cpu())
    for k, s in sd["adam"]["state"].items():
        n = adam_names[k]
        assert_same_bits(s["exp_avg"].numpy().ravel(), om[n], n)
        assert_same_bits(s["exp_avg_sq"].numpy().ravel(), ov[n], n)
    # restore into a fresh CPU model + optimizer (runner.py:62-63) and continue identically
    saved = copy.deepcopy(sd)
    model2 = copy.deepcopy(cpu_model)
    opt2 = HybridMuonAdamW(model2, lr=.003, muon_lr=.02)
    opt2.load_state_dict(saved)
    for m, o in ((cpu_model, opt_c), (model2, opt2)):
        o.zero_grad(set_to_none=True)
        _engine_grads(m, 9)
        o.step()
    for (n, p), (_, q) in zip(cpu_model.named_parameters(), model2.named_parameters()):
        assert torch.equal(p, q), n


class Uneven(nn.Module):
    """Hidden Linear layers of different sizes (one not a multiple of 64 elements)."""

    def __init__(self):
        super().__init__()
        self.a = nn.Linear(64, 192, bias=False)
        self.b = nn.Linear(192, 70, bias=False)
        self.c = nn.Linear(70, 33, bias=True)
        self.lm_head = nn.Linear(33, 16, bias=False)


@pytest.mark.parametrize("model_cls,pinned,parts", [(Tiny, False, 2), (Uneven, False, 2),
                                                    (Tiny, True, 2), (Uneven, True, 2),
                                                    (Tiny, False, 1), (Uneven, False, 3),
                                                    (Tiny, True, 5)])
def test_hybrid_on_cpu_masters_equals_device_masters(model_cls, pinned, parts):
    """Per-matrix streamed updates (each staging chunk one whole matrix, updated as it
    arrives) and the whole-batch fallback (uneven sizes, 5000-element chunks that cut
    matrices) both equal the device-resident optimizer bit for bit over three steps,
    masters and momenta, with pageable and with pinned (pin_host_tensors) masters, and
    with the matrices in 1, 2, 3 or more parts (more parts than matrices: one each)."""
    torch.manual_seed(4)
    cpu_model = model_cls()
    dev_model = copy.deepcopy(cpu_model).to(DEV)
    if pinned:
        pin_host_tensors(cpu_model.parameters())
    opt_c = HybridMuonAdamW(cpu_model, lr=.003, muon_lr=.02)
    opt_c.stream_parts = parts
    opt_d = HybridMuonAdamW(dev_model, lr=.003, muon_lr=.02)
    idx = list(range(len(opt_c.muon)))
    if model_cls is Uneven:
        opt_c._muon_masters.chunk = 5000
    assert opt_c._muon_masters.whole_tensor_chunks(idx) == (model_cls is Tiny)
    for step in range(3):
        _engine_grads(cpu_model, 10 + step)
        for (_, pc), (_, pd) in zip(cpu_model.named_parameters(), dev_model.named_parameters()):
            pd.grad = pc.grad.to(DEV)
        opt_c.step()
        opt_d.step()
    for (n, pc), (_, pd) in zip(cpu_model.named_parameters(), dev_model.named_parameters()):
        assert torch.equal(pc.detach(), pd.detach().cpu()), n
    for i, m in opt_d.momentum.items():
        assert torch.equal(opt_c.momentum[i].cpu(), m.cpu()), i


@pytest.mark.parametrize("model_cls,which,parts", [(Tiny, "all", None), (Tiny, "some", None),
                                                   (Uneven, "all", None), (Uneven, "muon", None),
                                                   (Tiny, "all", 3), (Uneven, "muon", 2)])
def test_hybrid_on_cpu_masters_takes_device_gradients(model_cls, which, parts):
    """step({p: g}) with gradients on the GPU (an engine's device stage buffers,
    engine.py:67, before Slot.flush copies them to CPU p.grad, :75-88): no gradient
    upload for those, and the same bits as the CPU-gradient step over three steps --
    masters, momenta, AdamW moments -- with every gradient on the device, every other
    one, or only the Muon ones, in the default and in fixed numbers of streamed parts.
    A parameter missing from the mapping is not stepped."""
    torch.manual_seed(5)
    model_a = model_cls()
    model_b = copy.deepcopy(model_a)
    opt_a = HybridMuonAdamW(model_a, lr=.003, muon_lr=.02)
    opt_b = HybridMuonAdamW(model_b, lr=.003, muon_lr=.02)
    opt_b.stream_parts = parts  # None: one part per 6 matrices with device gradients
    muon_ids = {id(p) for p in opt_b.muon}
    names = [n for n, _ in model_a.named_parameters()]
    for step in range(3):
        _engine_grads(model_a, 20 + step)
        skip = names[-1] if step == 1 else None   # absent from the mapping this step
        grads = {}
        for k, ((n, pa), (_, pb)) in enumerate(zip(model_a.named_parameters(),
                                                   model_b.named_parameters())):
            if n == skip:
                pa.grad = None
                continue
            on_device = (which == "all" or (which == "some" and k % 2 == 0)
                         or (which == "muon" and id(pb) in muon_ids))
            grads[pb] = pa.grad.to(DEV) if on_device else pa.grad.clone()
        before = opt_b._muon_grads.bytes_h2d
        opt_a.step()
        opt_b.step(grads)
        if which in ("all", "muon"):
            assert opt_b._muon_grads.bytes_h2d == before  # no Muon gradient went up
        assert all(p.grad is None for p in model_b.parameters())
    for (n, pa), (_, pb) in zip(model_a.named_parameters(), model_b.named_parameters()):
        assert pb.device.type == "cpu"
        assert torch.equal(pa.detach(), pb.detach()), n
    for i, m in opt_a.momentum.items():
        assert torch.equal(m.cpu(), opt_b.momentum[i].cpu()), i
    sa, sb = opt_a.state_dict()["adam"]["state"], opt_b.state_dict()["adam"]["state"]
    for k in sa:
        for key in ("exp_avg", "exp_avg_sq", "step"):
            assert torch.equal(sa[k][key], sb[k][key]), (k, key)


def test_optimizers_sharing_the_copy_streams_interleave():
    """Every staging object and the Muon side stream use one stream per role and device
    (staging.shared_stream).  Two CPU-master optimizers stepped alternately through those
    shared streams equal device-resident twins bit for bit, masters and momenta."""
    torch.manual_seed(7)
    cpu = [Tiny(), Uneven()]
    dev = [copy.deepcopy(m).to(DEV) for m in cpu]
    opt_c = [HybridMuonAdamW(m, lr=.003, muon_lr=.02) for m in cpu]
    opt_d = [HybridMuonAdamW(m, lr=.003, muon_lr=.02) for m in dev]
    assert opt_c[0]._muon_masters._copy is opt_c[1]._muon_grads._copy
    assert opt_c[0]._muon_masters._copy is opt_c[1].adam._staging._copy
    for step in range(3):
        for k, (cm, dm) in enumerate(zip(cpu, dev)):
            _engine_grads(cm, 20 + 10 * k + step)
            for (_, pc), (_, pd) in zip(cm.named_parameters(), dm.named_parameters()):
                pd.grad = pc.grad.to(DEV)
        for o in opt_c + opt_d:
            o.step()
    assert opt_c[0]._ns_stream is opt_c[1]._ns_stream
    for cm, dm, oc, od in zip(cpu, dev, opt_c, opt_d):
        for (n, pc), (_, pd) in zip(cm.named_parameters(), dm.named_parameters()):
            assert torch.equal(pc.detach(), pd.detach().cpu()), n
        for i, m in od.momentum.items():
            assert torch.equal(oc.momentum[i].cpu(), m.cpu()), i


@pytest.mark.parametrize("poisoned", ["norm.weight", "up.weight", "down.weight"])
def test_hybrid_on_cpu_masters_raises_before_any_mutation(poisoned):
    torch.manual_seed(1)
    model = Tiny()
    twin = copy.deepcopy(model)
    opt, opt2 = HybridMuonAdamW(model, lr=.003), HybridMuonAdamW(twin, lr=.003)
    for o, m in ((opt, model), (opt2, twin)):
        _engine_grads(m, 1)
        o.step()
    before = copy.deepcopy(model.state_dict())
    saved = copy.deepcopy(opt.state_dict())
    _engine_grads(model, 2)
    dict(model.named_parameters())[poisoned].grad.view(-1)[3] = float("inf")
    with pytest.raises(FloatingPointError):
        opt.step()
    for k, v in model.state_dict().items():
        assert torch.equal(v, before[k]), k
    after = opt.state_dict()
    for i, m in after["momentum"].items():
        assert torch.equal(m, saved["momentum"][i]), i
    for k, s in after["adam"]["state"].items():
        assert torch.equal(s["exp_avg"], saved["adam"]["state"][k]["exp_avg"])
    for o, m in ((opt, model), (opt2, twin)):
        _engine_grads(m, 3)
        o.step()
    for (n, p), (_, q) in zip(model.named_parameters(), twin.named_parameters()):
        assert torch.equal(p, q), n


def test_fused_adamw_on_cpu_masters_raises_before_any_mutation():
    """on_overflow="raise" with CPU masters: a non-finite gradient raises with the CPU masters
    and the moments untouched, and the next finite step equals that of an optimizer that never
    saw the poisoned one."""
    gen = torch.Generator().manual_seed(5)
    shapes = [(300, 70), (70,), (128, 300)]
    params = [torch.randn(s, generator=gen) * .02 for s in shapes]
    twin = [p.clone() for p in params]
    kw = dict(lr=1e-3, betas=(.9, .95), weight_decay=.1, on_overflow="raise")
    opt, opt2 = FusedAdamW(params, **kw), FusedAdamW(twin, **kw)
    opt._staging.chunk = 7000
    g1 = [torch.randn(s, generator=gen) * 1e-3 for s in shapes]
    opt.step([g.clone() for g in g1])
    opt2.step([g.clone() for g in g1])
    before = [p.clone() for p in params]
    moments = copy.deepcopy(opt.state_dict()["state"])
    bad = [torch.randn(s, generator=gen) * 1e-3 for s in shapes]
    bad[2].view(-1)[12345] = float("nan")
    with pytest.raises(FloatingPointError):
        opt.step(bad)
    for p, b in zip(params, before):
        assert torch.equal(p, b)
    after = opt.state_dict()["state"]
    for k, st in moments.items():
        assert torch.equal(after[k]["exp_avg"], st["exp_avg"])
        assert torch.equal(after[k]["exp_avg_sq"], st["exp_avg_sq"])
    g3 = [torch.randn(s, generator=gen) * 1e-3 for s in shapes]
    opt.step([g.clone() for g in g3])
    opt2.step([g.clone() for g in g3])
    for p, q in zip(params, twin):
        assert torch.equal(p, q)


def test_mixed_devices_are_rejected():
    model = Tiny()
    model.norm.to(DEV)
    with pytest.raises(ValueError, match="on the GPU or all on the CPU"):
        HybridMuonAdamW(model)
    with pytest.raises(ValueError, match="one device"):
        FusedAdamW([torch.zeros(4), torch.zeros(4, device=DEV)])


@pytest.mark.parametrize("chunk,pinned", [(None, False), (5000, False), (None, True)])
def test_fused_adamw_resident_masters(chunk, pinned):
    """resident_masters=True: after its first step the optimizer keeps the masters' device
    mirrors and uploads only the gradients (the masters come back as before), bit-exact
    with the device-resident optimizer; a master modified in place on the host between
    steps (its version counter moves) is uploaded again."""
    masters, grads = config1_inputs()
    cpu = [m.clone() for m in masters]
    if pinned:
        pin_host_tensors(cpu)
    dev = [m.to(DEV) for m in masters]
    groups = lambda ps: [dict(params=[p for p in ps if p.ndim == 2], weight_decay=CONFIG1["wd_2d"]),
                         dict(params=[p for p in ps if p.ndim == 1], weight_decay=0.0)]
    kw = dict(lr=CONFIG1["lr"], betas=CONFIG1["betas"], eps=CONFIG1["eps"])
    opt_c = FusedAdamW(groups(cpu), resident_masters=True, **kw)
    opt_d = FusedAdamW(groups(dev), **kw)
    if chunk is not None:
        opt_c._staging.chunk = chunk
    flat_c = [p for g in opt_c.param_groups for p in g["params"]]
    flat_d = [p for g in opt_d.param_groups for p in g["params"]]
    index = {id(p): i for i, p in enumerate(cpu)}
    nbytes = 4 * sum(p.numel() for p in flat_c)
    for t in range(1, 7):
        gs = grads(t)
        for p in flat_c:
            p.grad = gs[index[id(p)]].clone()
        for pc, pd in zip(flat_c, flat_d):
            pd.grad = pc.grad.to(DEV)
        if t == 4:  # the host changes two masters in place: they must go up again
            with torch.no_grad():
                for k in (0, 4):
                    flat_c[k].mul_(.5)
                    flat_d[k].mul_(.5)
        up0 = opt_c._staging.bytes_h2d
        opt_c.step()
        opt_d.step()
        up = opt_c._staging.bytes_h2d - up0
        if t == 4:
            assert up > 0
            if chunk is not None:  # only the chunks holding the two changed masters
                assert up < nbytes
        else:
            assert up == 0  # masters stayed resident (the initial upload is the constructor's)
        for pc, pd in zip(flat_c, flat_d):
            assert torch.equal(pc, pd.cpu()), t


def test_hybrid_resident_masters_follow_host_changes():
    """HybridMuonAdamW(resident_masters=True) on CPU masters against a device-resident twin
    over 7 steps, bit-exact, with host changes between steps that the optimizer must see:
    an in-place op on a parameter, a parameter's .data rebound to new storage,
    model.load_state_dict, and a write through .data followed by invalidate_masters()."""
    torch.manual_seed(11)
    cpu_model = Tiny()
    dev_model = copy.deepcopy(cpu_model).to(DEV)
    opt_c = HybridMuonAdamW(cpu_model, lr=.003, muon_lr=.02, resident_masters=True)
    opt_d = HybridMuonAdamW(dev_model, lr=.003, muon_lr=.02)
    pc = dict(cpu_model.named_parameters())
    pd = dict(dev_model.named_parameters())
    muon_up = []
    for step in range(7):
        with torch.no_grad():
            if step == 2:  # in place on the parameter: its version counter moves
                pc["up.weight"].mul_(.5); pd["up.weight"].mul_(.5)
                pc["norm.weight"].add_(.25); pd["norm.weight"].add_(.25)
            if step == 3:  # new storage
                pc["down.weight"].data = pc["down.weight"].data * 2
                pd["down.weight"].data = pd["down.weight"].data * 2
            if step == 4:  # a checkpoint restore
                state = {k: v * 1.5 for k, v in cpu_model.state_dict().items()}
                cpu_model.load_state_dict(state)
                dev_model.load_state_dict({k: v.to(DEV) for k, v in state.items()})
            if step == 5:  # invisible to the version counter: the caller invalidates
                pc["gate.weight"].data.add_(.125); pd["gate.weight"].add_(.125)
                pc["lm_head.weight"].data.mul_(.75); pd["lm_head.weight"].mul_(.75)
                opt_c.invalidate_masters()
        _engine_grads(cpu_model, 40 + step)
        for n, p in cpu_model.named_parameters():
            pd[n].grad = p.grad.to(DEV)
        up0 = opt_c._muon_masters.bytes_h2d
        opt_c.step()
        opt_d.step()
        muon_up.append(opt_c._muon_masters.bytes_h2d - up0)
        for n, p in cpu_model.named_parameters():
            assert torch.equal(p.detach(), pd[n].detach().cpu()), (step, n)
    muon_bytes = 4 * sum(p.numel() for p in opt_c.muon)
    assert muon_up[0] == muon_bytes                  # first step: every master goes up
    assert muon_up[1] == 0 and muon_up[6] == 0       # untouched: none
    assert 0 < muon_up[2] < muon_bytes and 0 < muon_up[3] < muon_bytes
    assert muon_up[4] == muon_bytes and muon_up[5] == muon_bytes
