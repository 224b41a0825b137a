"""Pins the CPU oracle's AdamW against torch and against closed forms.

The oracle (oracle/morph_oracle.c) rounds sqrt and division correctly (IEEE).
torch's CPU sqrt on the build host is *not* correctly rounded (it returns the
float one ulp below the correctly rounded root for ~0.6% of inputs; see
test_torch_cpu_sqrt_is_not_correctly_rounded), so against torch:
  * exp_avg / exp_avg_sq never involve sqrt and must match bit for bit;
  * masters match bit for bit whenever every sqrt of the step is exact
    (golden adamw_exact_sqrt.npz, beta2 = 0, 12-bit gradients);
  * masters otherwise agree to within what a one-ulp change of the
    denominator can cause, checked as max|dw| / max|w| <= 1e-6 per tensor.
"""
import json
import math

import numpy as np
import pytest
import torch

from tests.golden.make_golden import CONFIG1, config1_inputs, sha


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def test_torch_cpu_sqrt_is_not_correctly_rounded():
    """Documents why masters are compared to torch with a tolerance."""
    x = torch.rand(100000, generator=torch.Generator().manual_seed(0)) * 1e-6
    exact = np.sqrt(x.numpy().astype(np.float64)).astype(np.float32)  # RNE of the true root
    assert (np.sqrt(x.numpy()) == exact).all()  # numpy / libm: correctly rounded
    diff = x.sqrt().numpy().view(np.int32).astype(np.int64) - exact.view(np.int32)
    assert set(np.unique(diff)) <= {-1, 0}  # never more than one ulp, always low


def test_config1_moments_bitexact_and_masters_close(oracle, golden_dir):
    """BASELINE config 1 through the oracle vs torch.optim.AdamW (golden SHA-256)."""
    ref = json.loads((golden_dir / "config1.json").read_text())
    masters, grads = config1_inputs()
    W = [m.numpy().ravel().copy() for m in masters]
    M = [np.zeros_like(w) for w in W]
    V = [np.zeros_like(w) for w in W]
    for t in range(1, CONFIG1["steps"] + 1):
        for i, g in enumerate(grads(t)):
            wd = CONFIG1["wd_2d"] if g.ndim == 2 else 0.0
            hp = oracle.torch_adamw_hp(CONFIG1["lr"], *CONFIG1["betas"], CONFIG1["eps"], wd, t)
            oracle.adamw(g.numpy().ravel(), W[i], M[i], V[i], hp)
    for i, tref in enumerate(ref["tensors"]):
        assert sha(M[i]) == tref["sha_m"]
        assert sha(V[i]) == tref["sha_v"]
        idx = np.array(tref["sample_index"])
        w_ref = np.array(tref["sample_w"], np.float32)
        assert np.abs(W[i][idx] - w_ref).max() / np.abs(W[i]).max() <= 1e-6


def test_config1_against_live_torch_adamw(oracle):
    """Same run, against torch.optim.AdamW in this process, element by element."""
    masters, grads = config1_inputs()
    params = [torch.nn.Parameter(m.clone()) for m in masters]
    groups = [dict(params=[p for p in params if p.ndim == 2], weight_decay=.1),
              dict(params=[p for p in params if p.ndim == 1], weight_decay=0.)]
    opt = torch.optim.AdamW(groups, lr=3e-4, betas=(.9, .95), eps=1e-8, foreach=False)
    W = [m.numpy().ravel().copy() for m in masters]
    M = [np.zeros_like(w) for w in W]
    V = [np.zeros_like(w) for w in W]
    for t in range(1, 11):
        gs = grads(t)
        for p, g in zip(params, gs):
            p.grad = g.clone()
        # the denominators torch will use at this step, to tell sqrt rounding apart
        opt.step()
        for i, g in enumerate(gs):
            hp = oracle.torch_adamw_hp(3e-4, .9, .95, 1e-8, .1 if g.ndim == 2 else 0., t)
            oracle.adamw(g.numpy().ravel(), W[i], M[i], V[i], hp)
        for i, p in enumerate(params):
            st = opt.state[p]
            assert (bits(M[i]) == bits(st["exp_avg"].numpy().ravel())).all()
            assert (bits(V[i]) == bits(st["exp_avg_sq"].numpy().ravel())).all()
            w_ref = p.detach().numpy().ravel()
            assert np.abs(W[i] - w_ref).max() / np.abs(w_ref).max() <= 1e-6


def _finish_step(w, m, v_sqrt, hp):
    """The master's part of torch's step after the moments, in numpy binary32 (one IEEE
    rounding per operation, as torch's CPU kernels round them), with the square root of
    the new second moment given: p *= 1 - lr * wd (adam.py:416-419, when wd != 0);
    d = sqrt(v) / bias_correction2_sqrt + eps; p = p + (-step_size * m) / d (544-547)."""
    f = np.float32
    if hp.flags & 4:  # MORPH_HP_APPLY_DECAY
        w = w * f(hp.decay)
    d = v_sqrt / f(hp.bias_correction2_sqrt) + f(hp.eps)
    return w + (f(hp.neg_step_size) * m) / d


def test_config1_every_master_difference_is_torchs_sqrt(oracle):
    """Per element, over config 1's 10 steps: the master update restated in binary32 with
    torch's own sqrt of the (bit-exact) second moment gives torch.optim.AdamW's masters bit
    for bit, and with the correctly rounded sqrt gives the oracle's (which the GPU kernel
    equals bit for bit).  So the masters differ from torch only where torch's CPU sqrt
    rounds differently, element by element -- not merely within a norm-wise bound."""
    masters, grads = config1_inputs()
    params = [torch.nn.Parameter(m.clone()) for m in masters]
    groups = [dict(params=[p for p in params if p.ndim == 2], weight_decay=.1),
              dict(params=[p for p in params if p.ndim == 1], weight_decay=0.)]
    opt = torch.optim.AdamW(groups, lr=3e-4, betas=(.9, .95), eps=1e-8, foreach=False)
    W = [m.numpy().ravel().copy() for m in masters]          # oracle (correctly rounded sqrt)
    T = [w.copy() for w in W]                                 # restatement, torch's sqrt
    I = [w.copy() for w in W]                                 # restatement, IEEE sqrt
    M = [np.zeros_like(w) for w in W]
    V = [np.zeros_like(w) for w in W]
    differing = 0
    for t in range(1, 11):
        gs = grads(t)
        for p, g in zip(params, gs):
            p.grad = g.clone()
        opt.step()
        for i, g in enumerate(gs):
            hp = oracle.torch_adamw_hp(3e-4, .9, .95, 1e-8, .1 if g.ndim == 2 else 0., t)
            oracle.adamw(g.numpy().ravel(), W[i], M[i], V[i], hp)
            assert (bits(M[i]) == bits(opt.state[params[i]]["exp_avg"].numpy().ravel())).all()
            T[i] = _finish_step(T[i], M[i], torch.from_numpy(V[i]).sqrt().numpy(), hp)
            I[i] = _finish_step(I[i], M[i], np.sqrt(V[i]), hp)
            w_torch = params[i].detach().numpy().ravel()
            assert (bits(T[i]) == bits(w_torch)).all(), (t, i)
            assert (bits(I[i]) == bits(W[i])).all(), (t, i)
            differing += int((bits(W[i]) != bits(w_torch)).sum())
    assert differing > 0  # the comparison is not vacuous: torch's sqrt did round differently


def test_first_step_bitexact_where_torch_sqrt_is_exact(oracle):
    """From identical inputs, masters differ only where torch's sqrt rounds low."""
    gen = torch.Generator().manual_seed(5)
    n = 50000
    w0 = torch.randn(n, generator=gen) * .02
    m0 = torch.randn(n, generator=gen) * 1e-4
    v0 = torch.rand(n, generator=gen) * 1e-8
    g = torch.randn(n, generator=gen) * 1e-3
    p = torch.nn.Parameter(w0.clone())
    opt = torch.optim.AdamW([p], lr=1e-3, betas=(.9, .95), eps=1e-8, weight_decay=.1,
                            foreach=False)
    p.grad = g.clone()
    opt.step()  # creates zero state; overwrite and redo a genuine step 2
    st = opt.state[p]
    p.data.copy_(w0)
    st["exp_avg"].copy_(m0)
    st["exp_avg_sq"].copy_(v0)
    st["step"].fill_(1.)
    opt.step()
    W, M, V = w0.numpy().copy(), m0.numpy().copy(), v0.numpy().copy()
    oracle.adamw(g.numpy(), W, M, V, oracle.torch_adamw_hp(1e-3, .9, .95, 1e-8, .1, 2))
    assert (bits(M) == bits(st["exp_avg"].numpy())).all()
    assert (bits(V) == bits(st["exp_avg_sq"].numpy())).all()
    v_new = st["exp_avg_sq"].clone()
    sqrt_ok = (v_new.sqrt().numpy() == np.sqrt(v_new.numpy()))
    assert sqrt_ok.mean() > 0.98
    w_ref = p.detach().numpy()
    assert (bits(W)[sqrt_ok] == bits(w_ref)[sqrt_ok]).all()
    assert np.abs(W - w_ref).max() / np.abs(w_ref).max() <= 1e-6


@pytest.mark.parametrize("case", ["b1_0.9_wd", "b1_0.3_nowd"])
def test_exact_sqrt_golden_bitexact(oracle, golden_dir, case):
    """beta2 = 0 with 12-bit grads: every sqrt exact, so masters must match bit for bit.

    beta1 = 0.3 puts torch's lerp weight at 0.7, its large-weight formula.
    """
    z = np.load(golden_dir / "adamw_exact_sqrt.npz")
    lr, beta1, beta2, eps, wd, steps = z[case + "_hyper"]
    w = z[case + "_w0"].copy()
    m = np.zeros_like(w)
    v = np.zeros_like(w)
    for t, g in enumerate(z[case + "_grads"], start=1):
        oracle.adamw(g, w, m, v, oracle.torch_adamw_hp(lr, beta1, beta2, eps, wd, t))
    assert int(steps) == len(z[case + "_grads"])
    assert (bits(w) == bits(z[case + "_w"])).all()
    assert (bits(m) == bits(z[case + "_m"])).all()
    assert (bits(v) == bits(z[case + "_v"])).all()


def test_disk_update_restatement_matches_oracle(oracle):
    """streamtrain/disk.py:209-215 through torch ops vs the oracle with disk constants."""
    rng = np.random.RandomState(11)
    n = 3001
    state = np.stack([(rng.randn(n) * .02).astype(np.float32), np.zeros(n, np.float32),
                      np.zeros(n, np.float32)])
    w, m, v = [state[i].copy() for i in range(3)]
    for step, clip in ((1, .37), (2, 1.0), (5, .05)):
        grad = torch.from_numpy((rng.randn(n) * 1e-2).astype(np.float32))
        oracle.disk_update_torch(state, grad, step, .003, clip, chunk_elements=1000)
        oracle.adamw(grad.numpy(), w, m, v, oracle.disk_adamw_hp(step, .003, clip))
        assert (bits(m) == bits(state[1])).all()
        assert (bits(v) == bits(state[2])).all()
        assert np.abs(w - state[0]).max() / np.abs(state[0]).max() <= 1e-6


def test_disk_update_chunking_is_invisible(oracle):
    """Chunk size changes no byte of DiskState.update's result (elementwise op)."""
    rng = np.random.RandomState(2)
    n = 777
    base = np.stack([(rng.randn(n) * .02).astype(np.float32), np.zeros(n, np.float32),
                     np.zeros(n, np.float32)])
    grad = torch.from_numpy(rng.randn(n).astype(np.float32))
    outs = []
    for chunk in (1, 7, 256, 1048576):
        s = base.copy()
        oracle.disk_update_torch(s, grad, 1, .01, .5, chunk_elements=chunk)
        outs.append(s)
    for s in outs[1:]:
        assert (bits(s) == bits(outs[0])).all()


def test_state_cache_known_answer(oracle, golden_dir):
    """The explicit vectors of the reference's tests/test_state_cache.py:21-46."""
    z = np.load(golden_dir / "state_cache_kat.npz")
    w = np.array([1.0, -2.0, 0.5], np.float32)
    m = np.zeros(3, np.float32)
    v = np.zeros(3, np.float32)
    for (step, grad, clip), key in (((1, [2.0, -1.0, 0.5], 0.25), "after_t1"),
                                    ((3, [-0.3, 1.2, 5.0], 0.1), "after_t3")):
        oracle.adamw(np.array(grad, np.float32), w, m, v, oracle.disk_adamw_hp(step, .003, clip))
        exp = z[key]
        assert (bits(m) == bits(exp[1])).all()
        assert (bits(v) == bits(exp[2])).all()
        np.testing.assert_allclose(w, exp[0], rtol=1e-6, atol=0)


def _textbook_adamw(w, m, v, g, lr, b1, b2, eps, wd, t):
    """Loshchilov & Hutter decoupled AdamW in float64 (independent of op order)."""
    w = w * (1 - lr * wd)
    m = b1 * m + (1 - b1) * g
    v = b2 * v + (1 - b2) * g * g
    mhat = m / (1 - b1 ** t)
    vhat = v / (1 - b2 ** t)
    w = w - lr * mhat / (np.sqrt(vhat) + eps)
    return w, m, v


def test_matches_textbook_adamw_in_float64(oracle):
    """Three steps against the float64 textbook update: catches a dropped term or sign."""
    rng = np.random.RandomState(4)
    n = 4096
    w = (rng.randn(n) * .05).astype(np.float32)
    W, M, V = w.astype(np.float64), np.zeros(n), np.zeros(n)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    for t in (1, 2, 3):
        g = (rng.randn(n) * 1e-2).astype(np.float32)
        oracle.adamw(g, w, m, v, oracle.torch_adamw_hp(1e-2, .9, .95, 1e-8, .1, t))
        W, M, V = _textbook_adamw(W, M, V, g.astype(np.float64), 1e-2, .9, .95, 1e-8, .1, t)
    assert np.abs(m - M).max() <= 1e-6 * np.abs(M).max()
    assert np.abs(v - V).max() <= 1e-6 * np.abs(V).max()
    assert np.abs(w - W).max() <= 1e-6 * np.abs(W).max()


def test_first_step_closed_form(oracle):
    """Step 1 from m = v = 0: w1 = w0 (1 - lr wd) - lr g / (|g| + eps') exactly in real numbers."""
    rng = np.random.RandomState(9)
    g = (rng.randn(1000) * 1e-3).astype(np.float32)
    w = (rng.randn(1000) * .02).astype(np.float32)
    w0 = w.astype(np.float64)
    m = np.zeros_like(w)
    v = np.zeros_like(w)
    lr, wd, eps = 3e-4, .1, 1e-8
    oracle.adamw(g, w, m, v, oracle.torch_adamw_hp(lr, .9, .95, eps, wd, 1))
    gd = g.astype(np.float64)
    expect = w0 * (1 - lr * wd) - lr * gd / (np.abs(gd) + eps)
    # float32 rounds w0*(1-lr*wd) and the step to ~6e-8 of |w0| <= .1: 1e-8 absolute bound
    np.testing.assert_allclose(w, expect, rtol=2e-6, atol=1e-8)
    np.testing.assert_allclose(m, .1 * gd, rtol=1e-6)
    np.testing.assert_allclose(v, .05 * gd * gd, rtol=1e-6)


def test_loss_scale_unscale_and_clip_order(oracle):
    """g = (g16 / scale) * clip, in that order, each rounded (disk.py:447 then 210)."""
    g16 = np.array([1.0, 3.0, 65504.0, -7.5, 0.0, 6.1e-5], np.float16)
    m = np.zeros(g16.size, np.float32)
    hp = oracle.torch_adamw_hp(1.0, .5, .5, 0.0, 0.0, 1, scale=1024.0, clip=.3)
    oracle.adamw(g16, np.zeros_like(m), m, np.zeros_like(m), hp)
    # m1 = fma(.5, g - 0, 0) = .5 * g exactly, so m1 exposes the unscaled, clipped g
    g = (torch.from_numpy(g16).float() / 1024.0) * .3
    assert (m == (.5 * g).numpy()).all()


def test_non_power_of_two_scale_divides(oracle):
    """A scale that is not 2^k is a true division, as torch's g.float()/loss_scale."""
    g = np.array([1.0, 2.0, 3.0, 7.0], np.float32)
    hp = oracle.torch_adamw_hp(1.0, .5, .5, 0.0, 0.0, 1, scale=3.0)
    assert hp.flags & oracle.HP_DIVIDE_SCALE
    m = np.zeros(4, np.float32)
    oracle.adamw(g, np.zeros(4, np.float32), m, np.zeros(4, np.float32), hp)
    assert (m == np.float32(.5) * (torch.from_numpy(g) / 3.0).numpy()).all()
