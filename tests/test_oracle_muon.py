"""Pins the oracle's Muon arithmetic.

Elementwise (oracle/morph_oracle.c oracle_muon_momentum / oracle_muon_apply) against
torch CPU running the reference's own op sequence, streamtrain/optimizer.py:58-61:

    momentum.lerp_(p.grad, .05)                      (58)
    update = orthogonalize(p.grad.lerp(momentum, .95))   (59; the blend is checked here)
    update *= max(1, p.shape[0] / p.shape[1]) ** .5  (60)
    p.mul_(1 - lr * weight_decay).add_(update, alpha=-lr)   (61)

bit for bit, over several steps with a fresh gradient each step (so the momentum is
not a multiple of the gradient), both update scales (1 for [3072, 6144], sqrt(2)
for [6144, 3072]) and odd shapes.

The bf16 Newton-Schulz emulation (oracle.reference.newton_schulz_bf16_emulated),
the tolerance reference of the GPU chain, against:
  * the scalar recurrence on diagonal inputs, where every matrix product has one
    non-zero term and is exact, so each entry follows the quintic of
    tests/test_training.py:50-64 with the GPU's bf16 roundings -- bit for bit;
  * the FP32 reference (streamtrain/optimizer.py:13-22) with the roundings turned
    off -- to fp32 noise, in both orientations; a flipped coefficient sign fails it.
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import reference as R
from tests.helpers import assert_same_bits


@pytest.mark.parametrize("shape", [(3072, 6144), (70, 45)])
def test_momentum_and_nesterov_blend_match_torch(shape):
    gen = torch.Generator().manual_seed(sum(shape))
    m_torch = torch.zeros(shape)  # optimizer.py:56-57: zeros_like(p) on first use
    m_oracle = np.zeros(shape, np.float32)
    for step in range(5):
        g = torch.randn(shape, generator=gen) * 1e-3
        m_torch.lerp_(g, .05)
        u_torch = g.lerp(m_torch, .95)
        u_oracle = R.muon_momentum(g.numpy(), m_oracle)
        assert_same_bits(m_oracle, m_torch.numpy(), f"momentum, step {step}")
        assert_same_bits(u_oracle, u_torch.numpy(), f"Nesterov blend, step {step}")


@pytest.mark.parametrize("shape", [(3072, 6144), (6144, 3072), (45, 70), (70, 45)])
@pytest.mark.parametrize("bf16_update", [True, False])
def test_master_update_matches_torch(shape, bf16_update):
    gen = torch.Generator().manual_seed(3 * sum(shape) + bf16_update)
    lr, wd = .02, .01
    p_torch = torch.randn(shape, generator=gen) * .02
    p_oracle = p_torch.numpy().copy()
    scale = max(1, shape[0] / shape[1]) ** .5
    for step in range(5):
        update = torch.randn(shape, generator=gen) / math.sqrt(max(shape))
        if bf16_update:  # what the GPU chain hands over: bf16 values
            update = update.to(torch.bfloat16).float()
        u = update.clone()
        u *= scale
        p_torch.mul_(1 - lr * wd).add_(u, alpha=-lr)
        R.muon_apply(p_oracle, update.numpy(), R.f32(scale), R.f32(1 - lr * wd), R.f32(-lr))
        assert_same_bits(p_oracle, p_torch.numpy(), f"master, step {step}")


def test_muon_step_sequence_matches_torch_with_fresh_gradients():
    """Momentum, blend and update together, as muon_reference_step runs them, with the
    orthogonalisation replaced by a fixed map so the comparison stays elementwise."""
    gen = torch.Generator().manual_seed(5)
    shape = (96, 48)
    p_t = torch.randn(shape, generator=gen) * .02
    m_t = torch.zeros(shape)
    p_o, m_o = p_t.numpy().copy(), np.zeros(shape, np.float32)
    for step in range(5):
        g = torch.randn(shape, generator=gen) * 1e-3
        m_t.lerp_(g, .05)
        upd = (g.lerp(m_t, .95) * 50).to(torch.bfloat16).float()
        upd *= max(1, shape[0] / shape[1]) ** .5
        p_t.mul_(1 - .02 * .01).add_(upd, alpha=-.02)
        u_o = R.muon_momentum(g.numpy(), m_o)
        upd_o = (torch.from_numpy(u_o) * 50).to(torch.bfloat16).float().numpy()
        R.muon_apply(p_o, upd_o, R.f32(2 ** .5), R.f32(1 - .02 * .01), R.f32(-.02))
        assert_same_bits(m_o, m_t.numpy(), "momentum")
        assert_same_bits(p_o, p_t.numpy(), "master")


# -- bf16 Newton-Schulz emulation ------------------------------------------------------
def _f32_rne(value):
    """Round an exact rational to the nearest binary32 (ties to even)."""
    x = np.float32(float(value))
    cands = [np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))]

    def key(y):
        return (abs(Fraction(float(y)) - value), int(np.array(y).view(np.uint32)) & 1)
    return min(cands, key=key)


def _bf16(x):
    return float(torch.tensor(float(x), dtype=torch.float32).to(torch.bfloat16).float())


def _fma(a, b, c):
    return float(_f32_rne(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))))


def _mul(a, b):
    return float(_f32_rne(Fraction(float(a)) * Fraction(float(b))))


def _add(a, b):
    return float(_f32_rne(Fraction(float(a)) + Fraction(float(b))))


def scalar_recurrence(d, steps=5, coeffs=(3.4445, -4.775, 2.0315)):
    """Each diagonal entry through the quintic with the GPU chain's roundings
    (B' = bf16(fma(b, A, c A^2) + a), x' = bf16(B' x), the first iteration scaled by 1/den)."""
    a, b, c = (R.f32(v) for v in coeffs)
    den = float(np.float32(math.sqrt(math.fsum(float(v) ** 2 for v in d))) + np.float32(1e-7))
    inv_den = float(np.float32(1) / np.float32(den))
    inv_den2 = R.f32(1.0 / (den * den))
    xs = [_bf16(v) for v in d]
    for it in range(steps):
        out = []
        for x in xs:
            A = _bf16(_mul(x * x, inv_den2) if it == 0 else x * x)  # x * x: exact in fp32
            B = _bf16(_add(_fma(b, A, _mul(A * A, c)), a))           # B' = B + a on the diagonal
            x = _bf16(_mul(B * x, inv_den) if it == 0 else B * x)   # B * x: exact in fp32
            out.append(x)
        xs = out
    return xs


@pytest.mark.parametrize("m,n", [(6, 10), (10, 6), (40, 40)])
def test_emulation_on_diagonal_inputs_is_the_scalar_recurrence(m, n):
    rng = np.random.RandomState(m * n)
    k = min(m, n)
    # 6-bit values: every square and the sum of squares is exact in binary64
    d = (rng.randint(1, 64, size=k) * 2.0 ** rng.randint(-12, -6, size=k)).astype(np.float32)
    G = torch.zeros(m, n)
    G[range(k), range(k)] = torch.from_numpy(d)
    X = R.newton_schulz_bf16_emulated(G)
    expect = scalar_recurrence(d)
    got = X[range(k), range(k)].numpy()
    assert_same_bits(got, np.array(expect, np.float32), "diagonal")
    off = X.clone()
    off[range(k), range(k)] = 0
    assert not off.any()


@pytest.mark.parametrize("shape", [(96, 160), (160, 96), (64, 64)])
def test_emulation_without_rounding_is_the_fp32_reference(shape):
    g = torch.randn(shape, generator=torch.Generator().manual_seed(sum(shape))) * 1e-3
    ref = R.orthogonalize_fp32(g)
    emu = R.newton_schulz_bf16_emulated(g, rounding=False)
    assert emu.shape == ref.shape
    assert float((emu - ref).norm() / ref.norm()) <= 2e-5
    # the same check fails a wrong sign on one coefficient
    wrong = R.newton_schulz_bf16_emulated(g, coeffs=(3.4445, 4.775, 2.0315), rounding=False)
    assert not float((wrong - ref).norm() / ref.norm()) <= 0.1  # (it diverges to NaN)


def test_emulation_error_is_the_bf16_level():
    """With the roundings on, the emulation sits at the bf16 level from FP32: well above
    fp32 noise, well below the quintic's own deviation from orthogonality."""
    g = torch.randn(256, 512, generator=torch.Generator().manual_seed(4)) * 1e-3
    ref = R.orthogonalize_fp32(g)
    rel = float((R.newton_schulz_bf16_emulated(g) - ref).norm() / ref.norm())
    assert 2e-3 <= rel <= 3e-2, rel


def test_emulation_without_iterations_is_the_normalised_input():
    g = torch.randn(70, 45, generator=torch.Generator().manual_seed(6)) * 1e-3
    out = R.newton_schulz_bf16_emulated(g, steps=0)
    ref = g / (g.norm() + 1e-7)
    assert bool(((out - ref).abs() <= ref.abs() * 2 ** -7).all())


def _unfused_chain_emulated(u, steps=5, coeffs=(3.4445, -4.775, 2.0315)):
    """The chain before the quintic's linear term moved onto B's diagonal, with its own
    rounding points: B = bf16(fma(b, A, c A A^T)), X' = bf16(fma(a, X, B X)) (the first
    iteration's products and X0 scaled by 1/den^2 and 1/den); otherwise as
    newton_schulz_bf16_emulated (optimizer.py:13-22)."""
    x = u.float()
    transpose = x.shape[0] > x.shape[1]
    if transpose:
        x = x.T
    x = x.contiguous()
    rnd = lambda t: t.to(torch.bfloat16).float()
    den = np.float32(math.sqrt(float(x.double().square().sum()))) + np.float32(1e-7)
    inv_den = np.float32(1) / den
    inv_den2 = R.f32(1.0 / (float(den) * float(den)))
    a, b, c = (R.f32(v) for v in coeffs)
    X = rnd(x)
    for it in range(steps):
        first = it == 0
        A = rnd(X @ X.T * inv_den2 if first else X @ X.T)
        B = rnd(R._fma32(b, A, A @ A.T * c))
        BX = B @ X
        X = rnd(R._fma32(a, X * float(inv_den), BX * float(inv_den)) if first
                else R._fma32(a, X, BX))
    return X.T if transpose else X


@pytest.mark.parametrize("shape", [(64, 128), (200, 96), (384, 768), (768, 1536)])
def test_linear_term_on_the_diagonal_is_no_further_from_fp32(shape):
    """Carrying a on B's diagonal (B' = cAA + bA + aI, one rounding) instead of a separate
    a X term moved the chain's rounding points; measured on the GPU tests' inputs it is
    closer to the FP32 reference than the unfused chain, never further (distances: folded
    0.0126 / 0.0098 / 0.0105 / 0.0094 against unfused 0.0149 / 0.0126 / 0.0107 / 0.0106)."""
    g = torch.randn(shape, generator=torch.Generator().manual_seed(sum(shape))) * 1e-3
    ref = R.orthogonalize_fp32(g)
    folded = float((R.newton_schulz_bf16_emulated(g) - ref).norm() / ref.norm())
    unfused = float((_unfused_chain_emulated(g) - ref).norm() / ref.norm())
    assert folded <= unfused, (folded, unfused)
    assert 2e-3 <= unfused <= 3e-2  # both at the bf16 level
