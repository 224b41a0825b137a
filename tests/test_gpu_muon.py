"""GPU parity of the Muon path: bf16 MFMA GEMM, Newton-Schulz, Muon step, HybridMuonAdamW.

The reference orthogonalises in FP32 (streamtrain/optimizer.py:13-22); the
BASELINE asks for bf16 on MFMA, so Newton-Schulz is compared with a tolerance:
- the GEMM building block against the exact (float64) product of its bf16
  inputs: error within one bf16 rounding of the result plus fp32 accumulation;
- orthogonalize against the FP32 reference: the relative Frobenius error is at
  most 1.5x that of the oracle's bf16 emulation of the same chain (same rounding
  points, torch fp32 products; oracle.reference.newton_schulz_bf16_emulated),
  singular values inside the quintic's band [0.6, 1.2] (FP32 gives [0.68, 1.14]);
- on diagonal inputs, where every product has one non-zero term and is exact,
  bit for bit equal to that emulation (the quintic of tests/test_training.py:50-64
  with the chain's bf16 roundings);
and every elementwise part bit for bit: momentum/Nesterov against the oracle's
restatement (itself bit-exact with torch, tests/test_oracle_muon.py), the master
update against the oracle applied to the GPU's own Newton-Schulz output.
"""
import copy

import numpy as np
import pytest
import torch
from torch import nn

from morph_amd import muon
from tests.helpers import assert_same_bits

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def rand_bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("b,M,N,K", [(1, 256, 256, 64), (3, 512, 768, 192), (2, 768, 256, 512)])
def test_gemm_nt_against_exact_product(b, M, N, K):
    P, Q, D = rand_bf16((b, M, K), 1), rand_bf16((b, N, K), 2), rand_bf16((b, M, N), 3)
    alpha, beta = 2.0315, -4.775
    out_t = torch.empty((b, N, M), dtype=torch.bfloat16, device=DEV)
    C = muon.gemm_nt(P.to(DEV), Q.to(DEV), D.to(DEV), alpha, beta, out_t=out_t).cpu()
    Pd, Qd, Dd = P.double(), Q.double(), D.double()
    exact = alpha * Pd @ Qd.transpose(1, 2) + beta * Dd
    # bound: one bf16 rounding of the result + fp32 accumulation over K terms
    mag = abs(alpha) * Pd.abs() @ Qd.abs().transpose(1, 2) + abs(beta) * Dd.abs()
    err = (C.double() - exact).abs()
    assert (err <= 2 ** -8 * exact.abs() + 1e-6 * K * mag + 1e-30).all()
    assert torch.equal(out_t.cpu(), C.transpose(1, 2))


@pytest.mark.parametrize("b,M,N,K", [(1, 256, 256, 64), (3, 512, 768, 192), (2, 768, 512, 512)])
def test_gemm_q_kn_equals_the_nt_form_bit_for_bit(b, M, N, K):
    """Q stored [K, N] (transposing LDS reads) gives the same fragments, so the same bits as
    passing Q^T in [N, K]; with D, alpha, beta and the transposed copy."""
    P, Q, D = rand_bf16((b, M, K), 4), rand_bf16((b, N, K), 5), rand_bf16((b, M, N), 6)
    Pd, Qd, Dd = P.to(DEV), Q.to(DEV), D.to(DEV)
    Qkn = Qd.transpose(1, 2).contiguous()
    ta = torch.empty((b, N, M), dtype=torch.bfloat16, device=DEV)
    tb = torch.empty((b, N, M), dtype=torch.bfloat16, device=DEV)
    ca = muon.gemm_nt(Pd, Qd, Dd, 3.4445, 1.0, out_t=ta)
    cb = muon.gemm_nt(Pd, Qkn, Dd, 3.4445, 1.0, out_t=tb, q_kn=True)
    assert torch.equal(ca, cb) and torch.equal(ta, tb)
    exact = P.double() @ Q.double().transpose(1, 2)
    C = muon.gemm_nt(Pd, Qkn, q_kn=True).cpu().double()
    mag = P.double().abs() @ Q.double().abs().transpose(1, 2)
    assert ((C - exact).abs() <= 2 ** -8 * exact.abs() + 1e-6 * K * mag + 1e-30).all()


@pytest.mark.parametrize("alpha", [1 + 2 ** -8, 1 + 3 * 2 ** -8, 1 / 3, -0.7, 2.0 ** -140, 7.5e37])
def test_gemm_output_rounding_is_round_to_nearest_even(alpha):
    """C = alpha * I Q^T is one fp32 product alpha * q rounded once to bf16.  With q a
    power of two, 1 + 2^-8 and 1 + 3 * 2^-8 land exactly on ties (to even: down and
    up); 2^-140 gives fp32 denormals, 7.5e37 overflows bf16.  Bits must equal torch's
    CPU conversion (round to nearest even) of the same fp32 product, in C and in Ct."""
    g = torch.Generator().manual_seed(21)
    Q = torch.randn(256, 256, generator=g)
    Q[:64] = torch.sign(Q[:64]) * 2.0 ** torch.randint(-20, 20, (64, 256), generator=g).float()
    Q = Q.to(torch.bfloat16)
    P = torch.eye(256, dtype=torch.bfloat16)
    out_t = torch.empty((256, 256), dtype=torch.bfloat16, device=DEV)
    C = muon.gemm_nt(P.to(DEV), Q.to(DEV), None, alpha, out_t=out_t).cpu()
    expect = (torch.tensor(alpha, dtype=torch.float32) * Q.float().T).to(torch.bfloat16)
    assert torch.equal(C.view(torch.int16), expect.view(torch.int16))
    assert torch.equal(out_t.cpu().view(torch.int16), expect.T.contiguous().view(torch.int16))


def test_gemm_nt_in_place_output_over_D():
    """D may alias C: the epilogue reads each D element before it writes that C element."""
    P, Q = rand_bf16((256, 256), 4).to(DEV), rand_bf16((512, 256), 5).to(DEV)
    X = rand_bf16((256, 512), 6).to(DEV)
    expect = muon.gemm_nt(P, Q, X.clone(), 1.0, 3.4445)
    muon.gemm_nt(P, Q, X, 1.0, 3.4445, out=X)
    assert torch.equal(X, expect)


@pytest.mark.parametrize("b,M,K", [(1, 256, 64), (2, 1024, 320), (3, 768, 768)])
def test_gemm_nt_symmetric_mode(b, M, K):
    """Upper-triangle tiles + mirror: exactly symmetric, equal to the full product's bound,
    and the upper triangle equals the full computation bit for bit."""
    X = rand_bf16((b, M, K), 7).to(DEV)
    full = muon.gemm_nt(X, X)
    sym = muon.gemm_nt(X, X, symmetric=True)
    assert torch.equal(sym, sym.transpose(1, 2))
    upper = torch.triu(torch.ones(M // 256, M // 256, dtype=torch.bool)).repeat_interleave(
        256, 0).repeat_interleave(256, 1).to(DEV)
    assert torch.equal(sym[:, upper], full[:, upper])
    # with a symmetric D and alpha/beta, as in B = c A A^T + b A
    A = sym
    B = muon.gemm_nt(A, A, A, 2.0315, -4.775, symmetric=True)
    Ad = A.double().cpu()
    exact = 2.0315 * Ad @ Ad.transpose(1, 2) - 4.775 * Ad
    mag = 2.0315 * Ad.abs() @ Ad.abs().transpose(1, 2) + 4.775 * Ad.abs()
    assert ((B.double().cpu() - exact).abs() <= 2 ** -8 * exact.abs() + 1e-6 * M * mag).all()
    assert torch.equal(B, B.transpose(1, 2))


def test_orthogonalize_diagonal_closed_form():
    """tests/test_training.py:50-64: diag(.0975, .195) -> quintic on each singular value."""
    g = torch.diag(torch.tensor([.0975, .195])).to(DEV)
    out = muon.orthogonalize(g).cpu().double()
    d = torch.tensor([.0975, .195], dtype=torch.float64)
    d = d / (d.norm() + 1e-7)
    for _ in range(5):
        d = 3.4445 * d - 4.775 * d ** 3 + 2.0315 * d ** 5
    torch.testing.assert_close(out, torch.diag(d), rtol=1.5e-2, atol=1e-6)


# Relative Frobenius distance from the FP32 reference of the chain as it was before the
# quintic's linear term moved onto B's diagonal (B = bf16(b A + c A A^T), X' = bf16(a X +
# B X)), emulated on the CPU with the same inputs: a bound that does not move with the
# emulation of the current chain (tests/test_oracle_muon.py shows the current chain is
# the closer of the two on these shapes).
UNFUSED_DISTANCE = {(64, 128): 0.01485, (200, 96): 0.01256, (384, 768): 0.01067,
                    (6144, 3072): 0.00880}


@pytest.mark.parametrize("shape", [(64, 128), (200, 96), (384, 768), (6144, 3072)])
def test_orthogonalize_against_fp32_reference(shape):
    """Within 1.5x of the bf16 emulation's distance from the FP32 reference, and within
    1.15x of the unfused chain's (a fixed number per shape)."""
    from oracle import reference as R
    torch.backends.cuda.matmul.allow_tf32 = False
    g = torch.randn(shape, generator=torch.Generator().manual_seed(sum(shape))) * 1e-3
    gd = g.to(DEV)
    ref = R.orthogonalize_fp32(gd)
    emu = R.newton_schulz_bf16_emulated(gd)
    out = muon.orthogonalize(gd)
    rel = float((out - ref).norm() / ref.norm())
    rel_emu = float((emu - ref).norm() / ref.norm())
    print(f"shape {shape}: GPU {rel:.5f}, bf16 emulation {rel_emu:.5f} from FP32")
    assert rel <= 1.5 * rel_emu, (rel, rel_emu)
    assert rel <= 1.15 * UNFUSED_DISTANCE[shape], (rel, UNFUSED_DISTANCE[shape])
    if max(shape) <= 1024:
        sv = torch.linalg.svdvals(out.cpu().double())
        assert 0.6 <= float(sv.min()) and float(sv.max()) <= 1.2


@pytest.mark.parametrize("m,n", [(200, 300), (300, 200), (256, 512)])
def test_orthogonalize_diagonal_bitexact_vs_emulation(m, n):
    """A diagonal [m, n] input: every product of the chain has one non-zero term, so the
    fp32 accumulation is exact and the GPU must equal the emulation bit for bit (the
    emulation equals the scalar recurrence there, tests/test_oracle_muon.py)."""
    from oracle import reference as R
    rng = np.random.RandomState(m + n)
    k = min(m, n)
    # 6-bit values: the binary64 sum of squares is exact in any order
    d = (rng.randint(1, 64, size=k) * 2.0 ** rng.randint(-12, -6, size=k)).astype(np.float32)
    G = torch.zeros(m, n)
    G[range(k), range(k)] = torch.from_numpy(d)
    out = muon.orthogonalize(G.to(DEV)).cpu()
    emu = R.newton_schulz_bf16_emulated(G)
    assert_same_bits(out.numpy(), emu.numpy(), "diagonal Newton-Schulz")


@pytest.mark.parametrize("shape", [(200, 300), (300, 200)])
def test_a_nonfinite_call_leaves_nothing_for_the_next(shape):
    """Shapes off the 256 tile have zero padding in the workspace.  A NaN or inf input
    turns it into NaN during the chain (0 * NaN); the next call of the same shape --
    orthogonalize, or a Muon step whose chain ran on an infinite gradient because the
    caller passed no gate -- must equal the same call on a fresh workspace."""
    from morph_amd import kernels
    ws = muon.Workspaces()
    gen = torch.Generator().manual_seed(sum(shape) + 1)
    g = (torch.randn(shape, generator=gen) * 1e-3).to(DEV)
    bad = g.clone()
    bad[3, 5] = float("nan")
    assert torch.isnan(muon.orthogonalize(bad, workspaces=ws)).any()
    out = muon.orthogonalize(g, workspaces=ws)
    assert torch.isfinite(out).all()
    assert torch.equal(out, muon.orthogonalize(g, workspaces=muon.Workspaces()))
    # a Muon step with the gate left to the caller: the chain runs on the infinity
    p0 = (torch.randn(shape, generator=gen) * .02).to(DEV)
    p, m = p0.clone(), torch.zeros_like(p0)
    inf_grad = g.clone()
    inf_grad[7, 1] = float("inf")
    flag = kernels.new_flag(DEV)
    muon.muon_step([p], [inf_grad], [m], .02, .01, workspaces=ws, found_inf=flag)
    assert flag.item() == 1
    p.copy_(p0)
    m.zero_()
    muon.muon_step([p], [g], [m], .02, .01, workspaces=ws)
    q, mq = p0.clone(), torch.zeros_like(p0)
    muon.muon_step([q], [g], [mq], .02, .01, workspaces=muon.Workspaces())
    assert torch.equal(p, q) and torch.equal(m, mq) and torch.isfinite(p).all()


def test_orthogonalize_batches_same_shape_matrices():
    gs = [torch.randn(96, 160, generator=torch.Generator().manual_seed(i)) * 1e-3 for i in range(5)]
    batched = muon.orthogonalize([g.to(DEV) for g in gs])
    for g, b in zip(gs, batched):
        assert torch.equal(muon.orthogonalize(g.to(DEV)), b)


@pytest.mark.parametrize("shape", [(96, 160), (160, 96), (70, 45)])
def test_orthogonalize_without_iterations_is_the_normalised_input(shape):
    """steps=0: X = G / (|G| + 1e-7) (optimizer.py:18), here bf16(bf16(G) / den): two bf16
    roundings of the FP32 value, so within 2^-7 of it elementwise, in both orientations."""
    G = torch.randn(shape, generator=torch.Generator().manual_seed(sum(shape))) * 1e-3
    out = muon.orthogonalize(G.to(DEV), steps=0).cpu()
    ref = G / (G.norm() + 1e-7)
    assert out.shape == ref.shape
    assert bool(((out - ref).abs() <= ref.abs() * 2 ** -7).all())


def on_device(t, offset):
    """t on the GPU, `offset` elements past the start of a fresh allocation."""
    buf = torch.zeros(t.numel() + offset, dtype=t.dtype, device=DEV)
    buf[offset:] = t.reshape(-1).to(DEV)
    return buf[offset:].view(t.shape)


@pytest.mark.parametrize("shape,offset", [
    ((128, 256), 0), ((100, 300), 0), ((45, 70), 0), ((96, 96), 0), ((1, 300), 0),
    ((300, 100), 0), ((70, 45), 0), ((300, 1), 0), ((4100, 1024), 0), ((4096, 640), 0),
    ((256, 640), 1), ((640, 256), 1), ((640, 256), 2), ((512, 768), 0), ((768, 512), 0)])
def test_muon_step_elementwise_bitexact(shape, offset):
    """momentum/Nesterov and the master update match the oracle bit for bit: the flat
    passes (X in the stored layout: (128, 256) whole blocks, (100, 300) a partial last
    block, (45, 70) rows not a multiple of 4, (96, 96) square, (1, 300) a single row) and
    the transposing tile passes ((300, 100) and (70, 45) partial tiles only, (300, 1) a
    single column, (4100, 1024) whole tiles and a partial last band, (4096, 640) whole
    momentum tiles and a partial last column of apply tiles); with `offset`, parameter,
    momentum and gradient start off a 16-byte boundary, so every pass takes its
    element-wise path.  (512, 768) and (768, 512) have no operand padding: their update
    rides on the last Newton-Schulz product's epilogue (morph_muon_newton_schulz_finish)."""
    from oracle import reference as R
    gen = torch.Generator().manual_seed(7)
    p0 = torch.randn(shape, generator=gen) * .02
    m0 = torch.randn(shape, generator=gen) * 1e-3
    g = torch.randn(shape, generator=gen) * 1e-3
    lr, wd = .02, .01
    p, m = on_device(p0, offset), on_device(m0, offset)
    muon.muon_step([p], [on_device(g, offset)], [m], lr, wd)
    om = m0.numpy().copy()
    u = R.muon_momentum(g.numpy(), om)  # momentum in place, returns the Nesterov blend
    assert_same_bits(m.cpu().numpy(), om, "momentum")
    U = muon.orthogonalize(torch.from_numpy(u).to(DEV)).cpu().numpy()
    op = p0.numpy().copy()
    scale = R.f32(max(1, shape[0] / shape[1]) ** .5)
    R.muon_apply(op, U, scale, R.f32(1 - lr * wd), R.f32(-lr))
    assert_same_bits(p.cpu().numpy(), op, "param")


def emulated_muon_step(p, g, m, lr, wd):
    """optimizer.py:55-61 with the oracle's elementwise steps (bit-exact with torch) and
    the bf16 Newton-Schulz emulation: the tolerance reference of the GPU step."""
    from oracle import reference as R
    u = R.muon_momentum(g, m)
    U = R.newton_schulz_bf16_emulated(torch.from_numpy(u)).numpy()
    scale = R.f32(max(1, p.shape[0] / p.shape[1]) ** .5)
    R.muon_apply(p, np.ascontiguousarray(U), scale, R.f32(1 - lr * wd), R.f32(-lr))


@pytest.mark.parametrize("shape", [(256, 512), (512, 256)])
def test_muon_step_against_fp32_reference_update(shape):
    """Three steps with a fresh gradient each (the momentum is then no multiple of the
    gradient, so the Nesterov blend shows in the update): momentum bit-exact with the
    reference's torch arithmetic, the accumulated update within 1.5x of the emulated
    bf16 step's distance from the FP32 reference."""
    from oracle import reference as R
    gen = torch.Generator().manual_seed(8 + shape[0])
    p0 = torch.randn(shape, generator=gen) * .02
    p, m = p0.clone().to(DEV), torch.zeros(shape, device=DEV)
    rp, rm = p0.clone(), torch.zeros(shape)
    ep, em = p0.numpy().copy(), np.zeros(shape, np.float32)
    for _ in range(3):
        g = torch.randn(shape, generator=gen) * 1e-3
        muon.muon_step([p], [g.to(DEV)], [m], .02, .01)
        R.muon_reference_step(rp, g, rm, .02, .01)
        emulated_muon_step(ep, g.numpy(), em, .02, .01)
    assert torch.equal(m.cpu(), rm)  # momentum is elementwise torch arithmetic: exact
    du, dr, de = (p.cpu() - p0), (rp - p0), (torch.from_numpy(ep) - p0)
    rel = float((du - dr).norm() / dr.norm())
    rel_emu = float((de - dr).norm() / dr.norm())
    assert rel <= 1.5 * rel_emu, (rel, rel_emu)


class Tiny(nn.Module):
    """Hidden Linear layers (Muon), a LayerNorm and an lm_head (AdamW)."""

    def __init__(self):
        super().__init__()
        self.up = nn.Linear(64, 192, bias=True)
        self.down = nn.Linear(192, 64, bias=False)
        self.norm = nn.LayerNorm(64)
        self.lm_head = nn.Linear(64, 32, bias=False)


def _grads(model, seed):
    gen = torch.Generator().manual_seed(seed)
    for p in model.parameters():
        p.grad = (torch.randn(p.shape, generator=gen) * 1e-3).to(p.device)


def test_hybrid_partition_and_adam_group_match_torch():
    """optimizer.py:25-31 partition; the AdamW group equals torch.optim.AdamW (betas .9/.95)."""
    torch.manual_seed(0)
    cpu = Tiny()
    gpu = copy.deepcopy(cpu).to(DEV)
    opt = muon.HybridMuonAdamW(gpu, lr=.003)
    assert [id(p) for p in opt.muon] == [id(gpu.up.weight), id(gpu.down.weight)]
    adam_ref = [p for n, p in cpu.named_parameters() if n not in ("up.weight", "down.weight")]
    ref = torch.optim.AdamW(adam_ref, lr=.003, weight_decay=.01, betas=(.9, .95), foreach=False)
    for step in range(3):
        _grads(gpu, step)
        _grads(cpu, step)
        opt.step()
        ref.step()
    opt.adam.resolve()
    for n, p in gpu.named_parameters():
        if n in ("up.weight", "down.weight"):
            continue
        q = dict(cpu.named_parameters())[n]
        st, qs = opt.adam.state[p], ref.state[q]
        assert torch.equal(st["exp_avg"].cpu(), qs["exp_avg"])
        assert torch.equal(st["exp_avg_sq"].cpu(), qs["exp_avg_sq"])
        assert (p.detach().cpu() - q.detach()).abs().max() <= 1e-6 * q.detach().abs().max()


def test_adam_group_bitexact_with_torch_on_the_reference_known_answer():
    """tests/test_training.py:9-28's known answer: every AdamW-group gradient 0.2 for three
    steps; the group equals torch.optim.AdamW(betas .9/.95, foreach=False) with rtol = atol = 0
    (masters included: this input never meets torch's 1-ulp CPU sqrt), then a NaN gradient
    raises with the whole model untouched."""
    torch.manual_seed(3)
    cpu = Tiny()
    gpu = copy.deepcopy(cpu).to(DEV)
    opt = muon.HybridMuonAdamW(gpu, lr=.003)
    names = [n for n, _ in cpu.named_parameters() if n not in ("up.weight", "down.weight")]
    ref_params = [dict(cpu.named_parameters())[n] for n in names]
    ref = torch.optim.AdamW(ref_params, lr=.003, weight_decay=.01, betas=(.9, .95), foreach=False)
    for _ in range(3):
        for n, p in gpu.named_parameters():
            p.grad = torch.full_like(p, .2) if n in names else torch.zeros_like(p)
        for q in ref_params:
            q.grad = torch.full_like(q, .2)
        opt.step()
        ref.step()
    for n, q in zip(names, ref_params):
        torch.testing.assert_close(dict(gpu.named_parameters())[n].detach().cpu(), q.detach(),
                                   rtol=0, atol=0)
    before = {k: v.clone() for k, v in gpu.state_dict().items()}
    dict(gpu.named_parameters())[names[0]].grad.fill_(float("nan"))
    with pytest.raises(FloatingPointError):
        opt.step()
    for k, v in gpu.state_dict().items():
        torch.testing.assert_close(v, before[k], rtol=0, atol=0)


@pytest.mark.parametrize("poisoned,bad", [("norm.weight", float("nan")),
                                          ("up.weight", float("inf")),
                                          ("down.weight", float("nan"))])
def test_hybrid_nonfinite_raises_before_any_mutation(poisoned, bad):
    """optimizer.py:49-51 / tests/test_training.py:22-27: an AdamW-group gradient (caught by
    the detector) or a Muon gradient (caught in the momentum pass) raises with parameters,
    momenta and AdamW state untouched; the next finite step then equals the step of an
    optimizer that never saw the poisoned one."""
    torch.manual_seed(1)
    gpu = Tiny().to(DEV)
    twin = copy.deepcopy(gpu)
    opt, opt2 = muon.HybridMuonAdamW(gpu, lr=.003), muon.HybridMuonAdamW(twin, lr=.003)
    for o, m in ((opt, gpu), (opt2, twin)):
        _grads(m, 1)
        o.step()
    before = copy.deepcopy(gpu.state_dict())
    mom = {i: t.clone() for i, t in opt.momentum.items()}
    _grads(gpu, 2)
    dict(gpu.named_parameters())[poisoned].grad.view(-1)[5] = bad
    with pytest.raises(FloatingPointError):
        opt.step()
    for k, v in gpu.state_dict().items():
        assert torch.equal(v, before[k]), k
    for i, t in opt.momentum.items():
        assert torch.equal(t, mom[i]), i
    for o, m in ((opt, gpu), (opt2, twin)):
        _grads(m, 3)
        o.step()
    for (k, v), (k2, v2) in zip(gpu.state_dict().items(), twin.state_dict().items()):
        assert torch.equal(v, v2), k
    for i in opt.momentum:
        assert torch.equal(opt.momentum[i], opt2.momentum[i]), i


def test_hybrid_muon_diagonal_matches_scalar_newton_schulz():
    """tests/test_training.py:50-64 on the GPU, to bf16 tolerance."""
    model = nn.Sequential(nn.Linear(2, 2, bias=False), nn.LayerNorm(2)).to(DEV)
    opt = muon.HybridMuonAdamW(model, lr=.02)
    weight = model[0].weight
    before = weight.detach().clone()
    weight.grad = torch.diag(torch.tensor([1., 2.])).to(DEV)
    diagonal = torch.tensor([.0975, .195], dtype=torch.float64)
    diagonal = diagonal / (diagonal.norm() + 1e-7)
    for _ in range(5):
        diagonal = 3.4445 * diagonal - 4.775 * diagonal ** 3 + 2.0315 * diagonal ** 5
    opt.step()
    expected = before * (1 - .02 * .01) - .02 * torch.diag(diagonal.float()).to(DEV)
    torch.testing.assert_close(weight.detach(), expected, rtol=1e-5, atol=3e-4)


def test_hybrid_state_dict_roundtrip():
    a = Tiny().to(DEV)
    b = copy.deepcopy(a)
    oa = muon.HybridMuonAdamW(a, lr=.003)
    _grads(a, 3)
    oa.step()
    ob = muon.HybridMuonAdamW(b, lr=.003)
    # as after torch.save / torch.load: load_state_dict keeps on-device tensors by
    # reference (value.to(device), optimizer.py:68), so the state is copied first
    ob.load_state_dict(copy.deepcopy(oa.state_dict()))
    b.load_state_dict(a.state_dict())
    for m in (a, b):
        _grads(m, 4)
    oa.step()
    ob.step()
    for (n, p), (_, q) in zip(a.named_parameters(), b.named_parameters()):
        assert torch.equal(p, q), n


@pytest.mark.parametrize("rows,cols,steps", [(256, 512, 5), (512, 256, 5), (512, 768, 2),
                                             (768, 512, 1), (192, 320, 5), (320, 192, 1)])
def test_update_in_the_last_product_equals_the_finish_pass(rows, cols, steps):
    """morph_muon_newton_schulz_finish carries the master update in the last X' = B' X
    product's epilogue when the operand has no padding -- both orientations in one batch,
    so the epilogue writes p rows from the tile's rows and from its columns, scale
    sqrt(max(1, r/c)) per matrix; with steps == 1 the last product is also the first,
    which carries 1/den -- and falls back to the finish pass otherwise ((192, 320),
    (320, 192)).  Either way parameters and momenta are bit-identical to
    prepare + newton_schulz + finish."""
    import ctypes
    from morph_amd import _lib
    L = _lib.lib()
    gen = torch.Generator().manual_seed(rows + cols + steps)
    shapes = [(rows, cols), (cols, rows), (rows, cols), (cols, rows)]
    p0 = [torch.randn(s, generator=gen) * .02 for s in shapes]
    m0 = [torch.randn(s, generator=gen) * 1e-3 for s in shapes]
    g = [(torch.randn(s, generator=gen) * 1e-3).to(DEV) for s in shapes]
    hp = muon._step_hp(rows, cols, .02, .01, steps)
    results = []
    for fused in (True, False):
        p, m = [t.to(DEV) for t in p0], [t.to(DEV) for t in m0]
        ws = torch.zeros(L.morph_muon_workspace_bytes(rows, cols, 4), dtype=torch.uint8,
                         device=DEV)
        wsp, sh = ctypes.c_void_p(ws.data_ptr()), _lib.stream_handle()
        arr = (_lib.MuonMatrix * 4)()
        for i in range(4):
            arr[i].grad, arr[i].momentum, arr[i].param = (g[i].data_ptr(), m[i].data_ptr(),
                                                          p[i].data_ptr())
            arr[i].transposed = int(shapes[i] != (rows, cols))
        _lib.check(L.morph_muon_prepare(arr, 4, rows, cols, ctypes.byref(hp), 0, wsp, ws.numel(),
                                        None, sh))
        if fused:
            _lib.check(L.morph_muon_newton_schulz_finish(arr, 4, rows, cols, ctypes.byref(hp), wsp,
                                                         ws.numel(), sh))
        else:
            _lib.check(L.morph_muon_newton_schulz(4, rows, cols, ctypes.byref(hp), wsp, ws.numel(),
                                                  sh))
            _lib.check(L.morph_muon_finish(arr, 4, rows, cols, ctypes.byref(hp), 0, wsp, ws.numel(),
                                           sh))
        torch.cuda.synchronize()
        results.append((p, m))
    for i in range(4):
        assert torch.equal(results[0][0][i], results[1][0][i]), i
        assert torch.equal(results[0][1][i], results[1][1][i]), i
        assert not torch.equal(results[0][0][i].cpu(), p0[i])  # the update happened


def test_one_call_c_entry_equals_phased_path():
    """morph_muon_step (C convenience) == prepare + newton_schulz_finish as the Python layer runs them."""
    import ctypes
    from morph_amd import _lib
    gen = torch.Generator().manual_seed(9)
    shape = (192, 320)
    p0, m0, g = (torch.randn(shape, generator=gen) * s for s in (.02, 1e-3, 1e-3))
    pa, ma = p0.to(DEV), m0.to(DEV)
    muon.muon_step([pa], [g.to(DEV)], [ma], .02, .01)
    pb, mb, gb = p0.to(DEV), m0.to(DEV), g.to(DEV)
    ws = torch.zeros(_lib.lib().morph_muon_workspace_bytes(*shape, 1), dtype=torch.uint8, device=DEV)
    arr = (_lib.MuonMatrix * 1)()
    arr[0].grad, arr[0].momentum, arr[0].param = gb.data_ptr(), mb.data_ptr(), pb.data_ptr()
    hp = muon._hp(update_scale=1.0, decay=1 - .02 * .01, neg_lr=-.02)
    _lib.check(_lib.lib().morph_muon_step(arr, 1, *shape, ctypes.byref(hp),
                                          ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                          _lib.stream_handle()))
    assert torch.equal(pa, pb) and torch.equal(ma, mb)


def test_mixed_orientation_batch_equals_separate_batches():
    """[r, c] and [c, r] matrices share one batch (one Newton-Schulz operand shape);
    every matrix comes out bit-identical to running it alone, scale sqrt(max(1, r/c))
    per matrix as optimizer.py:60 computes it."""
    gen = torch.Generator().manual_seed(11)
    shapes = [(192, 448), (448, 192), (192, 448), (448, 192)]
    p0 = [torch.randn(s, generator=gen) * .02 for s in shapes]
    m0 = [torch.randn(s, generator=gen) * 1e-3 for s in shapes]
    g = [(torch.randn(s, generator=gen) * 1e-3).to(DEV) for s in shapes]
    pa, ma = [t.to(DEV) for t in p0], [t.to(DEV) for t in m0]
    muon.muon_step(pa, g, ma, .02, .01)  # one batch of four
    for i in range(len(shapes)):
        pb, mb = p0[i].to(DEV), m0[i].to(DEV)
        muon.muon_step([pb], [g[i]], [mb], .02, .01)
        assert torch.equal(pa[i], pb) and torch.equal(ma[i], mb), i
    outs = muon.orthogonalize(g)
    for i in range(len(shapes)):
        assert torch.equal(outs[i], muon.orthogonalize(g[i])), i


def test_more_than_64_matrices_run_as_several_batches():
    """A shape's matrices go to the library 64 per call: 70 of them (both orientations) come
    out bit-identical to running each alone, and so does orthogonalize."""
    gen = torch.Generator().manual_seed(13)
    shapes = [(96, 64) if i % 3 == 0 else (64, 96) for i in range(70)]
    p0 = [torch.randn(s, generator=gen) * .02 for s in shapes]
    m0 = [torch.randn(s, generator=gen) * 1e-3 for s in shapes]
    g = [(torch.randn(s, generator=gen) * 1e-3).to(DEV) for s in shapes]
    pa, ma = [t.to(DEV) for t in p0], [t.to(DEV) for t in m0]
    muon.muon_step(pa, g, ma, .02, .01)
    for i in (0, 1, 63, 64, 69):
        pb, mb = p0[i].to(DEV), m0[i].to(DEV)
        muon.muon_step([pb], [g[i]], [mb], .02, .01)
        assert torch.equal(pa[i], pb) and torch.equal(ma[i], mb), i
    outs = muon.orthogonalize(g)
    for i in (2, 64, 68):
        assert torch.equal(outs[i], muon.orthogonalize(g[i])), i


def test_transposed_flag_equals_passing_the_transposed_shape():
    """C ABI: a [c, r] matrix flagged transposed under (rows, cols) = (r, c) equals the
    same matrix passed unflagged as (c, r)."""
    import ctypes
    from morph_amd import _lib
    gen = torch.Generator().manual_seed(12)
    r, c = 256, 576
    p0, m0, g = (torch.randn(c, r, generator=gen) * s for s in (.02, 1e-3, 1e-3))
    g = g.to(DEV)
    results = []
    for rows, cols, transposed in ((r, c, 1), (c, r, 0)):
        p, m = p0.to(DEV), m0.to(DEV)
        ws = torch.zeros(_lib.lib().morph_muon_workspace_bytes(rows, cols, 1), dtype=torch.uint8,
                         device=DEV)
        arr = (_lib.MuonMatrix * 1)()
        arr[0].grad, arr[0].momentum, arr[0].param = g.data_ptr(), m.data_ptr(), p.data_ptr()
        arr[0].transposed = transposed
        scale = (c / r) ** .5
        hp = muon._hp(update_scale=scale if not transposed else 1.0,
                      update_scale_transposed=scale if transposed else 1.0,
                      decay=1 - .02 * .01, neg_lr=-.02)
        _lib.check(_lib.lib().morph_muon_step(arr, 1, rows, cols, ctypes.byref(hp),
                                              ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                              _lib.stream_handle()))
        results.append((p, m))
    assert torch.equal(results[0][0], results[1][0]) and torch.equal(results[0][1], results[1][1])
