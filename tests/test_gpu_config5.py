"""BASELINE config 5 at its full workload: HybridMuonAdamW.step (streamtrain/optimizer.py:47-62)
over 42 hidden matrices of the 5B SwiGLU preset (14 blocks of W_gate, W_up [6144, 3072] and
W_down [3072, 6144], one Newton-Schulz batch of [3072, 6144] operands) plus the 326-vector
(1,001,472-parameter) AdamW group, for three steps with a fresh gradient each.

Checked, for every one of the 42 matrices:
  * the momentum after each step bit for bit against the reference's torch CPU
    arithmetic (momentum.lerp_(g, .05), optimizer.py:58);
  * the accumulated master update against the FP32 reference chain (the Nesterov blend
    g.lerp(m, .95), orthogonalize in FP32, sqrt(max(1, r/c)) scale, decay, -lr;
    optimizer.py:58-61) within 1.5x the distance of the same chain with the oracle's bf16
    Newton-Schulz emulation (oracle.reference.newton_schulz_bf16_emulated);
and the AdamW group bit for bit against the oracle (masters and both moments).
The FP32 and emulated chains run their products with torch's fp32 GEMM on the GPU.
"""
import numpy as np
import pytest
import torch

import bench
from morph_amd.muon import HybridMuonAdamW
from oracle import reference as R
from tests.helpers import assert_same_bits

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
LR, MUON_LR, WD = 3e-4, 0.02, .01  # bench's config-5 optimizer; weight decay: the reference default


def test_config5_three_full_steps():
    torch.backends.cuda.matmul.allow_tf32 = False
    model = bench.Config5(DEV)
    opt = HybridMuonAdamW(model, lr=LR, muon_lr=MUON_LR)
    assert len(opt.muon) == 42
    vectors = [p for g in opt.adam.param_groups for p in g["params"]]
    assert len(vectors) == 326 and sum(p.numel() for p in vectors) == 1_001_472
    print("config 5: 42 x [3072, 6144] Muon + 326 AdamW vectors, 3 steps", flush=True)
    p0 = [p.detach().clone() for p in opt.muon]
    ref_p = [p.clone() for p in p0]
    emu_p = [p.clone() for p in p0]
    ref_m = [torch.zeros(p.shape) for p in opt.muon]  # CPU, as optimizer.py:56-57 on CPU masters
    aw = [p.detach().cpu().numpy().ravel().copy() for p in vectors]
    am = [np.zeros_like(w) for w in aw]
    av = [np.zeros_like(w) for w in aw]
    gen = torch.Generator(device=DEV).manual_seed(55)
    decay = 1 - MUON_LR * WD
    for step in range(1, 4):
        for p in model.parameters():
            p.grad = torch.randn(p.shape, generator=gen, device=DEV) * 1e-3
        opt.step()
        torch.cuda.synchronize()
        for i, p in enumerate(opt.muon):
            g = p.grad.cpu()
            ref_m[i].lerp_(g, .05)
            u = g.lerp(ref_m[i], .95).to(DEV)
            assert torch.equal(opt.momentum[i].cpu(), ref_m[i]), f"momentum {i}, step {step}"
            scale = max(1, p.shape[0] / p.shape[1]) ** .5
            ref_p[i].mul_(decay).add_(R.orthogonalize_fp32(u) * scale, alpha=-MUON_LR)
            emu_p[i].mul_(decay).add_(R.newton_schulz_bf16_emulated(u) * scale, alpha=-MUON_LR)
        for k, p in enumerate(vectors):
            hp = R.torch_adamw_hp(LR, .9, .95, 1e-8, WD, step)
            R.adamw(p.grad.cpu().numpy().ravel(), aw[k], am[k], av[k], hp)
        print(f"step {step} checked: momenta of 42 matrices bit-exact", flush=True)
    worst = 0.0
    for i, p in enumerate(opt.muon):
        du, dr, de = p.detach() - p0[i], ref_p[i] - p0[i], emu_p[i] - p0[i]
        rel = float((du - dr).norm() / dr.norm())
        rel_emu = float((de - dr).norm() / dr.norm())
        worst = max(worst, rel / rel_emu)
        assert rel <= 1.5 * rel_emu, (i, tuple(p.shape), rel, rel_emu)
    print(f"update: worst GPU / emulation distance from FP32 = {worst:.3f}", flush=True)
    opt.adam.resolve()
    for k, p in enumerate(vectors):
        st = opt.adam.state[p]
        assert st["step"] == 3
        assert_same_bits(p.detach().cpu().numpy().ravel(), aw[k], f"AdamW master {k}")
        assert_same_bits(st["exp_avg"].cpu().numpy().ravel(), am[k], f"exp_avg {k}")
        assert_same_bits(st["exp_avg_sq"].cpu().numpy().ravel(), av[k], f"exp_avg_sq {k}")
