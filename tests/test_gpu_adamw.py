"""GPU parity: the fused AdamW kernel vs the CPU oracle, bit for bit.

Inputs are generated on the CPU with seeded generators and copied to the
GPU, so the kernel and the oracle see identical bits.  Masters, moments and
the export copy must match the oracle exactly (the oracle rounds sqrt and
division correctly, as the kernel does).
"""
import numpy as np
import pytest
import torch

from morph_amd import hyper, kernels
from tests.helpers import (TORCH_TO_ORACLE, assert_same_bits, export_bits, oracle_export_bits,
                           oracle_hp_for, to_oracle)

pytestmark = pytest.mark.gpu

DEV = "cuda"


def make_case(n, grad_dtype, seed, scale=1.0, offset=0):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n + offset, generator=g) * .02
    m = torch.randn(n + offset, generator=g) * 1e-4
    v = torch.rand(n + offset, generator=g) * 1e-8
    grad = (torch.randn(n + offset, generator=g) * 1e-4 * scale).to(grad_dtype)
    return w, m, v, grad


def product_hp(kind, step, scale=1.0, clip=None, lr=3e-4, betas=(.9, .95), wd=.1):
    if kind == "disk":
        return hyper.disk_constants(step=step, lr=lr, clip=clip, loss_scale=scale)
    return hyper.adamw_constants(lr=lr, beta1=betas[0], beta2=betas[1], eps=1e-8,
                                 weight_decay=wd, step=step, loss_scale=scale, clip=clip)


def run_and_compare(n, grad_dtype, out_dtype, steps, seed, kind="torch", scale=1.0, clip=None,
                    offset=0, wd=.1, betas=(.9, .95)):
    from oracle import reference as R
    w, m, v, grad = make_case(n, grad_dtype, seed, scale, offset)
    dw, dm, dv = (t.to(DEV) for t in (w, m, v))
    dg = grad.to(DEV)
    sl = slice(offset, offset + n)
    out = torch.empty(n + offset, dtype=out_dtype, device=DEV) if out_dtype is not None else None
    ow, om, ov = (to_oracle(t[sl]).copy() for t in (w, m, v))
    og = to_oracle(grad[sl])
    for step in range(1, steps + 1):
        hp = product_hp(kind, step, scale, clip, wd=wd, betas=betas)
        kernels.adamw_step(dw[sl], dm[sl], dv[sl], dg[sl], hp,
                           out=out[sl] if out is not None else None)
        ohp = oracle_hp_for(kind, step, scale=scale, clip=clip, wd=wd, betas=betas)
        oout = R.adamw(og, ow, om, ov, ohp, out_dtype=TORCH_TO_ORACLE[out_dtype],
                       grad_dtype=TORCH_TO_ORACLE[grad_dtype])
    torch.cuda.synchronize()
    assert_same_bits(dw[sl].cpu().numpy(), ow, "master")
    assert_same_bits(dm[sl].cpu().numpy(), om, "exp_avg")
    assert_same_bits(dv[sl].cpu().numpy(), ov, "exp_avg_sq")
    if out is not None:
        assert_same_bits(export_bits(out[sl]), oracle_export_bits(oout, out_dtype), "export")
    if offset:
        # bytes outside the view are untouched
        assert torch.equal(dw[:offset].cpu(), w[:offset])


@pytest.mark.parametrize("grad_dtype,out_dtype,scale", [
    (torch.float16, torch.float16, 65536.), (torch.bfloat16, torch.bfloat16, 1.),
    (torch.float32, None, 1.), (torch.float16, torch.bfloat16, 1024.),
    (torch.bfloat16, torch.float16, 2.), (torch.float32, torch.float32, 1.),
    (torch.float16, None, 128.), (torch.float32, torch.float16, 1.)])
@pytest.mark.parametrize("n", [1, 3, 4, 5, 4095, 4096, 4097, 65539, 1000003])
def test_fused_adamw_bitexact(grad_dtype, out_dtype, scale, n):
    run_and_compare(n, grad_dtype, out_dtype, steps=3, seed=n, scale=scale)


@pytest.mark.parametrize("offset", [1, 2, 3, 5])
def test_unaligned_views_take_the_scalar_path(offset):
    run_and_compare(20001, torch.float16, torch.float16, steps=2, seed=offset, scale=65536.,
                    offset=offset)


def test_disk_constants_with_clip():
    """DiskState.update's constants: betas (.9, .999), wd .01, gradient * clip."""
    run_and_compare(100003, torch.float32, None, steps=4, seed=7, kind="disk", clip=.37, wd=.01)


def test_large_lerp_weight_and_divided_scale():
    """beta1 = .3 -> torch's other lerp formula; scale 3 -> true division."""
    run_and_compare(50001, torch.float16, torch.float16, steps=3, seed=8, scale=3.0,
                    betas=(.3, .5))


def test_zero_weight_decay_is_exact_identity():
    run_and_compare(70001, torch.bfloat16, torch.bfloat16, steps=3, seed=9, wd=0.0)


def test_skip_flag_leaves_every_byte_untouched():
    w, m, v, grad = make_case(300001, torch.float16, 3, 65536.)
    dw, dm, dv, dg = (t.to(DEV) for t in (w, m, v, grad))
    out = torch.full((300001,), 7.0, dtype=torch.float16, device=DEV)
    flag = torch.ones(1, dtype=torch.int32, device=DEV)
    kernels.adamw_step(dw, dm, dv, dg, product_hp("torch", 1, 65536.), out=out, skip_flag=flag)
    torch.cuda.synchronize()
    assert torch.equal(dw.cpu(), w) and torch.equal(dm.cpu(), m) and torch.equal(dv.cpu(), v)
    assert bool((out == 7.0).all())
    flag.zero_()
    kernels.adamw_step(dw, dm, dv, dg, product_hp("torch", 1, 65536.), out=out, skip_flag=flag)
    torch.cuda.synchronize()
    assert not torch.equal(dw.cpu(), w)


def test_multi_tensor_launch_splits_and_mixes_constants():
    """100 tensors (more than one launch holds), 12 constant sets, sizes incl. 0."""
    from oracle import reference as R
    rng = np.random.RandomState(0)
    sizes = [int(s) for s in rng.choice([0, 1, 7, 4096, 5000, 33333, 131072], size=100)]
    cases = [make_case(n, torch.float16, 100 + i, 1024.) for i, n in enumerate(sizes)]
    dev = [[t.to(DEV) for t in c] for c in cases]
    outs = [torch.empty(n, dtype=torch.bfloat16, device=DEV) for n in sizes]
    hp_index = [(i // 9) % 12 for i in range(100)]  # runs of one constant set: 48-tensor launches
    batch = kernels.AdamwBatch([d[0] for d in dev], [d[1] for d in dev], [d[2] for d in dev],
                               [d[3] for d in dev], outs, hp_index)
    lrs = [1e-4 * (k + 1) for k in range(12)]
    hps = [hyper.adamw_constants(lr=lrs[k], beta1=.9, beta2=.95, eps=1e-8,
                                 weight_decay=.1 * (k % 2), step=k + 1, loss_scale=1024.)
           for k in range(12)]
    batch.launch(hps)
    torch.cuda.synchronize()
    for i, ((w, m, v, g), d, o) in enumerate(zip(cases, dev, outs)):
        k = hp_index[i]
        ow, om, ov = to_oracle(w).copy(), to_oracle(m).copy(), to_oracle(v).copy()
        ohp = R.torch_adamw_hp(lrs[k], .9, .95, 1e-8, .1 * (k % 2), k + 1, scale=1024.)
        oo = R.adamw(to_oracle(g), ow, om, ov, ohp, out_dtype=R.DTYPE_BF16)
        assert_same_bits(d[0].cpu().numpy(), ow, f"master[{i}]")
        assert_same_bits(d[1].cpu().numpy(), om, f"exp_avg[{i}]")
        assert_same_bits(d[2].cpu().numpy(), ov, f"exp_avg_sq[{i}]")
        assert_same_bits(export_bits(o), oo, f"export[{i}]")


def test_launch_larger_than_the_infinity_cache_runs_descending_bit_exact():
    """A launch whose gradients exceed 256 MB runs its chunks in descending order (it reads
    the gradient lines the detector left in the Infinity Cache first).  Elementwise, so the
    bits are the ascending order's: three FP32-gradient tensors (288 MB of gradients in
    one launch) with ragged sizes, one of them an unaligned view (scalar path), against
    the oracle over two steps with different constants."""
    from oracle import reference as R
    sizes = [40_000_003, 31_999_997, 5]
    offsets = [0, 1, 0]
    cases = [make_case(n, torch.float32, 300 + i, offset=o)
             for i, (n, o) in enumerate(zip(sizes, offsets))]
    assert sum(4 * n for n in sizes) > 256 << 20
    views = [[t.to(DEV)[o:] for t in c] for c, o in zip(cases, offsets)]
    outs = [torch.empty(n, dtype=torch.float16, device=DEV) for n in sizes]
    batch = kernels.AdamwBatch([v[0] for v in views], [v[1] for v in views],
                               [v[2] for v in views], [v[3] for v in views], outs)
    ora = [[to_oracle(t[o:]).copy() for t in c] for c, o in zip(cases, offsets)]
    for step in (1, 2):
        batch.launch([hyper.adamw_constants(lr=3e-4 * step, beta1=.9, beta2=.95, eps=1e-8,
                                            weight_decay=.1, step=step)])
        ohp = R.torch_adamw_hp(3e-4 * step, .9, .95, 1e-8, .1, step)
        oouts = [R.adamw(o[3], o[0], o[1], o[2], ohp, out_dtype=R.DTYPE_F16) for o in ora]
    torch.cuda.synchronize()
    for i, (v, o, out, oo) in enumerate(zip(views, ora, outs, oouts)):
        assert_same_bits(v[0].cpu().numpy(), o[0], f"master[{i}]")
        assert_same_bits(v[1].cpu().numpy(), o[1], f"exp_avg[{i}]")
        assert_same_bits(v[2].cpu().numpy(), o[2], f"exp_avg_sq[{i}]")
        assert_same_bits(export_bits(out), oo.view(np.uint16), f"export[{i}]")


def test_special_values_in_masters_and_grads():
    """Subnormal, zero, huge and export-overflowing values round like the oracle."""
    from oracle import reference as R
    w = torch.tensor([0.0, -0.0, 1e-40, -3e-39, 7e4, -1e5, 65504.0, 1.0, 3.4e38] * 113)
    m = torch.zeros_like(w)
    v = torch.zeros_like(w)
    g = torch.tensor([0.0, 1e-7, -6e-8, 65504.0, -2.0, 1e-3, 0.5, -0.0, 1.0] * 113,
                     dtype=torch.float16)
    dw, dm, dv, dg = (t.to(DEV) for t in (w, m, v, g))
    out = torch.empty(w.numel(), dtype=torch.float16, device=DEV)
    ow, om, ov = to_oracle(w).copy(), to_oracle(m).copy(), to_oracle(v).copy()
    for step in (1, 2):
        kernels.adamw_step(dw, dm, dv, dg, product_hp("torch", step, 1.0), out=out)
        oo = R.adamw(to_oracle(g), ow, om, ov, oracle_hp_for("torch", step),
                     out_dtype=R.DTYPE_F16)
    torch.cuda.synchronize()
    assert_same_bits(dw.cpu().numpy(), ow, "master")
    assert_same_bits(dm.cpu().numpy(), om, "exp_avg")
    assert_same_bits(dv.cpu().numpy(), ov, "exp_avg_sq")
    assert_same_bits(export_bits(out), oo.view(np.uint16), "export")


def test_stamped_one_tensor_step_equals_the_plain_step():
    """adamw_step with a DispatchTimer pair (the one-tensor morph_adamw_multi that stamps the
    dispatch) writes the same bytes as morph_adamw_fused and times a positive interval."""
    gen = torch.Generator().manual_seed(99)
    n = 1 << 20
    w = torch.randn(n, generator=gen) * .02
    g = (torch.randn(n, generator=gen) * 1e-3).to(DEV)
    hp = hyper.disk_constants(step=1, lr=3e-4, clip=0.5)
    runs = []
    timer = kernels.DispatchTimer(1)
    for events in (None, timer.next()):
        p, m, v = w.to(DEV), torch.zeros(n, device=DEV), torch.zeros(n, device=DEV)
        out = torch.empty(n, dtype=torch.float16, device=DEV)
        kernels.adamw_step(p, m, v, g, hp, out=out, events=events)
        torch.cuda.synchronize()
        runs.append((p, m, v, out))
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    assert timer.elapsed_ms()[0] > 0
