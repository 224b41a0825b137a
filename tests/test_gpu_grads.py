"""GPU parity of the stage-gradient window (morph_grad_accumulate, morph_sumsq_total).

Accumulation must equal the reference's torch ops (oracle.accumulate_torch) bit for
bit; the non-finite flag must equal torch.isfinite over the accumulated window; the
FP64 norm must equal the reference's chunked sum exactly on dyadic inputs (where
FP64 sums are exact in any order) and to 1e-12 relative otherwise, and be
deterministic run to run.
"""
import math

import pytest
import torch

from morph_amd import grads as G
from oracle import reference as R
from tests.helpers import assert_same_bits

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
SHAPES = [(1,), (7,), (2047,), (2048,), (2049,), (3, 1000), (1025, 33), (4096,)]


def oracle_window(micro_grads, scale):
    """The reference's loop: zeroed FP32 window, add_(g.float() / scale) per micro-batch."""
    window = [torch.zeros(s) for s in SHAPES]
    for grads in micro_grads:
        for dst, g in zip(window, grads):
            if g is not None:
                R.accumulate_torch(dst, g, scale)
    return window


def micro_batches(dtype, k, seed, scale, with_none=True):
    gen = torch.Generator().manual_seed(seed)
    out = []
    for m in range(k):
        grads = []
        for i, s in enumerate(SHAPES):
            if with_none and (i + m) % 5 == 3:
                grads.append(None)  # parameter without a gradient in this micro-batch
            else:
                grads.append((torch.randn(s, generator=gen) * 1e-3 * scale).to(dtype))
        out.append(grads)
    return out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("scale", [1.0, 65536.0, 3.0])
def test_accumulate_bitexact_vs_reference_ops(dtype, scale):
    mbs = micro_batches(dtype, 4, 1, scale)
    window = G.StageGradients(SHAPES, DEV)
    window.flat.fill_(float("nan"))  # stale contents: the first pass must overwrite
    window.zero_()
    for k, grads in enumerate(mbs):
        window.accumulate([g.to(DEV) if g is not None else None for g in grads], scale,
                          final=(k == len(mbs) - 1))
    expect = oracle_window(mbs, scale)
    for got, exp in zip(window.views, expect):
        assert_same_bits(got.cpu().numpy(), exp.numpy(), "window")
    assert not window.found_inf()
    ref = R.norm_squared_torch(expect)
    assert abs(window.norm_squared() - ref) <= 1e-12 * ref


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_unaligned_gradient_views(dtype):
    """Gradients that start off a 16-byte boundary (views one element into their
    allocation) take the lane-strided path; the window, flag and norm are unchanged."""
    def on_device(g):
        if g is None:
            return None
        buf = torch.zeros(g.numel() + 1, dtype=g.dtype, device=DEV)
        buf[1:] = g.reshape(-1).to(DEV)
        return buf[1:].view(g.shape)

    mbs = micro_batches(dtype, 3, 5, 65536.0)
    window = G.StageGradients(SHAPES, DEV)
    window.zero_()
    for k, grads in enumerate(mbs):
        window.accumulate([on_device(g) for g in grads], 65536.0, final=(k == len(mbs) - 1))
    expect = oracle_window(mbs, 65536.0)
    for got, exp in zip(window.views, expect):
        assert_same_bits(got.cpu().numpy(), exp.numpy(), "window")
    assert not window.found_inf()
    ref = R.norm_squared_torch(expect)
    assert abs(window.norm_squared() - ref) <= 1e-12 * ref


def test_first_pass_turns_negative_zero_into_positive_zero():
    window = G.StageGradients([(5,)], DEV).zero_()
    g = torch.tensor([-0.0, 0.0, -0.0, 1.0, -0.0], dtype=torch.float16, device=DEV)
    window.accumulate([g], 128.0, final=True)
    assert not torch.signbit(window.views[0]).any()


def test_norm_exact_on_dyadic_inputs_and_deterministic():
    gen = torch.Generator().manual_seed(3)
    shapes = [(1048577,), (3000, 7), (2048,)]
    ks = [torch.randint(-2047, 2048, s, generator=gen) for s in shapes]
    grads = [(k.double() / 1024).float() for k in ks]
    exact = sum(int((k.long() ** 2).sum()) for k in ks) / 2 ** 20
    assert R.norm_squared_torch(grads) == exact
    values = []
    for _ in range(2):
        window = G.StageGradients(shapes, DEV).zero_()
        window.accumulate([g.to(DEV) for g in grads], 1.0, final=True)
        values.append(window.norm_squared())
    assert values[0] == exact and values[1] == exact


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("poison", [float("inf"), float("-inf"), float("nan")])
def test_nonfinite_flag_matches_isfinite(dtype, poison):
    mbs = micro_batches(dtype, 3, 4, 1.0, with_none=False)
    where = (5, 17)  # shape index, flat position
    mbs[1][where[0]].view(-1)[where[1]] = poison
    window = G.StageGradients(SHAPES, DEV).zero_()
    for k, grads in enumerate(mbs):
        window.accumulate([g.to(DEV) for g in grads], 1.0, final=(k == 2))
    expect = oracle_window(mbs, 1.0)
    assert window.found_inf() == (not all(torch.isfinite(t).all() for t in expect))
    assert window.found_inf()
    assert not math.isfinite(window.norm_squared())


def test_fp16_overflow_after_accumulation_is_flagged():
    """Finite fp16 gradients whose FP32 sum overflows still read as finite per element;
    the flag follows the accumulated window, as the reference's norm does."""
    big = torch.full((4,), 3e38, dtype=torch.float32, device=DEV)
    window = G.StageGradients([(4,)], DEV).zero_()
    window.accumulate([big], 1.0)
    window.accumulate([big], 1.0, final=True)
    assert window.found_inf()


def test_many_tensors_span_several_launches():
    shapes = [(257 + 13 * i,) for i in range(45)]  # more than one launch's 32 tensors
    gen = torch.Generator().manual_seed(8)
    grads = [(torch.randn(s, generator=gen) * 1e-2).to(torch.float16) for s in shapes]
    window = G.StageGradients(shapes, DEV).zero_()
    window.accumulate([g.to(DEV) for g in grads], 65536.0)
    window.accumulate([g.to(DEV) for g in grads], 65536.0, final=True)
    for view, g in zip(window.views, grads):
        d = torch.zeros(g.shape)
        R.accumulate_torch(d, g, 65536.0)
        R.accumulate_torch(d, g, 65536.0)
        assert_same_bits(view.cpu().numpy(), d.numpy(), "window")
    ref = R.norm_squared_torch([v.cpu() for v in window.views])
    assert abs(window.norm_squared() - ref) <= 1e-12 * ref


def test_config2_window_full_size_against_torch_on_gpu():
    """The 5B-preset stage window (N = 56,623,104, FP16 gradients x 2^16, 4 micro-batches):
    bit-exact against the same torch ops run on the GPU (power-of-two scale, so torch's
    reciprocal multiply and this kernel give identical bits), norm to 1e-12."""
    shapes = [(6144, 3072), (6144, 3072), (3072, 6144)]
    gen = torch.Generator(device=DEV).manual_seed(2)
    window = G.StageGradients(shapes, DEV).zero_()
    ref = [torch.zeros(s, device=DEV) for s in shapes]
    for k in range(4):
        grads = [(torch.randn(s, generator=gen, device=DEV) * 1e-4 * 65536).half() for s in shapes]
        window.accumulate(grads, 65536.0, final=(k == 3))
        for d, g in zip(ref, grads):
            d.add_(g.float() / 65536.0)
    for got, exp in zip(window.views, ref):
        assert torch.equal(got.view(torch.int32), exp.view(torch.int32))
    ref_norm = sum(float(t.double().square().sum()) for t in ref)
    assert abs(window.norm_squared() - ref_norm) <= 1e-12 * ref_norm
    assert not window.found_inf()


def test_clip_coefficient_matches_reference_expression():
    for n2 in (0.0, 0.25, 1.0, 4.0, 1e6):
        norm = math.sqrt(n2)
        assert G.clip_coefficient(n2, 1.0) == min(1., 1.0 / (norm + 1e-6))


@pytest.mark.parametrize("poison", [False, True])
def test_window_flag_into_the_optimizer_replaces_the_detector(poison):
    """The final accumulate pass writes its non-finite flag into FusedAdamW's step state
    and step(..., checked=True) skips the detector: the same masters, moments, exports,
    skip decision and loss scale as the ordinary step on the same window."""
    from morph_amd import DynamicLossScale, FusedAdamW
    shapes = [(300, 200), (4097,), (64, 64)]
    gen = torch.Generator().manual_seed(11)
    masters = [torch.randn(s, generator=gen) * .02 for s in shapes]
    micro = [[(torch.randn(s, generator=gen) * 1e-4 * 1024).half() for s in shapes]
             for _ in range(3)]
    if poison:
        micro[1][1][17] = float("inf")
    results = []
    for checked in (False, True):
        opt = FusedAdamW([m.to(DEV) for m in masters], lr=3e-4, betas=(.9, .95),
                         weight_decay=.1, loss_scale=DynamicLossScale(1024., 2000),
                         export_dtype=torch.float16, sync=True)
        window = G.StageGradients(shapes, DEV).zero_()
        for k, grads in enumerate(micro):
            window.accumulate([g.to(DEV) for g in grads], 1.0, final=(k == 2),
                              found_inf=opt.found_inf if checked else None)
        assert window.found_inf() == poison
        applied = opt.step(window.views, checked=checked)
        assert applied == (not poison)
        results.append(opt)
    a, b = results
    assert a.loss_scale.scale == b.loss_scale.scale == (512. if poison else 1024.)
    for p, q in zip([p for g in a.param_groups for p in g["params"]],
                    [p for g in b.param_groups for p in g["params"]]):
        assert torch.equal(p, q)
        for key in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(a.state[p][key], b.state[q][key])
    for x, y in zip(a.exports, b.exports):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))


def test_tied_embedding_sum_through_the_windows():
    """disk.py:455-462 / sparse_disk.py:126-130: the head stage holds its embedding gradient,
    stage 0 adds it (one FP32 add) before the update; the norm counts the sum once.  Here the
    head stage accumulates into its own window and stage 0's final pass takes that FP32 view
    with scale 1 (x * 1 is exact, so the add is the reference's): views bit-exact, norm over
    stage 0 only."""
    gen = torch.Generator().manual_seed(13)
    emb, other = (96, 64), (64, 128)
    scale = 1024.0
    head_micro = [(torch.randn(emb, generator=gen) * 1e-3 * scale).half() for _ in range(2)]
    stage0_micro = [[(torch.randn(s, generator=gen) * 1e-3 * scale).half() for s in (emb, other)]
                    for _ in range(3)]
    tied = G.StageGradients([emb], DEV).zero_()
    for k, g in enumerate(head_micro):
        tied.accumulate([g.to(DEV)], scale, final=(k == 1))
    window = G.StageGradients([emb, other], DEV).zero_()
    for grads in stage0_micro:
        window.accumulate([g.to(DEV) for g in grads], scale)
    window.accumulate([tied.views[0], None], 1.0, final=True)
    # the reference's ops on the CPU
    held = torch.zeros(emb)
    for g in head_micro:
        held.add_(g.float() / scale)
    ref = [torch.zeros(emb), torch.zeros(other)]
    for grads in stage0_micro:
        for d, g in zip(ref, grads):
            d.add_(g.float() / scale)
    ref[0].add_(held)
    for got, exp in zip(window.views, ref):
        assert torch.equal(got.cpu().view(torch.int32), exp.view(torch.int32))
    ref_norm = sum(float(piece.double().square().sum()) for t in ref
                   for piece in t.flatten().split(1048576))
    assert abs(window.norm_squared() - ref_norm) <= 1e-12 * ref_norm
    assert not window.found_inf()
