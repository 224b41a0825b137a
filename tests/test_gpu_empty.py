"""Empty inputs through every GPU entry point: zero-element tensors are accepted, launch
nothing for themselves and leave the other tensors' results unchanged."""
import pytest
import torch

from morph_amd import FusedAdamW, fp8, kernels
from morph_amd import grads as G

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def test_fp8_empty_roundtrip():
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        enc, sc = fp8.pack_fp8(torch.empty(0, dtype=dtype, device=DEV))
        assert enc.numel() == 0 and sc.numel() == 0
        assert fp8.unpack_fp8(enc, sc, dtype).numel() == 0


def test_detector_with_empty_tensors():
    empty = torch.empty(0, dtype=torch.float16, device=DEV)
    flag = kernels.new_flag()
    kernels.flag_clear(flag)
    kernels.nonfinite_or([empty], flag)
    assert flag.item() == 0
    kernels.nonfinite_or([empty, torch.tensor([1.0, float("inf")], device=DEV).half(), empty], flag)
    assert flag.item() == 1


def test_fused_adamw_with_an_empty_parameter():
    """The same steps with and without a zero-element parameter give identical bits."""
    gen = torch.Generator().manual_seed(3)
    shapes = [(10,), (3, 4), (257,)]
    init = [torch.randn(s, generator=gen) * .02 for s in shapes]
    grads = [[torch.randn(s, generator=gen) * 1e-3 for s in shapes] for _ in range(3)]

    def run(with_empty):
        ps = [torch.nn.Parameter(t.clone().to(DEV)) for t in init]
        if with_empty:
            ps.insert(1, torch.nn.Parameter(torch.empty(0, device=DEV)))
        opt = FusedAdamW(ps, lr=3e-4, betas=(.9, .95), weight_decay=.1)
        for gs in grads:
            full = [g.to(DEV) for g in gs]
            if with_empty:
                full.insert(1, torch.empty(0, device=DEV))
            for p, g in zip(ps, full):
                p.grad = g
            opt.step()
        torch.cuda.synchronize()
        return [p.detach().cpu() for p in ps if p.numel()]

    for a, b in zip(run(True), run(False)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_stage_gradients_with_an_empty_shape():
    g = torch.randn(5, generator=torch.Generator().manual_seed(1)).half()
    window = G.StageGradients([(0,), (5,)], DEV)
    window.zero_()
    window.accumulate([torch.empty(0, dtype=torch.float16, device=DEV), g.to(DEV)], 2.0,
                      final=True)
    assert window.views[0].numel() == 0
    assert torch.equal(window.views[1].cpu(), g.float() / 2.0)
    assert not window.found_inf()
    assert window.norm_squared() == pytest.approx(float((g.double() / 2.0).pow(2).sum()), rel=1e-12)
