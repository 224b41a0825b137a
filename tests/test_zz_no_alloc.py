"""The allocation-free final accumulate pass against the existing entry points.

morph_grad_accumulate_final_noalloc (FP64 partials in the library's own device array)
must equal morph_grad_accumulate(..., MORPH_ACCUM_FINAL) into a caller workspace
followed by morph_sumsq_total: the FP32 window, the non-finite flag and the FP64 sum of
squares bit for bit.  Two calls in a row, the second over a smaller input (the array
keeps the first call's partials beyond what the second writes; they must not leak in).
Both called through the C ABI.
"""
import ctypes

import pytest
import torch

from morph_amd import _lib

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _descs(grads, dsts):
    arr = (_lib.AccumTensor * len(dsts))()
    for i, (g, d) in enumerate(zip(grads, dsts)):
        arr[i].grad = g.data_ptr() if g is not None else None
        arr[i].dst = d.data_ptr()
        arr[i].numel = d.numel()
    return arr


def _run(shapes, dtype, scale, poison, seed, noalloc):
    gen = torch.Generator().manual_seed(seed)
    L = _lib.lib()
    sh = _lib.stream_handle()
    code = _lib.dtype_code(dtype)
    micro = [[(torch.randn(s, generator=gen) * 1e-3 * scale).to(dtype).to(DEV) for s in shapes]
             for _ in range(2)]
    if poison:
        micro[1][-1].view(-1)[3] = float("inf")
    micro[1][0] = None  # a parameter without a gradient in the last micro-batch
    dsts = [torch.empty(s, device=DEV) for s in shapes]
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    total = torch.full((), -1.0, dtype=torch.float64, device=DEV)
    _lib.check(L.morph_grad_accumulate(_descs(micro[0], dsts), len(dsts), code, scale,
                                       _lib.ACCUM_OVERWRITE, None, None, 0, sh))
    arr = _descs(micro[1], dsts)
    if noalloc:
        _lib.check(L.morph_grad_accumulate_final_noalloc(
            arr, len(dsts), code, scale, 0, ctypes.c_void_p(flag.data_ptr()),
            ctypes.c_void_p(total.data_ptr()), sh))
    else:
        n = L.morph_grad_partials(arr, len(dsts))
        partials = torch.empty(n, dtype=torch.float64, device=DEV)
        _lib.check(L.morph_grad_accumulate(arr, len(dsts), code, scale, _lib.ACCUM_FINAL,
                                           ctypes.c_void_p(flag.data_ptr()),
                                           ctypes.c_void_p(partials.data_ptr()), n, sh))
        _lib.check(L.morph_sumsq_total(ctypes.c_void_p(partials.data_ptr()), n,
                                       ctypes.c_void_p(total.data_ptr()), 0, sh))
    torch.cuda.synchronize()
    return [d.cpu() for d in dsts], int(flag.item()), float(total.item())


CALLS = [  # (shapes, gradient dtype, loss scale, poisoned): the second call is smaller
    ([(3000, 700), (4097,), (33,), (2048, 512)], torch.float16, 65536.0, False),
    ([(100, 50), (7,), (1025,)], torch.bfloat16, 3.0, True),
]


def test_noalloc_final_pass_equals_workspace_form_twice():
    for k, (shapes, dtype, scale, poison) in enumerate(CALLS):
        print(f"call {k}: {len(shapes)} tensors, {dtype}, scale {scale}", flush=True)
        ref = _run(shapes, dtype, scale, poison, 100 + k, noalloc=False)
        got = _run(shapes, dtype, scale, poison, 100 + k, noalloc=True)
        for a, b in zip(ref[0], got[0]):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32))
        assert ref[1] == got[1] == int(poison)
        assert ref[2] == got[2]
        if not poison:
            assert ref[2] > 0


def test_noalloc_rejects_bad_arguments_before_any_launch():
    L = _lib.lib()
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    total = torch.zeros((), dtype=torch.float64, device=DEV)
    d = torch.zeros(16, device=DEV)
    arr = _descs([None], [d])
    fp, tp = ctypes.c_void_p(flag.data_ptr()), ctypes.c_void_p(total.data_ptr())
    sh = _lib.stream_handle()
    assert L.morph_grad_accumulate_final_noalloc(arr, 1, 1, 1.0, 2, fp, tp, sh) == -1  # FINAL implied
    assert L.morph_grad_accumulate_final_noalloc(arr, 1, 1, 1.0, 0, None, tp, sh) == -1
    assert L.morph_grad_accumulate_final_noalloc(arr, 1, 1, 1.0, 0, fp, None, sh) == -1
    assert L.morph_grad_accumulate_final_noalloc(arr, 1, 9, 1.0, 0, fp, tp, sh) == -2
