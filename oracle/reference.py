"""CPU oracle for MORPH's mixed-precision optimizer step.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py import this module, and only as the checker or
the timed CPU baseline.  The product package (morph_amd) never imports it.

Contents, each restating the reference (paths relative to the MORPH repo):
  * host constant computation -- torch/optim/adam.py:414-419, 528-547 and
    streamtrain/disk.py:210-214;
  * LossScale -- streamtrain/precision.py:6-17 (DynamicLossScale);
  * adamw()/nonfinite_any()/f32_to_f16()/f32_to_bf16() -- ctypes bindings of
    the C restatement in oracle/morph_oracle.c (element arithmetic);
  * disk_update_torch() -- streamtrain/disk.py:203-216 run with torch CPU ops;
  * orthogonalize_fp32()/muon_reference_step() -- streamtrain/optimizer.py:13-22,
    52-61 in FP32 torch CPU;
  * export_fp16_reference() -- streamtrain/export.py:16-43 (numpy FP16 encoding,
    per-shard SHA-256, the morph-fp16-shards-v1 manifest) without the run lock
    and with the model passed in;
  * pack_fp8_torch()/unpack_fp8_torch() -- streamtrain/precision.py:24-37 with
    torch CPU ops (float8_e4m3fn conversion);
  * accumulate_torch()/norm_squared_torch() -- the stage-gradient window of
    streamtrain/sparse_disk.py:104-108 / disk.py:446-448 and the FP64 norm pass
    disk.py:466-468 / sparse_disk.py:136, with torch CPU ops.

Pinning (tests/test_oracle_*.py): accumulate_torch against numpy's IEEE
binary32 arithmetic, norm_squared_torch against exact rational sums (math.fsum)
on inputs whose FP64 sums are exact; the C restatement is checked bit-exact
against torch.optim.AdamW(foreach=False) and against disk_update_torch; both
are checked against float64 closed forms of the first step; LossScale against
the reference's known answers (tests/test_fp16.py:59-72); conversions against
numpy/torch rounding; orthogonalize against the diagonal closed form of
tests/test_training.py:50-64 and against invariants.
"""
import ctypes
import math
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
LIB_PATH = ROOT / "lib" / "libmorph_oracle.so"

DTYPE_NONE, DTYPE_F32, DTYPE_F16, DTYPE_BF16 = -1, 0, 1, 2
HP_DIVIDE_SCALE, HP_APPLY_CLIP, HP_APPLY_DECAY, HP_LERP_LARGE = 1, 2, 4, 8


class HP(ctypes.Structure):
    """Mirror of morph_adamw_hp (include/morph_optim.h)."""
    _fields_ = [(name, ctypes.c_float) for name in (
        "scale", "inv_scale", "clip", "decay", "lerp_weight", "beta2",
        "one_minus_beta2", "bias_correction2_sqrt", "neg_step_size", "eps")] + [
        ("flags", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


def f32(x):
    """Round a Python float once to binary32, as torch does with a scalar operand."""
    return float(np.float32(x))


def _pow2(x):
    mantissa, _ = math.frexp(x)
    return x > 0 and mantissa == 0.5


def _hp(scale, clip, decay, apply_decay, lerp_weight, beta2, one_minus_beta2,
        bc2_sqrt, neg_step_size, eps):
    flags = 0
    if not _pow2(scale):
        flags |= HP_DIVIDE_SCALE
    if clip is not None:
        flags |= HP_APPLY_CLIP
    if apply_decay:
        flags |= HP_APPLY_DECAY
    if abs(lerp_weight) >= 0.5:
        flags |= HP_LERP_LARGE
    return HP(f32(scale), f32(1.0 / scale), f32(1.0 if clip is None else clip), f32(decay),
              f32(lerp_weight), f32(beta2), f32(one_minus_beta2), f32(bc2_sqrt),
              f32(neg_step_size), f32(eps), flags, 0)


def torch_adamw_hp(lr, beta1, beta2, eps, weight_decay, step, scale=1.0, clip=None):
    """Constants of torch's _single_tensor_adam for step `step` (1-based).

    torch/optim/adam.py:414-419: p.mul_(1 - lr * weight_decay) when wd != 0;
    457: exp_avg.lerp_(grad, 1 - beta1); 476: mul_(beta2).addcmul_(.., 1 - beta2);
    528-547: bias_correction1 = 1 - beta1 ** step, step_size = lr / bc1,
    bias_correction2_sqrt = (1 - beta2 ** step) ** 0.5,
    denom = sqrt(v) / bc2_sqrt + eps, p.addcdiv_(m, denom, value=-step_size).
    `step` is a float there (state_steps tensor .item()).
    """
    step = float(step)
    bias_correction1 = 1 - beta1 ** step
    bias_correction2 = 1 - beta2 ** step
    step_size = lr / bias_correction1
    bias_correction2_sqrt = bias_correction2 ** 0.5
    return _hp(scale, clip, 1 - lr * weight_decay, weight_decay != 0, 1 - beta1, beta2,
               1 - beta2, bias_correction2_sqrt, -step_size, eps)


def disk_adamw_hp(step, lr, clip, scale=1.0):
    """Constants of DiskState.update (streamtrain/disk.py:210-214).

    g = gradient * clip; first.lerp_(g, .1); second.mul_(.999).addcmul_(g, g,
    value=.001); denominator = sqrt(second) / math.sqrt(1 - .999**step) + 1e-8;
    weight.mul_(1 - lr*.01).addcdiv_(first, denominator, value=-lr/(1 - .9**step)).
    Decay is always applied there (wd .01 on every parameter).
    """
    return _hp(scale, clip, 1 - lr * .01, True, .1, .999, .001,
               math.sqrt(1 - .999 ** step), -lr / (1 - .9 ** step), 1e-8)


class LossScale:
    """Restatement of DynamicLossScale (streamtrain/precision.py:6-17)."""

    def __init__(self, scale=128., growth_interval=2000):
        self.scale = float(scale)
        self.good_steps = 0
        self.growth_interval = growth_interval

    def overflow(self):  # precision.py:9-11
        if self.scale <= 1:
            raise FloatingPointError('FP16 overflow at minimum loss scale; state unchanged')
        self.scale = max(1., self.scale / 2)
        self.good_steps = 0

    def success(self):  # precision.py:12-14
        self.good_steps += 1
        if self.good_steps >= self.growth_interval:
            self.scale = min(self.scale * 2, 65536.)
            self.good_steps = 0

    def state_dict(self):
        return dict(scale=self.scale, good_steps=self.good_steps,
                    growth_interval=self.growth_interval)


# ---------------------------------------------------------------- C oracle --
_lib = None


def lib():
    """Load (building first if needed) the C restatement."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        handle = ctypes.CDLL(str(LIB_PATH))
        vp, i64, f = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
        handle.oracle_adamw.argtypes = [vp, ctypes.c_int, vp, vp, vp, vp, ctypes.c_int, i64,
                                        ctypes.POINTER(HP)]
        handle.oracle_adamw.restype = None
        handle.oracle_nonfinite_any.argtypes = [vp, ctypes.c_int, i64]
        handle.oracle_nonfinite_any.restype = ctypes.c_int
        for name in ("oracle_f32_to_f16", "oracle_f32_to_bf16", "oracle_f16_to_f32"):
            getattr(handle, name).argtypes = [vp, vp, i64]
            getattr(handle, name).restype = None
        handle.oracle_muon_momentum.argtypes = [vp, vp, vp, i64, f, f]
        handle.oracle_muon_momentum.restype = None
        handle.oracle_muon_apply.argtypes = [vp, vp, i64, f, f, f]
        handle.oracle_muon_apply.restype = None
        _lib = handle
    return _lib


def build():
    """Compile oracle/morph_oracle.c with the committed Makefile."""
    import subprocess
    subprocess.run(["make", "-s", "-C", str(ROOT)], check=True)


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def _dtype_code(a):
    if a.dtype == np.float32:
        return DTYPE_F32
    if a.dtype == np.float16:
        return DTYPE_F16
    raise TypeError(f"unsupported array dtype {a.dtype}; pass bf16 as uint16 with dtype=DTYPE_BF16")


def adamw(grad, w, m, v, hp, out_dtype=DTYPE_NONE, grad_dtype=None):
    """One AdamW step in place on contiguous float32 arrays w/m/v.

    grad: float32 / float16 array, or uint16 bit patterns with grad_dtype=DTYPE_BF16.
    Returns the export copy (float16 array, uint16 bf16 bits, float32) or None.
    """
    for a in (w, m, v):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    grad = np.ascontiguousarray(grad)
    if grad_dtype is None:
        grad_dtype = _dtype_code(grad)
    n = w.size
    assert grad.size == n and m.size == n and v.size == n
    out = None
    if out_dtype == DTYPE_F16:
        out = np.empty(n, np.float16)
    elif out_dtype == DTYPE_BF16:
        out = np.empty(n, np.uint16)
    elif out_dtype == DTYPE_F32:
        out = np.empty(n, np.float32)
    lib().oracle_adamw(_ptr(grad), grad_dtype, _ptr(w), _ptr(m), _ptr(v), _ptr(out), out_dtype,
                       n, ctypes.byref(hp))
    return out


def nonfinite_any(grad, dtype=None):
    grad = np.ascontiguousarray(grad)
    if dtype is None:
        dtype = _dtype_code(grad)
    return bool(lib().oracle_nonfinite_any(_ptr(grad), dtype, grad.size))


def f32_to_f16(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_f16(_ptr(x), _ptr(y), x.size)
    return y


def f32_to_bf16(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_bf16(_ptr(x), _ptr(y), x.size)
    return y


def muon_momentum(grad, momentum, mom_w=.05, nesterov_w=.95):
    """In place on momentum; returns the Nesterov blend (optimizer.py:58-59)."""
    u = np.empty_like(grad)
    lib().oracle_muon_momentum(_ptr(grad), _ptr(momentum), _ptr(u), grad.size, mom_w, nesterov_w)
    return u


def muon_apply(p, update, scale, decay, neg_lr):
    """In place on p: p = p*decay + (update*scale)*neg_lr (optimizer.py:60-61)."""
    lib().oracle_muon_apply(_ptr(p), _ptr(update), p.size, scale, decay, neg_lr)


# ------------------------------------------------ torch-CPU restatements --
def disk_update_torch(state, gradient, step, lr, clip, chunk_elements=1048576, fault=None):
    """DiskState.update's arithmetic on an in-RAM [3, N] float32 array.

    Follows streamtrain/disk.py:207-216 op for op (torch CPU ops on chunk
    copies, then a stacked write-back); `fault` is called after each partial
    write as at disk.py:216.  No file I/O: the memmap is replaced by `state`.
    """
    import torch
    size = state.shape[1]
    flat = gradient.flatten()
    for start in range(0, size, chunk_elements):
        end = min(start + chunk_elements, size)
        weight, first, second = [torch.from_numpy(state[i, start:end].copy()) for i in range(3)]
        g = flat[start:end] * clip
        first.lerp_(g, .1)
        second.mul_(.999).addcmul_(g, g, value=.001)
        denominator = second.sqrt().div_(math.sqrt(1 - .999 ** step)).add_(1e-8)
        weight.mul_(1 - lr * .01).addcdiv_(first, denominator, value=-lr / (1 - .9 ** step))
        state[:, start:end] = np.stack((weight.numpy(), first.numpy(), second.numpy()))
        if fault is not None:
            fault('partial_state_write')


def orthogonalize_fp32(gradient, steps=5):
    """streamtrain/optimizer.py:13-22 in FP32 (torch CPU or whatever device gradient is on)."""
    x = gradient.float()
    transpose = x.shape[0] > x.shape[1]
    if transpose:
        x = x.T
    x = x / (x.norm() + 1e-7)
    for _ in range(steps):
        gram = x @ x.T
        x = 3.4445 * x + (-4.775 * gram + 2.0315 * (gram @ gram)) @ x
    return x.T if transpose else x


def muon_reference_step(param, grad, momentum, lr, weight_decay):
    """One Muon update of one matrix, streamtrain/optimizer.py:55-61, FP32 torch."""
    momentum.lerp_(grad, .05)
    update = orthogonalize_fp32(grad.lerp(momentum, .95))
    update *= max(1, param.shape[0] / param.shape[1]) ** .5
    param.mul_(1 - lr * weight_decay).add_(update, alpha=-lr)
    return update


def _fma32(a, b, c):
    """fp32 fma(a, b, c) with `a` an fp32 scalar and b, c fp32 tensors: the product of two
    binary32 values is exact in binary64, so one binary64 add and one rounding to
    binary32 give the fused result (except where that add itself rounds, which needs
    exponents 29+ bits apart)."""
    return (b.double() * float(a) + c.double()).float()


def newton_schulz_bf16_emulated(u, steps=5, coeffs=(3.4445, -4.775, 2.0315), rounding=True):
    """The bf16 Newton-Schulz chain of the GPU kernels, emulated with torch fp32 products.

    Same algorithm as streamtrain/optimizer.py:13-22 (transpose the taller matrix,
    X / (|X|_F + 1e-7), `steps` quintic iterations, transpose back), with the
    quintic's linear term carried on B's diagonal (a X + B X = (B + a I) X) and the
    GPU's rounding points:
      den = fp32(sqrt(sum u^2 in binary64)) + fp32(1e-7);  X0 = bf16(u)
      iteration 0:  A  = bf16(fp32(1 / den^2) * X0 X0^T)
                    B' = bf16(fma(b, A, c * A A^T) + a on the diagonal)
                    X  = bf16((1 / den) * B' X0)
      later:        A = bf16(X X^T); B' as above; X = bf16(B' X)
    with every product accumulated in fp32 (here: torch's fp32 matmul of the bf16
    values, exact per term, in its own summation order).  rounding=False skips the
    bf16 roundings (X0 = u), which leaves the FP32 reference up to fp32 rounding.
    Returns an fp32 tensor in u's layout (the values of the bf16 result).
    """
    import torch
    x = u.float()
    transpose = x.shape[0] > x.shape[1]
    if transpose:
        x = x.T
    x = x.contiguous()
    rnd = (lambda t: t.to(torch.bfloat16).float()) if rounding else (lambda t: t)
    den = np.float32(math.sqrt(float(x.double().square().sum()))) + np.float32(1e-7)
    inv_den = np.float32(1) / den
    inv_den2 = f32(1.0 / (float(den) * float(den)))
    a, b, c = (f32(v) for v in coeffs)
    X = rnd(x)
    for it in range(steps):
        first = it == 0
        A = X @ X.T
        A = rnd(A * inv_den2 if first else A)
        B = _fma32(b, A, A @ A.T * c)
        B.diagonal().add_(a)  # one fp32 add, on the diagonal only
        B = rnd(B)
        BX = B @ X
        X = rnd(BX * float(inv_den) if first else BX)
    if steps == 0:
        X = rnd(X / float(den))
    return X.T if transpose else X


def accumulate_torch(destination, gradient, loss_scale):
    """sparse_disk.py:106-107 (disk.py:447 on the CPU): the per-micro-batch unscale + add."""
    destination.add_(gradient.detach().float() / loss_scale)


def norm_squared_torch(gradients, chunk=1048576):
    """disk.py:466-468 / sparse_disk.py:136: FP64 sum of squares over 1M-element pieces."""
    total = 0.0
    for g in gradients:
        for piece in g.flatten().split(chunk):
            total += piece.double().square().sum().item()
    return total


def pack_fp8_torch(value, block_size=256):
    """precision.py:24-30: E4M3FN bytes + FP32 per-block scale."""
    import torch
    flat = value.detach().float().flatten()
    padding = (-flat.numel()) % block_size
    padded = torch.nn.functional.pad(flat, (0, padding)).reshape(-1, block_size)
    scales = (padded.abs().amax(1) / 448.).clamp_min(1e-30)
    encoded = (padded / scales[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(
        torch.uint8).flatten()[:flat.numel()]
    return encoded, scales


def unpack_fp8_torch(encoded, scales, dtype=None, block_size=256):
    """precision.py:33-37."""
    import torch
    dtype = dtype or torch.float16
    size = encoded.numel()
    padding = (-size) % block_size
    padded = torch.nn.functional.pad(encoded, (0, padding))
    values = padded.view(torch.float8_e4m3fn).float().reshape(-1, block_size)
    return (values * scales[:, None]).to(dtype).flatten()[:size]


def e4m3fn_value(byte):
    """E4M3FN decoded from the format definition (1-4-3, bias 7, no inf, S.1111.111 = NaN)."""
    sign = -1.0 if byte & 0x80 else 1.0
    e, m = (byte >> 3) & 0xF, byte & 7
    if e == 15 and m == 7:
        return float("nan")
    if e == 0:
        return sign * m * 2.0 ** -9
    return sign * (1 + m / 8) * 2.0 ** (e - 7)


def export_fp16_reference(state_dir, output, model, chunk_elements=1048576, durable=False):
    """export.py:16-43 on the CPU: same checks, encoding, hashing, manifest.  durable: flush
    and fsync each shard as export.py:35 does (left out where only the bytes matter)."""
    import hashlib
    import json
    from pathlib import Path
    state_dir, output = Path(state_dir), Path(output)
    manifest = json.loads((state_dir / "manifest.json").read_text())
    if manifest["dirty"]:
        raise ValueError("cannot export an incomplete optimizer transaction")
    entries = {name: dict(shape=list(p.shape), size=p.numel(), file=f"{i:05}.bin")
               for i, (name, p) in enumerate(model.named_parameters())}
    if entries != manifest["entries"]:
        raise ValueError("disk state tensor schema differs")
    output.mkdir(parents=True, exist_ok=False)
    weights = {}
    for name, entry in entries.items():
        source = np.memmap(state_dir / entry["file"], dtype=np.float32, mode="r", shape=(3, entry["size"]))
        path = output / entry["file"]
        digest = hashlib.sha256()
        with path.open("wb") as handle:
            for start in range(0, entry["size"], chunk_elements):
                value = np.asarray(source[0, start:start + chunk_elements])
                if not np.isfinite(value).all() or np.abs(value).max(initial=0) > 65504:
                    raise ValueError("weights cannot be represented by finite FP16")
                encoded = value.astype("<f2").tobytes()
                handle.write(encoded)
                digest.update(encoded)
            if durable:
                handle.flush()
                os.fsync(handle.fileno())
        del source
        weights[name] = dict(file=path.name, shape=entry["shape"], dtype="float16",
                             sha256=digest.hexdigest())
    canonical = {id(p): n for n, p in model.named_parameters()}
    aliases = {n: canonical[id(p)] for n, p in model.named_parameters(remove_duplicate=False)
               if canonical[id(p)] != n}
    result = dict(format="morph-fp16-shards-v1", config=model.config.to_dict(), step=manifest["step"],
                  weights=weights, aliases=aliases,
                  lm_head=dict(kind="tied_embedding_projection", weight="embedding.weight"),
                  parameters=sum(e["size"] for e in entries.values()), optimizer_included=False,
                  buffers="deterministically reconstructed from config",
                  source_precision="float32 masters", export_precision="float16")
    (output / "manifest.json").write_text(json.dumps(result))
    return result


def cpu_threads():
    return len(os.sched_getaffinity(0))
