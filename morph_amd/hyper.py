"""Host-side AdamW constants for the fused kernel.

Each constant is evaluated in Python double precision with the same
expression the reference uses and then rounded once to fp32, which is what
torch's CPU kernels do with a Python scalar operand.  The kernel then
reproduces torch's per-element rounding (see include/morph_optim.h).
"""
import math
import struct

from ._lib import (AdamwHP, HP_APPLY_CLIP, HP_APPLY_DECAY, HP_DIVIDE_SCALE,
                   HP_LERP_LARGE)


def to_f32(x):
    """Round-to-nearest-even of a double to binary32, returned as a Python float."""
    return struct.unpack("<f", struct.pack("<f", x))[0]


def is_power_of_two(x):
    if not (x > 0 and math.isfinite(x)):
        return False
    return math.frexp(x)[0] == 0.5


def _pack(*, scale, clip, decay, apply_decay, lerp_weight, beta2, one_minus_beta2,
          bias_correction2_sqrt, neg_step_size, eps):
    if not (scale > 0 and math.isfinite(scale)):
        raise ValueError(f"loss scale must be positive and finite, got {scale}")
    flags = 0
    if not is_power_of_two(scale):
        flags |= HP_DIVIDE_SCALE
    if clip is not None:
        flags |= HP_APPLY_CLIP
    if apply_decay:
        flags |= HP_APPLY_DECAY
    if abs(lerp_weight) >= 0.5:  # torch's lerp switches formula at |w| >= 0.5
        flags |= HP_LERP_LARGE
    return AdamwHP(
        to_f32(scale), to_f32(1.0 / scale), to_f32(1.0 if clip is None else clip),
        to_f32(decay), to_f32(lerp_weight), to_f32(beta2), to_f32(one_minus_beta2),
        to_f32(bias_correction2_sqrt), to_f32(neg_step_size), to_f32(eps), flags, 0)


def adamw_constants(*, lr, beta1, beta2, eps, weight_decay, step, loss_scale=1.0, clip=None):
    """Constants of torch.optim.AdamW (foreach=False) for 1-based `step`.

    torch/optim/adam.py:416-419 (decoupled decay factor, skipped at wd == 0),
    457 (lerp weight 1 - beta1), 476 (beta2, 1 - beta2), 528-547 (bias
    corrections with `step` as a float, step size, sqrt via ** 0.5).
    """
    if step < 1:
        raise ValueError("step is 1-based")
    t = float(step)
    bias_correction1 = 1 - beta1 ** t
    bias_correction2 = 1 - beta2 ** t
    return _pack(scale=loss_scale, clip=clip, decay=1 - lr * weight_decay,
                 apply_decay=weight_decay != 0, lerp_weight=1 - beta1, beta2=beta2,
                 one_minus_beta2=1 - beta2, bias_correction2_sqrt=bias_correction2 ** 0.5,
                 neg_step_size=-(lr / bias_correction1), eps=eps)


def disk_constants(*, step, lr, clip, loss_scale=1.0):
    """Constants of DiskState.update (streamtrain/disk.py:210-214).

    That path hard-codes betas (0.9, 0.999), eps 1e-8 and weight decay 0.01 on
    every parameter, multiplies the gradient by `clip`, and takes the second
    bias correction's root with math.sqrt.
    """
    if step < 1:
        raise ValueError("step is 1-based")
    return _pack(scale=loss_scale, clip=clip, decay=1 - lr * .01, apply_decay=True,
                 lerp_weight=.1, beta2=.999, one_minus_beta2=.001,
                 bias_correction2_sqrt=math.sqrt(1 - .999 ** step),
                 neg_step_size=-lr / (1 - .9 ** step), eps=1e-8)
