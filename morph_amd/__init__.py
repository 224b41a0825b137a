"""MI355X-native mixed-precision optimizer step for MORPH's streamed trainer.

Python host code over hand-written gfx950 HIP kernels reached through the C
ABI in include/morph_optim.h.  There is no CPU fallback: every entry point
requires the built library (python -m morph_amd.build) and GPU tensors.
"""
from .precision import DynamicLossScale
from .optimizer import FusedAdamW
from .staging import pin_host_tensors

__all__ = ["DynamicLossScale", "FusedAdamW", "pin_host_tensors"]
