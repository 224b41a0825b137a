"""ctypes binding of libmorph_optim.so (the C ABI in include/morph_optim.h).

The shared library is built in-tree by morph_amd.build into morph_amd/lib/.
It links the same HIP runtime soname torch carries (libamdhip64.so.7), so
torch is imported first: the dynamic loader then resolves the library's HIP
calls to the runtime torch already loaded, and torch's streams and device
pointers are valid in both.  There is no fallback: when the library is missing
every entry point raises.
"""
import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must load the HIP runtime before the library)

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libmorph_optim.so"
ABI_VERSION = 9

DTYPE_NONE, DTYPE_F32, DTYPE_F16, DTYPE_BF16 = -1, 0, 1, 2
HP_DIVIDE_SCALE, HP_APPLY_CLIP, HP_APPLY_DECAY, HP_LERP_LARGE = 1, 2, 4, 8

# Every symbol include/morph_optim.h declares.
EXPORTS = (
    "morph_abi_version", "morph_strerror", "morph_flag_clear", "morph_nonfinite_or",
    "morph_nonfinite_or_multi", "morph_adamw_fused", "morph_adamw_multi",
    "morph_adamw_multi_dev", "morph_step_end", "morph_nonfinite_or_close",
    "morph_grad_partials", "morph_grad_accumulate", "morph_grad_accumulate_final_noalloc",
    "morph_sumsq_total", "morph_convert_f32", "morph_fp8_pack", "morph_fp8_unpack",
    "morph_gemm_nt_bf16",
    "morph_muon_workspace_bytes", "morph_muon_step", "morph_muon_orthogonalize",
    "morph_muon_prepare", "morph_muon_newton_schulz", "morph_muon_finish",
    "morph_muon_finish_range", "morph_muon_newton_schulz_finish", "morph_host_copy",
)
GEMM_TILE_M, GEMM_TILE_N, GEMM_TILE_K = 256, 256, 64
GEMM_SYMMETRIC = 1
GEMM_Q_KN = 2
ACCUM_ELEMS_PER_BLOCK, ACCUM_OVERWRITE, ACCUM_FINAL = 2048, 1, 2
NOALLOC_MAX_PARTIALS = 1 << 20
FP8_BLOCK = 256
FATAL_MIN_SCALE = 1


class MorphError(RuntimeError):
    """A negative status returned by the C ABI."""


class AdamwHP(ctypes.Structure):
    """morph_adamw_hp."""
    _fields_ = [(name, ctypes.c_float) for name in (
        "scale", "inv_scale", "clip", "decay", "lerp_weight", "beta2",
        "one_minus_beta2", "bias_correction2_sqrt", "neg_step_size", "eps")] + [
        ("flags", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


class AdamwTensor(ctypes.Structure):
    """morph_adamw_tensor."""
    _fields_ = [("grad", ctypes.c_void_p), ("param", ctypes.c_void_p),
                ("exp_avg", ctypes.c_void_p), ("exp_avg_sq", ctypes.c_void_p),
                ("out", ctypes.c_void_p), ("numel", ctypes.c_int64),
                ("hp_index", ctypes.c_int32), ("clock_index", ctypes.c_int32)]


class StepState(ctypes.Structure):
    """morph_step_state (device-resident step control, 72 bytes)."""
    _fields_ = [("scale", ctypes.c_double), ("scale_cap", ctypes.c_double),
                ("good_steps", ctypes.c_int64), ("growth_interval", ctypes.c_int64),
                ("applied", ctypes.c_int64), ("skipped", ctypes.c_int64),
                ("found_inf", ctypes.c_uint32 * 2), ("fatal", ctypes.c_uint32),
                ("last_found_inf", ctypes.c_uint32), ("dynamic", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32)]


class AdamwSched(ctypes.Structure):
    """morph_adamw_sched."""
    _fields_ = [("lr", ctypes.c_double), ("bias_correction1", ctypes.c_void_p),
                ("bias_correction2_sqrt", ctypes.c_void_p), ("table_len", ctypes.c_int64)]


class AccumTensor(ctypes.Structure):
    """morph_accum_tensor."""
    _fields_ = [("grad", ctypes.c_void_p), ("dst", ctypes.c_void_p), ("numel", ctypes.c_int64)]


class MuonMatrix(ctypes.Structure):
    """morph_muon_matrix."""
    _fields_ = [("grad", ctypes.c_void_p), ("momentum", ctypes.c_void_p),
                ("param", ctypes.c_void_p), ("transposed", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("momentum_out", ctypes.c_void_p)]


class MuonHP(ctypes.Structure):
    """morph_muon_hp."""
    _fields_ = [(name, ctypes.c_float) for name in (
        "momentum_weight", "nesterov_weight", "a", "b", "c", "update_scale", "decay",
        "neg_lr")] + [("ns_steps", ctypes.c_int32), ("update_scale_transposed", ctypes.c_float)]


_lib = None
_load_lock = threading.Lock()


def lib():
    """The loaded library (loaded once, by whichever thread asks first); raises if
    it has not been built."""
    if _lib is None:
        with _load_lock:
            if _lib is None:
                _load()
    return _lib


def _load():
    global _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build the HIP library first "
            "(python -m morph_amd.build); morph_amd has no CPU fallback")
    handle = ctypes.CDLL(str(LIB_PATH))
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    sig = {
        "morph_abi_version": ([], i32),
        "morph_strerror": ([i32], ctypes.c_char_p),
        "morph_flag_clear": ([vp, vp], i32),
        "morph_nonfinite_or": ([vp, i32, i64, vp, vp], i32),
        "morph_nonfinite_or_multi": ([vp, vp, i32, i32, vp, vp], i32),
        "morph_adamw_fused": ([vp, i32, vp, vp, vp, vp, i32, i64, ctypes.POINTER(AdamwHP),
                               vp, vp], i32),
        "morph_adamw_multi": ([ctypes.POINTER(AdamwTensor), i32, i32, i32,
                               ctypes.POINTER(AdamwHP), i32, vp, vp, vp, vp], i32),
        "morph_adamw_multi_dev": ([ctypes.POINTER(AdamwTensor), i32, i32, i32,
                                   ctypes.POINTER(AdamwHP), ctypes.POINTER(AdamwSched), i32,
                                   vp, vp, i32, vp, vp, vp], i32),
        "morph_step_end": ([vp, vp, vp, i32, i32, vp], i32),
        "morph_nonfinite_or_close": ([vp, vp, i32, i32, vp, i32, vp, vp, i32, vp], i32),
        "morph_grad_partials": ([ctypes.POINTER(AccumTensor), i32], i64),
        "morph_grad_accumulate": ([ctypes.POINTER(AccumTensor), i32, i32, ctypes.c_double, i32,
                                   vp, vp, i64, vp], i32),
        "morph_grad_accumulate_final_noalloc": ([ctypes.POINTER(AccumTensor), i32, i32,
                                                 ctypes.c_double, i32, vp, vp, vp], i32),
        "morph_sumsq_total": ([vp, i64, vp, i32, vp], i32),
        "morph_convert_f32": ([vp, vp, i32, i64, vp, vp], i32),
        "morph_fp8_pack": ([vp, i32, i64, vp, vp, vp], i32),
        "morph_fp8_unpack": ([vp, vp, i64, vp, i32, vp], i32),
        "morph_gemm_nt_bf16": ([vp, vp, vp, vp, vp] + [i64] * 14 +
                               [ctypes.c_float, ctypes.c_float, i32, vp], i32),
        "morph_muon_workspace_bytes": ([i64, i64, i32], ctypes.c_size_t),
        "morph_muon_step": ([ctypes.POINTER(MuonMatrix), i32, i64, i64,
                             ctypes.POINTER(MuonHP), vp, ctypes.c_size_t, vp], i32),
        "morph_muon_orthogonalize": ([ctypes.POINTER(MuonMatrix), i32, i64, i64,
                                      ctypes.POINTER(MuonHP), vp, ctypes.c_size_t, vp], i32),
        "morph_muon_prepare": ([ctypes.POINTER(MuonMatrix), i32, i64, i64,
                                ctypes.POINTER(MuonHP), i32, vp, ctypes.c_size_t, vp, vp], i32),
        "morph_muon_newton_schulz": ([i32, i64, i64, ctypes.POINTER(MuonHP), vp,
                                      ctypes.c_size_t, vp], i32),
        "morph_muon_finish": ([ctypes.POINTER(MuonMatrix), i32, i64, i64,
                               ctypes.POINTER(MuonHP), i32, vp, ctypes.c_size_t, vp], i32),
        "morph_muon_finish_range": ([ctypes.POINTER(MuonMatrix), i32, i64, i64,
                                     ctypes.POINTER(MuonHP), i32, i32, i32, vp, ctypes.c_size_t,
                                     vp], i32),
        "morph_muon_newton_schulz_finish": ([ctypes.POINTER(MuonMatrix), i32, i64, i64,
                                             ctypes.POINTER(MuonHP), vp, ctypes.c_size_t, vp],
                                            i32),
        "morph_host_copy": ([vp, vp, ctypes.c_size_t, i32], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(handle, name)
        fn.argtypes, fn.restype = args, res
    version = handle.morph_abi_version()
    if version != ABI_VERSION:
        raise ImportError(f"{LIB_PATH} has ABI {version}, expected {ABI_VERSION}")
    _lib = handle


def check(status):
    if status != 0:
        raise MorphError(f"morph status {status}: {lib().morph_strerror(status).decode()}")


def dtype_code(dtype):
    if dtype is None:
        return DTYPE_NONE
    try:
        return {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16,
                torch.bfloat16: DTYPE_BF16}[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16")


def stream_handle(stream=None):
    """Raw hipStream_t of a torch stream (default: the current one)."""
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def require_device_tensor(t, name):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on the GPU (got {t.device}); morph_amd has no CPU path")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
