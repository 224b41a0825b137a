"""Build libmorph_optim.so for gfx950 in-tree (python -m morph_amd.build).

Flags that matter for results:
  -ffp-contract=off       no implicit multiply-add fusion: the kernels round
                          exactly where torch's CPU kernels round, and fuse
                          only where __fmaf_rn says so;
  -packed-fp32-ops off    no packed FP32 instructions in device code.
  -fhip-fp32-correctly-rounded-divide-sqrt
                          fp32 `/` and sqrt lower to IEEE correctly
                          rounded sequences (hipcc's default, made explicit).
"""
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SOURCES = ["abi.hip", "adamw.hip", "nonfinite.hip", "step.hip", "grads.hip", "convert.hip", "fp8.hip", "gemm.hip", "muon.hip", "hostcopy.hip"]
OUTPUT = PKG / "lib" / "libmorph_optim.so"
ARCH = os.environ.get("MORPH_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def build(output=OUTPUT, extra_flags=(), quiet=True):
    output = Path(output)
    output.parent.mkdir(parents=True, exist_ok=True)
    tmp = output.with_name(output.name + ".tmp")
    cmd = [hipcc(), *FLAGS, *extra_flags, "-o", str(tmp),
           *[str(PKG / "csrc" / s) for s in SOURCES]]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(cmd)}")
    if not quiet:
        # The host pass warns that it does not know the packed-fp32 feature; drop that noise.
        noise = "is not a recognized feature for this target"
        sys.stderr.write("".join(l + "\n" for l in proc.stderr.splitlines() if noise not in l))
    os.replace(tmp, output)
    return output


if __name__ == "__main__":
    print(build(quiet=False))
