"""In-tree build of the gfx950 device library (lib/libq3t_hip.so).

hipcc flags: -ffp-contract=off keeps every fp32 rounding where the kernels
write it (no implicit fused multiply-add); the packed-fp32-ops target feature
is disabled so the compiler emits no packed fp32 instructions.
"""
import os
import subprocess

from .device import PKG_DIR

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("Q3T_OFFLOAD_ARCH", "gfx950")
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def build_device_lib(verbose=False):
    src = os.path.join(PKG_DIR, "csrc", "q3t_dev.hip")
    out_dir = os.path.join(PKG_DIR, "lib")
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "libq3t_hip.so")
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", *HIP_FLAGS, "-shared", "-o", tmp, src]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + r.stderr[-4000:])
    os.replace(tmp, out)
    if verbose:
        print(" ".join(cmd))
    return out
