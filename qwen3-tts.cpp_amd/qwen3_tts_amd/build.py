"""In-tree build of the gfx950 device library (lib/libq3t_hip.so).

hipcc flags: -ffp-contract=off keeps every fp32 rounding where the kernels
write it (no implicit fused multiply-add); the packed-fp32-ops target feature
is disabled so the compiler emits no packed fp32 instructions.  Matrix-core
accumulators live in ordinary vector registers (-amdgpu-mfma-vgpr-form): the
vocoder GEMM's K loop, unrolled by two steps, otherwise copied every
accumulator between the two register files each step (2.35 -> 2.27-2.30 ms
per 73-frame window), and the prefill and multi-stream GEMMs gain 1-1.5%;
the results are the same.
"""
import os
import subprocess

from .device import PKG_DIR

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("Q3T_OFFLOAD_ARCH", "gfx950")
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


SRC_FLAGS = {"q3t_dev.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"], "q3t_voc.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd, verbose):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + r.stderr[-4000:])
    if verbose:
        print(" ".join(cmd))


def build_device_lib(verbose=False):
    out_dir = os.path.join(PKG_DIR, "lib")
    obj_dir = os.path.join(out_dir, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    objs = []
    for src, extra in SRC_FLAGS.items():
        obj = os.path.join(obj_dir, src.replace(".hip", ".o"))
        _run([HIPCC, f"--offload-arch={ARCH}", *HIP_FLAGS, *extra, "-c", "-o", obj,
              os.path.join(PKG_DIR, "csrc", src)], verbose)
        objs.append(obj)
    out = os.path.join(out_dir, "libq3t_hip.so")
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", tmp, *objs], verbose)
    os.replace(tmp, out)
    return out


def build_facade(verbose=False):
    """libqwen3tts_amd.so: the drop-in TTSTransformer + GGUF reader (host C++,
    g++), linked against the device library; plus the C++ facade test driver."""
    csrc = os.path.join(PKG_DIR, "csrc")
    lib_dir = os.path.join(PKG_DIR, "lib")
    out = os.path.join(lib_dir, "libqwen3tts_amd.so")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-o", out + ".tmp",
           os.path.join(csrc, "tts_transformer.cpp"), os.path.join(csrc, "audio_tokenizer_decoder.cpp"),
           os.path.join(csrc, "gguf_reader.cpp"),
           "-L" + lib_dir, "-lq3t_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("g++ (facade) failed:\n" + r.stderr[-4000:])
    os.replace(out + ".tmp", out)
    root = os.path.dirname(PKG_DIR)
    for name in ("test_transformer_dev", "test_vocoder_dev", "test_gguf_config"):
        test_src = os.path.join(root, "tests", "cpp", name + ".cpp")
        test_bin = os.path.join(lib_dir, name)
        if not os.path.exists(test_src):
            continue
        cmd = ["g++", "-O2", "-std=c++17", "-I" + csrc, "-o", test_bin, test_src, "-L" + lib_dir,
               "-lqwen3tts_amd", "-lq3t_hip", "-Wl,-rpath," + lib_dir, "-Wl,-rpath,$ORIGIN"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("g++ (facade test) failed:\n" + r.stderr[-4000:])
    if verbose:
        print("built", out)
    return out
