"""Build the gfx950 sparse_attn libraries in-tree (no JIT cache, no ninja).

Outputs, all under ``kernelgen-challenge_amd/lib/``:

* ``libsparse_attn_gfx950.so`` -- HIP kernels + C-ABI (``include/sparse_attn.h``),
  built by ``hipcc --offload-arch=gfx950`` only.
* ``libhc_sinkhorn_gfx950.so`` -- the track-02 ``hc_split_sinkhorn`` kernels +
  C-ABI (``include/hc_sinkhorn.h``), built the same way.
* ``libfused_moe_gfx950.so`` -- the track-03 ``fused_moe`` kernels + C-ABI
  (``include/fused_moe.h``), built the same way.
* ``libsa_noalloc_gfx950.so`` -- the allocation-free entry point
  ``sa_forward_noalloc`` (``include/sparse_attn_noalloc.h``) and its 48 MiB
  device array, linked to ``libsparse_attn_gfx950.so``: only processes that
  load it hold the array.
* ``sa_torch_ext.so`` -- the PyTorch-ROCm operators ``torch.ops.sa_amd.*``
  (host C++ against torch's headers), linked to the two libraries above with
  an ``$ORIGIN`` rpath.
* ``libsa_host_test.so`` -- g++ build of the host-side validation and launch
  planning, for CPU tests of the C-ABI's argument handling.

Run ``python kernelgen-challenge_amd/build.py``; every call rebuilds.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO, "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")

HIP_LIB = os.path.join(LIB_DIR, "libsparse_attn_gfx950.so")
HC_LIB = os.path.join(LIB_DIR, "libhc_sinkhorn_gfx950.so")
FM_LIB = os.path.join(LIB_DIR, "libfused_moe_gfx950.so")
NOALLOC_LIB = os.path.join(LIB_DIR, "libsa_noalloc_gfx950.so")
TORCH_EXT = os.path.join(LIB_DIR, "sa_torch_ext.so")
HOST_TEST_LIB = os.path.join(LIB_DIR, "libsa_host_test.so")

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

# Packed-fp32 VALU forms are kept out of every gfx950 code object.
# -amdgpu-mfma-vgpr-form: compiler-generated MFMAs accumulate in VGPRs. The
# shared-row kernel issues its O += P . V MFMAs as inline assembly with AGPR
# accumulators (all 256 AGPRs hold O) and its S = K . Q^T MFMAs through the
# compiler; without the flag the compiler also gives S AGPRs and shuffles
# part of O through VGPRs every step.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def _run(cmd, verbose, strict=False):
    """Run one compiler command. Its diagnostics are always printed (hipcc's
    host-pass note that it does not know the packed-fp32 feature aside, which
    is harmless); with ``strict`` any of them fails the build."""
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"build step failed ({res.returncode}): {cmd[0]} ... {cmd[-1]}")
    noise = [ln for ln in (res.stdout + res.stderr).splitlines()
             if ln.strip() and "packed-fp32-ops" not in ln]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")
        if strict:
            raise RuntimeError(f"build step printed diagnostics (treated as errors): {cmd[-3]}")


def _atomic_target(path):
    return path + f".tmp{os.getpid()}"


def build_hip_lib(verbose=False):
    hipcc = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    for src, out in (("sparse_attn_gfx950.hip", HIP_LIB), ("hc_sinkhorn_gfx950.hip", HC_LIB),
                     ("fused_moe_gfx950.hip", FM_LIB)):
        tmp = _atomic_target(out)
        _run([hipcc, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}",
              os.path.join(CSRC, src), "-o", tmp], verbose, strict=True)
        os.replace(tmp, out)
    tmp = _atomic_target(NOALLOC_LIB)
    _run([hipcc, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}",
          os.path.join(CSRC, "sa_noalloc_gfx950.hip"), f"-L{LIB_DIR}", "-lsparse_attn_gfx950",
          "-Wl,-rpath,$ORIGIN", "-o", tmp], verbose, strict=True)
    os.replace(tmp, NOALLOC_LIB)


def build_torch_ext(verbose=False):
    import torch
    from torch.utils import cpp_extension

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = cpp_extension.include_paths() + [os.path.join(ROCM, "include"), INCLUDE]
    libdirs = cpp_extension.library_paths()
    tmp = _atomic_target(TORCH_EXT)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1",
           "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=sa_torch_ext",
           "-Wno-deprecated-declarations"]
    cmd += [f"-I{p}" for p in incs]
    cmd += [f"-isystem{sysconfig.get_paths()['include']}"]
    cmd += [os.path.join(CSRC, "sa_torch.cpp"), "-o", tmp]
    cmd += [f"-L{p}" for p in libdirs] + [f"-L{LIB_DIR}", f"-L{ROCM}/lib"]
    cmd += ["-lsparse_attn_gfx950", "-lhc_sinkhorn_gfx950", "-lfused_moe_gfx950", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
            "-ltorch_hip", "-ltorch_python", "-lamdhip64", "-Wl,-rpath,$ORIGIN"]
    cmd += [f"-Wl,-rpath,{p}" for p in libdirs]
    _run(cmd, verbose)
    os.replace(tmp, TORCH_EXT)


def build_host_test_lib(verbose=False):
    tmp = _atomic_target(HOST_TEST_LIB)
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
          f"-I{INCLUDE}", f"-I{CSRC}", os.path.join(CSRC, "sa_host_test.cpp"),
          "-o", tmp], verbose)
    os.replace(tmp, HOST_TEST_LIB)


def build(verbose=False):
    os.makedirs(LIB_DIR, exist_ok=True)
    build_hip_lib(verbose)
    build_torch_ext(verbose)
    build_host_test_lib(verbose)


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
    print(f"built {HIP_LIB}\n      {HC_LIB}\n      {FM_LIB}\n      {NOALLOC_LIB}\n      {TORCH_EXT}\n"
          f"      {HOST_TEST_LIB}")
