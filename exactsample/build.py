"""Builds the gfx950 library and the PyTorch op binding in place.

    python -m exactsample.build            # both
    python -m exactsample.build --lib-only # the C-ABI library only

Outputs (next to this file):
  libexactsample_amd.so       HIP kernels + the C ABI of include/exactsample_amd.h
  _exactsample_ops.so         the exactsample::verify_out torch op (links the above)

hipcc cross-compiles for gfx950 without a GPU. Every HIP source is built with
-ffp-contract=off (the FP32 error bounds assume no fused multiply-add
contraction) and with packed FP32 instructions disabled.
"""
import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libexactsample_amd.so")
OPS = os.path.join(HERE, "_exactsample_ops.so")
KERNEL_UNITS = ["es_f32.hip", "es_bf16.hip", "es_f16.hip", "es_f64.hip", "es_api.hip", "es_selftest.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("EXACTSAMPLE_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    noise = "is not a recognized feature for this target"
    text = "\n".join(line for line in proc.stdout.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{text}")
    return text


def build_library(jobs=None):
    """Compiles the HIP units in parallel and links libexactsample_amd.so."""
    tmp = tempfile.mkdtemp(prefix="es_build_")
    try:
        objects = [os.path.join(tmp, unit.replace(".hip", ".o")) for unit in KERNEL_UNITS]
        commands = [[HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, unit), "-o", obj]
                    for unit, obj in zip(KERNEL_UNITS, objects)]
        workers = jobs or min(len(commands), os.cpu_count() or 1)
        with concurrent.futures.ThreadPoolExecutor(workers) as pool:
            list(pool.map(_run, commands))
        staged = LIB + ".tmp"
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", staged])
        os.replace(staged, LIB)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return LIB


def build_ops():
    """Compiles the torch op binding (host C++ only, no device code) against the built library."""
    import torch
    import torch.utils.cpp_extension as ce
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    includes = [f"-I{p}" for p in ce.include_paths(device_type="cuda")] + [f"-I{INCLUDE}"]
    libdirs = [f"-L{p}" for p in ce.library_paths(device_type="cuda")]
    staged = OPS + ".tmp"
    # g++ as PyTorch itself is built, so C++ symbol mangling matches libtorch.
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *includes, os.path.join(CSRC, "binding.cpp"), "-o", staged,
        *libdirs, "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        f"-L{HERE}", "-lexactsample_amd", "-Wl,-rpath,$ORIGIN",
    ]
    _run(cmd)
    os.replace(staged, OPS)
    return OPS


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--lib-only", action="store_true")
    parser.add_argument("--jobs", type=int)
    args = parser.parse_args(argv)
    print(build_library(args.jobs), flush=True)
    if not args.lib_only:
        print(build_ops(), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
