"""Build driver: configures and builds the CMake project (gfx950 only) in-tree.

``build()`` always re-runs CMake (configure + build), in-tree:
``vkwr_amd/libvkwr_amd.so`` (HIP kernels, C ABI of include/vkwr_amd.h) and the
torch extension modules ``vkwr/_v1_*_C.so``, ``vkwr/_rwkv7_C.so`` and
``vkwr/_sampling_C.so``.
"""
import os
import subprocess
import sys
import sysconfig

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD_DIR = os.path.join(ROOT, "_build")


def build(verbose=False, jobs=None):
    import torch  # noqa: F401  (only for its install location)

    torch_dir = os.path.dirname(torch.__file__)
    py_inc = sysconfig.get_paths()["include"]
    jobs = jobs or min(16, os.cpu_count() or 4)
    cfg = ["cmake", "-S", ROOT, "-B", BUILD_DIR, "-G", "Ninja",
           f"-DTORCH_DIR={torch_dir}", f"-DPYTHON_INCLUDE_DIR={py_inc}",
           "-DCMAKE_HIP_COMPILER=/opt/rocm/llvm/bin/clang++",
           "-DCMAKE_PREFIX_PATH=/opt/rocm", "-DCMAKE_BUILD_TYPE=Release"]
    out = None if verbose else subprocess.PIPE
    for cmd in (cfg, ["cmake", "--build", BUILD_DIR, "-j", str(jobs)]):
        p = subprocess.run(cmd, stdout=out, stderr=subprocess.STDOUT, text=True)
        if p.returncode != 0:
            if p.stdout:
                sys.stderr.write(p.stdout[-20000:])
            raise RuntimeError(f"vkwr_amd build failed: {' '.join(cmd)}")


if __name__ == "__main__":
    build(verbose=True)
