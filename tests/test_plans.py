"""Kernel planners against what their kernels assume (CPU only, no GPU call).

tests/plan_invariants.cpp calls the planners exported by the built libqmm4.so (row-split, its
x-in-registers form, row-phase, K-split verify, GEMM) over a grid of shapes (1-4096 rows, 16-262144 columns,
K = 128-20480) and CU counts (1-304), and checks every accepted plan: dynamic LDS within 160 KB,
output columns covered exactly once, K slices and units that tile K, each loop form only in the
configuration its launch path instantiates, stream-K workgroups between 1 and the unit count
within the workspace. The planners pick the kernel for the reference's quantized_matmul
(packed_linear.py:83-104 routes by rows), so a plan that broke one of these would launch a kernel
outside its assumptions.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "mlx-tree-spec_amd", "mlx_tree_spec_amd")
LIB = os.path.join(LIBDIR, "libqmm4.so")


def test_planners_keep_kernel_invariants(tmp_path):
    if not os.path.exists(LIB):
        pytest.skip("libqmm4.so is not built (run __graft_entry__.build())")
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ is not available")
    exe = tmp_path / "plan_invariants"
    cmd = [cxx, "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "mlx-tree-spec_amd", "csrc"),
           os.path.join(ROOT, "tests", "plan_invariants.cpp"), "-L", LIBDIR, "-lqmm4",
           f"-Wl,-rpath,{LIBDIR}", "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert build.returncode == 0, build.stderr[-4000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stdout[-4000:] + run.stderr[-2000:]
    assert "violations: 0" in run.stdout
    checked = int(run.stdout.split("plans checked:")[1].split(",")[0])
    assert checked > 10000, run.stdout
