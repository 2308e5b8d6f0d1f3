"""Build libqmm4.so (the gfx950 kernels + C ABI) in-tree with hipcc.

    python -m mlx_tree_spec_amd.build      (with mlx-tree-spec_amd/ on sys.path)

Objects compile in parallel; the library is linked to a temporary name and renamed, so a reader
never sees a half-written file.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
PROJ_DIR = os.path.dirname(PKG_DIR)
REPO_DIR = os.path.dirname(PROJ_DIR)
CSRC = os.path.join(PROJ_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_NAME = "libqmm4.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
# The benchmark's measurement floors (an empty launch, a streaming read): csrc/floor/, a library
# of its own that only bench.py loads.
FLOOR_DIR = os.path.join(CSRC, "floor")
FLOOR_PATH = os.path.join(PKG_DIR, "libqmm4_floor.so")
ARCH = os.environ.get("QMM4_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in device code. hipcc's host pass warns that
# it does not know the feature; that warning is harmless.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC,
]


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src: str, obj: str) -> None:
    cmd = ["hipcc", *HIPCC_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")


def _link(srcs: list[str], out: str) -> None:
    with tempfile.TemporaryDirectory(prefix="qmm4_build_") as tmp:
        objs = [os.path.join(tmp, os.path.basename(s) + ".o") for s in srcs]
        with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
            list(ex.map(_compile, srcs, objs))
        out_tmp = out + f".tmp{os.getpid()}"
        # --no-undefined: a kernel whose host stub the compiler dropped fails here, not at load time.
        cmd = ["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", *objs, "-o", out_tmp]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
        os.replace(out_tmp, out)


def build(verbose: bool = False) -> str:
    _link(sources(), LIB_PATH)
    _link(sorted(os.path.join(FLOOR_DIR, f) for f in os.listdir(FLOOR_DIR) if f.endswith(".hip")), FLOOR_PATH)
    if verbose:
        print(f"built {LIB_PATH} and {FLOOR_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
