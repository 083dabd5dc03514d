"""In-tree build of ``libpararnn_amd.so`` (gfx950) with hipcc.

The library is a plain C-ABI shared object (declarations in
``include/pararnn_amd.h``); it is loaded with ctypes by ``pararnn_amd._lib``.
Building needs only ROCm's hipcc, no GPU.  Every HIP source is compiled with
packed-fp32 instructions disabled (``-packed-fp32-ops``) and with MFMA results
in ordinary VGPRs (``-amdgpu-mfma-vgpr-form``: no accumulator-register reads in
the MFMA step loops).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)  # pararnn-torch_amd/
CSRC = os.path.join(ROOT, "csrc")
REPO = os.path.dirname(ROOT)
INCLUDE = os.path.join(REPO, "include")
LIB_NAME = "libpararnn_amd.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    exe = os.path.join(rocm, "bin", "hipcc")
    if os.path.exists(exe):
        return exe
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; pararnn_amd needs ROCm to build")
    return found


def _flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-mllvm", "-amdgpu-mfma-vgpr-form=1",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
    ]


# Per-file compiler options on top of _flags() (measured on the bench lines;
# other files were unchanged or slower with them):
#  * the wide-head adjoint walk runs ~8% faster under the iterative ILP
#    scheduler (the forward walks slower);
#  * the sLSTM kernels with the scheduler's AMDGPU register pressure
#    trackers: the fused Newton launch 1.87 -> 1.80 ms at config 3, the
#    packed-stream line ~1.5% faster.
_FILE_FLAGS = {
    "gru_wide_rev.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
    "slstm_diag.hip": ["-mllvm", "-amdgpu-use-amdgpu-trackers=1"],
    "slstm_packed.hip": ["-mllvm", "-amdgpu-use-amdgpu-trackers=1"],
}


def sources() -> list[str]:
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip")
    )


def build(verbose: bool = False) -> str:
    """Compile every ``csrc/*.hip`` and link ``pararnn_amd/libpararnn_amd.so``."""
    hipcc = _hipcc()
    obj_dir = os.path.join(ROOT, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    srcs = sources()

    def compile_one(src: str) -> str:
        obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
        cmd = [hipcc, *_flags(), *_FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
