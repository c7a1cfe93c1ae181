"""Build recipe for the gfx950 shared library ``libtpf_amd.so``.

Every HIP source under ``csrc/`` is compiled with hipcc for gfx950 only and
linked into one C-ABI shared library that sits next to this file.  The
library exports plain ``extern "C"`` entry points (declared in
``include/tpf_amd.h``); Python reaches them through ``ctypes``.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libtpf_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME
BUILD_DIR = PKG_DIR / "_build"
ARCH = "gfx950"

# Packed FP32 VALU ops are disabled for all device code (hipcc -O3 otherwise
# forms v_pk_* f32 instructions from ordinary float code).
DEVICE_FLAGS = [
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # Keep MFMA accumulators in ordinary VGPRs (no v_accvgpr copies around
    # the softmax / epilogue code that reads them).
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
]


# Per-source extra flags.  attention.hip: the kernels never test for NaN
# and take scores that are finite or -inf, so fmaxf needs no NaN quieting
# (without the flag every v_max of an MFMA result is preceded by a
# canonicalising v_max: six VALU instructions per 32 x 32 score block).
FILE_FLAGS = {"attention.hip": ["-fno-honor-nans"]}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the TurboPairFormer MI355X library needs ROCm's hipcc")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source for gfx950 and link ``libtpf_amd.so`` (always rebuilds)."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    common = [
        "-O3",
        "-std=c++17",
        "-fPIC",
        f"--offload-arch={ARCH}",
        f"-I{CSRC}",
        f"-I{PKG_DIR.parent / 'include'}",
        "-Wno-unused-command-line-argument",
    ]
    objs = []
    cmds = []
    for src in sources():
        obj = BUILD_DIR / (src.stem + ".o")
        objs.append(obj)
        extra = (DEVICE_FLAGS + FILE_FLAGS.get(src.name, [])) if src.suffix == ".hip" else []
        lang = ["-x", "hip"] if src.suffix == ".hip" else []
        cmds.append([hipcc, *common, *extra, *lang, "-c", str(src), "-o", str(obj)])

    def run(cmd):
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{res.stderr}")
        return res

    jobs = jobs or min(8, max(1, len(cmds)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(run, cmds))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    run([hipcc, "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
