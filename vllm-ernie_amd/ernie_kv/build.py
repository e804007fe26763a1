"""Build ``libernie_kv.so`` for gfx950 with hipcc, in-tree.

The library is a plain C-ABI shared object (``include/ernie_kv.h``); no torch
headers are involved.  Kernels whose arithmetic the CPU oracle mirrors bit for
bit (append/quant, compressor, indexer scoring) are compiled with
``-ffp-contract=off`` so hipcc cannot fuse a multiply-add the oracle does not
perform; the decode kernel (tolerance-checked) keeps contraction on.

Usage: ``python -m ernie_kv.build`` (from ``vllm-ernie_amd/``) or
``ernie_kv.build.build()``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR.parent / "csrc"
LIB_PATH = PKG_DIR / "libernie_kv.so"
ARCH = os.environ.get("EKV_OFFLOAD_ARCH", "gfx950")

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # Packed FP32 arithmetic stays off: hipcc must not emit v_pk_{add,mul,fma}_f32.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]
EXACT = ["-ffp-contract=off"]
# MFMA results in ordinary VGPRs rather than accumulation registers, so the
# indexer's page loops use them without a copy back (the scores they feed
# are the same).
MFMA_VGPR = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
SOURCES = {
    "ekv_status.cpp": [],
    "ekv_append.hip": EXACT,
    "ekv_hca.hip": EXACT,
    "ekv_indexer.hip": EXACT + MFMA_VGPR,
    "ekv_decode.hip": [],
    "ekv_quant.hip": EXACT,
    "ekv_mxfp4.hip": EXACT,
    "ekv_pages.hip": EXACT,
}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the ERNIE KV library needs ROCm's hipcc")
    return path


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")


def build(verbose: bool = False) -> Path:
    """Compile every source and link ``libernie_kv.so`` next to this module."""
    from concurrent.futures import ThreadPoolExecutor

    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix="ekv_build_") as tmp:
        objs, cmds = [], []
        for src, extra in SOURCES.items():
            obj = Path(tmp) / (Path(src).stem + ".o")
            cmds.append([cc, *COMMON, *extra, "-I", str(CSRC), "-c", str(CSRC / src), "-o", str(obj)])
            if verbose:
                print(" ".join(cmds[-1]), flush=True)
            objs.append(str(obj))
        # one compiler process per source, at most as many as the cores allow
        workers = max(1, min(len(cmds), len(os.sched_getaffinity(0)), 8))
        with ThreadPoolExecutor(workers) as pool:
            list(pool.map(_run, cmds))
        out_tmp = LIB_PATH.with_suffix(".so.tmp")
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(out_tmp)])
        os.replace(out_tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv)
    print(p)
