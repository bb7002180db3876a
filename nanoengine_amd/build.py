"""Build the gfx950 HIP library ``libdsa_amd.so`` in-tree with hipcc.

Run ``python -m nanoengine_amd.build`` (or ``__graft_entry__.build()``); the
library lands next to this file so it travels with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "libdsa_amd.so"
# measurement kernels for `bench.py --micro`, kept out of the product library
MICROBENCH_SRC = "microbench.hip"
MICROBENCH_LIB = PKG_DIR / "libdsa_microbench.so"
SOURCES = ["capi.hip", "topk.hip", "indexer.hip", "sparse_mla.hip", "cache_store.hip",
           "indexer_prologue.hip", "prefill_logits.hip", "sparse_mla_prefill.hip",
           "prefill_topk.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-result",
    # No packed-fp32 instructions in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# MFMA results in VGPRs where the accumulators feed VALU work (ReLU, top-k
# keys) every step and AGPR-resident results would cost a copy each time. The
# sparse-MLA kernels and the prologue use the compiler's default register
# assignment.
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
PER_FILE_FLAGS = {
    "capi.hip": VGPR_FORM,
    "topk.hip": VGPR_FORM,
    "indexer.hip": VGPR_FORM,
    "cache_store.hip": VGPR_FORM,
    "sparse_mla.hip": [],
    "sparse_mla_prefill.hip": [],
    "indexer_prologue.hip": [],
    "prefill_logits.hip": VGPR_FORM,
    "prefill_topk.hip": VGPR_FORM,
}


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 (in parallel) and link the shared library."""
    from concurrent.futures import ThreadPoolExecutor

    with tempfile.TemporaryDirectory(prefix="dsa_build_") as tmp:
        objs = [os.path.join(tmp, Path(s).stem + ".o") for s in SOURCES]
        cmds = [[hipcc(), *HIPCC_FLAGS, *PER_FILE_FLAGS[s], "-c", str(CSRC / s), "-o", o]
                for s, o in zip(SOURCES, objs)]
        cmds.append([hipcc(), *HIPCC_FLAGS, "-shared", str(CSRC / MICROBENCH_SRC), "-o", str(MICROBENCH_LIB)])
        with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as pool:
            list(pool.map(lambda c: _run(c, verbose), cmds))
        _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(LIB_PATH), *objs], verbose)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
