"""Build recipe for libsage_mi355x.so (gfx950 only).

Compiles the HIP sources under ``csrc/`` with ``hipcc`` into one in-tree
shared library.  Packed fp32 VALU instructions are disabled
(``-packed-fp32-ops``); no fast-math flags are used, so fp32 division stays
correctly rounded, which the quantization codes depend on.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libsage_mi355x.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
# the measurement build: the same library with per-phase s_memtime timing of
# the attention kernel's pipelined loop (sage_phase_read), for bench.py
# --phase-timing; never loaded by the product path
PHASE_LIB_PATH = os.path.join(HERE, "libsage_mi355x_phase.so")
SOURCES = ["sage_quant.hip", "sage_attn.hip", "sage_mask.hip", "sage_bwd.hip", "sage_capi.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
    ]


def _link(cc: str, objs: list[str], tmp: str, path: str) -> None:
    tmp_lib = os.path.join(tmp, os.path.basename(path))
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_lib]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    shutil.copyfile(tmp_lib, path + ".tmp")
    os.replace(path + ".tmp", path)


def build(verbose: bool = False, phase_timing: bool = False) -> str:
    """Compile every source and link LIB_PATH atomically; returns LIB_PATH.
    With phase_timing, builds PHASE_LIB_PATH (-DSAGE_PHASE_TIMING) instead."""
    cc = hipcc()
    extra = ["-DSAGE_PHASE_TIMING"] if phase_timing else []
    out_path = PHASE_LIB_PATH if phase_timing else LIB_PATH
    with tempfile.TemporaryDirectory(prefix="sage_build_") as tmp:
        srcs = SOURCES
        objs = [os.path.join(tmp, src + ".o") for src in srcs]

        def compile_one(i: int) -> None:
            cmd = [cc, *flags(), *extra, "-c", os.path.join(CSRC, srcs[i]), "-o", objs[i]]
            if verbose:
                print(" ".join(cmd), flush=True)
            res = subprocess.run(cmd, capture_output=True, text=True)
            if res.returncode != 0:
                raise RuntimeError(f"hipcc failed on {srcs[i]}:\n{res.stderr}")

        # one hipcc process per source file, at most four at a time
        with concurrent.futures.ThreadPoolExecutor(max_workers=min(4, len(srcs))) as pool:
            for f in [pool.submit(compile_one, i) for i in range(len(srcs))]:
                f.result()
        _link(cc, objs, tmp, out_path)
    return out_path


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, phase_timing="--phase-timing" in sys.argv))
