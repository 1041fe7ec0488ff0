"""Compile the gfx950 HIP library ``libllattn_gfx950.so`` in-tree with hipcc.

Usage: ``python -m llattn_amd._build`` (from ``local-latent-attention_amd/``) or
``__graft_entry__.build()``.  Always recompiles.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
SRC_DIR = PKG_DIR.parent / "csrc"
INCLUDE_DIR = PKG_DIR.parents[1] / "include"
LIB_NAME = "libllattn_gfx950.so"
SOURCES = ("llattn_abi.cpp", "llattn_pool.hip", "llattn_latent.hip", "llattn_local.hip", "llattn_local_wide.hip",
           "llattn_gemm.hip", "llattn_gemm_f32.hip",
           "llattn_colsum.hip", "llattn_cast.hip", "llattn_norm.hip",
           "llattn_xent.hip")
ARCH = "gfx950"

# -packed-fp32-ops off: hipcc must not emit packed fp32 arithmetic for this target.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fno-gpu-rdc",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-inline-asm",
]


# Per-source additions: the wide-window backward keeps its MFMA accumulators in VGPRs (no AGPRs), so that a
# wave's whole 256-register budget at two waves per SIMD is usable without copies between register files.
EXTRA_FLAGS = {"llattn_local_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the llattn HIP library needs ROCm's hipcc to build")
    return path


def build(verbose: bool = False) -> Path:
    """Compile every source and link the shared library next to this file."""
    cc = hipcc()
    out = PKG_DIR / LIB_NAME
    with tempfile.TemporaryDirectory(prefix="llattn_build_") as tmp:
        objs, procs = [], []
        for src in SOURCES:
            obj = Path(tmp) / (Path(src).stem + ".o")
            cmd = [cc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), f"-I{INCLUDE_DIR}", f"-I{SRC_DIR}", "-c",
                   str(SRC_DIR / src), "-o", str(obj)]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
            objs.append(str(obj))
        failed = []
        for src, p in procs:
            log, _ = p.communicate()
            log = "\n".join(l for l in log.splitlines() if "packed-fp32-ops" not in l)
            if p.returncode != 0:
                failed.append(f"--- {src} ---\n{log}")
            elif verbose and log.strip():
                print(log)
        if failed:
            raise RuntimeError("hipcc failed:\n" + "\n".join(failed))
        tmp_out = Path(tmp) / LIB_NAME
        link = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp_out), *objs]
        r = subprocess.run(link, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
        os.replace(tmp_out, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
