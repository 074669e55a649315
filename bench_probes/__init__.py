"""Measurement probes that bench.py runs beside the attention kernels.

Not part of the product: the C-ABI library (grout_amd/libgrout_attn_hip.so)
neither contains nor loads them.  ``build()`` compiles ``*.hip`` in this folder
for gfx950 into ``bench_probes/libgrout_probe.so``:

* ``mfma_ceiling.hip``: the sustained v_mfma_f32_32x32x16_f16 rate for
  operand data distributed like the prefill kernel's;
* ``hbm_read.hip``: the sustained HBM read rate of a plain streaming kernel.
* ``hbm_copy.hip``: the sustained rate of a plain streaming copy (read + write).
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgrout_probe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def sources() -> list[str]:
    return sorted(os.path.join(HERE, f) for f in os.listdir(HERE) if f.endswith(".hip"))


def build(verbose: bool = False) -> str:
    """Compile and link the probes (one hipcc call; a few seconds)."""
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           *sources(), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"probe build failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def lib_path() -> str:
    """The probe library, built first when it is missing."""
    if not os.path.exists(LIB_PATH):
        build()
    return LIB_PATH
