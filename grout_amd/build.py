"""Build libgrout_attn_hip.so (the C-ABI library) in-tree with hipcc for gfx950.

Usage: ``python -m grout_amd.build [--verbose]``.  Each ``csrc/*.hip`` file is
compiled separately (in parallel) and linked into ``grout_amd/libgrout_attn_hip.so``.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libgrout_attn_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 VALU forms are disabled for every HIP file (hipcc's host pass
# warns that it does not know the feature; that is harmless).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Single-lane counter RMWs stay plain atomics: the wave-aggregating rewrite
    # consumes the returned value right after issue, i.e. waits a memory round
    # trip where the kernel only needs the value at its end.
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    # MFMAs accumulate in ordinary VGPRs: the decode accumulators are also
    # touched by VALU (rare rescale), and the AGPR form would copy them into
    # and out of the accumulation registers around every MFMA.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
]


#: Flags for single files: gfx940+ kernel-argument preload, so the pointers a
#: kernel reads first arrive in SGPRs at dispatch instead of through a
#: kernel-argument load.  The decode attention kernels take the device
#: position pointer as their first argument (its load then goes out at the
#: first instruction); the decode-layer kernels (GEMV, norms, SiLU, argmax)
#: take their tensors first (Qwen3-32B token step 12.866 -> 12.819 ms).
FILE_FLAGS = {
    "attn_decode.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=2"],
    "decode_layer.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=5"],
}


def sources(d: str = CSRC) -> list[str]:
    return sorted(os.path.join(d, f) for f in os.listdir(d) if f.endswith(".hip"))


def _compile(src: str, verbose: bool, extra: list[str]) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), *extra, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in line and line.strip())
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{out}")
    if verbose and out:
        print(out, flush=True)
    return obj


def _link(objs: list[str], path: str, verbose: bool) -> None:
    tmp = path + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, path)


def build(verbose: bool = False, extra: list[str] | None = None) -> str:
    """Compile every csrc/*.hip for gfx950 and link the C-ABI library."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    extra = list(extra or [])
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(len(srcs), 8)) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, extra), srcs))
    _link(objs, LIB_PATH, verbose)
    return LIB_PATH


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--verbose", "-v", action="store_true")
    ap.add_argument("--resource-usage", action="store_true",
                    help="print per-kernel VGPR/AGPR/LDS usage from the compiler")
    args = ap.parse_args(argv)
    extra = ["-Rpass-analysis=kernel-resource-usage"] if args.resource_usage else []
    path = build(verbose=args.verbose or args.resource_usage, extra=extra)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
