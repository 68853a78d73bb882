"""Build libunicache_hip.so (gfx950) in-tree with hipcc.

Usage: ``python -m unicache_amd.build`` or ``unicache_amd.build.build()``.
The library lands next to this file, where ``unicache_amd._native`` loads it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libunicache_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = os.environ.get("UNICACHE_HIP_ARCH", "gfx950")

SOURCES = [
    "uc_api.hip",
    "uc_pack.hip",
    "uc_decode.hip",
    "uc_decode_mfma.hip",
    "uc_attn_mq.hip",
    "uc_merge.hip",
    "uc_h2o.hip",
    "uc_h2o_mfma.hip",
    "uc_compact.hip",
    "uc_stream.hip",
    "uc_parts.hip",
]

# -ffp-contract=off keeps the pack/dequant arithmetic bit-exact (no implicit
# FMA); hot loops request FMAs explicitly.  Packed fp32 instructions are
# disabled for every kernel.
COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the MI355X kernels need ROCm's hipcc")
    return path


# Per-source flags.  The decode kernel rescales its MFMA output accumulators
# in VALU code; keeping MFMA results in VGPRs avoids moving them between AGPRs
# and VGPRs every iteration.
SOURCE_FLAGS = {
    "uc_decode_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: str, obj: str, extra: list[str]) -> None:
    cmd = [_hipcc(), *COMMON_FLAGS, *SOURCE_FLAGS.get(src, []), *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stdout}\n{proc.stderr}")


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> str:
    """Compile every kernel source and link the shared library; return its path."""

    extra = list(extra_flags or [])
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    sources = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    objs = [os.path.join(objdir, s.replace(".hip", ".o")) for s in sources]
    workers = max(1, min(len(sources), int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        futures = [pool.submit(_compile, s, o, extra) for s, o in zip(sources, objs)]
        for fut in futures:
            fut.result()
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True, extra_flags=sys.argv[1:])
