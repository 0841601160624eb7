"""Build the in-tree HIP library ``sgl_amd_mono/moe/libmkmoe.so`` for gfx950.

    python sgl-amd-mono_amd/build.py          # rebuild
    python sgl-amd-mono_amd/build.py --check  # print the kernels' register / LDS use

The library holds the kernels and the C ABI of ``include/mkmoe.h``. It is built
in place (not installed) so that the same file runs wherever the tree is copied.
"""

from __future__ import annotations

import argparse
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT = ROOT / "sgl_amd_mono" / "moe" / "libmkmoe.so"
SOURCES = [CSRC / "mkmoe_kernels.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # no packed fp32 instructions in the device code
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def build(check: bool = False, verbose: bool = False) -> Path:
    """Compile the library (always; a few tens of seconds) and return its path."""
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, *(str(s) for s in SOURCES), "-o", str(tmp)]
    if check:
        cmd.append("-Rpass-analysis=kernel-resource-usage")
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode})")
    if check:
        keep = ("Function Name", "VGPRs:", "ScratchSize", "LDS Size", "Occupancy")
        for line in res.stderr.splitlines():
            if any(k in line for k in keep):
                print(line.split("remark:")[-1].replace("[-Rpass-analysis=kernel-resource-usage]", "").strip())
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true")
    args = ap.parse_args()
    print(build(check=args.check, verbose=True))
