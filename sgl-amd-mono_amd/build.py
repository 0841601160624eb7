"""Build the in-tree HIP library ``sgl_amd_mono/moe/libmkmoe.so`` for gfx950.

    python sgl-amd-mono_amd/build.py             # rebuild
    python sgl-amd-mono_amd/build.py --check     # and print the kernels' register / LDS use
    python sgl-amd-mono_amd/build.py --timeline  # the diagnostic build with phase stamps
                                                 # (libmkmoe_tl.so; bench.py --timeline)
    python sgl-amd-mono_amd/build.py --lds       # the LDS budget per shape (a host program)

The library holds the kernels and the C ABI of ``include/mkmoe.h`` and
``include/mkmoe_seam.h``. It is built in place (not installed) so that the same
file runs wherever the tree is copied. The MoE source compiles in parts, in
parallel: one object per compiled MoE shape (``MKMOE_UNIT`` 0 .. 8) and one for
the host code (``MKMOE_UNIT`` 9); the FFN seam's source (``csrc/mkmoe_seam.hip``)
is one more object; then one link. The test hooks of ``include/mkmoe_testing.h``
(``csrc/mkmoe_testing.hip``) build alongside, as ``libmkmoe_testing.so``.
"""

from __future__ import annotations

import argparse
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT = ROOT / "sgl_amd_mono" / "moe" / "libmkmoe.so"
OUT_TIMELINE = ROOT / "sgl_amd_mono" / "moe" / "libmkmoe_tl.so"
OUT_TESTING = ROOT / "sgl_amd_mono" / "moe" / "libmkmoe_testing.so"
SOURCE = CSRC / "mkmoe_kernels.hip"
SEAM_SOURCE = CSRC / "mkmoe_seam.hip"
TESTING_SOURCE = CSRC / "mkmoe_testing.hip"
UNITS = (0, 1, 2, 3, 4, 5, 6, 7, 8, 9)  # the compiled shapes, then the host code
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # no packed fp32 instructions in the device code
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> subprocess.CompletedProcess:
    return subprocess.run(cmd, capture_output=True, text=True)


def build(check: bool = False, verbose: bool = False, timeline: bool = False) -> Path:
    """Compile the library (always; about 30 s with the parts in parallel) and return its path;
    the product build also compiles the test hooks' library (libmkmoe_testing.so)."""
    out = OUT_TIMELINE if timeline else OUT
    defs = ["-DMKMOE_TIMELINE"] if timeline else []
    with tempfile.TemporaryDirectory(prefix="mkmoe_build_") as tmpd:
        objs = [Path(tmpd) / f"unit{u}.o" for u in UNITS] + [Path(tmpd) / "seam.o"]
        cmds = []
        for u, o in zip(UNITS, objs):
            cmds.append([HIPCC, *FLAGS, *defs, f"-DMKMOE_UNIT={u}", "-c", str(SOURCE), "-o", str(o)])
        cmds.append([HIPCC, *FLAGS, "-c", str(SEAM_SOURCE), "-o", str(objs[-1])])
        testing_tmp = OUT_TESTING.with_suffix(".so.tmp")
        if not timeline:
            cmds.append([HIPCC, *FLAGS, "-shared", str(TESTING_SOURCE), "-o", str(testing_tmp)])
        if check:
            for cmd in cmds:
                cmd.append("-Rpass-analysis=kernel-resource-usage")
        if verbose:
            print(" ".join(cmds[0]), flush=True)
        jobs = min(len(cmds), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
        with ThreadPoolExecutor(jobs) as ex:
            results = list(ex.map(_run, cmds))
        for cmd, res in zip(cmds, results):
            if res.returncode != 0:
                sys.stderr.write(res.stdout + res.stderr)
                raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}")
        if check:
            keep = ("Function Name", "VGPRs:", "ScratchSize", "LDS Size", "Occupancy")
            for res in results:
                for line in res.stderr.splitlines():
                    if any(k in line for k in keep):
                        print(line.split("remark:")[-1].replace("[-Rpass-analysis=kernel-resource-usage]", "").strip())
        tmp = out.with_suffix(".so.tmp")
        link = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *(str(o) for o in objs), "-o", str(tmp)]
        res = _run(link)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"link failed ({res.returncode})")
        os.replace(tmp, out)
        if not timeline:
            os.replace(testing_tmp, OUT_TESTING)
    return out


def lds_budget() -> str:
    """The persistent launch's LDS budget per compiled shape (a markdown table): a host program
    built from csrc/mkmoe_lds.hip, which sizes each stage's member of the LDS union."""
    with tempfile.TemporaryDirectory(prefix="mkmoe_lds_") as tmpd:
        exe = Path(tmpd) / "mkmoe_lds"
        res = _run([HIPCC, *FLAGS, str(CSRC / "mkmoe_lds.hip"), "-o", str(exe)])
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"mkmoe_lds build failed ({res.returncode})")
        res = _run([str(exe)])
        if res.returncode != 0:
            raise RuntimeError(f"mkmoe_lds failed ({res.returncode})")
        return res.stdout


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true")
    ap.add_argument("--timeline", action="store_true")
    ap.add_argument("--lds", action="store_true", help="print the LDS budget per shape (no library build)")
    args = ap.parse_args()
    if args.lds:
        print(lds_budget(), end="")
    else:
        print(build(check=args.check, verbose=True, timeline=args.timeline))
