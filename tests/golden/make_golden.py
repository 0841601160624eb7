"""Write the golden vectors of the decode MoE block (run from the repository root).

    python tests/golden/make_golden.py

For a few small cases (one preset and row count each) it stores, from the
oracle's seeded CPU inputs: the input rows' bits, a CRC-32 of every generated
weight tensor the case reads (the dense ones and each routed expert's), and
the oracle's expert ids, routing weights and bf16 output bits. The tests check
the oracle against these files (``tests/test_golden.py``) and the HIP kernel
against them (``tests/test_gpu_parity.py``), so a change in either, or in the
seeded generation, shows up as a fixture mismatch.

``fp4_table.json`` holds the e2m1 table of the reference's golden model
(``test/kernels/deepseek_v41/check_ffn.py:23-40``), copied as data.
"""

from __future__ import annotations

import sys
import zlib
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "sgl-amd-mono_amd")]

from oracle import gen  # noqa: E402
from oracle import moe as om  # noqa: E402
from sgl_amd_mono.moe.presets import workload_dict  # noqa: E402

CASES = [("cfg1_plumbing_fp8", 4), ("cfg2_tp4_fp8", 1), ("cfg3_tp4_mxfp4", 1), ("cfg5_tp2_mxfp4_norm", 1), ("plumbing_fp8_softplus", 4)]
HERE = Path(__file__).resolve().parent


def crc(t: torch.Tensor) -> int:
    return zlib.crc32(t.contiguous().view(torch.uint8).numpy().tobytes()) if t.dtype != torch.uint8 else zlib.crc32(t.contiguous().numpy().tobytes())


def case_file(workload: str, rows: int) -> Path:
    return HERE / f"moe_{workload}_r{rows}.npz"


def compute(workload: str, rows: int, seed: int = 0) -> dict:
    p = workload_dict(workload)
    x = gen.make_x(p, rows, seed)
    dense = gen.make_dense(p, seed)
    ex = gen.LazyExperts(p, seed)
    res = om.moe_partial(x, dense, p, experts=ex)
    experts = sorted(ex.cache)
    crcs = [crc(dense[k]) for k in sorted(dense)]
    for e in experts:
        crcs += [crc(t) for t in ex.cache[e]]
    return {
        "x_bits": x.view(torch.int16).numpy(),
        "dense_names": np.array(sorted(dense)),
        "experts": np.array(experts, dtype=np.int32),
        "crc": np.array(crcs, dtype=np.uint32),
        "ids": res["ids"].astype(np.int32),
        "weights_bits": res["weights"].astype(np.float32).view(np.uint32),
        "out_bits": res["out"].view(torch.int16).numpy(),
    }


def main() -> None:
    for wl, r in CASES:
        d = compute(wl, r)
        np.savez_compressed(case_file(wl, r), **d)
        print(f"{case_file(wl, r).name}: experts {d['experts'].tolist()}")
    fp4 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    import json

    (HERE / "fp4_table.json").write_text(json.dumps({"source": "test/kernels/deepseek_v41/check_ffn.py:23-40", "e2m1": fp4}) + "\n")


if __name__ == "__main__":
    main()
