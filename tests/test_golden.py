"""The oracle against the committed golden vectors (tests/golden/), on the CPU.

The fixtures hold the seeded inputs' bits and CRCs, and the expert ids, routing
weights and bf16 output bits of small cases of every preset; they were written
by ``tests/golden/make_golden.py``. A change in the oracle's arithmetic, its
routing, or the seeded generation fails here. The same fixtures pin the HIP
kernel in ``test_gpu_parity.py``.
"""

import json
import sys
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(HERE))

import make_golden as mg  # noqa: E402
from sgl_amd_mono.moe.presets import workload_dict  # noqa: E402


@pytest.mark.parametrize("workload,rows", mg.CASES)
def test_oracle_reproduces_fixture(workload, rows):
    want = np.load(mg.case_file(workload, rows))
    got = mg.compute(workload, rows)
    assert np.array_equal(got["x_bits"], want["x_bits"]), "seeded x"
    assert np.array_equal(got["experts"], want["experts"]), "experts read"
    assert np.array_equal(got["crc"], want["crc"]), "seeded weights"
    assert np.array_equal(got["ids"], want["ids"]), "expert ids"
    assert np.array_equal(got["weights_bits"], want["weights_bits"]), "routing weights"
    assert np.array_equal(got["out_bits"], want["out_bits"]), "output bits"


def test_fixture_invariants():
    for workload, rows in mg.CASES:
        f = np.load(mg.case_file(workload, rows))
        ids = f["ids"]
        assert ids.shape[0] == rows
        assert all(len(set(r)) == len(r) for r in ids.tolist()), "distinct experts a row"
        assert set(np.unique(ids).tolist()) == set(f["experts"].tolist()), "the experts read are the ones picked"
        w = f["weights_bits"].view(np.float32)
        scale = workload_dict(workload)["routed_scale"]
        np.testing.assert_allclose(w.sum(axis=1), scale, rtol=1e-6)


def test_fp4_table_is_the_reference_table():
    from oracle import formats as fm

    ref = json.loads((HERE / "fp4_table.json").read_text())["e2m1"]
    got = list(fm.FP4_VALUES)
    assert got == ref and [np.signbit(v) for v in got] == [np.signbit(v) for v in ref]
