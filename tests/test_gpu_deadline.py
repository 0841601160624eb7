"""The device deadline path, forced from the host (no wait is made to hang).

A runner whose deadline is one tick (10 ns) gives up every wait at once: the
routing reads part sums that have not landed (the unset marker, a NaN, so every
choice is -inf and the row picks experts 0 .. topk-1 with weight 0), the
hand-offs pass with their data half written, and the launch ends normally. Every
address a launch derives from hand-off data is clamped (expert ids to [0, E),
pick slots to the step's picks), so a launch that gave up stays within its
buffers. The test asserts the error words (code, stage, workgroup, count) and
that ``clear_errors`` (a full workspace reset) restores a launch bit-identical
to a launch on a fresh workspace. The reference's guard test does the same
from its side (``test/kernels/test_guard_hip.py``, ``common/guard.py:69-89``).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("workload,rows", [("cfg2_tp4_fp8", 8), ("cfg2_tp4_fp8", 24), ("cfg3_tp4_mxfp4", 8)])
def test_deadline_gives_up_then_clear_restores(workload, rows):
    from test_gpu_parity import _case, _runner

    from sgl_amd_mono.moe import _lib

    c = _case(workload, rows)
    x = c.x[:rows].contiguous()
    ref_run = _runner(c)
    ref = ref_run.moe(c.w, x).clone()
    torch.cuda.synchronize()
    ref_run.raise_on_device_error()

    print(f"\n{workload} R={rows}: a launch with a one-tick deadline", flush=True)
    run = _runner(c, deadline_s=1e-8)
    out = run.moe(c.w, x)
    torch.cuda.synchronize()
    e = run.read_errors()
    print(f"  error words {e}", flush=True)
    assert e[_lib.ERRW_CODE] == 1, e  # MKMOE_DEVERR_DEADLINE
    assert e[_lib.ERRW_STAGE] in _lib.STAGES, e
    assert 0 <= e[_lib.ERRW_BLOCK] < 256, e
    # one record a wave a wait at most: 8 waves x 256 workgroups x (3 waits + the routing poll)
    assert 1 <= e[_lib.ERRW_COUNT] <= 8 * 256 * 4, e
    with pytest.raises(RuntimeError, match="deadline"):
        run.raise_on_device_error()
    assert out.shape == ref.shape

    # the reset restores the workspace; the next launch equals the fresh workspace's bit for bit
    run.deadline_s = 2.0
    run.clear_errors()
    assert run.read_errors() == [0] * _lib.ERRW_WORDS
    out2 = run.moe(c.w, x)
    torch.cuda.synchronize()
    run.raise_on_device_error()
    assert torch.equal(out2.view(torch.int16), ref.view(torch.int16)), "launch after clear_errors"
    assert bool((run.region("router_parts_polled") == 0xFF).all()), "polled part sums left unset"


@pytest.mark.parametrize(
    "workload,rows,stage,wg",
    [
        ("cfg2_tp4_fp8", 8, 4, 5),  # the gate_up hand-off (C)
        ("cfg2_tp4_fp8", 24, 3, 17),  # the routing hand-off (above 8 rows)
        ("cfg3_tp4_mxfp4", 16, 6, 200),  # stage Q's hand-off
        ("cfg3_tp4_mxfp4", 1, 2, 0),  # the polled router part sums and the x codes
        ("cfg3_tp4_mxfp4", 1, 3, 10),  # the published routing (a workgroup of the early shared gate_up)
        ("cfg2_tp4_fp8", 4, 3, 200),  # the shared intermediate, before the shared down
        ("cfg5_tp2_mxfp4_norm", 24, 1, 255),  # the RMSNorm's hand-off (above 16 rows: below, none)
    ],
)
def test_fault_injection_stalls_one_wait(workload, rows, stage, wg):
    """A wait stalled by the test fault injection (one workgroup, one stage: the reference's
    SGLANG_AMD_MONO_FAULT_INJECT, common/guard.py:69-89) runs to its deadline: the error words
    name that wait (its stage and workgroup, the fault word set; the waits it holds up may reach
    their deadlines first), the launch ends, and clear_errors restores a launch bit-identical to
    a fresh workspace's."""
    from test_gpu_parity import _case, _runner

    from sgl_amd_mono.moe import _lib

    c = _case(workload, rows)
    x = c.x[:rows].contiguous()
    ref_run = _runner(c)
    ref = ref_run.moe(c.w, x).clone()
    torch.cuda.synchronize()
    ref_run.raise_on_device_error()
    assert ref_run.read_errors() == [0] * _lib.ERRW_WORDS

    print(f"\n{workload} R={rows}: workgroup {wg}'s wait at stage {stage} stalled (deadline 1 ms)", flush=True)
    run = _runner(c, deadline_s=1e-3)
    run.moe(c.w, x, fault=(stage, wg))
    torch.cuda.synchronize()
    e = run.read_errors()
    print(f"  error words {e}", flush=True)
    assert e[_lib.ERRW_CODE] == 1, e  # MKMOE_DEVERR_DEADLINE
    assert e[_lib.ERRW_FAULT] == 1, e
    assert (e[_lib.ERRW_STAGE], e[_lib.ERRW_BLOCK]) == (stage, wg), e
    assert e[_lib.ERRW_COUNT] >= 1, e

    run.deadline_s = 2.0
    run.clear_errors()
    assert run.read_errors() == [0] * _lib.ERRW_WORDS
    out2 = run.moe(c.w, x)
    torch.cuda.synchronize()
    run.raise_on_device_error()
    assert torch.equal(out2.view(torch.int16), ref.view(torch.int16)), "launch after clear_errors"
