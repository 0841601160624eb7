"""The entry point that allocates nothing (mkmoe_forward_static) against mkmoe_forward.

It runs the same kernel on the same arithmetic, with the workspace in the library's static
device array instead of a caller's allocation, so its outputs and routing must equal
mkmoe_forward's bit for bit: two calls in a row on the static array, the second with fewer
rows (the array keeps the first call's contents), each against mkmoe_forward on the same
inputs. Through the C ABI (ctypes), on an MI355X.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _static(run, w, x, opts=None):
    from sgl_amd_mono.moe import _lib

    rows = x.shape[0]
    p = run.preset
    out = torch.empty(rows, p.hidden, dtype=torch.bfloat16, device="cuda")
    ids = torch.empty(rows, p.topk, dtype=torch.int32, device="cuda")
    wts = torch.empty(rows, p.topk, dtype=torch.float32, device="cuda")
    ws_ = w.c_struct()
    rc = _lib.lib().mkmoe_forward_static(
        ctypes.byref(run.shape), ctypes.byref(ws_), x.data_ptr(), rows, out.data_ptr(), ids.data_ptr(),
        wts.data_ptr(), None if opts is None else ctypes.byref(opts), torch.cuda.current_stream().cuda_stream,
    )  # fmt: skip
    _lib.check(rc, "mkmoe_forward_static")
    return out, ids, wts


@pytest.mark.parametrize("workload,rows,rows2", [("cfg2_tp4_fp8", 24, 8), ("cfg3_tp4_mxfp4", 8, 1)])
def test_static_workspace_equals_forward(workload, rows, rows2):
    import sys
    from pathlib import Path

    sys.path.insert(0, str(Path(__file__).resolve().parent))
    from gpu_case import build

    from sgl_amd_mono.moe.runner import MoeRunner

    c = build(workload, rows)
    run = MoeRunner(c.preset, "cuda")
    for r in (rows, rows2):
        print(f"\n{workload}: mkmoe_forward_static, {r} rows", flush=True)
        x = c.x[:r].contiguous()
        ids = torch.empty(r, c.p["topk"], dtype=torch.int32, device="cuda")
        wts = torch.empty(r, c.p["topk"], dtype=torch.float32, device="cuda")
        want = run.moe(c.w, x, topk_ids=ids, topk_w=wts)
        got, gids, gwts = _static(run, c.w, x)
        torch.cuda.synchronize()
        run.raise_on_device_error()
        assert torch.equal(gids, ids), "expert ids"
        assert torch.equal(gwts.view(torch.int32), wts.view(torch.int32)), "routing weights"
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), "output"


def test_static_workspace_refuses_before_any_launch():
    """A call beyond the compiled limits (here more rows than any shape takes) is refused with a
    status code and enqueues nothing; every compiled shape's layout fits the array (a CPU test
    checks the sizes), so the array's own size limit is checked before the launch as well."""
    from sgl_amd_mono.moe import _lib

    from sgl_amd_mono.moe.presets import PRESETS

    shape = _lib.shape_of(PRESETS["dsv3_tp2_mxfp4_norm"], 48)
    shape.max_rows = 49  # beyond the largest compiled row count: refused as rows, before the array
    x = torch.zeros(1, 7168, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros(1, 7168, dtype=torch.bfloat16, device="cuda")
    w = _lib.Weights(*([x.data_ptr()] * 11))
    rc = _lib.lib().mkmoe_forward_static(ctypes.byref(shape), ctypes.byref(w), x.data_ptr(), 1, out.data_ptr(),
                                         None, None, None, torch.cuda.current_stream().cuda_stream)
    assert rc == -3  # MKMOE_ERR_ROWS
