"""Pin the oracle's exact GEMV order (``oracle/exact.py``): fp64 closeness and a scalar restatement."""

import numpy as np
import pytest
import torch

from oracle import exact as ex
from oracle import formats as fm
from oracle import gen
from oracle import moe as om


def _fp8_case(n, k, t, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=g) * 0.02
    x = torch.randn(t, k, generator=g)
    wq, ws = fm.quant_fp8_b128(w)
    xq, xs = fm.group_fp8_quant(x, 128)
    return wq, ws, xq, xs


def _fp4_case(n, k, t, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=g) * 0.02
    x = torch.randn(t, k, generator=g)
    wq, ws = fm.quant_mxfp4(w)
    xq, xs = fm.mxfp8_quant(x)
    return wq, ws, xq, xs


@pytest.mark.parametrize("k", [512, 1024, 7168])
def test_fp8_gemv_close_to_fp64(k):
    wq, ws, xq, xs = _fp8_case(256, k, 3, k)
    got = ex.gemv_fp8_b128(wq, ws, xq, xs)
    ref = fm.group_fp8_dequant(xq, xs).double() @ fm.deq_fp8_b128(wq, ws).double().T
    err = np.abs(got - ref.numpy()).max() / np.abs(ref.numpy()).max()
    assert err < 1e-5, err


@pytest.mark.parametrize("k", [512, 1024, 7168])
def test_fp4_gemv_close_to_fp64(k):
    wq, ws, xq, xs = _fp4_case(128, k, 3, k)
    got = ex.gemv_mxfp4(wq, ws, xq, xs)
    ref = fm.mxfp8_dequant(xq, xs).double() @ fm.deq_mxfp4(wq, ws).double().T
    err = np.abs(got - ref.numpy()).max() / np.abs(ref.numpy()).max()
    assert err < 1e-5, err


def _scalar_gemv(wv, xv, scale, ce, lpr=None):
    """Index by index: chunk sums in element order, scaled, chunk c to lane c % LPR, lane sums, tree."""
    f = np.float32
    n, k = wv.shape
    c_n = k // ce
    if lpr is None:
        lpr = 64 if c_n % 64 == 0 else 32 if c_n % 32 == 0 else 16 if c_n % 16 == 0 else 8
    out = np.zeros((xv.shape[0], n), np.float32)
    for t in range(xv.shape[0]):
        for r in range(n):
            lanes = [f(0)] * lpr
            for c in range(c_n):
                d = f(0)
                for i in range(ce):
                    d = f(d + f(xv[t, c * ce + i] * wv[r, c * ce + i]))
                lanes[c % lpr] = f(lanes[c % lpr] + scale(t, r, c, d))
            while len(lanes) > 1:
                h = len(lanes) // 2
                lanes = [f(lanes[i] + lanes[i + h]) for i in range(h)]
            out[t, r] = lanes[0]
    return out


@pytest.mark.parametrize("lpr", [None, 8])
def test_fp8_gemv_scalar_restatement(lpr):
    wq, ws, xq, xs = _fp8_case(3, 512, 2, 11)
    wv = fm.e4m3_to_f32(wq).numpy()
    xv = fm.e4m3_to_f32(xq).numpy()
    wsn, xsn = ws.numpy(), xs.numpy()
    f = np.float32

    def scale(t, r, c, d):
        return f(d * f(wsn[r // 128, c // 8] * xsn[t, c // 8]))

    want = _scalar_gemv(wv, xv, scale, 16, lpr)
    got = ex.gemv_fp8_b128(wq, ws, xq, xs, lpr)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("lpr", [None, 8])
def test_fp4_gemv_scalar_restatement(lpr):
    wq, ws, xq, xs = _fp4_case(3, 1024, 2, 12)
    wv = fm.fp4_unpack(wq).numpy()
    xv = fm.e4m3_to_f32(xq).numpy()
    wsn, xsn = ws.numpy().astype(np.int32), xs.numpy().astype(np.int32)

    def scale(t, r, c, d):
        return np.float32(np.ldexp(d, wsn[r, c] + xsn[t, c] - 254))

    want = _scalar_gemv(wv, xv, scale, 32, lpr)
    got = ex.gemv_mxfp4(wq, ws, xq, xs, lpr)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_lanes_per_row_matches_kernel_rule():
    # the kernel's gate_up rows: 64 lanes when the chunks divide by 64, else 32, 16, 8
    assert ex.lanes_per_row(7168 // 16) == 64  # FP8 gate_up rows
    assert ex.lanes_per_row(7168 // 32) == 32  # MXFP4 gate_up rows
    assert ex.lanes_per_row(1024 // 32) == 32
    # the down rows: 8 lanes a row, whatever the width
    assert ex.DOWN_LANES == 8


def test_lane_count_changes_the_sum():
    # the restatement is sensitive to the lane count it is given: a kernel that dealt its
    # down chunks to 16 or 32 lanes would not match the oracle's 8
    wq, ws, xq, xs = _fp8_case(64, 512, 4, 13)
    a = ex.gemv_fp8_b128(wq, ws, xq, xs, 8)
    for other in (16, 32):
        b = ex.gemv_fp8_b128(wq, ws, xq, xs, other)
        assert not np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_silu_exact_close_to_torch():
    z = np.linspace(-12, 12, 10001).astype(np.float32)
    got = ex.silu_exact(z)
    ref = torch.nn.functional.silu(torch.from_numpy(z).double()).numpy()
    assert np.abs(got - ref).max() <= 4e-7 * np.abs(ref).max()


@pytest.mark.parametrize("fmt", ["fp8_b128", "mxfp4"])
def test_exact_and_golden_order_agree(fmt):
    p = dict(
        hidden=1024, experts=16, topk=4, n_group=4, topk_group=2, inter=256, shared_inter=256,
        routed_scale=2.5, swiglu_limit=10.0, router_parts=2, norm_eps=None, renorm=True, routed_fmt=fmt,
    )  # fmt: skip
    x = gen.make_x(p, 6, 5)
    w = gen.make_dense(p, 5)
    exs = gen.LazyExperts(p, 5)
    a = om.moe_partial(x, w, p, experts=exs, exact=True)["out"].float()
    b = om.moe_partial(x, w, p, experts=exs, exact=False)["out"].float()
    assert float((a - b).norm() / b.norm()) < 1e-2
