"""Pin the golden MoE partial (``oracle/moe.py``): GEMMs against fp64, the combine order, invariants."""

import numpy as np
import pytest
import torch

from oracle import formats as fm
from oracle import gen
from oracle import moe as om
from sgl_amd_mono.moe.presets import PRESETS, workload_dict

TINY = dict(
    hidden=1024, experts=16, topk=4, n_group=4, topk_group=2, inter=256, shared_inter=256,
    routed_scale=2.5, swiglu_limit=10.0, router_parts=2, norm_eps=None, renorm=True,
)  # fmt: skip


def _inputs(p, rows, seed=0):
    x = gen.make_x(p, rows, seed)
    w = gen.make_dense(p, seed)
    ex = gen.LazyExperts(p, seed)
    return x, w, ex


@pytest.mark.parametrize("fmt", ["fp8_b128", "mxfp4"])
def test_golden_against_fp64(fmt):
    """The golden partial against an fp64 evaluation of the same quantized operands and rounding points."""
    p = dict(TINY, routed_fmt=fmt)
    x, w, ex = _inputs(p, 5, seed=1)
    res = om.moe_partial(x, w, p, experts=ex)
    ids = torch.from_numpy(res["ids"].astype(np.int64))
    wts = torch.from_numpy(res["weights"]).double()
    xr = om.act_qdq(x, fmt).double()
    lim = 10.0
    y_k = torch.zeros(5, p["topk"], p["hidden"], dtype=torch.float64)
    for r in range(5):
        for k in range(p["topk"]):
            w13, w13_s, w2, w2_s = ex.get(int(ids[r, k]))
            h = xr[r] @ om.deq_weight(w13, w13_s, fmt).double().T
            g, u = h[: p["inter"]], h[p["inter"] :]
            mid = fm.bf((torch.nn.functional.silu(g.clamp(max=lim)) * u.clamp(-lim, lim)).float()).double()
            y_k[r, k] = om.act_qdq(mid.float()[None], fmt).double()[0] @ om.deq_weight(w2, w2_s, fmt).double().T
    routed = (y_k * wts[..., None]).sum(1)
    xs = om.act_qdq(x, om.FP8_B128).double()
    hs = xs @ fm.deq_fp8_b128(w["sgu"], w["sgu_s"]).double().T
    s = p["shared_inter"]
    smid = torch.nn.functional.silu(hs[:, :s].clamp(max=lim)) * hs[:, s:].clamp(-lim, lim)
    shared = om.act_qdq(smid.float(), om.FP8_B128).double() @ fm.deq_fp8_b128(w["sw2"], w["sw2_s"]).double().T
    ref = routed + shared
    got = res["out"].double()
    rel = float((got - ref).norm() / ref.norm())
    assert rel < 2e-2, rel


def test_combine_order_two_picks():
    """bf16 at every add, in top-k order: each step rounds, unlike the fp32 sum rounded once."""
    a = torch.tensor([1.0])
    b = torch.tensor([3 * 2.0**-10])  # exact in bf16; below half a bf16 ulp of 1.0 (2^-8)
    routed = torch.zeros(1)
    for v in (a, b, b):
        routed = fm.bf(routed + fm.bf(v))
    assert float(routed) == 1.0  # each add rounds back to 1.0
    assert float(fm.bf(a + 2 * b)) == 1.0078125  # the one-shot sum crosses half an ulp


def test_zero_shared_expert_leaves_routed():
    p = dict(TINY, routed_fmt="fp8_b128")
    x, w, ex = _inputs(p, 3, seed=2)
    w0 = dict(w, sw2=torch.zeros_like(w["sw2"]))
    res = om.moe_partial(x, w0, p, experts=ex)
    routed = torch.zeros(3, p["hidden"])
    for k in range(p["topk"]):
        routed = fm.bf(routed + res["per_k"][:, k])
    assert torch.equal(res["out"].float(), routed)


def test_unpicked_experts_never_read():
    p = dict(TINY, routed_fmt="mxfp4")
    x, w, ex = _inputs(p, 2, seed=3)
    res = om.moe_partial(x, w, p, experts=ex)
    picked = set(np.unique(res["ids"]).tolist())
    assert set(ex.cache) == picked


def test_workload_dicts_match_presets():
    for name, pr in PRESETS.items():
        d = pr.as_dict()
        assert d["hidden"] % 512 == 0 and (d["hidden"] // 512) % d["router_parts"] == 0
    d = workload_dict("cfg4_tp4_mxfp4_zipf")
    assert d["zipf_s"] == 1.2 and d["routed_fmt"] == "mxfp4"


def test_zipf_routing_is_skewed():
    p = workload_dict("cfg4_tp4_mxfp4_zipf")
    x = gen.make_x(p, 48, 0)
    w = gen.make_dense(p, 0)
    from oracle import routing as rt

    _, ids, _ = rt.route(x, w["gate_w"], w["bias"], p)
    st = om.union_stats(ids)
    assert st["max_rows_per_expert"] >= 20 and st["U"] < 150, st
