"""The fixed-order routing (``oracle.routing.route``, the kernel's order) against the golden's
own routing (``oracle.moe.routing_golden``: an fp32 matmul of unspecified order and torch's
score, check_ffn.py:201-206), on every benchmark workload's seeded inputs.

The reference makes the same cross-check between its kernel and the golden
(check_ffn.py:321-322,339-341). The fixed-order logits are first held to their own order's
error bound against the fp64 dot: each lane adds 8 products per 512-column chunk of a part,
the 64 lanes add as a six-level tree and the parts add in turn, so every logit is within
(8 C / P + 6 + P) 2^-24 sum |x_i w_i| of it (C chunks, P parts). The two routings may then
disagree only where two choices lie within the two routings' measured logit errors of each
other (evaluated through the score): such a row is allowed and counted; any other disagreement
fails (a transposed router operand, a part summed twice, a wrong score or a wrong tie rule would).
"""

import math

import numpy as np
import pytest
import torch

from oracle import gen
from oracle import moe as om
from oracle import routing as rt
from sgl_amd_mono.moe.presets import workload_dict

CASES = [("cfg1_plumbing_fp8", 4), ("plumbing_fp8_softplus", 24)] + [
    (w, r) for w in ("cfg2_tp4_fp8", "cfg3_tp4_mxfp4", "cfg5_tp2_mxfp4_norm") for r in (1, 8, 48)
] + [("cfg4_tp4_mxfp4_zipf", 48)]


def _score64(z: np.ndarray, scoring: str) -> np.ndarray:
    z = np.asarray(z, np.float64)
    if scoring == "sqrt_softplus":
        return np.sqrt(np.where(z > 20, z, np.log1p(np.exp(np.minimum(z, 20)))))
    return 1.0 / (1.0 + np.exp(-z))


def _exact_logits(xin, gate_w):
    xd, wd = xin.double(), gate_w.double()
    return (xd @ wd.T).numpy(), (xd.abs() @ wd.abs().T).numpy()


def _choice_bounds(exact, delta, bias, p):
    """[lo, hi] of every (row, expert) choice over the logits within ``delta`` of the exact ones
    (the score is increasing), widened by the fp32 rounding of the score and of score + bias."""
    sc = p.get("scoring", "sigmoid")
    b = bias.double().numpy()[None, :]
    lo = _score64(exact - delta, sc) + b
    hi = _score64(exact + delta, sc) + b
    pad = 2.0**-22 * np.maximum(np.abs(lo), np.abs(hi))
    return lo - pad, hi + pad


def _ambiguous(a: int, c: int, lo: np.ndarray, hi: np.ndarray) -> bool:
    return lo[a] <= hi[c] and lo[c] <= hi[a]


@pytest.mark.parametrize("workload,rows", CASES)
def test_routing_matches_golden(workload, rows):
    p = workload_dict(workload)
    x = gen.make_x(p, rows, 0)
    d = gen.make_dense(p, 0)
    xin = rt.rmsnorm_exact(x, d["norm"], p["norm_eps"]) if p["norm_eps"] is not None else x
    _, ids, wts = rt.route(xin, d["gate_w"], d["bias"], p)
    gids, gwts, _ = om.routing_golden(xin, d["gate_w"], d["bias"], p)
    fixed = rt.router_logits(xin, d["gate_w"], p["router_parts"]).astype(np.float64)
    golden = om.routing_golden(xin, d["gate_w"], d["bias"], p)[2].astype(np.float64)
    exact, absdot = _exact_logits(xin, d["gate_w"])
    chunks = p["hidden"] // 512
    order_bound = (8 * chunks // p["router_parts"] + 6 + p["router_parts"]) * 2.0**-24 * absdot
    assert np.all(np.abs(fixed - exact) <= order_bound), "fixed-order logits past their order's bound"
    delta = np.abs(fixed - exact) + np.abs(golden - exact)
    lo, hi = _choice_bounds(exact, delta, d["bias"], p)
    differ = 0
    for r in range(rows):
        if ids[r].tolist() == gids[r].tolist():
            # the same picks: the weights differ only by the logits' rounding
            rel = np.abs(wts[r] - gwts[r]) / np.abs(gwts[r])
            assert float(rel.max()) <= 1e-4, (r, rel.max())
            continue
        differ += 1
        for a, c in zip(ids[r].tolist(), gids[r].tolist()):
            if a != c:
                assert _ambiguous(a, c, lo[r], hi[r]), (r, a, c, lo[r][[a, c]], hi[r][[a, c]])
    print(f"{workload} R={rows}: {differ} of {rows} rows route differently (within the bound)")
    assert differ <= max(1, rows // 10)  # the reference's own tolerance is 10 % (check_ffn.py:341)


def test_a_transposed_router_fails():
    """A plausible mistake planted in the oracle (the router's operand read transposed within
    its 512-column chunks) is caught: its logits leave the order's bound and its ids differ."""
    p = workload_dict("cfg2_tp4_fp8")
    x = gen.make_x(p, 8, 0)
    d = gen.make_dense(p, 0)
    g = d["gate_w"].reshape(p["experts"], -1, 64, 8).transpose(2, 3).reshape(p["experts"], -1)
    _, ids, _ = rt.route(x, g, d["bias"], p)
    gids, _, _ = om.routing_golden(x, d["gate_w"], d["bias"], p)
    assert not np.array_equal(ids, gids)
    exact, absdot = _exact_logits(x, d["gate_w"])
    bad = rt.router_logits(x, g, p["router_parts"]).astype(np.float64)
    assert np.any(np.abs(bad - exact) > (8 * 14 // 7 + 6 + 7) * 2.0**-24 * absdot)


def test_ambiguity_bound_is_tight_enough():
    """The bound leaves real choices apart: on the cfg2 seeds no two of a row's top-9 choices
    are within it, so an accidental pass of _ambiguous is not how the test above passes."""
    p = workload_dict("cfg2_tp4_fp8")
    x = gen.make_x(p, 8, 0)
    d = gen.make_dense(p, 0)
    exact, _ = _exact_logits(x, d["gate_w"])
    fixed = rt.router_logits(x, d["gate_w"], p["router_parts"]).astype(np.float64)
    golden = om.routing_golden(x, d["gate_w"], d["bias"], p)[2].astype(np.float64)
    lo, hi = _choice_bounds(exact, np.abs(fixed - exact) + np.abs(golden - exact), d["bias"], p)
    mid = (lo + hi) / 2
    for r in range(8):
        top = np.argsort(-mid[r])[:9]
        for i in range(8):
            assert not _ambiguous(int(top[i]), int(top[i + 1]), lo[r], hi[r])
    assert math.isfinite(float(hi.max()))
