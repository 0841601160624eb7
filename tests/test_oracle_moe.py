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


# ---------------------------------------------------------------- moe_partial, crafted bits
# A layer built so that every value moe_partial computes is a short dyadic number: the
# router weight is zero (every logit 0, every score sigmoid(0) = 1/2, so the bias -e / 1000
# picks experts 0, 1, 2, 3 in that order, each weighing 1/2 * 2.0 / 2.0 = 1/2); x rows are
# (448, v, t, 0, ...), whose group-128 FP8 scale is 448 / 448 = 1 exactly, so the codes are x;
# every weight and block scale is an e4m3 value or 1. A gate row holds (A, B) at K 0, 1 and
# its up row (C, 0, D) at K 0..2, so gate = 448 A + v B and up = 448 C + t D exactly; the
# intermediate is nonzero in column 0 only, its requantized code is 448 and the down row
# (1 at K 0, for output columns 0..7) gives it back: each pick contributes bf16(mid / 2), the
# shared expert its smid. The values were searched so that each plausible misplacement of a
# rounding point (test_moe_partial_crafted_catches) changes at least one row's bits.
CRAFT = dict(
    hidden=1024, experts=16, topk=4, n_group=1, topk_group=1, inter=128, shared_inter=128,
    routed_fmt="fp8_b128", routed_scale=2.0, swiglu_limit=10.0, router_parts=2, norm_eps=None,
    renorm=True, scoring="sigmoid",
)  # fmt: skip
CRAFT_ROWS = ((0.3125, 0.875), (2.25, 4.0), (0.46875, 0.6875), (0.029296875, 1.875))  # (v, t)
CRAFT_SHARED = (0.0078125, -0.8125, 0.01953125, -0.4375)  # (A, B, C, D)
CRAFT_ROUTED = (  # experts 0..3
    (-0.015625, 0.0546875, -0.017578125, -7.0),
    (0.005859375, -2.5, -0.029296875, -0.03515625),
    (0.021484375, -0.021484375, 0.02734375, 1.125),
    (0.04296875, 0.001953125, -0.05078125, -0.234375),
)
# Worked by hand, row 0 (v 0.3125, t 0.875):
#   shared: g = 448 * 2^-7 - 0.3125 * 0.8125 = 3.24609375, bf16 3.25; u = 448 * 0.01953125 -
#     0.875 * 0.4375 = 8.3671875, bf16 8.375; smid = bf16(silu(3.25) * 8.375) = bf16(26.2028) = 26.25
#   expert 0: g = -6.98291015625, u = -14 (clamps to -10): mid = bf16(silu(g) * -10) = bf16(0.064713)
#     = 0.06494140625
#   expert 1: g = 1.84375, u = -13.15576171875 (-10): mid = bf16(-15.91878) = -15.9375
#   expert 2: g = 9.6182861328125, u = 13.234375 (10): mid = bf16(96.1765) = 96
#   expert 3: g = 19.25... (10), u = -22.95... (-10): mid = bf16(-99.99546) = -100
#   contributions mid / 2 in top-k order: 0.032470703125, -7.96875, 48, -50
#   chain: 0.032470703125; bf16(-7.936279296875) = -7.9375; bf16(40.0625) = 40 (the 0.25 grid of
#     [32, 64)); bf16(40 - 50) = -10; out = bf16(-10 + 26.25) = 16.25
#   rows 1-3 likewise: 8.625, 17.5, 13. Each mistake of MISTAKES changes at least one row.
CRAFT_OUT_BITS = (0x4182, 0x410A, 0x418C, 0x4150)  # out[r, 0:8] (16.25, 8.625, 17.5, 13); 0 elsewhere


def _craft_layer():
    from oracle import formats as fm

    p = dict(CRAFT)
    h, e, i, s = p["hidden"], p["experts"], p["inter"], p["shared_inter"]
    x = torch.zeros(len(CRAFT_ROWS), h)
    x[:, 0] = 448.0
    for r, (v, t) in enumerate(CRAFT_ROWS):
        x[r, 1], x[r, 2] = v, t

    def gate_up(a, b, c, d, n):
        w = torch.zeros(2 * n, h)
        w[0, 0], w[0, 1], w[n, 0], w[n, 2] = a, b, c, d
        return fm.e4m3_codes_from_f32(w)

    down = torch.zeros(h, i)
    down[:8, 0] = 1.0
    w = {
        "gate_w": torch.zeros(e, h, dtype=torch.bfloat16),
        "bias": -torch.arange(e, dtype=torch.float32) / 1000,
        "sgu": gate_up(*CRAFT_SHARED, s),
        "sgu_s": torch.ones(2 * s // 128, h // 128),
        "sw2": fm.e4m3_codes_from_f32(down),
        "sw2_s": torch.ones(h // 128, s // 128),
    }
    w13 = torch.zeros(e, 2 * i, h, dtype=torch.uint8)
    for k, abcd in enumerate(CRAFT_ROUTED):
        w13[k] = gate_up(*abcd, i)
    w2 = fm.e4m3_codes_from_f32(down)[None].repeat(e, 1, 1)
    src = om.ExpertSource(w13, torch.ones(e, 2 * i // 128, h // 128), w2, torch.ones(e, h // 128, i // 128))
    return p, x.to(torch.bfloat16), w, src


def _craft_bits(out):
    return [int(v) & 0xFFFF for v in out.view(torch.int16)[:, 0].tolist()]


@pytest.mark.parametrize("exact", [True, False])
def test_moe_partial_crafted_bits(exact):
    """moe_partial on the crafted layer: routing, and every output element's bits, as worked
    out by hand (CRAFT_OUT_BITS): the routed SwiGLU rounds once after the product, the shared
    SwiGLU at gate, up and product, the combine adds in top-k order with bf16 at every add and
    then adds the shared output (check_ffn.py:216-232)."""
    p, x, w, src = _craft_layer()
    res = om.moe_partial(x, w, p, experts=src, exact=exact)
    assert res["ids"].tolist() == [[0, 1, 2, 3]] * len(CRAFT_ROWS)
    assert np.all(res["weights"] == np.float32(0.5))
    out = res["out"]
    assert _craft_bits(out) == list(CRAFT_OUT_BITS)
    assert torch.equal(out[:, :8], out[:, :1].expand(-1, 8)) and not out[:, 8:].float().any()
    assert res["per_k"][0, :, 0].tolist() == [0.032470703125, -7.96875, 48.0, -50.0]


def _one_shot(per_k, shared):
    routed = per_k.sum(1)
    return om.fm.bf(routed + shared).to(torch.bfloat16), routed.abs()


_COMBINE = om.combine


def _reversed(per_k, shared):
    return _COMBINE(per_k.flip(1), shared)


def _shared_first(per_k, shared):
    acc = shared.clone()
    for k in range(per_k.shape[1]):
        acc = om.fm.bf(acc + per_k[:, k])
    return acc.to(torch.bfloat16), acc.abs()


def _no_per_add_round(per_k, shared):
    routed = torch.zeros_like(shared)
    for k in range(per_k.shape[1]):
        routed = routed + per_k[:, k]
    return om.fm.bf(routed + shared).to(torch.bfloat16), routed.abs()


def _np_bf(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


MISTAKES = {
    # the combine
    "one_shot_sum": ("combine", _one_shot),
    "reversed_order": ("combine", _reversed),
    "shared_added_first": ("combine", _shared_first),
    "no_bf16_per_add": ("combine", _no_per_add_round),
    # the shared SwiGLU (exact path: oracle.exact; golden path: oracle.moe)
    "shared_as_routed_rule": ("swiglu_shared", lambda g, u, lim: _routed_rule(g, u, lim)),
    "shared_gate_not_rounded": ("swiglu_shared", lambda g, u, lim: _shared_rule(g, u, lim, gate=False)),
    "shared_up_not_rounded": ("swiglu_shared", lambda g, u, lim: _shared_rule(g, u, lim, up=False)),
    "shared_silu_rounded": ("swiglu_shared", lambda g, u, lim: _shared_rule(g, u, lim, silu_bf=True)),
    # the routed SwiGLU
    "routed_as_shared_rule": ("swiglu_routed", lambda g, u, lim: _shared_rule(g, u, lim)),
    "routed_silu_rounded": ("swiglu_routed", lambda g, u, lim: _routed_rule(g, u, lim, silu_bf=True)),
    "routed_no_clamp": ("swiglu_routed", lambda g, u, lim: _routed_rule(g, u, 1e30)),
}


def _silu_np(z):
    z = np.asarray(z, np.float32)
    return (z / (np.float32(1) + np.exp(-z.astype(np.float64)))).astype(np.float32)


def _routed_rule(g, u, lim, silu_bf=False):
    g, u = np.asarray(g, np.float32), np.asarray(u, np.float32)
    s = _silu_np(np.minimum(g, np.float32(lim)))
    s = _np_bf(s) if silu_bf else s
    return _np_bf(s * np.clip(u, -np.float32(lim), np.float32(lim)))


def _shared_rule(g, u, lim, gate=True, up=True, silu_bf=False):
    g, u = np.asarray(g, np.float32), np.asarray(u, np.float32)
    gg = np.minimum(g, np.float32(lim))
    uu = np.clip(u, -np.float32(lim), np.float32(lim))
    s = _silu_np(_np_bf(gg) if gate else gg)
    s = _np_bf(s) if silu_bf else s
    return _np_bf(s * (_np_bf(uu) if up else uu))


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("mistake", sorted(MISTAKES))
def test_moe_partial_crafted_catches(mistake, exact, monkeypatch):
    """Each plausible misplacement of a rounding point, planted in the oracle, changes the
    crafted layer's bits: the crafted case pins moe_partial's combine and both SwiGLU rules."""
    from oracle import exact as ex

    what, fn = MISTAKES[mistake]
    if what == "combine":
        monkeypatch.setattr(om, "combine", fn)
    elif exact:
        monkeypatch.setattr(ex, what, fn)
    else:
        golden = {"swiglu_shared": "swiglu_shared_golden", "swiglu_routed": "swiglu_routed_golden"}[what]
        monkeypatch.setattr(om, golden, lambda g, u, lim: torch.from_numpy(fn(g.numpy(), u.numpy(), lim)))
    p, x, w, src = _craft_layer()
    out = om.moe_partial(x, w, p, experts=src, exact=exact)["out"]
    assert _craft_bits(out) != list(CRAFT_OUT_BITS)


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


# ---------------------------------------------------------------- the V4.1 shared expert, crafted bits
# The MX shared expert (FP8 with E8M0 32 x 32 scales, its activations and intermediate by the
# MXFP8 "vllm" rule, check_ffn.py:118-121,226-231). One row x = (448, 0, ...): its vllm code is
# 127, so its codes are x. Gate row 0 and up row 128 hold 1 at K 0, with block codes 119 and
# 20: g = 448 * 2^-8 = 1.75, u = 448 * 2^-107 = 1.75 * 2^-99 (no clamp). Worked by hand:
#   silu(1.75) = 1.75 / (1 + e^-1.75) = 1.4909173 (fp32); product 1.3045527 * 2^-98, bf16
#   smid = 1.3046875 * 2^-98 (167 / 128)
#   vllm: smid / 448 = 1.491 * 2^-107, so code 21 (2^-106); smid / 2^-106 = 334, e4m3 320 (the
#   step in [256, 448) is 32); back: 320 * 2^-106 = 1.25 * 2^-98
#   down row 32 holds 1 at K 0 with block code 227 (2^100): 1.25 * 2^2 = 5.0, bf16 0x40A0 in
#   column 32; every routed weight is zero, so out[0, 32] = bf16(0 + 5.0) and 0 elsewhere.
# The "aiter" rule (floor 1e-10) and group-128 (scale max(amax, 1e-10) / 448) both flush that
# intermediate to 0; block codes 126 at sgu_s[0, 4] and 125 at sw2_s[0, 1] are where a
# transposed scale index reads, and a 128-row block index reads the default 127.
MXC_OUT_BITS = 0x40A0


def _mx_shared_layer():
    p = dict(CRAFT, shared_fmt="fp8_mx32")
    h, e, i, s = p["hidden"], p["experts"], p["inter"], p["shared_inter"]
    x = torch.zeros(1, h)
    x[0, 0] = 448.0
    sgu = torch.zeros(2 * s, h)
    sgu[0, 0] = sgu[s, 0] = 1.0
    sgu_s = torch.full((2 * s // 32, h // 32), 127, dtype=torch.uint8)
    sgu_s[0, 0], sgu_s[4, 0], sgu_s[0, 4] = 119, 20, 126
    sw2 = torch.zeros(h, s)
    sw2[32, 0] = 1.0
    sw2_s = torch.full((h // 32, s // 32), 127, dtype=torch.uint8)
    sw2_s[1, 0], sw2_s[0, 1] = 227, 125
    w = {
        "gate_w": torch.zeros(e, h, dtype=torch.bfloat16),
        "bias": -torch.arange(e, dtype=torch.float32) / 1000,
        "sgu": fm.e4m3_codes_from_f32(sgu),
        "sgu_s": sgu_s,
        "sw2": fm.e4m3_codes_from_f32(sw2),
        "sw2_s": sw2_s,
    }
    src = om.ExpertSource(
        torch.zeros(e, 2 * i, h, dtype=torch.uint8), torch.ones(e, 2 * i // 128, h // 128),
        torch.zeros(e, h, i, dtype=torch.uint8), torch.ones(e, h // 128, i // 128),
    )  # fmt: skip
    return p, x.to(torch.bfloat16), w, src


def test_mx_shared_expert_crafted_bits():
    """moe_partial's MX shared expert on the crafted layer: the hand-worked 5.0 in column 32,
    zero elsewhere."""
    p, x, w, src = _mx_shared_layer()
    out = om.moe_partial(x, w, p, experts=src, exact=False)["out"]
    assert int(out.view(torch.int16)[0, 32]) & 0xFFFF == MXC_OUT_BITS
    assert out[0].float().nonzero().flatten().tolist() == [32]


def _deq_mx32_transposed(q, s):
    """Element (i, j) scaled by block (j / 32, i / 32) (wrapped into the scale grid)."""
    n, k = q.shape
    nb, kb = s.shape
    bi = (torch.arange(n)[:, None] // 32) % kb
    bj = (torch.arange(k)[None, :] // 32) % nb
    return fm.e4m3_to_f32(q) * fm.e8m0_to_f32(s)[bj, bi]


def _deq_mx32_blocks128(q, s):
    n, k = q.shape
    sf = fm.e8m0_to_f32(s).repeat_interleave(128, 0)[:n].repeat_interleave(128, 1)[:, :k]
    return fm.e4m3_to_f32(q) * sf


_ACT_QDQ = om.act_qdq
MX_MISTAKES = {
    "aiter_rule": ("act_qdq", lambda x, fmt: _ACT_QDQ(x, om.MXFP4 if fmt == om.FP8_MX32 else fmt)),
    "group128_rule": ("act_qdq", lambda x, fmt: _ACT_QDQ(x, om.FP8_B128 if fmt == om.FP8_MX32 else fmt)),
    "scales_transposed": ("deq", _deq_mx32_transposed),
    "scales_per_128": ("deq", _deq_mx32_blocks128),
}


@pytest.mark.parametrize("mistake", sorted(MX_MISTAKES))
def test_mx_shared_expert_crafted_catches(mistake, monkeypatch):
    """Each planted mistake (the shared expert's activations by another rule, its E8M0 block
    scales indexed transposed or per 128) changes the crafted layer's bits."""
    what, fn = MX_MISTAKES[mistake]
    if what == "act_qdq":
        monkeypatch.setattr(om, "act_qdq", fn)
    else:
        monkeypatch.setattr(fm, "deq_fp8_mx32", fn)
    p, x, w, src = _mx_shared_layer()
    out = om.moe_partial(x, w, p, experts=src, exact=False)["out"]
    assert int(out.view(torch.int16)[0, 32]) & 0xFFFF != MXC_OUT_BITS


def test_deq_fp8_mx32_hand_values():
    """deq_fp8_mx32 on a [64, 96] matrix with a distinct E8M0 code per 32 x 32 block: element
    (i, j) is e4m3(q[i, j]) * 2^(code[i / 32][j / 32] - 127), worked by hand at one element per
    block (e4m3 0x38 = 1.0, 0x3C = 1.5, 0xC4 = -3.0)."""
    q = torch.zeros(64, 96, dtype=torch.uint8)
    s = torch.tensor([[120, 127, 130], [126, 140, 100]], dtype=torch.uint8)
    q[0, 0], q[5, 40], q[31, 95], q[32, 0], q[40, 63], q[63, 64] = 0x38, 0x3C, 0xC4, 0x38, 0x3C, 0xC4
    d = fm.deq_fp8_mx32(q, s)
    want = {(0, 0): 2.0**-7, (5, 40): 1.5, (31, 95): -24.0, (32, 0): 0.5, (40, 63): 1.5 * 2.0**13,
            (63, 64): -3.0 * 2.0**-27}  # fmt: skip
    for (i, j), v in want.items():
        assert float(d[i, j]) == v, (i, j, float(d[i, j]), v)
    assert int((d != 0).sum()) == len(want)
