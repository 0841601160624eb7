"""Pins of the FFN seam's oracle (``oracle/seam.py``) against exact arithmetic, the reference
test's own fp64 residual, and the Sinkhorn gate's closed forms and invariants (CPU)."""

from __future__ import annotations

import math
import random
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import gen
from oracle import routing as rt
from oracle import seam as sm

F32 = np.float32
H = 5120


def _frac_round_f32(q: Fraction) -> np.float32:
    """Round an exact rational to the nearest fp32 (ties to even), by bisection on the fp32 grid."""
    lo = np.float32(float(q))  # within a few fp32 ulps
    for _ in range(4):
        if Fraction(float(lo)) > q:
            lo = np.nextafter(lo, np.float32(-np.inf))
        else:
            break
    while Fraction(float(np.nextafter(lo, np.float32(np.inf)))) <= q:
        lo = np.nextafter(lo, np.float32(np.inf))
    hi = np.nextafter(lo, np.float32(np.inf))
    dl, dh = q - Fraction(float(lo)), Fraction(float(hi)) - q
    if dl < dh:
        return lo
    if dh < dl:
        return hi
    return lo if (int(lo.view(np.uint32)) & 1) == 0 else hi


def _fma_exact(a, b, c) -> np.float32:
    return _frac_round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def test_fma32_matches_exact_rationals():
    rng = random.Random(5)
    cases = []
    for _ in range(3000):
        a = np.float32(rng.uniform(-4, 4) * 2.0 ** rng.randint(-20, 20))
        b = np.float32(rng.uniform(-4, 4) * 2.0 ** rng.randint(-20, 20))
        c = np.float32(rng.uniform(-4, 4) * 2.0 ** rng.randint(-40, 40))
        cases.append((a, b, c))
    # built to double-round: c + a b lies 2^-70 below the midpoint between 1 + 2^-23 and
    # 1 + 2^-22, so fp64 rounds it onto the midpoint and a plain cast would go up
    a0 = np.float32(2.0**-24 * (1 + 2.0**-23))
    b0 = np.float32(1 - 2.0**-23)
    c0 = np.float32(1 + 2.0**-23)
    cases += [(a0, b0, c0), (-a0, b0, -c0), (a0, -b0, np.float32(1 - 2.0**-22))]
    a, b, c = (np.array(v, F32) for v in zip(*cases))
    got = sm.fma32(a, b, c)
    want = np.array([_fma_exact(*t) for t in cases], F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert got[-3] == np.float32(1 + 2.0**-23)  # the plain fp64 -> fp32 cast gives 1 + 2^-22
    assert np.float32(float(a0) * float(b0) + float(c0)) != got[-3]


def _hc_post_fp64(i):
    """The reference test's fp64 hc_post (check_ffn.py:62-73): each element, and its largest term's |.|."""
    a = i["a"].double().numpy()
    r = i["res"].double().numpy()
    p = i["post"].double().numpy().reshape(len(a), -1)
    c = i["comb"].double().numpy()
    terms = np.concatenate(
        [(p[:, :, None] * a[:, None, :])[..., None], np.transpose(c[..., None] * r[:, :, None, :], (0, 2, 3, 1))], -1
    )
    return terms.sum(-1), np.abs(terms).max(-1)


def _bf16_ulp(x):
    return np.ldexp(1.0, np.frexp(np.abs(np.asarray(x, np.float64)))[1] - 8)


def _residual_ok(R, ref, big, share: float = 1e-4) -> bool:
    """Within half a bf16 ulp of the exact value plus the fp32 steps' error, and equal to its
    correctly rounded bf16 but for at most ``share`` of the elements (the reference's 0.01 %)."""
    err = np.abs(R.astype(np.float64) - ref)
    bound = 0.5 * _bf16_ulp(R) + 2.0**-18 * big
    rb = sm.bf16_round(ref.astype(F32))
    return bool((err <= bound).all() and (rb != R).mean() <= share)


@pytest.mark.parametrize("tokens", [1, 8, 48])
def test_residual_against_fp64_hc_post(tokens):
    i = gen.seam_inputs(tokens, H, 300 + tokens)
    R = sm.residual(i["a"].float().numpy(), i["res"].float().numpy(), i["post"].numpy(), i["comb"].numpy())
    ref, big = _hc_post_fp64(i)
    assert _residual_ok(R, ref, big)
    # a transposed comb (stream o's weight in new stream h) fails the same check
    ct = np.ascontiguousarray(np.transpose(i["comb"].numpy(), (0, 2, 1)))
    Rt = sm.residual(i["a"].float().numpy(), i["res"].float().numpy(), i["post"].numpy(), ct)
    assert not _residual_ok(Rt, ref, big)
    # so does a post applied to the wrong stream
    Rp = sm.residual(i["a"].float().numpy(), i["res"].float().numpy(), i["post"].numpy()[:, ::-1].copy(), i["comb"].numpy())
    assert not _residual_ok(Rp, ref, big)


def test_residual_last_term_is_fused():
    # v = -(1 + 2^-11) before the last term, whose product c3 r3 = 1 + 2^-11 + 2^-24 loses its
    # 2^-24 when rounded alone: fused, the column is 2^-24; rounded first, it would be 0
    a = np.zeros((1, H), F32)
    res = np.zeros((1, 4, H), F32)
    post = np.zeros((1, 4), F32)
    comb = np.zeros((1, 4, 4), F32)
    res[0, 0, 0] = 1.0
    comb[0, 0, 0] = -(1 + 2.0**-11)
    res[0, 3, 0] = 1 + 2.0**-12
    comb[0, 3, 0] = 1 + 2.0**-12
    R = sm.residual(a, res, post, comb)
    assert R[0, 0, 0] == np.float32(2.0**-24)
    assert np.float32(comb[0, 0, 0]) + np.float32(comb[0, 3, 0] * res[0, 3, 0]) == 0.0


@pytest.mark.parametrize("tokens", [1, 48])
def test_collapse_and_mix_sums_against_fp64(tokens):
    i = gen.seam_inputs(tokens, H, 400 + tokens)
    w = gen.seam_weights(H, 9)
    R = sm.residual(i["a"].float().numpy(), i["res"].float().numpy(), i["post"].numpy(), i["comb"].numpy())
    lin = sm.collapse(R, i["pre"].numpy())
    lin64 = (i["pre"].double().numpy()[:, :, None] * R.astype(np.float64)).sum(1)
    err = np.abs(lin - lin64)
    assert (err <= 0.5 * _bf16_ulp(lin) + 2.0**-20 * np.abs(R).max(1) * 4).all()
    sums = sm.mix_sums(sm.mix_partials(R, w["fn"].numpy()))
    Rf = R.reshape(tokens, -1).astype(np.float64)
    mix64 = Rf @ w["fn"].double().numpy().T
    sq64 = (Rf * Rf).sum(1)
    # fp32 sums of 20480 terms: relative to the sum of |terms|, within 2^-24 per add
    absum = np.abs(Rf) @ np.abs(w["fn"].double().numpy()).T
    assert (np.abs(sums[:, :24] - mix64) <= absum * 200 * 2.0**-24).all()
    assert (np.abs(sums[:, 24] - sq64) <= sq64 * 200 * 2.0**-24).all()
    # the slices are the right columns: each slice's partials against its own fp64 dot
    P = sm.mix_partials(R, w["fn"].numpy())
    s = 37
    cols = [o * H + 32 * s + c for o in range(4) for c in range(32)]
    ref = Rf[:, cols] @ w["fn"].double().numpy()[:, cols].T
    assert np.allclose(P[:, :24, s], ref, rtol=1e-5, atol=1e-7)


def test_gate_pre_post_against_math_exp():
    rng = np.random.default_rng(3)
    sums = np.zeros((16, 25), F32)
    sums[:, :24] = rng.normal(0, 3, (16, 24)).astype(F32)  # |z| up to about 30
    sums[:, 24] = rng.uniform(1e3, 3e4, 16).astype(F32)
    scale = np.array([0.7, 1.3, 0.9], F32)
    base = rng.normal(0, 0.1, 24).astype(F32)
    pre, post, _ = sm.gate(sums, scale, base, H)
    rstd = 1.0 / np.sqrt(sums[:, 24].astype(np.float64) / (4 * H) + 1e-20)
    v = sums[:, :24].astype(np.float64) * rstd[:, None]

    def sig(z):
        return 1.0 / (1.0 + np.exp(-z))

    # z's own fp32 roundings (v, then the fma) move sigmoid's tail by up to |z| 2^-22 relative
    zp = v[:, :4] * scale[0] + base[:4]
    zq = v[:, 4:8] * scale[1] + base[4:8]
    assert (np.abs(pre - (sig(zp) + 1e-6)) <= (sig(zp) + 1e-6) * (2e-7 + np.abs(zp) * 2.0**-22)).all()
    assert (np.abs(post - 2 * sig(zq)) <= 2 * sig(zq) * (2e-7 + np.abs(zq) * 2.0**-22)).all()


def test_sinkhorn_closed_forms_and_invariants():
    rng = np.random.default_rng(11)
    # logits a_r + b_c: exp(z) is a row scaling times a column scaling of all ones, so the
    # doubly stochastic limit is 1/4 everywhere (up to the 1e-6 added after the first row step)
    ar = rng.normal(0, 2, (8, 4, 1))
    bc = rng.normal(0, 2, (8, 1, 4))
    z = (ar + bc).astype(F32)
    cv = sm.sinkhorn(z)
    assert np.allclose(cv, 0.25, atol=5e-6)
    assert np.allclose(sm.sinkhorn(np.zeros((2, 4, 4), F32)), 0.25, atol=5e-6)
    # general logits: the columns sum to 1 (the last step), the rows nearly, and every cross
    # ratio P[r1][c1] P[r2][c2] / (P[r1][c2] P[r2][c1]) is exp(z) 's (scalings cancel)
    # (logits of spread 0.7 keep every entry above 1e-2, where the 1e-6 added after the first
    # row step moves a cross ratio by < 1e-4)
    z = rng.normal(0, 0.7, (64, 4, 4)).astype(F32)
    cv = sm.sinkhorn(z).astype(np.float64)
    assert np.allclose(cv.sum(1), 1.0, atol=3e-6)
    assert np.allclose(cv.sum(2), 1.0, atol=1e-5)
    for r1, r2, c1, c2 in [(0, 1, 0, 1), (0, 3, 2, 1), (2, 3, 3, 0), (1, 2, 0, 3)]:
        got = cv[:, r1, c1] * cv[:, r2, c2] / (cv[:, r1, c2] * cv[:, r2, c1])
        zz = z.astype(np.float64)
        want = np.exp(zz[:, r1, c1] + zz[:, r2, c2] - zz[:, r1, c2] - zz[:, r2, c1])
        assert np.allclose(got, want, rtol=2e-4), (r1, r2, c1, c2)
    # the row index is the logits' first: a transposed result breaks the cross ratios
    ct = np.transpose(cv, (0, 2, 1))
    got = ct[:, 0, 2] * ct[:, 3, 1] / (ct[:, 0, 1] * ct[:, 3, 2])
    want = np.exp(z[:, 0, 2] + z[:, 3, 1] - z[:, 0, 1] - z[:, 3, 2])
    assert not np.allclose(got, want, rtol=2e-4)


def test_gate_layout_pre_post_comb():
    # the 24 projections are pre 0..3, post 4..7, comb 8..23 row-major
    sums = np.zeros((1, 25), F32)
    sums[0, 24] = 4 * H  # rstd = 1
    base = np.zeros(24, F32)
    base[2] = 3.0
    base[5] = -2.0
    base[8 + 4 * 1 + 2] = 5.0  # comb[1][2] large
    pre, post, comb = sm.gate(sums, np.ones(3, F32), base, H)
    assert pre[0, 2] == rt.sigmoid_exact(np.float32(3.0)) + np.float32(1e-6)
    assert post[0, 1] == rt.sigmoid_exact(np.float32(-2.0)) * np.float32(2.0)
    assert np.argmax(comb[0]) == 4 * 1 + 2 and comb[0, 1, 2] > 0.8


@pytest.mark.parametrize("tokens", [1, 8])
def test_seam_norm_against_fp64(tokens):
    i = gen.seam_inputs(tokens, H, 500 + tokens)
    w = gen.seam_weights(H, 13)
    o = sm.ffn_seam(
        i["a"].float().numpy(), i["res"].float().numpy(), i["post"].numpy(), i["comb"].numpy(), i["pre"].numpy(),
        w["fn"].numpy(), w["scale"].numpy(), w["base"].numpy(), w["norm"].float().numpy(),
    )  # fmt: skip
    lin = o["lin"].astype(np.float64)
    ref = lin / np.sqrt((lin * lin).mean(1, keepdims=True) + 1e-20) * w["norm"].double().numpy()[None, :]
    assert (np.abs(o["normed"] - ref) <= _bf16_ulp(ref) * 1.0 + 1e-30).all()


def test_ffn_seam_outputs_shapes_and_determinism():
    i = gen.seam_inputs(3, H, 77)
    w = gen.seam_weights(H, 78)
    args = (
        i["a"].float().numpy(), i["res"].float().numpy(), i["post"].numpy(), i["comb"].numpy(), i["pre"].numpy(),
        w["fn"].numpy(), w["scale"].numpy(), w["base"].numpy(), w["norm"].float().numpy(),
    )  # fmt: skip
    o1, o2 = sm.ffn_seam(*args), sm.ffn_seam(*args)
    assert o1["res"].shape == (3, 4, H) and o1["normed"].shape == (3, H)
    assert o1["pre"].shape == (3, 4) and o1["post"].shape == (3, 4) and o1["comb"].shape == (3, 4, 4)
    for k in o1:
        assert np.array_equal(o1[k], o2[k])
    assert torch.isfinite(torch.from_numpy(o1["normed"])).all()
    assert math.isfinite(float(o1["comb"].sum()))
