"""Pin the oracle's routing (``oracle/routing.py``) and the kernel's host-built sigmoid and top-k.

Pins: fixed-order logits against an fp64 matmul and an index-by-index scalar
restatement; the fp64 sigmoid against math.exp and the C build of the
kernel's steps (bit for bit); the grouped top-k against exhaustive search of
group and expert subsets at E = 16, its invariants, and the C build (bit for
bit, ties included); the fixed-order RMSNorm against an fp64 RMSNorm.
"""

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import routing as rt


def test_router_logits_close_to_fp64():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 7168, generator=g).to(torch.bfloat16)
    w = (torch.randn(16, 7168, generator=g) / math.sqrt(7168)).to(torch.bfloat16)
    got = rt.router_logits(x, w, 7)
    ref = x.double() @ w.double().T
    assert np.abs(got - ref.numpy()).max() < 2e-5


def test_router_logits_scalar_restatement():
    """Index by index: lane l of chunk c holds elements 512 c + 8 l + j; parts of C / P chunks."""
    g = torch.Generator().manual_seed(1)
    h, parts = 1024, 2
    x = torch.randn(2, h, generator=g).to(torch.bfloat16)
    w = torch.randn(3, h, generator=g).to(torch.bfloat16)
    got = rt.router_logits(x, w, parts)
    xs, ws = x.float().numpy(), w.float().numpy()
    f = np.float32
    per = (h // 512) // parts
    for r in range(2):
        for e in range(3):
            logit = f(0)
            for p in range(parts):
                lanes = []
                for lane in range(64):
                    a = f(0)
                    for c in range(p * per, (p + 1) * per):
                        for j in range(8):
                            k = 512 * c + 8 * lane + j
                            a = f(a + f(xs[r, k] * ws[e, k]))
                    lanes.append(a)
                d = 32
                while d >= 1:
                    lanes = [f(lanes[i] + lanes[i + d]) for i in range(d)]
                    d //= 2
                logit = f(logit + lanes[0])
            assert got[r, e] == logit


def test_sigmoid_exact_accuracy():
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(20000) * 4, np.linspace(-70, 70, 2001)]).astype(np.float32)
    got = rt.sigmoid_exact(x)
    xc = np.clip(x.astype(np.float64), -60, 60)
    ref = np.array([1 / (1 + math.exp(-v)) for v in xc])
    # within half an fp32 ulp of the true value, plus fp64 slack
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= 0.5 * ulp + 1e-15)
    assert np.mean(got == ref.astype(np.float32)) > 0.9999


def test_host_sigmoid_bitexact():
    from sgl_amd_mono.moe import _lib

    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(100000) * 3, rng.uniform(-80, 80, 20000),
                        [0.0, -0.0, 60.0, -60.0, 1e-30, -1e-30]]).astype(np.float32)  # fmt: skip
    out = np.zeros_like(x)
    _lib.testing_lib().mkmoe_host_sigmoid(x.ctypes.data, out.ctypes.data, x.size)
    assert np.array_equal(out.view(np.uint32), rt.sigmoid_exact(x).view(np.uint32))


def _brute_topk(choice, scores, k, n_group, topk_group, scale):
    """Exhaustive: the group subset with the largest scores in (score desc, index asc) order,
    then the expert subset likewise, then the weights."""
    e = len(choice)
    per = e // n_group
    gs = []
    for g in range(n_group):
        top = sorted(choice[g * per : (g + 1) * per], reverse=True)
        gs.append(np.float32(top[0] + top[1]) if per > 1 else np.float32(top[0]))

    def rank_key(vals, idxs):
        return sorted(((-float(vals[i]), i) for i in idxs))

    best_groups = None
    for sub in itertools.combinations(range(n_group), topk_group):
        key = rank_key(gs, sub)
        # a subset is the top set iff every outside group ranks below every member
        outside = [g for g in range(n_group) if g not in sub]
        if all((-float(gs[o]), o) > key[-1] for o in outside):
            best_groups = sub
    allowed = [x for g in best_groups for x in range(g * per, (g + 1) * per)]
    order = [i for _, i in rank_key(choice, allowed)][:k]
    w = scores[order]
    total = np.float32(0)
    for v in w:
        total = np.float32(total + v)
    f = np.float32(np.float32(scale) / total)
    return np.array(order), (w * f).astype(np.float32)


@pytest.mark.parametrize("seed", range(20))
def test_grouped_topk_exhaustive(seed):
    rng = np.random.default_rng(seed)
    e, k, ng, tg = 16, 4, 4, 2
    scores = rt.sigmoid_exact(rng.standard_normal((1, e)).astype(np.float32))
    bias = (rng.standard_normal(e) * 0.02).astype(np.float32)
    if seed % 3 == 0:  # plant ties
        scores[0, 5] = scores[0, 9]
        bias[5] = bias[9]
    ids, wts = rt.grouped_topk(scores, bias, k, ng, tg, 2.5)
    choice = (scores[0] + bias).astype(np.float32)
    bid, bw = _brute_topk(choice, scores[0], k, ng, tg, 2.5)
    assert ids[0].tolist() == bid.tolist()
    assert np.array_equal(wts[0].view(np.uint32), bw.view(np.uint32))


def test_grouped_topk_invariants():
    rng = np.random.default_rng(7)
    scores = rt.sigmoid_exact(rng.standard_normal((64, 256)).astype(np.float32))
    bias = (rng.standard_normal(256) * 0.02).astype(np.float32)
    ids, wts = rt.grouped_topk(scores, bias, 8, 8, 4, 2.5)
    choice = scores + bias
    for r in range(64):
        assert len(set(ids[r].tolist())) == 8
        assert len({int(i) // 32 for i in ids[r]}) <= 4
        c = choice[r, ids[r]]
        assert np.all(c[:-1] >= c[1:])
        assert abs(float(wts[r].sum()) - 2.5) < 1e-5


def _host_topk(preset, scores, bias):
    from sgl_amd_mono.moe import _lib

    shape = _lib.shape_of(preset)
    ids = np.zeros(preset.topk, np.int32)
    w = np.zeros(preset.topk, np.float32)
    _lib.testing_lib().mkmoe_host_topk(
        __import__("ctypes").byref(shape), scores.ctypes.data, bias.ctypes.data, ids.ctypes.data, w.ctypes.data
    )
    return ids, w


@pytest.mark.parametrize("name", ["plumbing_fp8", "dsv3_tp4_fp8"])
def test_host_topk_bitexact(name):
    from sgl_amd_mono.moe.presets import PRESETS

    p = PRESETS[name]
    rng = np.random.default_rng(11)
    bias = np.ascontiguousarray((rng.standard_normal(p.experts) * 0.02).astype(np.float32))
    for t in range(200):
        scores = rt.sigmoid_exact(rng.standard_normal((1, p.experts)).astype(np.float32))
        if t % 4 == 0:  # ties across groups and within
            scores[0, : p.experts // 2] = scores[0, p.experts // 2 :]
        if t % 4 == 1:
            scores[0, :] = scores[0, 0]
        scores = np.ascontiguousarray(scores[0])
        ids, w = _host_topk(p, scores, bias)
        rid, rw = rt.grouped_topk(scores[None], bias, p.topk, p.n_group, p.topk_group, p.routed_scale)
        assert ids.tolist() == rid[0].tolist()
        assert np.array_equal(w.view(np.uint32), rw[0].view(np.uint32))


@pytest.mark.parametrize("seed", range(8))
def test_grouped_topk_nan_scores(seed):
    """A NaN score's choice is -inf and it weighs 0 (stages/moe.py:345-347): the oracle against
    brute force on the substituted choices, and the host build of the kernel's top-k."""
    from sgl_amd_mono.moe.presets import PRESETS

    rng = np.random.default_rng(100 + seed)
    e, k, ng, tg = 16, 4, 4, 2
    scores = rt.sigmoid_exact(rng.standard_normal((1, e)).astype(np.float32))
    bias = (rng.standard_normal(e) * 0.02).astype(np.float32)
    nan_at = rng.choice(e, size=1 + seed % 5, replace=False)
    scores[0, nan_at] = np.nan
    ids, wts = rt.grouped_topk(scores, bias, k, ng, tg, 2.5)
    choice = np.where(np.isnan(scores[0]), -np.inf, scores[0] + bias).astype(np.float32)
    bid, bw = _brute_topk(choice, np.nan_to_num(scores[0], nan=0.0), k, ng, tg, 2.5)
    assert ids[0].tolist() == bid.tolist()
    assert np.array_equal(wts[0].view(np.uint32), bw.view(np.uint32))
    assert not set(ids[0].tolist()) & set(nan_at.tolist())  # finite choices always win here
    # the kernel's host build, at 256 experts in 8 groups (NaN spread over several groups)
    p = PRESETS["dsv3_tp4_fp8"]
    sc = rt.sigmoid_exact(rng.standard_normal((1, p.experts)).astype(np.float32))[0]
    sc[rng.choice(p.experts, size=40, replace=False)] = np.nan
    bb = np.ascontiguousarray((rng.standard_normal(p.experts) * 0.02).astype(np.float32))
    sc = np.ascontiguousarray(sc)
    hid, hw = _host_topk(p, sc, bb)
    rid, rw = rt.grouped_topk(sc[None], bb, p.topk, p.n_group, p.topk_group, p.routed_scale)
    assert hid.tolist() == rid[0].tolist()
    assert np.array_equal(hw.view(np.uint32), rw[0].view(np.uint32))


def test_grouped_topk_all_nan_row():
    """Known answer: every score NaN -> every choice -inf, so groups and experts go by lower
    index (the first topk experts of group 0), and every weight is 0."""
    scores = np.full((1, 256), np.nan, np.float32)
    bias = np.zeros(256, np.float32)
    ids, wts = rt.grouped_topk(scores, bias, 8, 8, 4, 2.5)
    assert ids[0].tolist() == list(range(8))
    assert np.all(wts == 0)


def test_unset_part_sums_route_in_bounds():
    """A routing that gives up waiting reads the unset marker (0xFFFFFFFF, a NaN) as part sums:
    the kernel's host build maps it to a NaN score, and its top-k then returns in-range ids
    (0 .. topk-1 in the first groups) with weight 0, so nothing derived from them leaves a
    buffer."""
    from sgl_amd_mono.moe import _lib
    from sgl_amd_mono.moe.presets import PRESETS

    L = _lib.testing_lib()
    unset = np.full(4, 0xFFFFFFFF, np.uint32).view(np.float32)
    logit = np.zeros(4, np.float32)
    for _ in range(7):  # the parts added in order, as the kernel does
        logit = (logit + unset).astype(np.float32)
    sc = np.zeros(4, np.float32)
    L.mkmoe_host_sigmoid(logit.ctypes.data, sc.ctypes.data, 4)
    assert np.all(np.isnan(sc))
    for name in ("plumbing_fp8", "dsv3_tp4_fp8"):
        p = PRESETS[name]
        scores = np.full(p.experts, np.nan, np.float32)
        bias = np.ascontiguousarray((np.arange(p.experts) % 5).astype(np.float32) * np.float32(0.01))
        ids, w = _host_topk(p, scores, bias)
        assert ids.tolist() == list(range(p.topk)), ids
        assert np.all((ids >= 0) & (ids < p.experts)) and np.all(w == 0)


def test_rmsnorm_close_to_fp64():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(4, 7168, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(7168, generator=g)).to(torch.bfloat16)
    got = rt.rmsnorm_exact(x, w, 1e-6).float()
    xd = x.double()
    ref = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6) * w.double()
    ulp = torch.ldexp(torch.ones_like(ref), torch.frexp(ref.abs())[1] - 8)
    assert float(((got.double() - ref).abs() / ulp).max()) <= 1.0


def test_part_sums_never_take_the_unset_marker():
    """The polled copy of the router's part sums marks an unwritten word with 0xFFFFFFFF.
    No part sum takes that bit pattern: inputs with bf16 NaNs of every payload, infinities
    of both signs (inf - inf and 0 * inf generate NaNs) and ordinary values."""
    rng = np.random.default_rng(11)
    h, e, r, parts = 1024, 16, 6, 2
    x = torch.from_numpy(rng.standard_normal((r, h)).astype(np.float32)).to(torch.bfloat16)
    w = torch.from_numpy(rng.standard_normal((e, h)).astype(np.float32)).to(torch.bfloat16)
    xb, wb = x.view(torch.int16), w.view(torch.int16)
    specials = [0x7FFF, -1, 0x7FC1, -64, 0x7F80, -128, 0]  # NaNs (payloads), +inf, -inf, 0
    for i, v in enumerate(specials):
        xb[i % r, (37 * i) % h] = v
        wb[i % e, (37 * i + 5) % h] = v
    xb[r - 1, 0], wb[0, 0] = 0x7F80, 0  # 0 * inf
    xb[r - 1, 1], wb[1, 1] = 0x7F80, 0x3F80  # +inf ...
    xb[r - 1, 9], wb[1, 9] = -128, 0x3F80  # ... and -inf in one sum
    ps = rt.router_part_sums(x, w, parts)
    assert np.isnan(ps).any() and not (ps.view(np.uint32) == 0xFFFFFFFF).any()


def test_sqrt_softplus_against_math():
    """V4.1's score: softplus rounded to fp32, then the fp32 square root (the golden's
    ``F.softplus(logits).sqrt()``, check_ffn.py:203), against math.log1p / math.exp: equal to
    those two roundings of the true values but for a rare last-place tie, and never more than
    one fp32 ulp off."""
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(20000) * 6, np.linspace(-120, 40, 4001)]).astype(np.float32)
    got = rt.sqrt_softplus_exact(x)
    sp = np.array([v if v > 20 else math.log1p(math.exp(v)) for v in x.astype(np.float64)], np.float64)
    ref = np.sqrt(sp.astype(np.float32)).astype(np.float32)
    ulp = np.spacing(ref)
    assert np.all(np.abs(got.astype(np.float64) - ref.astype(np.float64)) <= ulp)
    assert np.mean(got == ref) > 0.9999


def test_sqrt_softplus_closed_forms():
    x = np.array([20.5, 33.0, 1e6, 0.0, -0.0, np.nan, -1000.0], np.float32)
    got = rt.sqrt_softplus_exact(x)
    assert np.array_equal(got[:3], np.sqrt(x[:3]))  # softplus(x) = x past 20
    assert got[3] == got[4] == np.sqrt(np.float32(math.log(2.0)))
    assert np.isnan(got[5]) and got[6] == 0.0
    # log1p against math.log1p over [0, 1]
    t = np.linspace(0.0, 1.0, 10001)
    ref = np.array([math.log1p(v) for v in t])
    assert np.max(np.abs(rt.log1p_01(t) - ref) / np.maximum(ref, 1e-300)) < 1e-15


def test_host_sqrt_softplus_bitexact():
    from sgl_amd_mono.moe import _lib

    rng = np.random.default_rng(6)
    x = np.concatenate([rng.standard_normal(100000) * 8, rng.uniform(-250, 60, 20000),
                        [0.0, -0.0, 20.0, 20.000002, -200.0, -1e-30]]).astype(np.float32)  # fmt: skip
    out = np.zeros_like(x)
    _lib.testing_lib().mkmoe_host_sqrt_softplus(x.ctypes.data, out.ctypes.data, x.size)
    assert np.array_equal(out.view(np.uint32), rt.sqrt_softplus_exact(x).view(np.uint32))


def test_global_topk_brute_force():
    """One group (V4.1): the top-k of choice = score + bias over every expert (a tie to the
    lower id) in that order, weights score * scale / their sum in that order; against every
    k-subset at E = 16."""
    rng = np.random.default_rng(7)
    e, k, scale = 16, 4, 1.5
    for trial in range(40):
        sc = rt.sqrt_softplus_exact(rng.standard_normal((1, e)).astype(np.float32))
        bias = (rng.integers(-2, 3, e) * 0.25).astype(np.float32) if trial % 2 else np.zeros(e, np.float32)
        if trial % 4 == 3:
            sc[0, 5] = sc[0, 9]  # a tie of choices
            bias[5] = bias[9]
        ids, wts = rt.grouped_topk(sc, bias, k, 1, 1, scale)
        ch = (sc[0] + bias).astype(np.float32)
        best = max(itertools.combinations(range(e), k), key=lambda s: sorted(((ch[i], -i) for i in s), reverse=True))
        want = sorted(best, key=lambda i: (-ch[i], i))
        assert ids[0].tolist() == want
        tot = np.float32(0.0)
        for i in want:
            tot = np.float32(tot + sc[0, i])
        f = np.float32(scale) / max(tot, np.float32(1e-20))
        assert np.array_equal(wts[0], (sc[0, want] * f).astype(np.float32))


def test_route_v41_scoring():
    """``route`` takes the preset's scorer."""
    import torch

    rng = np.random.default_rng(8)
    x = torch.from_numpy(rng.standard_normal((3, 1024)).astype(np.float32)).to(torch.bfloat16)
    gw = torch.from_numpy((rng.standard_normal((16, 1024)) / 32).astype(np.float32)).to(torch.bfloat16)
    p = dict(router_parts=2, topk=4, n_group=1, topk_group=1, routed_scale=1.5, scoring="sqrt_softplus")
    logit, ids, wts = rt.route(x, gw, np.zeros(16, np.float32), p)
    sc = rt.sqrt_softplus_exact(logit)
    want, ww = rt.grouped_topk(sc, np.zeros(16, np.float32), 4, 1, 1, 1.5)
    assert np.array_equal(ids, want) and np.array_equal(wts, ww)
    assert np.allclose(wts.sum(1), 1.5, rtol=1e-6)
