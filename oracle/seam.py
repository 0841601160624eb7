"""The FFN seam before the MoE block (DeepSeek-V4.1's mHC hyper-connection update, its
collapse to the layer input, the mix projection, the Sinkhorn gate and the RMSNorm), in the
exact order the seam kernels compute it.

TEST INFRASTRUCTURE ONLY (the oracle): imported by ``tests/`` and ``bench.py``'s CPU-baseline
leg, never by the product path.

The reference runs this seam at the head of its FFN launch (``gfx950/layer.py:569-577``, the
stages of ``gfx950/stages/seam.py``); its test's golden is SGLang's ``hc_boundary_fused_deferred``
and ``rmsnorm_with_sinkhorn`` (``test/kernels/deepseek_v41/check_ffn.py:264-276``), a
dependency absent here. Shapes: HC = 4 residual streams of the hidden width H, MIX = 24
projections (pre 4 | post 4 | comb 16), K = HC * H (``seam.py:45-55``).

Per token, with a the (all-reduced) attention output owed its post mix, res [HC][H], post
[HC], comb [HC][HC] (comb[h][o]: stream h's weight in new stream o), pre [HC]:

1. Residual (``seam.py:137-158``, fold, not SGLang's order): for each new stream o and
   column c, v = post[o] a[c] + res[0][c] comb[0][o]; v = v + comb[1][o] res[1][c];
   v = v + comb[2][o] res[2][c]; v = fma(comb[3][o], res[3][c], v); R[o][c] = bf16(v).
   Products are rounded on their own, only the last term is fused.
2. Collapse (``seam.py:103-118``): lin[c] = bf16(0 + pre[0] R[0][c] + ... + pre[3] R[3][c]),
   summed in stream order, products rounded.
3. Mix partials (the kernels' order; the reference's runs on fp32 MFMA, ``seam.py:218-248``):
   columns split into slices of 32; for slice s, projection j and stream o,
   q[j][o] = 0 + fn[j][o H + 32 s] R[o][32 s] + ... (the slice's 32 columns in order), and
   P[j][s] = ((q[j][0] + q[j][1]) + q[j][2]) + q[j][3]; the sum of squares of R over the
   slice the same way (P[24][s]).
4. Mix sums (``seam.py:265-284``): slices summed in groups of 8 (each in order from its
   first), then the groups in order from the first.
5. Gate (``seam.py:285-321``): rstd = 1 / sqrt(fma(sq, 1/K, 1e-20)); v = mix rstd;
   pre' = sigmoid(fma(v, scale[0], base)) + 1e-6 (j < 4); post' = 2 sigmoid(fma(v, scale[1],
   base)) (4 <= j < 8); the comb logits z = fma(v, scale[2], base) as a 4 x 4 matrix
   (row r = (j - 8) / 4): a row softmax exp(z - rowmax) (rows summed (e0 + e1) + (e2 + e3)),
   then cv = fma(e, 1 / rowsum, 1e-6); then cv /= colsum + 1e-6 (by a multiply with the
   reciprocal); then 19 more rounds of the row step and the column step, each dividing by
   its sum + 1e-6 the same way. The sigmoid and the exp are the kernels' exact fp64 ones
   (``routing.sigmoid_exact``, ``routing.exp_nonpos``), the reciprocals and square root IEEE
   fp32; the reference's are the hardware approximations (within its 1e-4 relative bound).
6. RMSNorm of lin with the norm weight (``routing.rmsnorm_exact``'s order; the reference's
   ``stage_norm``, ``seam.py:326-378``).

Parity pins (``tests/test_oracle_seam.py``): ``fma32`` against exact rational arithmetic,
including inputs built to double-round; the residual against the reference test's own fp64
``hc_post`` (``check_ffn.py:62-73``) within half a bf16 ulp of the largest term, and a
transposed comb failing it; the collapse and the mix sums against fp64 products; the gate's
pre and post against ``math.exp``; the Sinkhorn output against its closed forms (logits that
are a row term plus a column term give 1/4 everywhere), its cross ratios (those of exp(z)) and
its column sums; the norm against an fp64 RMSNorm.
"""

from __future__ import annotations

import numpy as np

from . import routing as rt

HC = 4
MIX = HC * (HC + 2)  # 24: pre 4 | post 4 | comb 16
PART = MIX + 1  # a slice's partials: the 24 mixes, then the sum of squares
COLS = 32  # columns a slice
GROUP = 8  # slices a gate group sums
MIX_EPS = 1e-20
HC_EPS = 1e-6
SINKHORN = 20
POST_MULT = 2.0

F32 = np.float32


def fma32(a, b, c) -> np.ndarray:
    """fp32 fma(a, b, c) rounded once (to nearest even), for finite inputs and result.

    a b is exact in fp64; s = fl64(a b + c) and its error e (TwoSum) hold the exact sum.
    Rounding s to fp32 is right unless s lies exactly halfway between two fp32 values and
    e != 0, where the exact sum is past (or short of) that midpoint: then the side e points to
    decides."""
    a = np.asarray(a, F32).astype(np.float64)
    b = np.asarray(b, F32).astype(np.float64)
    c = np.asarray(c, F32).astype(np.float64)
    p = a * b
    s = p + c
    bb = s - p
    e = (p - (s - bb)) + (c - bb)
    r = s.astype(F32)
    r64 = r.astype(np.float64)
    d = s - r64  # exact: s and r are within half an fp32 ulp
    toward = np.where(d > 0, np.inf, -np.inf).astype(F32)
    nb = np.nextafter(r, toward)
    half = (nb.astype(np.float64) - r64) * 0.5
    past = (d != 0) & (d == half) & (e != 0) & (np.sign(e) == np.sign(d))
    return np.where(past, nb, r).astype(F32)


def bf16_round(x) -> np.ndarray:
    """fp32 -> bf16 (nearest even) -> fp32, for finite x."""
    u = np.ascontiguousarray(x, F32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(F32)


def bf16_bits(x) -> np.ndarray:
    """bf16 bits (uint16) of the fp32 values x (already bf16-exact, or rounded here)."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def residual(a, res, post, comb) -> np.ndarray:
    """R [T][HC][H] (bf16-exact fp32) of a [T][H], res [T][HC][H], post [T][HC], comb [T][HC][HC] (step 1)."""
    a = np.asarray(a, F32)[:, None, :]
    r = np.asarray(res, F32)
    pst = np.asarray(post, F32).reshape(-1, HC)[:, :, None]
    cm = np.asarray(comb, F32).reshape(-1, HC, HC)  # [t][h][o]

    def c_(h):
        return cm[:, h, :][:, :, None]  # [t][o][1]

    v = (pst * a).astype(F32) + (r[:, 0:1, :] * c_(0)).astype(F32)
    v = v + (c_(1) * r[:, 1:2, :]).astype(F32)
    v = v + (c_(2) * r[:, 2:3, :]).astype(F32)
    v = fma32(np.broadcast_to(c_(3), v.shape), np.broadcast_to(r[:, 3:4, :], v.shape), v)
    return bf16_round(v)


def collapse(R, pre) -> np.ndarray:
    """lin [T][H] (bf16-exact) = bf16(sum_h pre[h] R[h]) in stream order (step 2)."""
    pr = np.asarray(pre, F32).reshape(-1, HC)
    acc = np.zeros(R.shape[::2], F32)
    for h in range(HC):
        acc = acc + (pr[:, h : h + 1] * R[:, h, :]).astype(F32)
    return bf16_round(acc)


def mix_partials(R, fn) -> np.ndarray:
    """P [T][PART][slices]: each slice's 24 mix partials and its sum of squares (step 3)."""
    t, hc, h = R.shape
    ns = h // COLS
    assert hc == HC and ns * COLS == h
    rv = R.reshape(t, 1, HC, ns, COLS)
    fv = np.asarray(fn, F32).reshape(1, MIX, HC, ns, COLS)
    q = np.zeros((t, MIX, HC, ns), F32)
    sq = np.zeros((t, HC, ns), F32)
    for cc in range(COLS):
        q = q + (fv[..., cc] * rv[..., cc]).astype(F32)
        x = R.reshape(t, HC, ns, COLS)[..., cc]
        sq = sq + (x * x).astype(F32)
    out = np.empty((t, PART, ns), F32)
    out[:, :MIX] = ((q[:, :, 0] + q[:, :, 1]) + q[:, :, 2]) + q[:, :, 3]
    out[:, MIX] = ((sq[:, 0] + sq[:, 1]) + sq[:, 2]) + sq[:, 3]
    return out


def mix_sums(P) -> np.ndarray:
    """[T][PART]: the slices' partials summed in groups of 8, then the groups in order (step 4)."""
    ns = P.shape[2]
    assert ns % GROUP == 0
    tot = None
    for g in range(ns // GROUP):
        acc = P[:, :, g * GROUP]
        for k in range(1, GROUP):
            acc = acc + P[:, :, g * GROUP + k]
        tot = acc if tot is None else tot + acc
    return tot


def _rcp(x) -> np.ndarray:
    return (F32(1.0) / np.asarray(x, F32)).astype(F32)


def sinkhorn(z) -> np.ndarray:
    """The comb gate of logits z [T][HC][HC] (step 5's matrix part)."""
    z = np.asarray(z, F32)
    m = np.maximum(np.maximum(z[:, :, 0], z[:, :, 1]), np.maximum(z[:, :, 2], z[:, :, 3]))
    y = (z - m[:, :, None]).astype(F32)
    e = rt.exp_nonpos(y.astype(np.float64)).astype(F32)
    eps = F32(HC_EPS)

    def rows(v):
        return (v[:, :, 0] + v[:, :, 1]) + (v[:, :, 2] + v[:, :, 3])

    def cols(v):
        return (v[:, 0, :] + v[:, 1, :]) + (v[:, 2, :] + v[:, 3, :])

    cv = fma32(e, np.broadcast_to(_rcp(rows(e))[:, :, None], e.shape), np.full(e.shape, eps, F32))
    cv = cv * _rcp(cols(cv) + eps)[:, None, :]
    for _ in range(SINKHORN - 1):
        cv = cv * _rcp(rows(cv) + eps)[:, :, None]
        cv = cv * _rcp(cols(cv) + eps)[:, None, :]
    return cv.astype(F32)


def gate(sums, scale, base, hidden: int):
    """pre' [T][HC], post' [T][HC], comb' [T][HC][HC] from the mix sums [T][PART] (step 5)."""
    sums = np.asarray(sums, F32)
    mix, sq = sums[:, :MIX], sums[:, MIX]
    d = fma32(sq, np.full_like(sq, F32(1.0 / (HC * hidden))), np.full_like(sq, F32(MIX_EPS)))
    rstd = _rcp(np.sqrt(d).astype(F32))
    v = (mix * rstd[:, None]).astype(F32)
    sc = np.asarray(scale, F32)
    bs = np.broadcast_to(np.asarray(base, F32)[None, :], v.shape)

    def aff(lo, hi, k):
        return fma32(v[:, lo:hi], np.full_like(v[:, lo:hi], sc[k]), bs[:, lo:hi])

    pre = (rt.sigmoid_exact(aff(0, HC, 0)) + F32(HC_EPS)).astype(F32)
    post = (rt.sigmoid_exact(aff(HC, 2 * HC, 1)) * F32(POST_MULT)).astype(F32)
    comb = sinkhorn(aff(2 * HC, MIX, 2).reshape(-1, HC, HC))
    return pre, post, comb


def rmsnorm(lin, w, eps: float) -> np.ndarray:
    """bf16-exact normed rows of lin [T][H] (step 6, ``routing.rmsnorm_exact``'s order)."""
    import torch

    x = torch.from_numpy(np.ascontiguousarray(lin, F32)).to(torch.bfloat16)
    wt = torch.from_numpy(np.ascontiguousarray(w, F32)).to(torch.bfloat16)
    return rt.rmsnorm_exact(x, wt, eps).float().numpy()


def ffn_seam(a, res, post, comb, pre, fn, scale, base, norm_w, norm_eps: float = 1e-20) -> dict:
    """Every output of the seam for bf16-exact fp32 a, res, norm_w and fp32 mixes and weights."""
    a = np.asarray(a, F32)
    t, h = a.shape
    R = residual(a, res, post, comb)
    lin = collapse(R, pre)
    P = mix_partials(R, fn)
    sums = mix_sums(P)
    pre_o, post_o, comb_o = gate(sums, scale, base, h)
    normed = rmsnorm(lin, norm_w, norm_eps)
    return dict(res=R, lin=lin, partials=P, sums=sums, pre=pre_o, post=post_o, comb=comb_o, normed=normed)
