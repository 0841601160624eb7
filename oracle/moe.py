"""The decode MoE block's golden model (one TP rank's pre-all-reduce partial), on the CPU.

TEST INFRASTRUCTURE ONLY (the oracle): imported by ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg, never by the
product path.

It restates ``golden_partial`` of ``test/kernels/deepseek_v41/check_ffn.py:209-232``
generalised over the presets (weight format, activation rule, routing, widths).
With ``exact=True`` (the default) every GEMV and SwiGLU follows the kernel's
fixed arithmetic order (``oracle.exact``), so the kernel's output must match
bit for bit; ``exact=False`` keeps the golden's fp32 matmuls and torch's silu
(the CPU baseline, and a cross-check within tolerance):

- routed experts, per expert e of the step's union (ascending id), its picks'
  rows: h = xr @ W13(e)^T in fp32; gate = h[:, :I], up = h[:, I:];
  mid = bf16(silu(min(gate, L)) * clamp(up, -L, L)); y = q(mid) @ W2(e)^T;
  per_k = bf16(y * w_k) (check_ffn.py:216-222)
- the routed sum in top-k order with bf16 at every add (check_ffn.py:223-225)
- the shared expert: hs = xs @ Wsgu^T; smid = bf16(silu(bf16(min(g, L))) *
  bf16(clamp(u, -L, L))); shared = bf16(q(smid) @ Wsw2^T) (check_ffn.py:226-231)
- out = bf16(routed + shared) (check_ffn.py:232)

q() is the preset's activation rule: MXFP8 "aiter" for MXFP4 routed experts
(check_ffn.py:212,221), per-token-group-128 FP8 with fp32 scales for FP8
128 x 128 weights (routed and shared). Routing is ``oracle.routing``'s exact
restatement (the kernel's order) rather than the golden's unordered fp32
matmul; the golden's own routing is kept as ``routing_golden`` for the
cross-check the reference makes (check_ffn.py:321-322,341).

Parity pins (tests/test_oracle_moe.py): each expert GEMM against an fp64
matmul of the dequantized operands; the combine order against a
hand-computed two-pick case; invariants (a zero shared expert leaves the
routed sum; an expert picked by no token is never read).
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import formats as fm
from . import routing as rt

FP8_B128 = "fp8_b128"
MXFP4 = "mxfp4"


def act_qdq(x: torch.Tensor, fmt: str) -> torch.Tensor:
    """The activation rule that feeds an expert GEMM of weight format ``fmt``."""
    if fmt == MXFP4:
        return fm.mxfp8_qdq(x)
    if fmt == FP8_B128:
        return fm.group_fp8_qdq(x, 128)
    raise ValueError(fmt)


def deq_weight(q: torch.Tensor, s: torch.Tensor, fmt: str) -> torch.Tensor:
    if fmt == MXFP4:
        return fm.deq_mxfp4(q, s)
    if fmt == FP8_B128:
        return fm.deq_fp8_b128(q, s)
    raise ValueError(fmt)


def silu(x: torch.Tensor) -> torch.Tensor:
    return F.silu(x)


def routing_golden(x: torch.Tensor, gate_w: torch.Tensor, bias: torch.Tensor, p: dict):
    """The golden's unordered fp32 routing (check_ffn.py:201-206), sigmoid grouped form."""
    logits = x.float() @ gate_w.float().T
    sc = torch.sigmoid(logits)
    ids, _ = rt.grouped_topk(
        sc.numpy(), bias.float().numpy(), p["topk"], p["n_group"], p["topk_group"], p["routed_scale"]
    )
    return ids


class ExpertSource:
    """Where the golden model reads expert e's quantized tensors (any mapping of e -> tensors)."""

    def __init__(self, w13, w13_s, w2, w2_s):
        self.w13, self.w13_s, self.w2, self.w2_s = w13, w13_s, w2, w2_s

    def get(self, e: int):
        return self.w13[e], self.w13_s[e], self.w2[e], self.w2_s[e]


def _qdq_codes(x: torch.Tensor, fmt: str):
    """(codes, scales) of the activation rule feeding weight format ``fmt``."""
    if fmt == MXFP4:
        return fm.mxfp8_quant(x)
    return fm.group_fp8_quant(x, 128)


def _gemv(wq, ws, xq, xs, fmt, lpr=None) -> np.ndarray:
    from . import exact as ex

    if fmt == MXFP4:
        return ex.gemv_mxfp4(wq, ws, xq, xs, lpr)
    return ex.gemv_fp8_b128(wq, ws, xq, xs, lpr)


def moe_partial(x: torch.Tensor, w: dict, p: dict, experts=None, exact: bool = True):
    """This rank's MoE partial of bf16 rows ``x`` [R, H].

    ``w`` holds CPU tensors: gate_w bf16 [E, H], bias fp32 [E], norm bf16 [H]
    (fused-norm preset only), sgu / sgu_s / sw2 / sw2_s (FP8 128 x 128 shared
    expert), and either the per-expert tensors w13 / w13_s / w2 / w2_s or an
    ``experts`` source with ``get(e)``. ``exact``: the kernel's GEMV and SwiGLU
    arithmetic (``oracle.exact``), bit for bit; otherwise the golden's fp32
    matmuls and torch's silu. Returns ids, weights, logits, the normed rows (if
    any), the per-pick contributions and the bf16 output.
    """
    from . import exact as ex

    lim = float(p["swiglu_limit"])
    r = x.shape[0]
    h = p["hidden"]
    inter = p["inter"]
    ish = p["shared_inter"]
    fmt = p["routed_fmt"]
    topk = p["topk"]
    if experts is None:
        experts = ExpertSource(w["w13"], w["w13_s"], w["w2"], w["w2_s"])
    xin = x
    if p.get("norm_eps") is not None:
        xin = rt.rmsnorm_exact(x, w["norm"], p["norm_eps"])
    logit, ids_np, wts_np = rt.route(xin, w["gate_w"], w["bias"], p)
    ids = torch.from_numpy(ids_np.astype(np.int64))
    wts = torch.from_numpy(wts_np)
    per_k = torch.zeros(r, topk, h)
    if exact:
        xq, xs = _qdq_codes(xin, fmt)
        xq2, xs2 = fm.group_fp8_quant(xin, 128)
        for e in ids.unique().tolist():
            rows, ks = (ids == e).nonzero(as_tuple=True)
            w13, w13_s, w2, w2_s = experts.get(e)
            hh = _gemv(w13, w13_s, xq[rows], xs[rows], fmt)
            mid = ex.swiglu_routed(hh[:, :inter], hh[:, inter:], lim)
            mq, ms = _qdq_codes(torch.from_numpy(mid), fmt)
            y = _gemv(w2, w2_s, mq, ms, fmt, ex.DOWN_LANES)
            per_k[rows, ks] = fm.bf(torch.from_numpy(y) * wts[rows, ks, None])
    else:
        xr = act_qdq(xin, fmt)
        for e in ids.unique().tolist():
            rows, ks = (ids == e).nonzero(as_tuple=True)
            w13, w13_s, w2, w2_s = experts.get(e)
            hh = xr[rows] @ deq_weight(w13, w13_s, fmt).T
            gate, up = hh[:, :inter], hh[:, inter:]
            mid = fm.bf(silu(gate.clamp(max=lim)) * up.clamp(-lim, lim))
            y = act_qdq(mid, fmt) @ deq_weight(w2, w2_s, fmt).T
            per_k[rows, ks] = fm.bf(y * wts[rows, ks, None])
    routed = torch.zeros(r, h)
    for k in range(topk):
        routed = fm.bf(routed + per_k[:, k])
    if ish > 0 and exact:
        hs = ex.gemv_fp8_b128(w["sgu"], w["sgu_s"], xq2, xs2)
        smid = ex.swiglu_shared(hs[:, :ish], hs[:, ish:], lim)
        smq, sms = fm.group_fp8_quant(torch.from_numpy(smid), 128)
        shared = fm.bf(torch.from_numpy(ex.gemv_fp8_b128(w["sw2"], w["sw2_s"], smq, sms, ex.DOWN_LANES)))
    elif ish > 0:
        xs_ = act_qdq(xin, FP8_B128)
        hs = xs_ @ fm.deq_fp8_b128(w["sgu"], w["sgu_s"]).T
        smid = fm.bf(silu(fm.bf(hs[:, :ish].clamp(max=lim))) * fm.bf(hs[:, ish:].clamp(-lim, lim)))
        shared = fm.bf(act_qdq(smid, FP8_B128) @ fm.deq_fp8_b128(w["sw2"], w["sw2_s"]).T)
    else:
        shared = torch.zeros(r, h)
    out = fm.bf(routed + shared).to(torch.bfloat16)
    return {
        "ids": ids_np,
        "weights": wts_np,
        "logits": logit,
        "normed": xin,
        "out": out,
        "per_k": per_k,
    }


def union_stats(ids: np.ndarray) -> dict:
    """U (distinct experts), the largest pick count of an expert and the pick count."""
    u, cnt = np.unique(ids, return_counts=True)
    return {"U": int(len(u)), "max_rows_per_expert": int(cnt.max()), "picks": int(ids.size)}
