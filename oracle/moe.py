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

Parity pins:
- tests/test_oracle_moe.py: the whole partial (both forms) on a crafted layer
  whose every value is a short dyadic number, against output bits worked out by
  hand: the routed SwiGLU rounded once after the product, the shared one at
  gate, up and product, the clamp, the combine in top-k order with bf16 at every
  add, then the shared output added; each misplaced rounding point or order,
  planted in the oracle, changes those bits (``combine``,
  ``swiglu_*_golden``, ``oracle.exact.swiglu_*``). Also the block against an
  fp64 evaluation of the same quantized operands, and an unpicked expert never
  read.
- tests/test_oracle_routing_golden.py: ``routing_golden`` (the golden's fp32
  matmul and torch's score) against the fixed-order routing on every benchmark
  workload's seeds: the same ids everywhere (a disagreement would be allowed
  only between choices within the two routings' measured logit errors), the
  weights within 1e-4; the fixed-order logits within their order's error bound.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import formats as fm
from . import routing as rt

FP8_B128 = "fp8_b128"
MXFP4 = "mxfp4"


FP8_MX32 = "fp8_mx32"  # e4m3 with E8M0 32 x 32 block scales (the V4.1 shared expert)


def act_qdq(x: torch.Tensor, fmt: str) -> torch.Tensor:
    """The activation rule that feeds an expert GEMM of weight format ``fmt``: MXFP8 "aiter"
    (MXFP4 weights), MXFP8 "vllm" (MX FP8 weights: check_ffn.py:212,231), group-128 FP8."""
    if fmt == MXFP4:
        return fm.mxfp8_qdq(x)
    if fmt == FP8_MX32:
        return fm.mxfp8_qdq(x, "vllm")
    if fmt == FP8_B128:
        return fm.group_fp8_qdq(x, 128)
    raise ValueError(fmt)


def has_exact(p: dict) -> bool:
    """Whether the preset has the fixed-order restatement (``exact=True``): the shapes whose
    GEMMs can run on the VALU GEMVs. The MX shared expert and the padded widths of the V4.1
    shape run on MFMA alone and are held to the golden's fp32-matmul form."""
    return p.get("shared_fmt", FP8_B128) == FP8_B128 and p.get("inter_real") is None


def deq_weight(q: torch.Tensor, s: torch.Tensor, fmt: str) -> torch.Tensor:
    if fmt == MXFP4:
        return fm.deq_mxfp4(q, s)
    if fmt == FP8_MX32:
        return fm.deq_fp8_mx32(q, s)
    if fmt == FP8_B128:
        return fm.deq_fp8_b128(q, s)
    raise ValueError(fmt)


def silu(x: torch.Tensor) -> torch.Tensor:
    return F.silu(x)


def swiglu_routed_golden(g: torch.Tensor, u: torch.Tensor, lim: float) -> torch.Tensor:
    """A routed expert's SwiGLU as the golden rounds it: bf16 once, after the product
    (``mid = bf(F.silu(gate.clamp(max=LIMIT)) * up.clamp(-LIMIT, LIMIT))``, check_ffn.py:220)."""
    return fm.bf(silu(g.clamp(max=lim)) * u.clamp(-lim, lim))


def swiglu_shared_golden(g: torch.Tensor, u: torch.Tensor, lim: float) -> torch.Tensor:
    """The shared expert's SwiGLU as the golden rounds it: bf16 at the clamped gate, at the
    clamped up and at the product (check_ffn.py:227-230)."""
    return fm.bf(silu(fm.bf(g.clamp(max=lim))) * fm.bf(u.clamp(-lim, lim)))


def combine(per_k: torch.Tensor, shared: torch.Tensor):
    """The weighted combine (check_ffn.py:223-225,232): the picks' bf16 contributions
    ``per_k`` [R, k, H] added in top-k order from 0 with bf16 at every add, then the shared
    expert's bf16 output added and rounded once more -> (out bf16 [R, H], the largest
    magnitude the bf16 chain held, fp32 [R, H])."""
    r, topk, h = per_k.shape
    routed = torch.zeros(r, h)
    chain = torch.zeros(r, h)
    for k in range(topk):
        routed = fm.bf(routed + per_k[:, k])
        chain = torch.maximum(chain, routed.abs())
    out = fm.bf(routed + shared).to(torch.bfloat16)
    return out, torch.maximum(chain, out.float().abs())


def routing_golden(x: torch.Tensor, gate_w: torch.Tensor, bias: torch.Tensor, p: dict):
    """The golden's own routing (check_ffn.py:201-206): logits by an fp32 matmul of
    unspecified order, the score by torch (``F.softplus(l).sqrt()`` for V4.1, ``torch.sigmoid``
    for the grouped DeepSeek-V3 presets), selection on score + bias (``topk`` of torch over one
    group; ``rt.grouped_topk`` over several), weights score * (scale / sum) -> (ids int32
    [R, k], weights fp32 [R, k], logits fp32 [R, E])."""
    logits = x.float() @ gate_w.float().T
    if p.get("scoring", "sigmoid") == "sqrt_softplus":
        sc = F.softplus(logits).sqrt()
    else:
        sc = torch.sigmoid(logits)
    scale = float(p["routed_scale"])
    if p["n_group"] == 1:
        ids = (sc + bias.float()).topk(p["topk"], dim=1).indices
        wt = sc.gather(1, ids)
        wts = wt * (scale / wt.sum(1, keepdim=True)) if p.get("renorm", True) else wt * scale
        return ids.numpy().astype(np.int32), wts.numpy().astype(np.float32), logits.numpy()
    ids, wts = rt.grouped_topk(
        sc.numpy(), bias.float().numpy(), p["topk"], p["n_group"], p["topk_group"], scale, p.get("renorm", True)
    )
    return ids, wts, logits.numpy()


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


def expert_contrib(tensors, xin_rows: torch.Tensor, w_rows: torch.Tensor, p: dict, exact: bool) -> torch.Tensor:
    """One routed expert's contributions bf16(y * w_k) [n, H] (fp32 holding bf16 values) for the
    n picks whose (normed) rows are ``xin_rows`` and routing weights ``w_rows``
    (check_ffn.py:216-222); ``exact``: the kernel's GEMV and SwiGLU order."""
    from . import exact as ex

    lim = float(p["swiglu_limit"])
    inter, fmt = p["inter"], p["routed_fmt"]
    w13, w13_s, w2, w2_s = tensors
    if exact:
        xq, xs = _qdq_codes(xin_rows, fmt)
        hh = _gemv(w13, w13_s, xq, xs, fmt)
        mid = ex.swiglu_routed(hh[:, :inter], hh[:, inter:], lim)
        mq, ms = _qdq_codes(torch.from_numpy(mid), fmt)
        y = torch.from_numpy(_gemv(w2, w2_s, mq, ms, fmt, ex.DOWN_LANES))
    else:
        xr = act_qdq(xin_rows, fmt)
        hh = xr @ deq_weight(w13, w13_s, fmt).T
        gate, up = hh[:, :inter], hh[:, inter:]
        mid = swiglu_routed_golden(gate, up, lim)
        y = act_qdq(mid, fmt) @ deq_weight(w2, w2_s, fmt).T
    return fm.bf(y * w_rows[:, None])


def _contrib_job(args):
    from . import gen

    p, seed, e, xin_rows, w_rows = args
    t = gen.LazyExperts(p, seed).get(e)
    g = expert_contrib(t, xin_rows, w_rows, p, False)
    return e, t, expert_contrib(t, xin_rows, w_rows, p, True) if has_exact(p) else g, g


def pool_contribs(p: dict, seed: int, xin: torch.Tensor, ids: np.ndarray, wts: np.ndarray, workers: int):
    """Every routed expert of a step, generated from its seed and computed in ``workers``
    processes started by spawn: -> (tensors, exact contributions, golden contributions),
    each a dict by expert id, the contributions in the pick order of ``moe_partial``."""
    import multiprocessing
    from concurrent.futures import ProcessPoolExecutor

    from . import gen

    idt = torch.from_numpy(ids.astype(np.int64))
    wt = torch.from_numpy(wts)
    jobs = []
    for e in idt.unique().tolist():
        rows, ks = (idt == e).nonzero(as_tuple=True)
        jobs.append((p, seed, e, xin[rows].clone(), wt[rows, ks].clone()))
    tensors, cx, cg = {}, {}, {}
    if workers <= 1 or len(jobs) < 8:
        results = map(_contrib_job, jobs)
    else:
        ctx = multiprocessing.get_context("spawn")
        pool = ProcessPoolExecutor(workers, mp_context=ctx, initializer=gen._one_thread)
        results = pool.map(_contrib_job, jobs)
    for e, t, x_, g_ in results:
        tensors[e], cx[e], cg[e] = t, x_, g_
    if workers > 1 and len(jobs) >= 8:
        pool.shutdown()
    return tensors, cx, cg


def moe_partial(x: torch.Tensor, w: dict, p: dict, experts=None, exact: bool = True, contribs: dict | None = None):
    """This rank's MoE partial of bf16 rows ``x`` [R, H].

    ``w`` holds CPU tensors: gate_w bf16 [E, H], bias fp32 [E], norm bf16 [H]
    (fused-norm preset only), sgu / sgu_s / sw2 / sw2_s (FP8 128 x 128 shared
    expert), and either the per-expert tensors w13 / w13_s / w2 / w2_s or an
    ``experts`` source with ``get(e)``. ``exact``: the kernel's GEMV and SwiGLU
    arithmetic (``oracle.exact``), bit for bit; otherwise the golden's fp32
    matmuls and torch's silu. ``contribs``: the routed experts' contributions
    already computed (``pool_contribs``) in the same mode. Returns ids, weights,
    logits, the normed rows (if any), the per-pick contributions and the bf16 output.
    The shared expert's format is ``p["shared_fmt"]`` (default FP8 128 x 128); with
    "fp8_mx32" its activations and intermediate take the MXFP8 "vllm" rule and its
    weights E8M0 32 x 32 scales (check_ffn.py:226-231); such presets have the golden's
    form alone (``has_exact``).
    """
    from . import exact as ex

    if exact and not has_exact(p):
        raise ValueError(f"{p.get('name', p)}: no fixed-order restatement (MFMA-only shape); use exact=False")
    sfmt = p.get("shared_fmt", FP8_B128)
    lim = float(p["swiglu_limit"])
    r = x.shape[0]
    h = p["hidden"]
    ish = p["shared_inter"]
    topk = p["topk"]
    if experts is None and contribs is None:
        experts = ExpertSource(w["w13"], w["w13_s"], w["w2"], w["w2_s"])
    xin = x
    if p.get("norm_eps") is not None:
        xin = rt.rmsnorm_exact(x, w["norm"], p["norm_eps"])
    logit, ids_np, wts_np = rt.route(xin, w["gate_w"], w["bias"], p)
    ids = torch.from_numpy(ids_np.astype(np.int64))
    wts = torch.from_numpy(wts_np)
    per_k = torch.zeros(r, topk, h)
    for e in ids.unique().tolist():
        rows, ks = (ids == e).nonzero(as_tuple=True)
        if contribs is not None:
            per_k[rows, ks] = contribs[e]
        else:
            per_k[rows, ks] = expert_contrib(experts.get(e), xin[rows], wts[rows, ks], p, exact)
    if exact:
        xq2, xs2 = fm.group_fp8_quant(xin, 128)
    if ish > 0 and exact:
        hs = ex.gemv_fp8_b128(w["sgu"], w["sgu_s"], xq2, xs2)
        smid = ex.swiglu_shared(hs[:, :ish], hs[:, ish:], lim)
        smq, sms = fm.group_fp8_quant(torch.from_numpy(smid), 128)
        shared = fm.bf(torch.from_numpy(ex.gemv_fp8_b128(w["sw2"], w["sw2_s"], smq, sms, ex.DOWN_LANES)))
    elif ish > 0:
        xs_ = act_qdq(xin, sfmt)
        hs = xs_ @ deq_weight(w["sgu"], w["sgu_s"], sfmt).T
        smid = swiglu_shared_golden(hs[:, :ish], hs[:, ish:], lim)
        shared = fm.bf(act_qdq(smid, sfmt) @ deq_weight(w["sw2"], w["sw2_s"], sfmt).T)
    else:
        shared = torch.zeros(r, h)
    out, chain = combine(per_k, shared)
    return {
        "chain_max": chain,
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
