"""Seeded CPU generation of one MoE layer's inputs and weights, per workload.

TEST INFRASTRUCTURE ONLY (the oracle side): imported by ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg.

Every tensor has its own CPU ``torch.Generator`` seeded base + a stable id, and
every routed expert is generated alone (seed base + 100000 + e), so the oracle
and a GPU test can materialise only the experts a step routes to. The
reference draws its inputs from device generators
(``test/kernels/deepseek_v41/check_ffn.py:133-134``), which cannot be
reproduced off the GPU; these are drawn on the CPU instead.

Distributions (per workload):
- x ~ N(0, 1) bf16 [R, H]
- router weight: N(0, 0.02) bf16 for the 1024-wide plumbing layer; N(0, 1/H)
  for the 7168-wide layers, so the logits x . w are ~N(0, 1)
- router bias ~ N(0, 0.02) fp32 (check_ffn.py:153-155)
- routed and shared expert weights ~ N(0, 0.02) fp32, then quantized (FP8 with
  fp32 128 x 128 scales, or MXFP4)
- RMSNorm weight 1 + N(0, 0.1) bf16 (check_ffn.py:152)
- the Zipf(1.2) stress: hidden element 0 of every row is 1.0 and router column
  0 holds bf16(log p_e) for p_e ~ rank(e)^-1.2 over a seeded permutation of the
  experts, so the logits are log p_e plus N(0, 1) noise.
- the V4.1 shape (an MX shared expert, padded routed widths) follows the reference
  test's ``make_weights`` (check_ffn.py:128-182) instead: router N(0, 0.02) bf16, bias
  N(0, 0.02) held in bf16; routed experts as random e2m1 bytes with E8M0 codes 118..122 over
  the rank's real columns and zeros in the loader's padding (gate and up rows I_real .. I, w2's
  K columns and scales past I_real); the shared expert N(0, 1) clamped to +-6 in e4m3 with E8M0
  32 x 32 codes 118..122.
"""

from __future__ import annotations

import math

import torch

from . import formats as fm
from .moe import FP8_B128, MXFP4

T_X, T_GATE, T_BIAS, T_NORM, T_SGU, T_SW2, T_ZIPF = 1, 2, 3, 4, 5, 6, 7
EXPERT_SEED = 100000


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(int(seed))


def randn(shape, seed: int, std: float = 1.0) -> torch.Tensor:
    return torch.randn(*shape, generator=_gen(seed)) * std


def make_x(p: dict, rows: int, seed: int) -> torch.Tensor:
    x = randn((rows, p["hidden"]), seed * 1000 + T_X)
    if p.get("zipf_s"):
        x[:, 0] = 1.0
    return x.to(torch.bfloat16)


def quant_weight(w: torch.Tensor, fmt: str):
    if fmt == FP8_B128:
        return fm.quant_fp8_b128(w)
    if fmt == MXFP4:
        return fm.quant_mxfp4(w)
    raise ValueError(fmt)


def _e8m0(shape, g: torch.Generator) -> torch.Tensor:
    return torch.randint(118, 123, shape, generator=g, dtype=torch.uint8)


def _v41(p: dict) -> bool:
    return p.get("shared_fmt") == "fp8_mx32"


def make_dense(p: dict, seed: int) -> dict:
    """The router, bias, norm and shared expert (everything but the routed experts)."""
    h, e = p["hidden"], p["experts"]
    if _v41(p):
        ish = p["shared_inter"]
        g = _gen(seed * 1000 + T_SGU)
        sgu = torch.randn(2 * ish, h, generator=g).clamp(-6, 6)
        sw2 = torch.randn(h, ish, generator=g).clamp(-6, 6)
        return {
            "gate_w": randn((e, h), seed * 1000 + T_GATE, 0.02).to(torch.bfloat16),
            "bias": randn((e,), seed * 1000 + T_BIAS, 0.02).to(torch.bfloat16).float(),
            "sgu": fm.e4m3_codes_from_f32(sgu),
            "sgu_s": _e8m0((2 * ish // 32, h // 32), g),
            "sw2": fm.e4m3_codes_from_f32(sw2),
            "sw2_s": _e8m0((h // 32, ish // 32), g),
        }
    std = 0.02 if h <= 1024 else 1.0 / math.sqrt(h)
    gate = randn((e, h), seed * 1000 + T_GATE, std)
    if p.get("zipf_s"):
        perm = torch.randperm(e, generator=_gen(seed * 1000 + T_ZIPF))
        rank = torch.empty(e)
        rank[perm] = torch.arange(1, e + 1, dtype=torch.float32)
        logp = -p["zipf_s"] * torch.log(rank)
        logp = logp - torch.logsumexp(logp, 0)
        gate[:, 0] = logp
    w = {
        "gate_w": gate.to(torch.bfloat16),
        "bias": randn((e,), seed * 1000 + T_BIAS, 0.02).float(),
    }
    if p.get("norm_eps") is not None:
        w["norm"] = (1 + randn((h,), seed * 1000 + T_NORM, 0.1)).to(torch.bfloat16)
    ish = p["shared_inter"]
    w["sgu"], w["sgu_s"] = fm.quant_fp8_b128(randn((2 * ish, h), seed * 1000 + T_SGU, 0.02))
    w["sw2"], w["sw2_s"] = fm.quant_fp8_b128(randn((h, ish), seed * 1000 + T_SW2, 0.02))
    return w


def _expert_job(args):
    p, seed, e = args
    return e, LazyExperts(p, seed).get(e)


def _one_thread():
    torch.set_num_threads(1)


class LazyExperts:
    """Routed expert e's quantized (w13, w13_s, w2, w2_s), generated on first use from seed + e."""

    def __init__(self, p: dict, seed: int):
        self.p, self.seed, self.cache = p, seed, {}

    def prefetch(self, es, workers: int) -> None:
        """Generate experts ``es`` in ``workers`` processes started by spawn (no GPU state is
        inherited): the same seeds, so the same tensors as ``get``."""
        todo = [int(e) for e in es if int(e) not in self.cache]
        if workers <= 1 or len(todo) < 8:
            for e in todo:
                self.get(e)
            return
        import multiprocessing
        from concurrent.futures import ProcessPoolExecutor

        ctx = multiprocessing.get_context("spawn")
        with ProcessPoolExecutor(workers, mp_context=ctx, initializer=_one_thread) as pool:
            for e, t in pool.map(_expert_job, [(self.p, self.seed, e) for e in todo]):
                self.cache[e] = t

    def get(self, e: int):
        if e not in self.cache and _v41(self.p):
            p = self.p
            h, i = p["hidden"], p["inter"]
            ir = p.get("inter_real") or i
            g = _gen(self.seed * 1000 + EXPERT_SEED + 4 * e)
            w13 = torch.zeros(2 * i, h // 2, dtype=torch.uint8)
            s13 = torch.zeros(2 * i, h // 32, dtype=torch.uint8)
            for half in (0, i):
                w13[half : half + ir] = torch.randint(0, 256, (ir, h // 2), generator=g, dtype=torch.uint8)
                s13[half : half + ir] = _e8m0((ir, h // 32), g)
            w2 = torch.zeros(h, i // 2, dtype=torch.uint8)
            s2 = torch.zeros(h, i // 32, dtype=torch.uint8)
            w2[:, : ir // 2] = torch.randint(0, 256, (h, ir // 2), generator=g, dtype=torch.uint8)
            s2[:, : ir // 32] = _e8m0((h, ir // 32), g)
            self.cache[e] = (w13, s13, w2, s2)
        if e not in self.cache:
            p = self.p
            h, i = p["hidden"], p["inter"]
            base = self.seed * 1000 + EXPERT_SEED + 4 * e
            w13 = randn((2 * i, h), base, 0.02)
            w2 = randn((h, i), base + 1, 0.02)
            self.cache[e] = quant_weight(w13, p["routed_fmt"]) + quant_weight(w2, p["routed_fmt"])
        return self.cache[e]


def expert_shapes(p: dict) -> dict:
    """Shapes and dtypes (as torch dtypes of the raw bytes) of the stacked routed-expert tensors."""
    e, h, i = p["experts"], p["hidden"], p["inter"]
    if p["routed_fmt"] == FP8_B128:
        return {
            "w13": ((e, 2 * i, h), torch.uint8),
            "w13_s": ((e, -(-2 * i // 128), -(-h // 128)), torch.float32),
            "w2": ((e, h, i), torch.uint8),
            "w2_s": ((e, -(-h // 128), -(-i // 128)), torch.float32),
        }
    return {
        "w13": ((e, 2 * i, h // 2), torch.uint8),
        "w13_s": ((e, 2 * i, h // 32), torch.uint8),
        "w2": ((e, h, i // 2), torch.uint8),
        "w2_s": ((e, h, i // 32), torch.uint8),
    }


# ---------------------------------------------------------------- the FFN seam (mHC) inputs
T_SEAM_X, T_SEAM_RES, T_SEAM_COMB, T_SEAM_POST, T_SEAM_PRE = 11, 12, 13, 14, 15
T_SEAM_FN, T_SEAM_SCALE, T_SEAM_BASE, T_SEAM_NORM = 16, 17, 18, 19
SEAM_HC = 4
SEAM_MIX = 24


def seam_inputs(tokens: int, hidden: int, seed: int) -> dict:
    """One step's seam inputs, with the distributions of the reference test's
    ``seam_inputs`` (check_ffn.py:236-251) on one rank: residual streams of RMS 1 (bf16), a
    Sinkhorn-normalised comb, post = 2 sigmoid(N), pre = sigmoid(N) + 1e-6, the attention
    output N(0, 0.5) (bf16)."""
    hc = SEAM_HC
    res = torch.randn(tokens, hc, hidden, generator=_gen(seed + T_SEAM_RES))
    res = (res * torch.rsqrt(res.pow(2).mean(-1, keepdim=True))).to(torch.bfloat16)
    comb = torch.rand(tokens, hc, hc, generator=_gen(seed + T_SEAM_COMB)) + 0.1
    for _ in range(20):
        comb = comb / comb.sum(-1, keepdim=True)
        comb = comb / comb.sum(-2, keepdim=True)
    post = torch.sigmoid(torch.randn(tokens, hc, generator=_gen(seed + T_SEAM_POST))) * 2
    pre = torch.sigmoid(torch.randn(tokens, hc, generator=_gen(seed + T_SEAM_PRE))) + 1e-6
    a = (torch.randn(tokens, hidden, generator=_gen(seed + T_SEAM_X)) * 0.5).to(torch.bfloat16)
    return dict(a=a, res=res, post=post.contiguous(), comb=comb.contiguous(), pre=pre.contiguous())


def seam_weights(hidden: int, seed: int) -> dict:
    """The seam's weights as the reference test draws them (check_ffn.py:149-152): fn
    N(0, 0.01) [24, 4 H] fp32, scale |N(0, 0.5)| + 0.5 [3], base N(0, 0.1) [24], the norm
    weight 1 + N(0, 0.1) bf16."""
    return dict(
        fn=randn((SEAM_MIX, SEAM_HC * hidden), seed + T_SEAM_FN, 0.01),
        scale=randn((3,), seed + T_SEAM_SCALE, 0.5).abs() + 0.5,
        base=randn((SEAM_MIX,), seed + T_SEAM_BASE, 0.1),
        norm=(1.0 + randn((hidden,), seed + T_SEAM_NORM, 0.1)).to(torch.bfloat16),
    )
