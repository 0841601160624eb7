"""Build one MoE layer on the GPU from the oracle's seeded CPU inputs, plus its oracle result.

Every expert that a checked row routes to holds its seeded weights (generated
on the CPU, expert by expert); every other expert holds random but finite bytes
drawn on the GPU, so a kernel that reads a wrong expert for a checked row
fails the comparison. Routing (cheap) is checked for every row; the output for
``check`` rows (all rows up to 8, else 8 rows spread over the step).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from oracle import gen
from oracle import moe as om
from oracle import routing as rt
from sgl_amd_mono.moe.presets import PRESETS, WORKLOADS, workload_dict
from sgl_amd_mono.moe.runner import MoeWeights


@dataclass
class Case:
    workload: str
    preset: object
    p: dict
    rows: int
    x: torch.Tensor  # device bf16 [R, H]
    w: MoeWeights
    ids: np.ndarray  # oracle ids [R, k]
    wts: np.ndarray  # oracle weights [R, k]
    parts: np.ndarray  # oracle router part sums [R, E, P]
    xin: torch.Tensor  # oracle normed (or raw) x, CPU bf16
    check: np.ndarray  # rows whose output the oracle computed
    ref: torch.Tensor  # oracle output bf16 [len(check), H] (the kernel's arithmetic order)
    golden: torch.Tensor  # the golden's fp32-matmul output bf16 [len(check), H]


def _random_fill(shape, dtype, fmt, kind, device, g):
    if dtype == torch.float32:  # fp32 block scales
        return torch.rand(shape, generator=g, device=device) * 1e-4 + 1e-4
    if kind == "scale":  # E8M0
        return torch.randint(118, 123, shape, generator=g, device=device, dtype=torch.uint8)
    t = torch.randint(0, 256, shape, generator=g, device=device, dtype=torch.uint8)
    if fmt == om.FP8_B128:  # no e4m3 NaN codes (0x7f, 0xff)
        t = torch.where((t & 0x7F) == 0x7F, t ^ 1, t)
    return t


def check_rows(rows: int) -> np.ndarray:
    if rows <= 8:
        return np.arange(rows)
    return np.unique(np.linspace(0, rows - 1, 8).round().astype(int))


def build(workload: str, rows: int, seed: int = 0, device="cuda") -> Case:
    p = workload_dict(workload)
    preset = PRESETS[WORKLOADS[workload]["preset"]]
    x = gen.make_x(p, rows, seed)
    dense = gen.make_dense(p, seed)
    xin = rt.rmsnorm_exact(x, dense["norm"], p["norm_eps"]) if p["norm_eps"] is not None else x
    parts = rt.router_part_sums(xin, dense["gate_w"], p["router_parts"])
    scores = rt.sigmoid_exact(rt.logits_from_parts(parts))
    ids, wts = rt.grouped_topk(scores, dense["bias"].numpy(), p["topk"], p["n_group"], p["topk_group"], p["routed_scale"])
    check = check_rows(rows)
    ex = gen.LazyExperts(p, seed)
    res = om.moe_partial(x[torch.from_numpy(check)], dense, p, experts=ex)
    assert np.array_equal(res["ids"], ids[check])
    golden = om.moe_partial(x[torch.from_numpy(check)], dense, p, experts=ex, exact=False)["out"]
    g = torch.Generator(device=device).manual_seed(1234 + seed)
    dev = {}
    for name, (shape, dtype) in gen.expert_shapes(p).items():
        kind = "scale" if name.endswith("_s") else "w"
        dev[name] = _random_fill(shape, dtype, p["routed_fmt"], kind, device, g)
    for e, (w13, w13_s, w2, w2_s) in ex.cache.items():
        dev["w13"][e].copy_(w13.to(device))
        dev["w13_s"][e].copy_(w13_s.to(device))
        dev["w2"][e].copy_(w2.to(device))
        dev["w2_s"][e].copy_(w2_s.to(device))
    w = MoeWeights(
        gate_w=dense["gate_w"].to(device),
        bias=dense["bias"].to(device),
        sgu=dense["sgu"].to(device),
        sgu_s=dense["sgu_s"].to(device),
        sw2=dense["sw2"].to(device),
        sw2_s=dense["sw2_s"].to(device),
        norm=dense["norm"].to(device) if "norm" in dense else None,
        **dev,
    )
    return Case(workload, preset, p, rows, x.to(device), w, ids, wts, parts, xin, check, res["out"], golden)


def errors(out: torch.Tensor, ref: torch.Tensor) -> dict:
    """max-abs, relative L2, cosine, and the largest difference in bf16 ulps of the reference."""
    a, b = out.float().cpu(), ref.float().cpu()
    d = (a - b).abs()
    ulp = torch.ldexp(torch.ones_like(b), torch.frexp(b.abs().clamp_min(2.0**-20))[1] - 8)
    return {
        "max_abs": float(d.max()),
        "rel_l2": float((a - b).norm() / b.norm()),
        "cos": float(torch.nn.functional.cosine_similarity(a.reshape(-1), b.reshape(-1), dim=0)),
        "max_ulp": float((d / ulp).max()),
        "n_over_2e-2": int((d > 2e-2).sum()),
        "nan": bool(torch.isnan(a).any()),
    }
