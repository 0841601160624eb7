"""The MoE block shapes the HIP library is compiled for (one TP rank's share).

The reference hardcodes one model's MoE (``sgl_amd_mono/deepseek_v41/__init__.py:11-37``,
``gfx950/stages/moe_shape.py:24``, ``gfx950/stages/dims.py:13-56``). Here the
block is parameterised; each preset is one compiled specialisation of the
kernel (``csrc/mkmoe_kernels.hip``), selected at run time by its shape.

Fields:
- hidden, experts, topk, n_group, topk_group: routing (DeepSeek-V3 ``noaux_tc``:
  sigmoid scores, bias for selection, top-2 sums per group)
- inter / shared_inter: a routed / the shared expert's intermediate width on
  this rank (the TP share)
- routed_fmt: "fp8_b128" (e4m3 with fp32 128 x 128 block scales) or "mxfp4"
  (e2m1 with an E8M0 scale per 32 K)
- shared_fmt: the shared expert's, "fp8_b128" (its activations and intermediate quantized
  per 128 with fp32 scales) or "fp8_mx32" (e4m3 with E8M0 32 x 32 block scales, fed by MXFP8
  of the "vllm" rule: V4.1's, ``gfx950/runner.py:143-146``, ``check_ffn.py:118-121,226-231``)
- inter_real: a routed expert's real width on this rank when the loader pads it with zero
  weights to ``inter`` (V4.1: 2304 / 4 = 576 padded to 640, ``stages/dims.py:13-46``)
- aiter_only: compiled for SGLang's loaded gfx950 layout of the MXFP4 experts alone
- routed_scale, swiglu_limit: the weights' scale after normalisation and the
  SwiGLU clamp (the reference's 1.5 and 10.0 at ``stages/moe.py:96-97``)
- router_parts: contiguous K parts of the router GEMV summed in order (the
  reference's ``PARTS`` at ``stages/router.py:18``)
- norm_eps: RMSNorm before the block (None: no norm)
- scoring: the router's score, "sigmoid" (DeepSeek-V3) or "sqrt_softplus" (V4.1:
  sqrt(softplus(logit)) with the bias for selection, ``check_ffn.py:201-206``)
- max_rows: the decode rows a launch takes at most (``spec.py:64``: 48)
"""

from __future__ import annotations

from dataclasses import asdict, dataclass

FMT_CODES = {"fp8_b128": 1, "mxfp4": 2, "fp8_mx32": 4}


@dataclass(frozen=True)
class MoePreset:
    name: str
    hidden: int
    experts: int
    topk: int
    n_group: int
    topk_group: int
    inter: int
    shared_inter: int
    routed_fmt: str
    routed_scale: float
    swiglu_limit: float
    router_parts: int
    norm_eps: float | None = None
    max_rows: int = 48
    renorm: bool = True
    scoring: str = "sigmoid"
    shared_fmt: str = "fp8_b128"
    inter_real: int | None = None
    aiter_only: bool = False

    def as_dict(self) -> dict:
        return asdict(self)

    @property
    def routed_expert_bytes(self) -> int:
        """HBM bytes of one routed expert (gate_up + down, weights + scales), at its real width
        (a padded layout's zero columns are not counted: they need not be read)."""
        h = self.hidden
        i = self.inter if self.inter_real is None else self.inter_real
        if self.routed_fmt == "mxfp4":
            return 3 * i * h // 2 + 3 * i * h // 32
        return 3 * i * h + 4 * (-(-2 * i // 128) * -(-h // 128) + -(-h // 128) * -(-i // 128))

    @property
    def shared_bytes(self) -> int:
        h, i = self.hidden, self.shared_inter
        if self.shared_fmt == "fp8_mx32":
            return 3 * i * h + 2 * i // 32 * (h // 32) + h // 32 * (i // 32)
        return 3 * i * h + 4 * (-(-2 * i // 128) * -(-h // 128) + -(-h // 128) * -(-i // 128))

    def algorithmic_bytes(self, rows: int, union: int) -> int:
        """B(R): the bytes one launch must move at least, for ``union`` distinct routed experts."""
        b = union * self.routed_expert_bytes + self.shared_bytes
        b += self.experts * self.hidden * 2 + self.experts * 4  # router weight (bf16) and bias
        b += 2 * rows * self.hidden * 2  # x in, out
        if self.norm_eps is not None:
            b += self.hidden * 2
        return b

    def flops(self, rows: int) -> int:
        return 2 * 3 * self.inter * self.hidden * rows * self.topk + 2 * 3 * self.shared_inter * self.hidden * rows + 2 * self.experts * self.hidden * rows


PRESETS = {
    # 1: the CPU-runnable plumbing layer
    "plumbing_fp8": MoePreset(
        "plumbing_fp8", hidden=1024, experts=16, topk=4, n_group=1, topk_group=1,
        inter=512, shared_inter=512, routed_fmt="fp8_b128", routed_scale=1.0,
        swiglu_limit=10.0, router_parts=2,
    ),
    # 2: DeepSeek-V3 shape, TP4 share, FP8 w8a8 128 x 128
    "dsv3_tp4_fp8": MoePreset(
        "dsv3_tp4_fp8", hidden=7168, experts=256, topk=8, n_group=8, topk_group=4,
        inter=512, shared_inter=512, routed_fmt="fp8_b128", routed_scale=2.5,
        swiglu_limit=10.0, router_parts=7,
    ),
    # 3 and 4: the same with MXFP4 routed experts (FP8 shared expert)
    "dsv3_tp4_mxfp4": MoePreset(
        "dsv3_tp4_mxfp4", hidden=7168, experts=256, topk=8, n_group=8, topk_group=4,
        inter=512, shared_inter=512, routed_fmt="mxfp4", routed_scale=2.5,
        swiglu_limit=10.0, router_parts=7,
    ),
    # 5: RMSNorm + MXFP4 experts + FP8 shared expert, TP2 share
    "dsv3_tp2_mxfp4_norm": MoePreset(
        "dsv3_tp2_mxfp4_norm", hidden=7168, experts=256, topk=8, n_group=8, topk_group=4,
        inter=1024, shared_inter=1024, routed_fmt="mxfp4", routed_scale=2.5,
        swiglu_limit=10.0, router_parts=7, norm_eps=1e-6,
    ),
    # DeepSeek-V4.1's MoE at TP4 (the reference's own model: stages/moe_shape.py:24,
    # stages/dims.py:13-56, check_ffn.py:13-18): hidden 5120, 384 experts top-6 by sqrt(softplus)
    # over one group, routed scale 1.5; MXFP4 routed experts in SGLang's loaded layout, the
    # rank's 576 columns padded to 640; the shared expert's 576 columns FP8 with E8M0 32 x 32
    # scales; the router in 5 parts of 1024 columns
    "v41_tp4": MoePreset(
        "v41_tp4", hidden=5120, experts=384, topk=6, n_group=1, topk_group=1,
        inter=640, shared_inter=576, routed_fmt="mxfp4", routed_scale=1.5,
        swiglu_limit=10.0, router_parts=5, scoring="sqrt_softplus", shared_fmt="fp8_mx32",
        inter_real=576, aiter_only=True,
    ),
    # ... at TP2: the rank's 1152 routed and shared columns (a multiple of 128, no padding)
    "v41_tp2": MoePreset(
        "v41_tp2", hidden=5120, experts=384, topk=6, n_group=1, topk_group=1, inter=1152,
        shared_inter=1152, routed_fmt="mxfp4", routed_scale=1.5, swiglu_limit=10.0, router_parts=5,
        scoring="sqrt_softplus", shared_fmt="fp8_mx32", aiter_only=True,
    ),
    # the plumbing layer routed as V4.1 routes (sqrt(softplus) scores over one group, the
    # routed scale 1.5 of check_ffn.py:14)
    "plumbing_fp8_softplus": MoePreset(
        "plumbing_fp8_softplus", hidden=1024, experts=16, topk=4, n_group=1, topk_group=1,
        inter=512, shared_inter=512, routed_fmt="fp8_b128", routed_scale=1.5,
        swiglu_limit=10.0, router_parts=2, scoring="sqrt_softplus",
    ),
}  # fmt: skip

# The workloads the tests and the benchmark run: a preset, the input
# distribution and the decode row counts
WORKLOADS = {
    "cfg1_plumbing_fp8": dict(preset="plumbing_fp8", rows=(4,)),
    "plumbing_fp8_softplus": dict(preset="plumbing_fp8_softplus", rows=(1, 4, 16, 24)),
    "cfg2_tp4_fp8": dict(preset="dsv3_tp4_fp8", rows=(1, 8, 48)),
    "cfg3_tp4_mxfp4": dict(preset="dsv3_tp4_mxfp4", rows=(1, 8, 48)),
    "cfg4_tp4_mxfp4_zipf": dict(preset="dsv3_tp4_mxfp4", rows=(48,), zipf_s=1.2),
    "cfg5_tp2_mxfp4_norm": dict(preset="dsv3_tp2_mxfp4_norm", rows=(1, 8, 48)),
    # parity stress cases: the Zipf skew on the other weight formats (experts picked by
    # more rows than one gate_up token group holds)
    "tp4_fp8_zipf": dict(preset="dsv3_tp4_fp8", rows=(16, 48), zipf_s=1.2),
    "tp2_mxfp4_norm_zipf": dict(preset="dsv3_tp2_mxfp4_norm", rows=(48,), zipf_s=1.2),
    # the reference's own MoE shape: DeepSeek-V4.1 at TP4, the experts in SGLang's layout
    "v41_tp4_mxfp4": dict(preset="v41_tp4", rows=(1, 8, 48)),
    "v41_tp2_mxfp4": dict(preset="v41_tp2", rows=(1, 8, 48)),
}


def workload_dict(name: str) -> dict:
    """The preset's fields plus the workload's input distribution (``zipf_s``)."""
    w = WORKLOADS[name]
    d = PRESETS[w["preset"]].as_dict()
    d["zipf_s"] = w.get("zipf_s")
    return d
