"""The MoE-block monokernel spec: DeepSeek-V3-shaped decode MoE on gfx950, backend ``amd``.

It keeps the reference spec's surface for the MoE path
(``sgl_amd_mono/deepseek_v41/spec.py``): a ``MonoSpec`` with per-ISA
``DeviceLimits`` (decode widths 1..48, TP 2 and 4, a persistent grid of 256
resident workgroups: ``:959-967``), per-output ``Numerics`` bounds
(``:287-318``), refusal reasons for the server configuration and for the
loaded model (``:331-404``), the FFN weights read in place off SGLang's
modules (``:484-530``) and a ``build`` that returns the object whose forward
the server calls (``:807-833,923-956``). Its forward is MoE-level: one layer's
MoE partial of this TP rank for the step's rows, before the all-reduce.

SGLang's module and attribute names read here (``mlp.gate.weight``,
``mlp.gate.e_score_correction_bias``, ``mlp.experts.w13_weight`` and its
scales, ``mlp.shared_experts.gate_up_proj`` / ``down_proj``,
``post_attention_layernorm``) are SGLang's DeepSeek-V3 ones; SGLang is not
installed here, so they are pinned only by the fake-model tests
(``tests/test_spec.py``).
"""

from __future__ import annotations

import dataclasses
import logging
import math

from .. import monospec as _local
from .presets import PRESETS, MoePreset

MAX_ROWS = 48
BLOCKS = 256
_log = logging.getLogger(__name__)


def _reg():
    from .. import registry

    return registry()


_R = _reg()
DeviceLimits, MonoSpec, Numerics, NumericsKind, Requirements = (
    getattr(_R, n, getattr(_local, n)) for n in ("DeviceLimits", "MonoSpec", "Numerics", "NumericsKind", "Requirements")
)

# The MoE fields of the HF config the presets are compiled for (DeepSeek-V3);
# moe_intermediate_size is the whole expert width, each TP rank holding 1/tp
HF_CONFIG = {
    "hidden_size": 7168,
    "n_routed_experts": 256,
    "num_experts_per_tok": 8,
    "n_group": 8,
    "topk_group": 4,
    "moe_intermediate_size": 2048,
    "n_shared_experts": 1,
    "scoring_func": "sigmoid",
    "topk_method": "noaux_tc",
    "norm_topk_prob": True,
}

# Per launch output against the normal path on the same GPU
NUMERICS = Numerics(
    NumericsKind.TOLERANCE,
    {
        # expert ids and routing weights as the normal path's routing picks them
        "moe.ids.max_abs": 0.0,
        "moe.weights.max_abs": 0.0,
        # the bf16 MoE partial against the dequantized fp32 golden
        "moe.out.max_abs": 2e-2,
        "moe.out.rel": 1e-2,
    },
)

FP8_B128, MXFP4 = "fp8_b128", "mxfp4"


def preset_for(hf_config, tp_size: int, routed_fmt: str, fuse_norm: bool = False) -> MoePreset | None:
    """The compiled preset for this model's MoE at ``tp_size`` (None: none compiled),
    with the model's routed scale and SwiGLU clamp (no clamp: +inf)."""
    get = lambda k, d=None: getattr(hf_config, k, d)  # noqa: E731
    inter = get("moe_intermediate_size", 0)
    if tp_size <= 0 or inter % tp_size:
        return None
    i = inter // tp_size
    s = i * (get("n_shared_experts", 0) or 0)
    for p in PRESETS.values():
        same = (
            p.hidden == get("hidden_size")
            and p.experts == get("n_routed_experts")
            and p.topk == get("num_experts_per_tok")
            and p.n_group == (get("n_group") or 1)
            and p.topk_group == (get("topk_group") or 1)
            and p.inter == i
            and p.shared_inter == s
            and p.routed_fmt == routed_fmt
            and (p.norm_eps is not None) == fuse_norm
        )
        if same:
            limit = get("swiglu_limit")
            return dataclasses.replace(
                p,
                routed_scale=float(get("routed_scaling_factor", p.routed_scale)),
                swiglu_limit=math.inf if limit is None else float(limit),
                norm_eps=float(get("rms_norm_eps", p.norm_eps)) if fuse_norm else None,
                renorm=bool(get("norm_topk_prob", True)),
            )
    return None


def routed_format(experts) -> str | None:
    """The routed experts' weight format off SGLang's fused-MoE module."""
    import torch

    w = getattr(experts, "w13_weight", None)
    if w is None:
        return None
    if w.dtype == torch.float8_e4m3fn and hasattr(experts, "w13_weight_scale_inv"):
        return FP8_B128
    if w.dtype in (torch.uint8, torch.float4_e2m1fn_x2) and _mx_scale_name(experts, "w13") is not None:
        return MXFP4
    return None


def _mx_scale_name(experts, which: str) -> str | None:
    """The attribute holding an MXFP4 tensor's E8M0 scales: ``*_weight_scale_inv`` where
    SGLang's gfx950 processing left them (the reference reads that name, deepseek_v41/spec.py:
    521-524), else ``*_weight_scale``."""
    for name in (f"{which}_weight_scale_inv", f"{which}_weight_scale"):
        if getattr(experts, name, None) is not None:
            return name
    return None


def _moe_layers(model) -> list[int]:
    """The layers whose MLP is a routed MoE (DeepSeek-V3: all but the first dense ones)."""
    return [i for i, layer in enumerate(model.model.layers) if hasattr(layer.mlp, "experts")]


def _weights(layer, preset: MoePreset, copies: dict, i: int):
    """Layer i's MoE tensors as the launch reads them (SGLang's, in place)."""
    import torch

    from .runner import MoeWeights

    mlp = layer.mlp
    e, sh = mlp.experts, mlp.shared_experts
    bias = mlp.gate.e_score_correction_bias
    if bias.dtype != torch.float32:  # the reference keeps an fp32 copy too (spec.py:519-521)
        bias = bias.float()
        copies["f32 router bias", i] = bias
    if preset.routed_fmt == FP8_B128:
        w13, w13_s, w2, w2_s = e.w13_weight, e.w13_weight_scale_inv, e.w2_weight, e.w2_weight_scale_inv
    else:
        # MXFP4 as SGLang holds it (deepseek_v41/spec.py:521-524 of the reference): the routed
        # experts are the router's rows (a fused shared expert or padding experts may follow
        # them in the tensors), the scales' bytes viewed as uint8, and a shuffled layout's flat
        # [E' rows][cols] scale matrix cut to the routed experts' rows. Views, not copies.
        n = mlp.gate.weight.shape[0]
        w13, w2 = e.w13_weight[:n], e.w2_weight[:n]
        w13_s = getattr(e, _mx_scale_name(e, "w13")).view(torch.uint8)
        w2_s = getattr(e, _mx_scale_name(e, "w2")).view(torch.uint8)
        if w13_s.dim() == 2:
            w13_s, w2_s = w13_s[: n * w13.shape[1]], w2_s[: n * w2.shape[1]]
        else:
            w13_s, w2_s = w13_s[:n], w2_s[:n]
    return MoeWeights(
        gate_w=mlp.gate.weight,
        bias=bias,
        w13=w13,
        w13_s=w13_s,
        w2=w2,
        w2_s=w2_s,
        sgu=sh.gate_up_proj.weight,
        sgu_s=sh.gate_up_proj.weight_scale_inv,
        sw2=sh.down_proj.weight,
        sw2_s=sh.down_proj.weight_scale_inv,
        norm=layer.post_attention_layernorm.weight if preset.norm_eps is not None else None,
    )


def weight_layout(experts) -> str:
    """The routed experts' layout as SGLang loaded them: "aiter" when its gfx950 processing
    shuffled them (the ``is_shuffled`` mark of mxfp4.py, spec.py:195 of the reference, which
    requires it: spec.py:369-370), else "row_major"."""
    return "aiter" if getattr(experts.w13_weight, "is_shuffled", False) else "row_major"


def _shape_reasons(w, preset: MoePreset, i: int) -> list[str]:
    """Each tensor against the preset's shape and dtype (no device needed)."""
    from .runner import shape_ok

    reasons = []
    for name, (shape, dtypes) in w.expected(preset).items():
        t = getattr(w, name)
        if t is None:
            reasons.append(f"layer {i}: MoE {name} missing")
        elif not shape_ok(name, t, shape) or t.dtype not in dtypes or not t.is_contiguous():
            reasons.append(f"layer {i}: MoE {name} is {tuple(t.shape)} {t.dtype}, want {shape} {dtypes[0]} contiguous")
    return reasons


def _config_disable_reasons(cfg, hf_config) -> list[str]:
    """What the requirements cannot state: the HIP library must be built and load."""
    from . import _lib

    reasons = []
    if not _lib.LIB_PATH.exists():
        reasons.append(f"needs the MoE HIP library {_lib.LIB_PATH.name} (sgl-amd-mono_amd/build.py)")
    else:
        try:
            _lib.lib()
        except (OSError, RuntimeError) as exc:
            reasons.append(f"the MoE HIP library does not load: {exc}")
    return reasons


def _model_disable_reasons(model, hf_config, copies: dict, tp_size: int | None = None, fuse_norm: bool = False) -> list[str]:
    """Why the loaded model cannot run on these kernels (empty: it can): per MoE layer,
    the routed format, its layout (row-major, or for MXFP4 SGLang's shuffled gfx950 layout,
    read in place; one layout for every layer), one shared expert, a compiled shape at this TP
    size, and every tensor's shape and dtype."""
    if tp_size is None:
        from sglang.srt.runtime_context import get_parallel  # type: ignore[import-not-found]

        tp_size = get_parallel().tp_size
    reasons = []
    layers = _moe_layers(model)
    if not layers:
        return ["no routed-MoE layers"]
    layouts = set()
    for i in layers:
        layer = model.model.layers[i]
        mlp = layer.mlp
        fmt = routed_format(mlp.experts)
        if fmt is None:
            reasons.append(f"layer {i}: routed experts neither FP8 128 x 128 nor MXFP4")
            continue
        layout = weight_layout(mlp.experts)
        layouts.add(layout)
        if layout == "aiter" and fmt != MXFP4:
            reasons.append(f"layer {i}: {fmt} MoE weights in a shuffled layout; the kernel reads those row-major")
        if getattr(mlp, "shared_experts", None) is None:
            reasons.append(f"layer {i}: needs one shared expert")
            continue
        preset = preset_for(hf_config, tp_size, fmt, fuse_norm)
        if preset is None:
            reasons.append(f"layer {i}: no compiled MoE shape for {fmt} experts at TP {tp_size}")
            continue
        reasons += _shape_reasons(_weights(layer, preset, copies, i), preset, i)
    if len(layouts) > 1:
        reasons.append("MoE layers in both the row-major and the shuffled layout")
    return reasons


class _Built:
    """One rank's MoE monokernel: the runner and each layer's weights."""

    def __init__(self, runner, layers: dict):
        self.runner, self._layers = runner, layers

    @property
    def layers(self) -> list[int]:
        return sorted(self._layers)

    def forward(self, plan, hidden_states, layer: int, out=None, topk_ids=None, topk_weights=None):
        """This rank's MoE partial of ``layer`` for the step's rows (bf16 [R, H], R <= 48),
        before the TP all-reduce; one launch on the current stream."""
        return self.runner.moe(self._layers[layer], hidden_states, out=out, topk_ids=topk_ids, topk_w=topk_weights)


def _tp_size(ctx) -> int:
    tp = getattr(ctx, "tp_size", None)
    if tp is None:
        from sglang.srt.runtime_context import get_parallel  # type: ignore[import-not-found]

        tp = get_parallel().tp_size
    return int(tp)


def _build(model, hf_config, ctx) -> _Built:
    from .runner import DEADLINE_S, MoeRunner

    tp = _tp_size(ctx)
    fuse_norm = bool(getattr(ctx, "fuse_norm", False))
    layers = {}
    preset = None
    layout = "row_major"
    for i in _moe_layers(model):
        layer = model.model.layers[i]
        layout = weight_layout(layer.mlp.experts)
        preset = preset_for(hf_config, tp, routed_format(layer.mlp.experts), fuse_norm)
        if preset is None:
            raise RuntimeError(f"layer {i}: no compiled MoE shape (model_disable_reasons refuses this model)")
        w = _weights(layer, preset, ctx.copies, i)
        w.check(preset)
        layers[i] = w
    device = next(iter(layers.values())).gate_w.device
    runner = MoeRunner(
        preset, device, max_rows=MAX_ROWS, deadline_s=getattr(ctx, "deadline_s", None) or DEADLINE_S, layout=layout
    )
    if layout == "aiter":
        _log.info("mkmoe: MoE experts read in place in SGLang's shuffled gfx950 layout")
    return _Built(runner, layers)


SPEC = MonoSpec(
    name="mkmoe_dsv3_hip",
    devices={
        "gfx950": DeviceLimits(
            widths=tuple(range(1, MAX_ROWS + 1)),
            tp_sizes=(2, 4),
            resident_blocks=BLOCKS,
        )
    },
    features=frozenset(),
    requires=Requirements(
        dtypes=frozenset({"bfloat16"}),
        server_args={"moe_runner_backend": frozenset({"auto", "triton"})},
        hf_config={**HF_CONFIG, "model_type": "deepseek_v3"},
    ),
    numerics=NUMERICS,
    model_disable_reasons=_model_disable_reasons,
    build=_build,
    api_version=1,
    config_disable_reasons=_config_disable_reasons,
)
