"""The FFN monokernel spec of DeepSeek-V4.1 (``DeepseekV4ForCausalLM``) on gfx950, backend ``amd``.

It keeps the reference spec's surface for the FFN path (``sgl_amd_mono/deepseek_v41/spec.py``):
a ``MonoSpec`` with the model's HF config as a requirement (``deepseek_v41/__init__.py:11-37``),
the gfx950 ``DeviceLimits`` (decode widths 1..48, a persistent grid of 256 resident workgroups:
``spec.py:959-967``), the per-output ``Numerics`` bounds, a ``load_tensor`` hook that keeps
this rank's shard of each layer's FP8 shared expert as the checkpoint holds it
(``spec.py:428-445``, ``_CKPT_SHARED`` at ``:67-72``), refusal reasons for the loaded model
(``:352-404``: the experts in aiter's shuffle, the shared expert seen), the FFN weights read in
place off SGLang's modules (``:484-530``) and a ``build`` whose forward runs one layer's FFN.

The TP 4 share (the rank's 576 routed columns padded to 640) and the TP 2 share (1152 columns)
are compiled, the reference's TP sizes (``spec.py:959-967``). The forward is the FFN's seam and
MoE block (``moe/ffn.py``); the attention TP reduce before it and the all-reduce after it need
peers.
"""

from __future__ import annotations

import logging
import re

from .. import monospec as _local
from .ffn import FfnRunner, FfnWeights
from .presets import PRESETS

MAX_ROWS = 48
BLOCKS = 256
# the compiled share of each TP size
PRESET_BY_TP = {2: "v41_tp2", 4: "v41_tp4"}
TP_SIZES = tuple(sorted(PRESET_BY_TP))
_log = logging.getLogger(__name__)


def _reg():
    from .. import registry

    return registry()


_R = _reg()
DeviceLimits, MonoSpec, Numerics, NumericsKind, Requirements = (
    getattr(_R, n, getattr(_local, n)) for n in ("DeviceLimits", "MonoSpec", "Numerics", "NumericsKind", "Requirements")
)

# The HF config fields the FFN path builds in (DeepSeek-V4.1-Flash; the reference's HF_CONFIG
# without its attention and indexer fields)
HF_CONFIG = dict(
    hidden_size=5120,
    moe_intermediate_size=2304,
    n_routed_experts=384,
    num_experts_per_tok=6,
    n_shared_experts=1,
    routed_scaling_factor=1.5,
    scoring_func="sqrtsoftplus",
    norm_topk_prob=True,
    topk_method="noaux_tc",
    hidden_act="silu",
    swiglu_limit=10.0,
    hc_mult=4,
    hc_sinkhorn_iters=20,
    hc_eps=1e-6,
    rms_norm_eps=1e-20,
)

# Per launch output against the normal path on the same GPU. The reference test's weights give
# outputs up to |out| ~ 30, so the partial is held to relative bounds (its own for this shape,
# ``spec.py:287-318``: the cosine of ``ffn.moe``)
NUMERICS = Numerics(
    NumericsKind.TOLERANCE,
    {
        "moe.ids.max_abs": 0.0,
        "moe.weights.max_abs": 0.0,
        "moe.out.rel": 1e-2,
        "moe.out.cosine": 0.9999,
    },
)

# the shared expert's projections, and the checkpoint names of their FP8 tensors as the model
# loader reads them (``layers.{i}.ffn.shared_experts.{w1,w2,w3}.{weight,scale}``; ``mtp.*``
# layers do not match)
SHARED = ("gate_proj", "up_proj", "down_proj")
CKPT_SHARED = re.compile(r"layers\.(?P<i>\d+)\.ffn\.shared_experts\.(?P<w>w[123])\.(?P<kind>weight|scale)")
CKPT_PROJ = {"w1": "gate_proj", "w3": "up_proj", "w2": "down_proj"}


def _parallel():
    """(tp_rank, tp_size) of this process (SGLang's runtime context)."""
    from sglang.srt.runtime_context import get_parallel  # type: ignore[import-not-found]

    p = get_parallel()
    return p.tp_rank, p.tp_size


def _moe_layers(model) -> list[int]:
    return [i for i, layer in enumerate(model.model.layers) if hasattr(getattr(layer, "mlp", None), "experts")]


def load_tensor(copies: dict, model, name: str, tensor, parallel=None) -> None:
    """Keep this rank's shard of a MoE layer's FP8 shared-expert tensor by its checkpoint name:
    gate and up split on their rows (the intermediate), down on its columns. ``parallel``:
    (tp_rank, tp_size), else SGLang's."""
    import torch

    m = CKPT_SHARED.fullmatch(name)
    if m is None:
        return
    i, proj = int(m["i"]), CKPT_PROJ[m["w"]]
    if i >= len(model.model.layers) or i not in _moe_layers(model):
        return
    rank, tp = _parallel() if parallel is None else parallel
    dim = 1 if proj == "down_proj" else 0
    t = tensor.view(torch.uint8)
    n = t.shape[dim] // tp
    dev = torch.cuda.current_device() if torch.cuda.is_available() else t.device
    copies["shared expert fp8", i, proj, m["kind"]] = t.narrow(dim, rank * n, n).to(dev).contiguous()


def _shared_seen(copies: dict, i: int) -> bool:
    return all(("shared expert fp8", i, p, k) in copies for p in SHARED for k in ("weight", "scale")) or all(
        ("shared expert fp8", i, p, k) in copies for p in ("gate_up", "down_proj") for k in ("weight", "scale")
    )


def _weights(layer, copies: dict, i: int) -> FfnWeights:
    """Layer i's FFN tensors as the launches read them: SGLang's in place, the shared expert
    from the checkpoint's shards (gate and up joined once into one tensor)."""
    import torch

    e, moe = layer.mlp.experts, layer.mlp
    n = moe.gate.weight.shape[0]  # the routed experts, before a fused shared one
    u8, e4m3 = torch.uint8, torch.float8_e4m3fn

    def gate_up(kind):
        key = ("shared expert fp8", i, "gate_up", kind)
        if key not in copies:
            copies[key] = torch.cat([copies.pop(("shared expert fp8", i, q, kind)) for q in SHARED[:2]])
        return copies[key]

    def down(kind):
        return copies["shared expert fp8", i, "down_proj", kind]

    bias = moe.gate.e_score_correction_bias
    if bias.dtype != torch.float32:  # the reference keeps an fp32 copy too (spec.py:518-520)
        bias = copies["f32 router bias", i] = bias.float()
    return FfnWeights(
        hc_ffn_fn=layer.hc_ffn_fn,
        hc_ffn_scale=layer.hc_ffn_scale,
        hc_ffn_base=layer.hc_ffn_base,
        ffn_norm=layer.post_attention_layernorm.weight,
        gate_w=moe.gate.weight,
        bias=bias,
        w13=e.w13_weight[:n],
        w13_s=e.w13_weight_scale_inv.view(u8)[: n * e.w13_weight.shape[1]],
        w2=e.w2_weight[:n],
        w2_s=e.w2_weight_scale_inv.view(u8)[: n * e.w2_weight.shape[1]],
        sgu=gate_up("weight").view(e4m3),
        sgu_s=gate_up("scale"),
        sw2=down("weight").view(e4m3),
        sw2_s=down("scale"),
    )


def _shape_reasons(w: FfnWeights, i: int, preset) -> list[str]:
    """Each MoE tensor against the compiled shape (no device needed)."""
    from .runner import shape_ok

    reasons = []
    for name, (shape, dtypes) in w.moe().expected(preset).items():
        t = getattr(w, name)
        if t is None:
            reasons.append(f"layer {i}: MoE {name} missing")
        elif not shape_ok(name, t, shape) or t.dtype not in dtypes or not t.is_contiguous():
            reasons.append(f"layer {i}: MoE {name} is {tuple(t.shape)} {t.dtype}, want {shape} {dtypes[0]} contiguous")
    return reasons


def _config_disable_reasons(cfg, hf_config) -> list[str]:
    from . import _lib

    if not _lib.LIB_PATH.exists():
        return [f"needs the MoE HIP library {_lib.LIB_PATH.name} (sgl-amd-mono_amd/build.py)"]
    try:
        _lib.lib()
    except (OSError, RuntimeError) as exc:
        return [f"the MoE HIP library does not load: {exc}"]
    return []


def _model_disable_reasons(model, hf_config, copies: dict, tp_size: int | None = None) -> list[str]:
    """Why the loaded model cannot run on these kernels (empty: it can): the TP size, and per
    MoE layer the experts in aiter's shuffle (the layout the kernel reads), the shared expert's
    FP8 shards seen by ``load_tensor``, and every tensor's shape and dtype."""
    if tp_size is None:
        tp_size = _parallel()[1]
    if tp_size not in TP_SIZES:
        return [f"the V4.1 FFN is compiled for TP {TP_SIZES} (this is TP {tp_size})"]
    layers = _moe_layers(model)
    if not layers:
        return ["no routed-MoE layers"]
    reasons = []
    for i in layers:
        layer = model.model.layers[i]
        if not getattr(layer.mlp.experts.w13_weight, "is_shuffled", False):
            reasons.append(f"layer {i}: MoE weights not in aiter's shuffle")
            continue
        if not _shared_seen(copies, i):
            reasons.append(f"layer {i}: the shared expert's FP8 tensors were not seen at load")
            continue
        reasons += _shape_reasons(_weights(layer, copies, i), i, PRESETS[PRESET_BY_TP[tp_size]])
    return reasons


class _Built:
    """One rank's V4.1 FFN monokernel: the runner and each layer's weights."""

    def __init__(self, runner: FfnRunner, layers: dict):
        self.runner, self._layers = runner, layers

    @property
    def layers(self) -> list[int]:
        return sorted(self._layers)

    def forward(self, plan, part, residual, post_mix, res_mix, pre_mix, layer: int, outs=None):
        """Layer ``layer``'s FFN for the step's rows: (out, res_out, post_out, comb_out,
        pre_out), ``DSV41MonoRunner.ffn``'s outputs; launches on the current stream."""
        return self.runner.ffn(self._layers[layer], part, residual, post_mix, res_mix, pre_mix, outs=outs)


def _build(model, hf_config, ctx) -> _Built:
    from .runner import DEADLINE_S

    tp = getattr(ctx, "tp_size", None)
    preset = PRESETS[PRESET_BY_TP[int(_parallel()[1] if tp is None else tp)]]
    layers = {}
    for i in _moe_layers(model):
        w = _weights(model.model.layers[i], ctx.copies, i)
        w.check(preset)
        layers[i] = w
    device = next(iter(layers.values())).gate_w.device
    runner = FfnRunner(
        preset, device, norm_eps=float(getattr(hf_config, "rms_norm_eps", HF_CONFIG["rms_norm_eps"])),
        max_rows=MAX_ROWS, deadline_s=getattr(ctx, "deadline_s", None) or DEADLINE_S,
    )  # fmt: skip
    _log.info("mkmoe: V4.1 FFN on %d layers, experts read in place in SGLang's shuffled gfx950 layout", len(layers))
    return _Built(runner, layers)


SPEC = MonoSpec(
    name="mkmoe_dsv41_ffn_hip",
    devices={"gfx950": DeviceLimits(widths=tuple(range(1, MAX_ROWS + 1)), tp_sizes=TP_SIZES, resident_blocks=BLOCKS)},
    features=frozenset(),
    requires=Requirements(
        dtypes=frozenset({"bfloat16"}),
        server_args={"moe_runner_backend": frozenset({"auto", "aiter"})},
        hf_config={**HF_CONFIG, "model_type": "deepseek_v41"},
        env={
            # the MXFP4 experts in aiter's gate / up interleaved layout (spec.py:986-990)
            "SGLANG_DSV4_FP4_EXPERTS": True,
            "SGLANG_DSV4_FP4_DEQUANT": False,
            "SGLANG_USE_AITER_MOE_GU_ITLV": True,
        },
    ),
    numerics=NUMERICS,
    model_disable_reasons=_model_disable_reasons,
    build=_build,
    api_version=1,
    config_disable_reasons=_config_disable_reasons,
    load_tensor=load_tensor,
)
