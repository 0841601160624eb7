"""The MoE monokernel spec on the CPU: the plugin entry point and registry, the
compiled-shape lookup, the per-output bounds, the refusal reasons on a fake
DeepSeek-V3 model (tensors on the meta device, no memory) and the weight mapping.

Follows the reference's spec unit tests (test/unit/test_deepseek_v41_spec.py),
which check the plugin registration, the numerics bounds and the model refusal
reasons with ``SimpleNamespace`` fakes of SGLang's modules.
"""

import math
from types import SimpleNamespace

import pytest
import torch

import sgl_amd_mono
from sgl_amd_mono import monospec
from sgl_amd_mono.moe import spec as mspec
from sgl_amd_mono.moe.presets import PRESETS

FP8 = torch.float8_e4m3fn
META = torch.device("meta")


def _hf(**over):
    return SimpleNamespace(**{**mspec.HF_CONFIG, "routed_scaling_factor": 2.5, "rms_norm_eps": 1e-6, **over})


def _t(shape, dtype):
    return torch.empty(shape, dtype=dtype, device=META)


def _moe_layer(tp=4, fmt="fp8_b128", e=256, h=7168, inter=2048, shuffled=False, shared=True, gate_dtype=torch.bfloat16,
               pad_experts=0):
    i = inter // tp
    n = e  # the router's experts; the fused-MoE tensors may hold pad_experts more
    if fmt == "fp8_b128":
        experts = SimpleNamespace(
            w13_weight=_t((e, 2 * i, h), FP8),
            w13_weight_scale_inv=_t((e, 2 * i // 128, h // 128), torch.float32),
            w2_weight=_t((e, h, i), FP8),
            w2_weight_scale_inv=_t((e, h // 128, i // 128), torch.float32),
        )
    else:
        e += pad_experts
        experts = SimpleNamespace(
            w13_weight=_t((e, 2 * i, h // 2), torch.uint8),
            w13_weight_scale=_t((e, 2 * i, h // 32), torch.uint8),
            w2_weight=_t((e, h, i // 2), torch.uint8),
            w2_weight_scale=_t((e, h, i // 32), torch.uint8),
        )
    if shuffled:
        experts.w13_weight = experts.w13_weight.clone()
        experts.w13_weight.is_shuffled = True
        if fmt != "fp8_b128":
            # SGLang's gfx950 processing, as the reference reads it (deepseek_v41/spec.py:
            # 521-524): fp4x2 weights, E8M0 scales as one flat [E' rows][cols] matrix a tensor,
            # under the name w13_weight_scale_inv
            experts.w13_weight = _t((e, 2 * i, h // 2), torch.float4_e2m1fn_x2)
            experts.w13_weight.is_shuffled = True
            experts.w2_weight = _t((e, h, i // 2), torch.float4_e2m1fn_x2)
            del experts.w13_weight_scale, experts.w2_weight_scale
            experts.w13_weight_scale_inv = _t((e * 2 * i, h // 32), torch.float8_e8m0fnu)
            experts.w2_weight_scale_inv = _t((e * h, i // 32), torch.float8_e8m0fnu)
    sh = None
    if shared:
        sh = SimpleNamespace(
            gate_up_proj=SimpleNamespace(weight=_t((2 * i, h), FP8), weight_scale_inv=_t((2 * i // 128, h // 128), torch.float32)),
            down_proj=SimpleNamespace(weight=_t((h, i), FP8), weight_scale_inv=_t((h // 128, i // 128), torch.float32)),
        )
    gate = SimpleNamespace(weight=_t((n, h), gate_dtype), e_score_correction_bias=_t((n,), torch.float32))
    return SimpleNamespace(
        mlp=SimpleNamespace(gate=gate, experts=experts, shared_experts=sh),
        post_attention_layernorm=SimpleNamespace(weight=_t((h,), torch.bfloat16)),
    )


def _model(layers):
    dense = SimpleNamespace(mlp=SimpleNamespace(gate_up_proj=None), post_attention_layernorm=None)
    return SimpleNamespace(model=SimpleNamespace(layers=[dense] + layers))


def test_the_plugin_registers_the_spec():
    # what SGLang's load_plugins() runs, from the sglang.srt.plugins entry point
    sgl_amd_mono.register_specs()
    reg = sgl_amd_mono.registry()
    found, why = reg.find_spec(backend=sgl_amd_mono.BACKEND, architectures=["DeepseekV3ForCausalLM"], isa="gfx950")
    assert found is mspec.SPEC, why
    none, why = reg.find_spec(backend=sgl_amd_mono.BACKEND, architectures=["DeepseekV3ForCausalLM"], isa="gfx942")
    assert none is None and "gfx942" in why
    none, why = reg.find_spec(backend="cuda", architectures=["DeepseekV3ForCausalLM"], isa="gfx950")
    assert none is None and "no spec" in why


def test_local_registry_checks_paths():
    with pytest.raises(ValueError):
        monospec.register(backend="amd", architecture="X", path="no_colon")


def test_limits_and_bounds():
    lim = mspec.SPEC.devices["gfx950"]
    assert lim.widths == tuple(range(1, 49)) and lim.tp_sizes == (2, 4) and lim.resident_blocks == 256
    # routing is exact; the partial is held to the golden's tolerance
    assert mspec.SPEC.numerics.bound("moe.ids.max_abs") == 0.0
    assert mspec.SPEC.numerics.bound("moe.weights.max_abs") == 0.0
    assert mspec.SPEC.numerics.bound("moe.out.max_abs") == 2e-2
    assert mspec.SPEC.numerics.bound("moe.out.rel") == 1e-2
    assert mspec.SPEC.api_version == monospec.MONOKERNEL_API_VERSION


def test_preset_lookup():
    hf = _hf()
    p = mspec.preset_for(hf, 4, "fp8_b128")
    assert p.name == "dsv3_tp4_fp8" and p.routed_scale == 2.5 and math.isinf(p.swiglu_limit)
    assert mspec.preset_for(hf, 4, "mxfp4").name == "dsv3_tp4_mxfp4"
    q = mspec.preset_for(_hf(swiglu_limit=10.0), 2, "mxfp4", fuse_norm=True)
    assert q.name == "dsv3_tp2_mxfp4_norm" and q.norm_eps == 1e-6 and q.swiglu_limit == 10.0
    assert mspec.preset_for(hf, 8, "fp8_b128") is None  # TP8: not compiled
    assert mspec.preset_for(hf, 2, "fp8_b128") is None
    assert mspec.preset_for(_hf(n_routed_experts=384), 4, "fp8_b128") is None  # Kimi-K2's 384 experts


def test_a_supported_model_has_no_reasons():
    for tp, fmt in ((4, "fp8_b128"), (4, "mxfp4")):
        m = _model([_moe_layer(tp, fmt), _moe_layer(tp, fmt)])
        assert mspec._model_disable_reasons(m, _hf(), {}, tp_size=tp) == []
    m = _model([_moe_layer(2, "mxfp4")])
    assert mspec._model_disable_reasons(m, _hf(), {}, tp_size=2, fuse_norm=True) == []


def test_refusal_reasons():
    hf = _hf()
    r = mspec._model_disable_reasons(_model([_moe_layer(shuffled=True)]), hf, {}, tp_size=4)
    assert any("shuffled" in x for x in r)
    r = mspec._model_disable_reasons(_model([_moe_layer(shared=False)]), hf, {}, tp_size=4)
    assert any("shared expert" in x for x in r)
    r = mspec._model_disable_reasons(_model([_moe_layer(tp=8)]), hf, {}, tp_size=8)
    assert any("no compiled MoE shape" in x for x in r)
    r = mspec._model_disable_reasons(_model([_moe_layer(gate_dtype=torch.float32)]), hf, {}, tp_size=4)
    assert any("gate_w" in x for x in r)
    layer = _moe_layer()
    layer.mlp.experts.w13_weight = _t((256, 1024, 7168), torch.bfloat16)
    r = mspec._model_disable_reasons(_model([layer]), hf, {}, tp_size=4)
    assert any("neither FP8" in x for x in r)
    assert mspec._model_disable_reasons(_model([]), hf, {}, tp_size=4) == ["no routed-MoE layers"]


def test_shuffled_mxfp4_is_read_in_place():
    """SGLang's gfx950 processing shuffles MXFP4 experts (is_shuffled, flat scale views):
    accepted and read in place in that layout (the reference requires it, spec.py:369-370);
    shuffled FP8 experts and a mix of layouts are refused."""
    hf = _hf()
    for tp, fuse in ((4, False), (2, True)):
        m = _model([_moe_layer(tp, "mxfp4", shuffled=True), _moe_layer(tp, "mxfp4", shuffled=True)])
        assert mspec._model_disable_reasons(m, hf, {}, tp_size=tp, fuse_norm=fuse) == []
        assert mspec.weight_layout(m.model.layers[1].mlp.experts) == "aiter"
    assert mspec.weight_layout(_moe_layer(4, "mxfp4").mlp.experts) == "row_major"
    mixed = _model([_moe_layer(4, "mxfp4", shuffled=True), _moe_layer(4, "mxfp4")])
    assert any("both" in x for x in mspec._model_disable_reasons(mixed, hf, {}, tp_size=4))
    layer = _moe_layer(4, "mxfp4", shuffled=True)
    ex = layer.mlp.experts
    w = mspec._weights(layer, PRESETS["dsv3_tp4_mxfp4"], {}, 1)
    assert w.w13.shape == ex.w13_weight.shape and w.w13.dtype == torch.float4_e2m1fn_x2
    assert w.w13_s.dtype == torch.uint8 and tuple(w.w13_s.shape) == (256 * 1024, 224)
    assert tuple(w.w2_s.shape) == (256 * 7168, 16)


def test_shuffled_mxfp4_with_padding_experts():
    """Fused-MoE tensors that hold more experts than the router (a fused shared expert or
    padding): the routed experts' rows are read (views, no copy), as the reference does
    (``e.w13_weight[:n]``, ``w13_weight_scale_inv.view(u8)[: n * rows]``)."""
    hf = _hf()
    layer = _moe_layer(4, "mxfp4", shuffled=True, pad_experts=1)
    ex = layer.mlp.experts
    assert ex.w13_weight.shape[0] == 257 and ex.w13_weight_scale_inv.shape[0] == 257 * 1024
    assert mspec._model_disable_reasons(_model([layer]), hf, {}, tp_size=4) == []
    w = mspec._weights(layer, PRESETS["dsv3_tp4_mxfp4"], {}, 1)
    assert w.w13.shape[0] == 256 and w.w2.shape[0] == 256
    assert tuple(w.w13_s.shape) == (256 * 1024, 224) and tuple(w.w2_s.shape) == (256 * 7168, 16)
    # row-major MXFP4 with a padding expert: its stacked tensors are cut alike
    layer = _moe_layer(4, "mxfp4", pad_experts=1)
    w = mspec._weights(layer, PRESETS["dsv3_tp4_mxfp4"], {}, 1)
    assert w.w13.shape[0] == 256 and w.w13_s.shape[0] == 256 and w.w2_s.shape[0] == 256
    assert mspec._model_disable_reasons(_model([layer]), hf, {}, tp_size=4) == []


def test_weights_read_in_place():
    layer = _moe_layer(4, "mxfp4")
    w = mspec._weights(layer, PRESETS["dsv3_tp4_mxfp4"], {}, 1)
    assert w.w13.data_ptr() == layer.mlp.experts.w13_weight.data_ptr() and w.w2_s.shape == layer.mlp.experts.w2_weight_scale.shape
    assert w.sgu is layer.mlp.shared_experts.gate_up_proj.weight and w.norm is None
    # a bf16 bias becomes an fp32 copy, kept in the copy table
    layer.mlp.gate.e_score_correction_bias = torch.zeros(256, dtype=torch.bfloat16)
    copies = {}
    w = mspec._weights(layer, PRESETS["dsv3_tp4_mxfp4"], copies, 3)
    assert w.bias.dtype == torch.float32 and copies["f32 router bias", 3] is w.bias


def test_config_reasons_name_a_missing_library(monkeypatch, tmp_path):
    from sgl_amd_mono.moe import _lib

    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libmkmoe.so")
    r = mspec._config_disable_reasons(None, _hf())
    assert r and "libmkmoe.so" in r[0]
