"""The DeepSeek-V4.1 FFN spec on the CPU: its registration, limits and bounds, the
checkpoint hook that keeps this rank's shard of the FP8 shared expert, the weight mapping off
SGLang's modules and the refusal reasons, on a fake model (tensors on the meta device).

Follows the reference's spec unit tests (test/unit/test_deepseek_v41_spec.py), which check the
plugin registration and the refusal reasons with ``SimpleNamespace`` fakes of SGLang's modules.
"""

from types import SimpleNamespace

import pytest
import torch

import sgl_amd_mono
from sgl_amd_mono.moe import spec_v41 as sv
from sgl_amd_mono.moe.presets import PRESETS

META = torch.device("meta")
FP4X2, E8M0, FP8 = torch.float4_e2m1fn_x2, torch.float8_e8m0fnu, torch.float8_e4m3fn
H, E, S_FULL = 5120, 384, 2304
I_PAD = {4: 640, 2: 1152}  # the loader's width of a rank's share (TP 4: 576 padded)
W2_COLS = {4: 24, 2: 40}  # w2's E8M0 columns, padded to a multiple of 8


def _t(shape, dtype):
    return torch.empty(shape, dtype=dtype, device=META)


def _layer(shuffled=True, pad_experts=0, experts=E, tp=4):
    e = experts + pad_experts
    i = I_PAD[tp]
    w13 = _t((e, 2 * i, H // 2), FP4X2)
    w13.is_shuffled = shuffled
    ex = SimpleNamespace(
        w13_weight=w13,
        w13_weight_scale_inv=_t((e * 2 * i, H // 32), E8M0),
        w2_weight=_t((e, H, i // 2), FP4X2),
        w2_weight_scale_inv=_t((e * H, W2_COLS[tp]), E8M0),
    )
    gate = SimpleNamespace(weight=_t((experts, H), torch.bfloat16), e_score_correction_bias=_t((experts,), torch.bfloat16))
    return SimpleNamespace(
        mlp=SimpleNamespace(gate=gate, experts=ex),
        hc_ffn_fn=_t((24, 4 * H), torch.float32),
        hc_ffn_scale=_t((3,), torch.float32),
        hc_ffn_base=_t((24,), torch.float32),
        post_attention_layernorm=SimpleNamespace(weight=_t((H,), torch.bfloat16)),
    )


def _model(layers):
    return SimpleNamespace(model=SimpleNamespace(layers=layers), config=SimpleNamespace(**sv.HF_CONFIG))


def _load_shared(copies, model, i, tp=4, rank=1):
    """The checkpoint's shared-expert tensors of layer i through the hook."""
    for w, shape in (("w1", (S_FULL, H)), ("w3", (S_FULL, H)), ("w2", (H, S_FULL))):
        sv.load_tensor(copies, model, f"layers.{i}.ffn.shared_experts.{w}.weight", _t(shape, FP8), (rank, tp))
        sv.load_tensor(copies, model, f"layers.{i}.ffn.shared_experts.{w}.scale",
                       _t((shape[0] // 32, shape[1] // 32), E8M0), (rank, tp))  # fmt: skip


def test_the_plugin_registers_the_v41_spec():
    sgl_amd_mono.register_specs()
    reg = sgl_amd_mono.registry()
    found, why = reg.find_spec(backend=sgl_amd_mono.BACKEND, architectures=["DeepseekV4ForCausalLM"], isa="gfx950")
    assert found is sv.SPEC, why
    none, why = reg.find_spec(backend=sgl_amd_mono.BACKEND, architectures=["DeepseekV4ForCausalLM"], isa="gfx942")
    assert none is None and "gfx942" in why


def test_limits_bounds_and_config():
    lim = sv.SPEC.devices["gfx950"]
    assert lim.widths == tuple(range(1, 49)) and lim.tp_sizes == (2, 4) and lim.resident_blocks == 256
    assert sv.SPEC.numerics.bound("moe.ids.max_abs") == 0.0 and sv.SPEC.numerics.bound("moe.out.cosine") == 0.9999
    req = sv.SPEC.requires.hf_config
    # the compiled presets are the config's TP 4 and TP 2 shares
    for tp, name in sv.PRESET_BY_TP.items():
        p = PRESETS[name]
        assert req["model_type"] == "deepseek_v41" and req["hidden_size"] == p.hidden
        assert req["n_routed_experts"] == p.experts and req["num_experts_per_tok"] == p.topk
        assert req["moe_intermediate_size"] // tp == (p.inter_real or p.inter) == p.shared_inter
        assert p.inter % 128 == 0 and p.inter - (p.inter_real or p.inter) < 128  # padded to 128 (dims.py)
        assert req["routed_scaling_factor"] == p.routed_scale and req["swiglu_limit"] == p.swiglu_limit
        assert req["scoring_func"] == "sqrtsoftplus" and p.scoring == "sqrt_softplus"
    assert sv.SPEC.load_tensor is sv.load_tensor


def test_load_tensor_keeps_the_rank_shard():
    """gate (w1) and up (w3) split on rows, down (w2) on columns; other names are ignored."""
    model = _model([_layer(), _layer()])
    copies = {}
    full = torch.arange(8 * 12, dtype=torch.uint8).reshape(8, 12)
    sv.load_tensor(copies, model, "layers.1.ffn.shared_experts.w1.weight", full, (1, 4))
    sv.load_tensor(copies, model, "layers.1.ffn.shared_experts.w2.weight", full, (2, 4))
    sv.load_tensor(copies, model, "mtp.0.ffn.shared_experts.w1.weight", full, (0, 4))
    sv.load_tensor(copies, model, "layers.9.ffn.shared_experts.w1.weight", full, (0, 4))  # no such layer
    sv.load_tensor(copies, model, "layers.1.ffn.experts.0.w1.weight", full, (0, 4))
    assert set(copies) == {("shared expert fp8", 1, "gate_proj", "weight"), ("shared expert fp8", 1, "down_proj", "weight")}
    assert torch.equal(copies["shared expert fp8", 1, "gate_proj", "weight"], full[2:4])
    d = copies["shared expert fp8", 1, "down_proj", "weight"]
    assert torch.equal(d, full[:, 6:9]) and d.is_contiguous()


def test_weights_mapping_and_a_loadable_model():
    layers = [_layer(pad_experts=16), _layer()]
    model = _model(layers)
    copies = {}
    for i in range(2):
        _load_shared(copies, model, i)
    assert sv._model_disable_reasons(model, model.config, copies, tp_size=4) == []
    w = sv._weights(layers[0], copies, 0)
    # the routed experts' rows only (padding experts follow them), the scales' bytes as uint8
    assert w.w13.shape == (E, 2 * I_PAD[4], H // 2) and w.w13_s.shape == (E * 2 * I_PAD[4], H // 32)
    assert w.w13_s.dtype == torch.uint8 and w.w2_s.shape == (E * H, 24)
    # the shared expert: gate and up joined (rows), the rank's columns of down, E8M0 32 x 32
    assert w.sgu.shape == (1152, H) and w.sgu.dtype == FP8 and w.sgu_s.shape == (36, 160)
    assert w.sw2.shape == (H, 576) and w.sw2_s.shape == (160, 18)
    assert w.bias.dtype == torch.float32 and ("f32 router bias", 0) in copies
    # the joined tensor is kept (its parts released), and a second mapping reuses it
    assert ("shared expert fp8", 0, "gate_up", "weight") in copies
    assert ("shared expert fp8", 0, "gate_proj", "weight") not in copies
    assert sv._weights(layers[0], copies, 0).sgu.shape == w.sgu.shape


def test_tp2_model_maps_and_loads():
    """TP 2: the rank's 1152 columns of every expert and of the shared expert."""
    layers = [_layer(tp=2), _layer(tp=2, pad_experts=8)]
    model = _model(layers)
    copies = {}
    for i in range(2):
        _load_shared(copies, model, i, tp=2, rank=0)
    assert sv._model_disable_reasons(model, model.config, copies, tp_size=2) == []
    w = sv._weights(layers[1], copies, 1)
    assert w.sgu.shape == (2304, H) and w.sgu_s.shape == (72, 160) and w.sw2.shape == (H, 1152)
    assert w.w2_s.shape == (E * H, 40)
    # TP 4's tensors at TP 2 are refused by shape
    m4 = _model([_layer()])
    c4 = {}
    _load_shared(c4, m4, 0, tp=4, rank=0)
    assert any("w13" in r for r in sv._model_disable_reasons(m4, m4.config, c4, tp_size=2))


def test_refusal_reasons():
    good = _layer()
    model = _model([good, _layer(shuffled=False), _layer(), _layer(experts=256)])
    copies = {}
    for i in (0, 1, 3):
        _load_shared(copies, model, i)
    why = sv._model_disable_reasons(model, model.config, copies, tp_size=4)
    assert any("layer 1" in r and "shuffle" in r for r in why)
    assert any("layer 2" in r and "shared expert" in r for r in why)
    assert any("layer 3" in r and "gate_w" in r for r in why)
    assert not any("layer 0" in r for r in why)
    assert "TP (2, 4)" in sv._model_disable_reasons(model, model.config, copies, tp_size=8)[0]


def test_ffn_runner_refuses_another_hidden_size():
    from sgl_amd_mono.moe.ffn import FfnRunner

    with pytest.raises(RuntimeError, match="hidden 5120"):
        FfnRunner("dsv3_tp4_fp8", "cpu")
