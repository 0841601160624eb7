"""Pin the oracle's number formats (``oracle/formats.py``) and the kernel's host-built e4m3 encoder.

Pins: the e4m3 code table against the bit-field definition and torch's
float8_e4m3fn; the encoder against brute-force nearest-value search with ties
to even; the FP4 table of the reference golden (check_ffn.py:23-40) against
the e2m1 bit fields; E8M0 against torch's float8_e8m0fnu; the MX scale codes
against their closed form; the weight quantizers against their specs.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import formats as fm


def _brute_e4m3(x: np.ndarray) -> np.ndarray:
    """Nearest e4m3 code by exhaustive search (ties: even mantissa), after the +-448 clamp."""
    tab = fm.e4m3_table()
    finite = np.where(np.isnan(tab), np.inf, tab)
    out = np.empty(x.shape, np.uint8)
    for i, v in enumerate(np.clip(x.astype(np.float64), -448, 448)):
        d = np.abs(finite - v)
        best = np.flatnonzero(d == d.min())
        if len(best) > 1:
            # tie: prefer the even mantissa; +0 and -0 tie at v == 0: keep the sign of v
            even = [c for c in best if (c & 1) == 0]
            best = even if even else best
            if v == 0 or (len(best) > 1):
                sgn = 0x80 if (np.signbit(v)) else 0
                best = [c for c in best if (c & 0x80) == sgn] or best
        out[i] = best[0]
    return out


def _edge_values() -> np.ndarray:
    tab = fm.e4m3_table()
    pos = np.sort(tab[(~np.isnan(tab)) & (tab >= 0)])
    pos = np.unique(pos)
    mids = (pos[1:] + pos[:-1]) / 2
    vals = np.concatenate([pos, mids, np.nextafter(mids.astype(np.float32), np.float32(0)),
                           np.nextafter(mids.astype(np.float32), np.float32(1000)),
                           [448.0, 449.0, 460.0, 1e6, 2.0**-10, 2.0**-12, 1e-30]])  # fmt: skip
    vals = vals.astype(np.float32)
    return np.concatenate([vals, -vals])


def test_e4m3_table_matches_torch():
    tab = fm.e4m3_table()
    t = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(tab), np.isnan(t))
    ok = ~np.isnan(tab)
    assert np.array_equal(tab[ok], t[ok].astype(np.float64))
    assert tab[0x7E] == 448.0 and tab[0x01] == 2.0**-9


def test_e4m3_encode_is_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([_edge_values(), rng.standard_normal(3000).astype(np.float32) * 30,
                        rng.standard_normal(1000).astype(np.float32) * 0.01])  # fmt: skip
    got = fm.e4m3_codes_from_f32(torch.from_numpy(x)).numpy()
    want = _brute_e4m3(x)
    # +-0 both decode to 0; compare values except keep NaN-free
    tab = fm.e4m3_table()
    assert np.array_equal(tab[got], tab[want]), x[tab[got] != tab[want]][:10]


def test_host_e4m3_encoder_matches_torch():
    from sgl_amd_mono.moe import _lib

    rng = np.random.default_rng(1)
    x = np.concatenate([_edge_values(), rng.standard_normal(200000).astype(np.float32) * 40,
                        (rng.standard_normal(200000) * 1e-3).astype(np.float32),
                        np.array([0.0, -0.0], np.float32)])  # fmt: skip
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.shape, np.uint8)
    _lib.testing_lib().mkmoe_host_e4m3_encode(x.ctypes.data, out.ctypes.data, x.size)
    want = fm.e4m3_codes_from_f32(torch.from_numpy(x)).numpy()
    assert np.array_equal(out, want), (x[out != want][:8], out[out != want][:8], want[out != want][:8])


def test_fp4_table_matches_bit_fields():
    for c, v in enumerate(fm.FP4_VALUES):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        mag = m * 0.5 if e == 0 else (1 + m / 2) * 2.0 ** (e - 1)
        assert v == (-mag if s else mag) and np.signbit(v) == bool(s)


def test_fp4_unpack_nibble_order():
    # byte 0x71: low nibble 1 -> element 0 = 0.5, high nibble 7 -> element 1 = 6.0
    v = fm.fp4_unpack(torch.tensor([[0x71, 0xF8]], dtype=torch.uint8))
    assert v.tolist() == [[0.5, 6.0, -0.0, -6.0]]


def test_e8m0_matches_torch():
    codes = torch.arange(0, 255, dtype=torch.int32).to(torch.uint8)
    want = codes.view(torch.float8_e8m0fnu).float()
    assert torch.equal(fm.e8m0_to_f32(codes), want)


def test_mx_code_closed_form_and_idempotence():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, 256, generator=g) * torch.exp2(torch.randint(-30, 20, (64, 1), generator=g).float())
    q, code = fm.mxfp8_quant(x)
    amax = x.reshape(64, -1, 32).abs().amax(-1).clamp_min(1e-10)
    s = torch.exp2(code.float() - 127)
    # the smallest power of two with amax / 448 <= 2^s (up to the fp32 product's rounding)
    assert bool(((amax * np.float32(1 / 448)) <= s).all())
    assert bool(((amax * np.float32(1 / 448)) > s / 2).all())
    y = fm.mxfp8_qdq(x)
    assert torch.equal(fm.mxfp8_qdq(y), y)


def test_group_fp8_bounds():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(8, 1024, generator=g) * 3
    q, s = fm.group_fp8_quant(x, 128)
    deq = fm.group_fp8_dequant(q, s, 128)
    qa = fm.e4m3_to_f32(q).abs().reshape(8, -1, 128)
    assert bool((qa <= 448).all()) and bool((qa.amax(-1) == 448).all())
    # e4m3 keeps 3 mantissa bits: relative error <= 2^-4 of the element (above the subnormals)
    rel = ((deq - x).abs() / x.abs().clamp_min(1e-3)).reshape(-1)
    big = x.abs().reshape(-1) > (s.repeat_interleave(128, -1).reshape(-1) * 2**-6)
    assert float(rel[big].max()) <= 2**-4 + 1e-6


def test_quant_fp8_b128_blocks():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(256, 384, generator=g) * 0.02
    q, s = fm.quant_fp8_b128(w)
    assert q.shape == (256, 384) and s.shape == (2, 3)
    blk = w.reshape(2, 128, 3, 128).abs().amax(dim=(1, 3))
    assert torch.allclose(s, blk / 448)
    deq = fm.deq_fp8_b128(q, s)
    assert float((deq - w).abs().max()) <= float(s.max()) * 16  # half an e4m3 ulp at 448 is 16


def _brute_e2m1(v: float) -> int:
    mags = np.array(fm.FP4_VALUES[:8])
    a = min(abs(v), 6.0)
    d = np.abs(mags - a)
    best = np.flatnonzero(d == d.min())
    c = best[0] if len(best) == 1 else [b for b in best if b % 2 == 0][0]
    return int(c) | (8 if v < 0 or (v == 0 and np.signbit(v)) else 0)


def test_mxfp4_quant_matches_ocp_rule():
    g = torch.Generator().manual_seed(6)
    w = torch.randn(8, 64, generator=g) * 0.02
    w[0, :32] = 0.0
    w[1, 0] = 1.0  # a block dominated by one value
    packed, code = fm.quant_mxfp4(w)
    assert packed.shape == (8, 32) and code.shape == (8, 2)
    assert int(code[0, 0]) == 0  # an all-zero block
    vals = fm.fp4_unpack(packed)
    for r in range(8):
        for b in range(2):
            blk = w[r, 32 * b : 32 * b + 32]
            amax = float(blk.abs().max())
            if amax == 0:
                continue
            x = int(np.floor(np.log2(amax))) - 2
            assert int(code[r, b]) == x + 127
            for j in range(32):
                want = fm.FP4_VALUES[_brute_e2m1(float(blk[j]) / 2.0**x)]
                assert float(vals[r, 32 * b + j]) == want
    deq = fm.deq_mxfp4(packed, code)
    assert deq.shape == w.shape


@pytest.mark.parametrize("fmt", ["fp8_b128", "mxfp4"])
def test_weight_roundtrip_error(fmt):
    from oracle.gen import quant_weight
    from oracle.moe import deq_weight

    g = torch.Generator().manual_seed(7)
    w = torch.randn(256, 512, generator=g) * 0.02
    q, s = quant_weight(w, fmt)
    rel = float((deq_weight(q, s, fmt) - w).norm() / w.norm())
    assert rel < (0.05 if fmt == "fp8_b128" else 0.2)


def test_host_library_exports():
    from sgl_amd_mono.moe import _lib

    import re
    from pathlib import Path

    L = _lib.lib()
    assert L.mkmoe_abi_version() == _lib.ABI_VERSION
    inc = Path(__file__).resolve().parents[1] / "include"

    def declared(names):
        out = set()
        for n in names:
            out |= set(re.findall(r"^(?:int|void|const char\*)\s+(mkmoe_\w+)\(", (inc / n).read_text(), re.M))
        return out

    # the product library: the drop-in surface (mkmoe.h, mkmoe_seam.h) and nothing else
    assert sorted(h.name for h in inc.glob("*.h")) == ["mkmoe.h", "mkmoe_seam.h", "mkmoe_testing.h"]
    product = declared(["mkmoe.h", "mkmoe_seam.h"])
    assert product == set(_lib.EXPORTS), product ^ set(_lib.EXPORTS)
    for name in _lib.EXPORTS:
        assert hasattr(L, name), name
    for name in _lib.TESTING_EXPORTS:
        assert not hasattr(L, name), f"{name} is a test hook, not part of the product library"
    assert ctypes.c_char_p(L.mkmoe_status_string(-2)).value
    # the test hooks' library: include/mkmoe_testing.h
    testing = declared(["mkmoe_testing.h"])
    assert testing == set(_lib.TESTING_EXPORTS), testing ^ set(_lib.TESTING_EXPORTS)
    T = _lib.testing_lib()
    for name in _lib.TESTING_EXPORTS:
        assert hasattr(T, name), name


def test_static_workspace_holds_every_compiled_shape():
    """mkmoe_forward_static's array (MKMOE_STATIC_WS_BYTES) holds the workspace of every
    compiled shape at the largest row count."""
    import re
    from pathlib import Path

    from sgl_amd_mono.moe import _lib
    from sgl_amd_mono.moe.presets import PRESETS

    header = (Path(__file__).resolve().parents[1] / "include" / "mkmoe.h").read_text()
    limit = eval(re.search(r"#define MKMOE_STATIC_WS_BYTES \((.+)\)", header).group(1).replace("u", ""))
    for p in PRESETS.values():
        n = ctypes.c_size_t()
        assert _lib.lib().mkmoe_workspace_bytes(ctypes.byref(_lib.shape_of(p, 48)), ctypes.byref(n)) == 0
        assert n.value <= limit, (p.name, n.value, limit)


def test_aiter_layout_shapes():
    """SGLang's loaded MXFP4 layout is a compiled shape of each MXFP4 preset (same workspace
    as the row-major one); the FP8 presets have none."""
    from sgl_amd_mono.moe import _lib
    from sgl_amd_mono.moe.presets import PRESETS

    L = _lib.lib()
    for p in PRESETS.values():
        if p.routed_fmt != "mxfp4":
            with pytest.raises(ValueError):
                _lib.shape_of(p, 48, "aiter")
            continue
        a, r = _lib.shape_of(p, 48, "aiter"), _lib.shape_of(p, 48)
        assert a.routed_fmt == _lib.FMT_MXFP4_AITER
        assert L.mkmoe_shape_supported(ctypes.byref(a)) == 1
        na, nr = ctypes.c_size_t(), ctypes.c_size_t()
        assert L.mkmoe_workspace_bytes(ctypes.byref(a), ctypes.byref(na)) == 0
        assert L.mkmoe_workspace_bytes(ctypes.byref(r), ctypes.byref(nr)) == 0
        assert na.value == nr.value


def test_mxfp8_vllm_rule_closed_form():
    """The "vllm" rule (check_ffn.py:99-101): the code of each 32-group is the smallest c in
    [0, 254] with fp32(max(amax, smallest normal) / 448) <= 2^(c - 127) (1 for a subnormal
    quotient, as code_ceil reads its exponent field); the values scaled by
    2^(127 - c), clamped to +-448, nearest even; quantize-dequantize is a projection."""
    from oracle import formats as fm

    g = torch.Generator().manual_seed(9)
    x = torch.randn(64, 256, generator=g) * torch.exp2(torch.randint(-30, 30, (64, 1), generator=g).float())
    x[0, :32] = 0.0
    x[1, :32] = 448.0 * 2.0**-3  # amax / 448 a power of two
    q, code = fm.mxfp8_quant(x, "vllm")
    amax = x.reshape(64, -1, 32).abs().amax(-1).clamp_min(torch.finfo(torch.float32).tiny)
    t = (amax / 448.0).double()
    for c, tv in zip(code.reshape(-1).tolist(), t.reshape(-1).tolist()):
        if tv < 2.0**-126:  # a subnormal quotient (the floored zero group): code_ceil gives 1
            assert c == 1
        else:
            assert 0 <= c <= 254 and tv <= 2.0 ** (c - 127) and tv > 2.0 ** (c - 128)
    assert code[1, 0] == 124
    d = fm.mxfp8_dequant(q, code)
    # a projection: the dequantized values quantize to themselves (the codes may drop by one
    # where a group's largest value rounded down to 224, whose quotient by 448 is a power of two)
    assert torch.equal(fm.mxfp8_qdq(d, "vllm"), d)
    qa, ca = fm.mxfp8_quant(x, "aiter")
    assert ca.min() >= 1 and code.min() == 1  # the zero group: vllm code 1 from the floor, too
    with pytest.raises(ValueError):
        fm.mxfp8_quant(x, "other")


def test_host_rejects_bad_options_before_any_device_call():
    """mkmoe_forward checks its options on the host first: a fault-injection stage the launch
    has no wait at, or a workgroup past the flag arrays, is MKMOE_ERR_ARG; valid options get
    as far as the pointer checks (MKMOE_ERR_NULL here). No GPU is touched."""
    from sgl_amd_mono.moe import _lib
    from sgl_amd_mono.moe.presets import PRESETS

    L = _lib.lib()
    shape = _lib.shape_of(PRESETS["dsv3_tp4_fp8"], 48)
    w = _lib.Weights()

    def fwd(**opts):
        o = _lib.Options(**opts)
        return L.mkmoe_forward(ctypes.byref(shape), ctypes.byref(w), None, 1, None, None, None, None, 0,
                               ctypes.byref(o), None)

    err_arg, err_null = -8, -1
    assert fwd() == err_null
    for stage in (1, 2, 3, 4, 6):
        assert fwd(fault_stage=stage, fault_workgroup=255) == err_null, stage
    assert fwd(fault_stage=5) == err_arg  # the down stage has no wait
    assert fwd(fault_stage=7) == err_arg
    assert fwd(fault_stage=-1) == err_arg
    assert fwd(fault_stage=4, fault_workgroup=256) == err_arg
    assert fwd(fault_stage=4, fault_workgroup=-1) == err_arg
    assert fwd(mfma_gate_rows=-1) == err_arg
    assert fwd(deadline_s=-1.0) == err_arg
