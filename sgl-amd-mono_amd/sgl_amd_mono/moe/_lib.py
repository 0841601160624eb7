"""ctypes binding of the in-tree HIP library (the C ABI of ``include/mkmoe.h`` and
``include/mkmoe_seam.h``), and of its test hooks' library (``include/mkmoe_testing.h``).

The library is loaded from this directory only. There is no fallback: a missing
or unloadable library raises, so a GPU run can never silently take another path.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmkmoe.so"
# the test hooks (hardware converts, the scaled MFMA, host builds of the exact arithmetic)
TESTING_LIB_PATH = Path(__file__).resolve().parent / "libmkmoe_testing.so"
# the diagnostic build with the persistent launch's phase stamps (build.py --timeline)
TIMELINE_LIB_PATH = Path(__file__).resolve().parent / "libmkmoe_tl.so"
TL_SLOTS = 32
TL_NAMES = (
    "start", "A done", "A arrived", "routed", "union", "A awaited", "gate_up", "C arrived",
    "C awaited", "D routed", "D shared", "end", "gate_up first unit", "gate_up wait", "down wait",
    "gate_up units", "gate_up fetch", "gate_up mfma", "gate_up sync", "gate_up emit", "gate_up sync2",
    "down quant", "down mfma", "parts landed", "scores", "Q done", "Q awaited", "down fetch", "down issue",
    "down units", "down first unit", "down barrier",
)  # fmt: skip

ABI_VERSION = 6  # MKMOE_ABI_VERSION of include/mkmoe.h that this binding follows
FMT_FP8_B128 = 1
FMT_MXFP4 = 2
FMT_MXFP4_AITER = 3  # MXFP4 in SGLang's loaded gfx950 layout (aiter's shuffles), read in place
FMT_FP8_MX32 = 4  # FP8 with E8M0 32 x 32 scales (the V4.1 shared expert)
SCORE_CODES = {"sigmoid": 0, "sqrt_softplus": 1}  # MKMOE_SCORE_*
ERRW_WORDS = 8
ERRW_CODE, ERRW_STAGE, ERRW_BLOCK, ERRW_COUNT, ERRW_FAULT = 0, 1, 2, 3, 4
REGIONS = {
    "x_normed": 0,
    "x_codes": 1,
    "x_scales": 2,
    "x_codes_shared": 3,
    "x_scales_shared": 4,
    "router_parts": 5,
    "ids": 6,
    "weights": 7,
    "shared_mid": 8,
    "mid": 9,
    "router_parts_polled": 10,
    "timeline": 11,
    "mid_codes": 12,
    "mid_scales": 13,
    "shared_mid_codes": 14,
    "shared_mid_scales": 15,
}
STAGES = {1: "norm", 2: "router + quantize", 3: "route", 4: "gate_up (routed + shared)", 5: "down (shared + routed) + combine", 6: "quantize the intermediates"}

# every symbol include/mkmoe.h and include/mkmoe_seam.h declare
EXPORTS = (
    "mkmoe_abi_version",
    "mkmoe_shape_supported",
    "mkmoe_workspace_bytes",
    "mkmoe_init_workspace",
    "mkmoe_forward",
    "mkmoe_forward_staged",
    "mkmoe_forward_static",
    "mkmoe_read_errors",
    "mkmoe_clear_errors",
    "mkmoe_workspace_region",
    "mkmoe_status_string",
    "mkmoe_seam_workspace_bytes",
    "mkmoe_seam_forward",
    "mkmoe_seam_gate",
)
# every symbol include/mkmoe_testing.h declares (libmkmoe_testing.so)
TESTING_EXPORTS = (
    "mkmoe_device_decode",
    "mkmoe_device_e4m3_sweep",
    "mkmoe_device_mfma_scaled",
    "mkmoe_host_e4m3_encode",
    "mkmoe_host_sigmoid",
    "mkmoe_host_sqrt_softplus",
    "mkmoe_host_topk",
)


class Shape(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int32),
        ("experts", ctypes.c_int32),
        ("topk", ctypes.c_int32),
        ("n_group", ctypes.c_int32),
        ("topk_group", ctypes.c_int32),
        ("inter", ctypes.c_int32),
        ("shared_inter", ctypes.c_int32),
        ("routed_fmt", ctypes.c_int32),
        ("router_parts", ctypes.c_int32),
        ("renorm", ctypes.c_int32),
        ("use_norm", ctypes.c_int32),
        ("max_rows", ctypes.c_int32),
        ("routed_scale", ctypes.c_float),
        ("swiglu_limit", ctypes.c_float),
        ("norm_eps", ctypes.c_float),
        ("scoring", ctypes.c_int32),
        ("shared_fmt", ctypes.c_int32),
    ]


class Options(ctypes.Structure):
    """``mkmoe_options``: a field left 0 takes the library's default."""

    _fields_ = [
        ("deadline_s", ctypes.c_double),
        ("mfma_gate_rows", ctypes.c_int32),
        ("mfma_down_rows", ctypes.c_int32),
        ("mxfp4_scaled_rows", ctypes.c_int32),
        ("mxfp4_scaled_down_rows", ctypes.c_int32),
        ("fault_stage", ctypes.c_int32),  # test fault injection: a stage code (STAGES), 0: none
        ("fault_workgroup", ctypes.c_int32),
    ]


class Weights(ctypes.Structure):
    _fields_ = [
        (n, ctypes.c_void_p)
        for n in ("gate_w", "bias", "w13", "w13_s", "w2", "w2_s", "sgu", "sgu_s", "sw2", "sw2_s", "norm")
    ]


class SeamIO(ctypes.Structure):
    """mkmoe_seam_io of include/mkmoe_seam.h."""

    _fields_ = [
        ("hidden", ctypes.c_int32),
        ("tokens", ctypes.c_int32),
        ("norm_eps", ctypes.c_float),
        ("flags", ctypes.c_int32),
    ] + [
        (n, ctypes.c_void_p)
        for n in (
            "a", "res", "post", "comb", "pre", "hc_fn", "hc_scale", "hc_base", "norm_w",
            "res_out", "normed", "post_out", "comb_out", "pre_out",
        )
    ]  # fmt: skip


SEAM_HC = 4
SEAM_MIX = 24
SEAM_HIDDEN = 5120
SEAM_MAX_TOKENS = 64
SEAM_GATE_LATER = 1

_lib = None


def use_timeline_build() -> None:
    """Load the diagnostic timeline build instead of the product library (before the first
    call of ``lib()``; raises when it has not been built)."""
    global LIB_PATH
    if _lib is not None and LIB_PATH != TIMELINE_LIB_PATH:
        raise RuntimeError("mkmoe: the product library is already loaded")
    LIB_PATH = TIMELINE_LIB_PATH


def lib() -> ctypes.CDLL:
    """The loaded library; raises when it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python sgl-amd-mono_amd/build.py` "
                "(the MoE block has no other implementation)"
            )
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i32, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t
        sp, wp, op = ctypes.POINTER(Shape), ctypes.POINTER(Weights), ctypes.POINTER(Options)
        L.mkmoe_abi_version.restype = ctypes.c_int
        L.mkmoe_shape_supported.argtypes = [sp]
        L.mkmoe_workspace_bytes.argtypes = [sp, ctypes.POINTER(sz)]
        L.mkmoe_init_workspace.argtypes = [sp, vp, sz, vp]
        fwd = [sp, wp, vp, i32, vp, vp, vp, vp, sz, op, vp]
        L.mkmoe_forward.argtypes = fwd
        L.mkmoe_forward_staged.argtypes = fwd
        L.mkmoe_forward_static.argtypes = [sp, wp, vp, i32, vp, vp, vp, op, vp]
        L.mkmoe_read_errors.argtypes = [vp, ctypes.POINTER(i32), i32, vp]
        L.mkmoe_clear_errors.argtypes = [sp, vp, sz, vp]
        L.mkmoe_workspace_region.argtypes = [sp, i32, ctypes.POINTER(sz), ctypes.POINTER(sz)]
        L.mkmoe_status_string.argtypes = [ctypes.c_int]
        L.mkmoe_status_string.restype = ctypes.c_char_p
        L.mkmoe_seam_workspace_bytes.argtypes = [i32, i32, ctypes.POINTER(sz)]
        L.mkmoe_seam_forward.argtypes = [ctypes.POINTER(SeamIO), vp, sz, vp]
        L.mkmoe_seam_gate.argtypes = [ctypes.POINTER(SeamIO), vp, sz, vp]
        if L.mkmoe_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"{LIB_PATH} has ABI {L.mkmoe_abi_version()}, this binding wants {ABI_VERSION}: rebuild it"
            )
        _lib = L
    return _lib


_testing_lib = None


def testing_lib() -> ctypes.CDLL:
    """The test hooks' library (include/mkmoe_testing.h); raises when it has not been built."""
    global _testing_lib
    if _testing_lib is None:
        if not TESTING_LIB_PATH.exists():
            raise RuntimeError(f"{TESTING_LIB_PATH} is missing: build it with `python sgl-amd-mono_amd/build.py`")
        T = ctypes.CDLL(str(TESTING_LIB_PATH))
        vp, i32 = ctypes.c_void_p, ctypes.c_int32
        T.mkmoe_device_decode.argtypes = [vp, vp, vp, i32, vp]
        T.mkmoe_device_e4m3_sweep.argtypes = [ctypes.c_uint32, ctypes.c_uint32, vp, vp, vp]
        T.mkmoe_device_mfma_scaled.argtypes = [vp, vp, vp, vp, vp, i32, i32, vp]
        for name in ("mkmoe_host_e4m3_encode", "mkmoe_host_sigmoid", "mkmoe_host_sqrt_softplus"):
            getattr(T, name).argtypes = [vp, vp, ctypes.c_int64]
            getattr(T, name).restype = None
        T.mkmoe_host_topk.argtypes = [ctypes.POINTER(Shape), vp, vp, vp, vp]
        T.mkmoe_host_topk.restype = None
        _testing_lib = T
    return _testing_lib


def status_string(rc: int) -> str:
    return lib().mkmoe_status_string(rc).decode()


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: {status_string(rc)} ({rc})")


LAYOUTS = ("row_major", "aiter")


def shape_of(preset, max_rows: int | None = None, layout: str | None = None) -> Shape:
    """The C shape of a ``presets.MoePreset`` whose routed experts are in ``layout``: row-major
    (include/mkmoe.h), or SGLang's loaded gfx950 layout of MXFP4 experts ("aiter"); by default
    the preset's own (aiter for a preset compiled for that layout alone, else row-major)."""
    from .presets import FMT_CODES

    if layout is None:
        layout = "aiter" if preset.aiter_only else "row_major"

    if layout not in LAYOUTS:
        raise ValueError(f"layout {layout!r}: one of {LAYOUTS}")
    if layout == "aiter" and preset.routed_fmt != "mxfp4":
        raise ValueError("the aiter layout is MXFP4's")
    if preset.aiter_only and layout != "aiter":
        raise ValueError(f"{preset.name} is compiled for SGLang's loaded (aiter) layout alone")

    return Shape(
        hidden=preset.hidden,
        experts=preset.experts,
        topk=preset.topk,
        n_group=preset.n_group,
        topk_group=preset.topk_group,
        inter=preset.inter,
        shared_inter=preset.shared_inter,
        routed_fmt=FMT_MXFP4_AITER if layout == "aiter" else FMT_CODES[preset.routed_fmt],
        router_parts=preset.router_parts,
        renorm=1 if preset.renorm else 0,
        use_norm=0 if preset.norm_eps is None else 1,
        max_rows=preset.max_rows if max_rows is None else max_rows,
        routed_scale=preset.routed_scale,
        swiglu_limit=preset.swiglu_limit,
        norm_eps=0.0 if preset.norm_eps is None else preset.norm_eps,
        scoring=SCORE_CODES[preset.scoring],
        shared_fmt=FMT_CODES[preset.shared_fmt],
    )
