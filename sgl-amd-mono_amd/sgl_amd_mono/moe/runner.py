"""Host runner of the decode MoE block: weights contract, workspace, and the call.

Mirrors the reference's host side for this path:
- ``MoeWeights`` / ``.check`` follow ``FFNWeights`` / ``.check``
  (``sgl_amd_mono/deepseek_v41/gfx950/runner.py:130-168``): the MoE tensors of
  one layer on this rank, read in place, with shapes, dtypes, contiguity and
  device checked before the first launch (a ``RuntimeError`` naming the tensor).
- ``MoeRunner.moe`` follows ``DSV41MonoRunner.ffn`` (``runner.py:436-510``):
  row checks in the manner of ``check_rows`` (``runner.py:94-105``), optional
  caller-provided outputs, one launch on the current stream, no host sync.
- The workspace replaces the runner's per-width scratch and epoch buffers
  (``runner.py:339-350``); it is allocated once, never inside a graph capture
  (``no_capture``, ``runner.py:122-127``).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, fields

import torch

from . import _lib
from .presets import PRESETS, MoePreset

FP8 = torch.float8_e4m3fn
FP4X2 = torch.float4_e2m1fn_x2
E8M0 = torch.float8_e8m0fnu


def no_capture(what: str) -> None:
    """Raise inside a graph capture: allocations and workspace set-up run eagerly."""
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError(f"mkmoe: {what} first reached inside a graph capture")


def _bytes_dtype(t: torch.Tensor, allowed: tuple) -> bool:
    return t.dtype in allowed


def shape_ok(name: str, t: torch.Tensor, shape: tuple) -> bool:
    """``t`` has ``shape``, or (MXFP4 scales) the same bytes as SGLang holds them: one
    [E * rows][cols] matrix a tensor (``deepseek_v41/gfx950/runner.py:169-172``)."""
    if tuple(t.shape) == shape:
        return True
    return name in ("w13_s", "w2_s") and len(shape) == 3 and t.dtype == torch.uint8 and tuple(t.shape) == (
        shape[0] * shape[1],
        shape[2],
    )


@dataclass
class MoeWeights:
    """One layer's MoE tensors on this rank, as the kernel reads them (in place).

    gate_w bf16 [E, H]; bias fp32 [E] (SGLang's e_score_correction_bias, as the
    reference keeps an fp32 copy: spec.py:519-521); norm bf16 [H] (fused-norm
    shapes only). Routed experts (stacked) w13 [E, 2I, ...] gate rows then up
    rows, w2 [E, H, ...]: FP8 e4m3 with fp32 [E, 2I/128, H/128] / [E, H/128,
    I/128] block scales, or MXFP4 packed e2m1 [E, 2I, H/2] / [E, H, I/2] with
    E8M0 [E, 2I, H/32] / [E, H, I/32]. Shared expert sgu e4m3 [2S, H] (gate
    rows then up rows) with fp32 [2S/128, H/128]; sw2 e4m3 [H, S] with fp32
    [H/128, S/128].
    """

    gate_w: torch.Tensor
    bias: torch.Tensor
    w13: torch.Tensor
    w13_s: torch.Tensor
    w2: torch.Tensor
    w2_s: torch.Tensor
    sgu: torch.Tensor
    sgu_s: torch.Tensor
    sw2: torch.Tensor
    sw2_s: torch.Tensor
    norm: torch.Tensor | None = None

    @staticmethod
    def expected(p: MoePreset) -> dict:
        """name -> (shape, accepted dtypes)."""
        e, h, i, s = p.experts, p.hidden, p.inter, p.shared_inter
        b8 = (FP8, torch.uint8)
        f32 = (torch.float32,)
        want = {
            "gate_w": ((e, h), (torch.bfloat16,)),
            "bias": ((e,), f32),
            "sgu": ((2 * s, h), b8),
            "sgu_s": ((-(-2 * s // 128), -(-h // 128)), f32),
            "sw2": ((h, s), b8),
            "sw2_s": ((-(-h // 128), -(-s // 128)), f32),
        }
        if p.shared_fmt == "fp8_mx32":  # E8M0 32 x 32 (gfx950/runner.py:163-166)
            want.update(sgu_s=((2 * s // 32, h // 32), (E8M0, torch.uint8)), sw2_s=((h // 32, s // 32), (E8M0, torch.uint8)))
        if p.routed_fmt == "fp8_b128":
            want.update(
                w13=((e, 2 * i, h), b8),
                w13_s=((e, -(-2 * i // 128), -(-h // 128)), f32),
                w2=((e, h, i), b8),
                w2_s=((e, -(-h // 128), -(-i // 128)), f32),
            )
        else:
            b4, sc = (FP4X2, torch.uint8), (E8M0, torch.uint8)
            want.update(
                w13=((e, 2 * i, h // 2), b4),
                w13_s=((e, 2 * i, h // 32), sc),
                w2=((e, h, i // 2), b4),
                # the loader pads w2_s's columns to a multiple of 8 (stages/dims.py:54-56)
                w2_s=((e, h, -(-i // 32 // 8) * 8), sc),
            )
        if p.norm_eps is not None:
            want["norm"] = ((h,), (torch.bfloat16,))
        return want

    def check(self, p: MoePreset, device=None) -> None:
        """Raise unless each tensor has the preset's shape and dtype and is contiguous on one GPU."""
        for name, (shape, dtypes) in self.expected(p).items():
            t = getattr(self, name)
            if t is None:
                raise RuntimeError(f"MoE {name}: missing, want {shape} {dtypes[0]}")
            dev_ok = t.is_cuda and (device is None or t.device == torch.device(device))
            if not (shape_ok(name, t, shape) and t.dtype in dtypes and t.is_contiguous() and dev_ok):
                raise RuntimeError(
                    f"MoE {name}: {tuple(t.shape)} {t.dtype} {t.device} contiguous={t.is_contiguous()}, "
                    f"want {shape} {dtypes[0]} contiguous on the GPU"
                )

    def c_struct(self) -> _lib.Weights:
        w = _lib.Weights()
        for f in fields(self):
            t = getattr(self, f.name)
            setattr(w, f.name, None if t is None else t.data_ptr())
        return w


# the library's defaults: launches with at least this many rows run the gate_up / down GEMMs
# on MFMA (every launch); fewer rows run the fixed-order VALU GEMVs, bit-identical to the
# oracle (mfma_rows=(49, 49) selects them at every row count)
MFMA_GATE_ROWS, MFMA_DOWN_ROWS = 1, 1
DEADLINE_S = 2.0
# MXFP4 shapes: launches with at least this many rows run the expert GEMMs on the scaled fp4 x
# fp8 MFMA (0: the library's default, never)
MXFP4_SCALED_ROWS = 0
# the down GEMM alone on the scaled MFMA from this many rows (0: the library's default, 8 rows on
# the shapes with inter <= 512, never on wider ones)
MXFP4_SCALED_DOWN_ROWS = 0


class MoeRunner:
    """The MoE block of one preset on one GPU: a workspace and the launch.

    ``deadline_s``, ``mfma_rows`` (gate_up rows, down rows) and ``mxfp4_scaled_rows``
    are this runner's per-call options (``mkmoe_options``); ``moe(...)`` overrides
    the GEMM choices for one call. Nothing is process-global. ``layout``: the routed
    experts' layout, "row_major" or (MXFP4) "aiter", SGLang's loaded gfx950 layout
    (``check_ffn.py:169-173``), read in place; with it every GEMM runs on MFMA."""

    def __init__(
        self,
        preset: MoePreset | str,
        device=None,
        max_rows: int | None = None,
        deadline_s: float = DEADLINE_S,
        mfma_rows: tuple[int, int] = (MFMA_GATE_ROWS, MFMA_DOWN_ROWS),
        mxfp4_scaled_rows: int = MXFP4_SCALED_ROWS,
        layout: str | None = None,
        mxfp4_scaled_down_rows: int = MXFP4_SCALED_DOWN_ROWS,
    ):
        self.preset = PRESETS[preset] if isinstance(preset, str) else preset
        if layout is None:  # a preset compiled for SGLang's loaded layout alone takes that one
            layout = "aiter" if self.preset.aiter_only else "row_major"
        self.layout = layout
        self.deadline_s = float(deadline_s)
        self.mfma_rows = (int(mfma_rows[0]), int(mfma_rows[1]))
        self.mxfp4_scaled_rows = int(mxfp4_scaled_rows)
        self.mxfp4_scaled_down_rows = int(mxfp4_scaled_down_rows)
        dev = torch.device("cuda") if device is None else torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError(f"mkmoe: {dev} is not a GPU")
        self.device = torch.device("cuda", torch.cuda.current_device() if dev.index is None else dev.index)
        self.lib = _lib.lib()
        self.shape = _lib.shape_of(self.preset, max_rows, layout)
        if not self.lib.mkmoe_shape_supported(ctypes.byref(self.shape)):
            raise RuntimeError(f"mkmoe: no compiled specialisation for {self.preset}")
        n = ctypes.c_size_t()
        _lib.check(self.lib.mkmoe_workspace_bytes(ctypes.byref(self.shape), ctypes.byref(n)), "workspace size")
        no_capture("workspace allocation")
        self.ws = torch.zeros(n.value, dtype=torch.uint8, device=self.device)
        _lib.check(
            self.lib.mkmoe_init_workspace(
                ctypes.byref(self.shape), self.ws.data_ptr(), self.ws.numel(), self._stream()
            ),
            "workspace init",
        )

    @property
    def max_rows(self) -> int:
        return self.shape.max_rows

    def supports(self, rows: int) -> bool:
        return 1 <= rows <= self.max_rows

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def moe(
        self,
        w: MoeWeights,
        x: torch.Tensor,
        out: torch.Tensor | None = None,
        topk_ids: torch.Tensor | None = None,
        topk_w: torch.Tensor | None = None,
        staged: bool = False,
        mfma_rows: tuple[int, int] | None = None,
        mxfp4_scaled_rows: int | None = None,
        fault: tuple[int, int] | None = None,
    ) -> torch.Tensor:
        """This rank's MoE partial of bf16 rows ``x`` [R, H] (before the all-reduce) -> bf16 [R, H].

        ``fault=(stage, workgroup)``: test fault injection for this call, as the reference's
        ``SGLANG_AMD_MONO_FAULT_INJECT`` (``common/guard.py:69-89``): that workgroup's wait at
        that stage (a code of ``_lib.STAGES``) runs to the deadline; the call's output is then
        not valid and ``clear_errors()`` restores the workspace."""
        p = self.preset
        rows = x.shape[0]
        if not self.supports(rows):
            raise RuntimeError(f"mkmoe: {rows} rows, want 1 .. {self.max_rows}")
        # every call: the kernel reads the weights with unbounded loads, so a tensor of the
        # wrong size must never reach it (a check is a few microseconds)
        w.check(p, self.device)
        bf = torch.bfloat16
        if out is None:
            no_capture("an output allocation")
            out = torch.empty(rows, p.hidden, dtype=bf, device=self.device)
        want = {"x": (x, p.hidden, bf), "out": (out, p.hidden, bf)}
        if topk_ids is not None:
            want["topk_ids"] = (topk_ids, p.topk, torch.int32)
        if topk_w is not None:
            want["topk_w"] = (topk_w, p.topk, torch.float32)
        for name, (t, size, dtype) in want.items():
            if not (t.dtype == dtype and t.numel() == rows * size and t.is_contiguous() and t.device == self.device):
                raise RuntimeError(
                    f"mkmoe {name}: {tuple(t.shape)} {t.dtype} {t.device}, want {rows} x {size} {dtype}"
                )
        fn = self.lib.mkmoe_forward_staged if staged else self.lib.mkmoe_forward
        ws_ = w.c_struct()
        gate, down = self.mfma_rows if mfma_rows is None else mfma_rows
        sc = self.mxfp4_scaled_rows if mxfp4_scaled_rows is None else int(mxfp4_scaled_rows)
        fs, fw = (0, 0) if fault is None else (int(fault[0]), int(fault[1]))
        opts = _lib.Options(
            deadline_s=self.deadline_s, mfma_gate_rows=int(gate), mfma_down_rows=int(down), mxfp4_scaled_rows=sc,
            mxfp4_scaled_down_rows=self.mxfp4_scaled_down_rows, fault_stage=fs, fault_workgroup=fw,
        )
        rc = fn(
            ctypes.byref(self.shape),
            ctypes.byref(ws_),
            x.data_ptr(),
            rows,
            out.data_ptr(),
            None if topk_ids is None else topk_ids.data_ptr(),
            None if topk_w is None else topk_w.data_ptr(),
            self.ws.data_ptr(),
            self.ws.numel(),
            ctypes.byref(opts),
            self._stream(),
        )
        _lib.check(rc, "mkmoe forward")
        return out

    def region(self, name: str, rows: int | None = None) -> torch.Tensor:
        """A view of a workspace region (for tests of intermediate results)."""
        off, n = ctypes.c_size_t(), ctypes.c_size_t()
        _lib.check(
            self.lib.mkmoe_workspace_region(ctypes.byref(self.shape), _lib.REGIONS[name], ctypes.byref(off), ctypes.byref(n)),
            "workspace region",
        )
        return self.ws[off.value : off.value + n.value]

    def read_errors(self) -> list[int]:
        """The device error words (synchronises the stream)."""
        words = (ctypes.c_int32 * _lib.ERRW_WORDS)()
        _lib.check(self.lib.mkmoe_read_errors(self.ws.data_ptr(), words, _lib.ERRW_WORDS, self._stream()), "read errors")
        return list(words)

    def raise_on_device_error(self) -> None:
        e = self.read_errors()
        if e[_lib.ERRW_CODE]:
            stage = _lib.STAGES.get(e[_lib.ERRW_STAGE], str(e[_lib.ERRW_STAGE]))
            raise RuntimeError(
                f"mkmoe: a device wait passed its deadline (stage {stage}, workgroup {e[_lib.ERRW_BLOCK]}, "
                f"{e[_lib.ERRW_COUNT]} waits)"
            )

    def clear_errors(self) -> None:
        """Reset the workspace after a device error: the error words, and the hand-off state
        (flags, polled router part sums) that a launch cut short by a deadline may leave."""
        no_capture("a workspace reset")
        _lib.check(
            self.lib.mkmoe_clear_errors(ctypes.byref(self.shape), self.ws.data_ptr(), self.ws.numel(), self._stream()),
            "clear errors",
        )
