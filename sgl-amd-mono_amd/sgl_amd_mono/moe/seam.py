"""Host runner of the FFN seam before the MoE block (DeepSeek-V4.1's mHC hyper-connections).

Mirrors the seam half of the reference's FFN launch:
- ``SeamWeights`` / ``.check`` are the seam's tensors of ``FFNWeights``
  (``sgl_amd_mono/deepseek_v41/gfx950/runner.py:130-136``): ``hc_ffn_fn`` [24, 4 H] fp32,
  ``hc_ffn_scale`` [3] fp32, ``hc_ffn_base`` [24] fp32, ``ffn_norm`` [H] bf16, read in place.
- ``SeamRunner.ffn_seam`` takes ``DSV41MonoRunner.ffn``'s seam arguments and returns its
  seam outputs (``runner.py:436-480``), with the same row checks (``check_rows``,
  ``runner.py:94-105``) and optional caller-provided outputs; the normed layer input, which
  the reference keeps in its launch's scratch for the MoE (``gfx950/layer.py:569-577``), is
  returned first. ``part`` is the attention output after the TP all-reduce (at TP 1, the
  rank's own), since the reduce itself needs peers.
Two launches on the current stream (include/mkmoe_seam.h), no host synchronisation; the
workspace for a token count is allocated on its first call, never inside a graph capture.
With ``gate_later`` the second launch is the norm alone and ``gate()`` runs the gate later,
off the path to the MoE block, as the reference runs its gates inside its MoE stage
(``gfx950/layer.py:579-586``).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from .runner import no_capture

HC, MIX, HIDDEN = _lib.SEAM_HC, _lib.SEAM_MIX, _lib.SEAM_HIDDEN
NORM_EPS = 1e-20  # the reference's RMS epsilon (check_ffn.py:21; seam.py:48)


@dataclass
class SeamWeights:
    """One layer's FFN-seam tensors on this rank (the reference's FFNWeights names)."""

    hc_ffn_fn: torch.Tensor
    hc_ffn_scale: torch.Tensor
    hc_ffn_base: torch.Tensor
    ffn_norm: torch.Tensor

    def check(self, device=None) -> None:
        """Raise unless each tensor has its shape and dtype and is contiguous on one GPU."""
        want = {
            "hc_ffn_fn": ((MIX, HC * HIDDEN), torch.float32),
            "hc_ffn_scale": ((3,), torch.float32),
            "hc_ffn_base": ((MIX,), torch.float32),
            "ffn_norm": ((HIDDEN,), torch.bfloat16),
        }
        for name, (shape, dtype) in want.items():
            t = getattr(self, name)
            dev_ok = t is not None and t.is_cuda and (device is None or t.device == torch.device(device))
            if t is None or not (tuple(t.shape) == shape and t.dtype == dtype and t.is_contiguous() and dev_ok):
                got = "missing" if t is None else f"{tuple(t.shape)} {t.dtype} {t.device}"
                raise RuntimeError(f"FFN seam {name}: {got}, want {shape} {dtype} contiguous on the GPU")


class SeamRunner:
    """The FFN seam on one GPU: per-token-count workspaces and the call."""

    def __init__(self, device=None, norm_eps: float = NORM_EPS):
        dev = torch.device("cuda") if device is None else torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError(f"mkmoe seam: {dev} is not a GPU")
        self.device = torch.device("cuda", torch.cuda.current_device() if dev.index is None else dev.index)
        self.norm_eps = float(norm_eps)
        self.lib = _lib.lib()
        self._ws: dict[int, torch.Tensor] = {}

    @staticmethod
    def supports(tokens: int) -> bool:
        return 1 <= tokens <= _lib.SEAM_MAX_TOKENS

    def workspace(self, tokens: int) -> torch.Tensor:
        ws = self._ws.get(tokens)
        if ws is None:
            n = ctypes.c_size_t()
            _lib.check(self.lib.mkmoe_seam_workspace_bytes(HIDDEN, tokens, ctypes.byref(n)), "seam workspace size")
            no_capture("the seam workspace")
            ws = self._ws[tokens] = torch.empty(n.value, dtype=torch.uint8, device=self.device)
        return ws

    def ffn_seam(
        self,
        w: SeamWeights,
        part: torch.Tensor,  # [M, H] bf16: the attention output, all-reduced
        residual: torch.Tensor,  # [M, 4, H] bf16
        post_mix: torch.Tensor,  # [M, 4, 1] or [M, 4] fp32
        res_mix: torch.Tensor,  # [M, 4, 4] fp32
        pre_mix: torch.Tensor,  # [M, 4] fp32
        outs: tuple | None = None,
        gate_later: bool = False,
    ) -> tuple:
        """-> (normed [M, H] bf16, res_out [M, 4, H] bf16, post_out [M, 4, 1], comb_out [M, 4, 4], pre_out [M, 4]).

        ``gate_later``: post_out, comb_out and pre_out are written by the next ``gate()`` call
        (after, say, the MoE launch), so that ``normed`` is ready first; the runner holds the
        call's tensors until then, and the workspace of this token count must not serve another
        call in between, so a call made while a gate_later call still waits for its gate is
        refused (its gate would be lost, and a call of the same token count would overwrite the
        partials that gate reads)."""
        pending = getattr(self, "_io", None)
        if pending is not None and pending.flags & _lib.SEAM_GATE_LATER:
            raise RuntimeError("mkmoe seam: a gate_later call waits for its gate(); call gate() first")
        M = part.shape[0]
        if not self.supports(M):
            raise RuntimeError(f"mkmoe seam: {M} rows, want 1 .. {_lib.SEAM_MAX_TOKENS}")
        w.check(self.device)
        bf, f32 = torch.bfloat16, torch.float32
        ins = {
            "part": (part, HIDDEN, bf),
            "residual": (residual, HC * HIDDEN, bf),
            "post": (post_mix, HC, f32),
            "comb": (res_mix, HC * HC, f32),
            "pre": (pre_mix, HC, f32),
        }
        if outs is None:
            no_capture("the seam's outputs")
            outs = (
                torch.empty(M, HIDDEN, dtype=bf, device=self.device),
                torch.empty(M, HC, HIDDEN, dtype=bf, device=self.device),
                torch.empty(M, HC, 1, dtype=f32, device=self.device),
                torch.empty(M, HC, HC, dtype=f32, device=self.device),
                torch.empty(M, HC, dtype=f32, device=self.device),
            )
        normed, res_out, post_out, comb_out, pre_out = outs
        outs_want = {
            "normed": (normed, HIDDEN, bf),
            "res_out": (res_out, HC * HIDDEN, bf),
            "post_out": (post_out, HC, f32),
            "comb_out": (comb_out, HC * HC, f32),
            "pre_out": (pre_out, HC, f32),
        }
        for name, (t, size, dtype) in {**ins, **outs_want}.items():
            if not (t.dtype == dtype and t.numel() == M * size and t.is_contiguous() and t.device == self.device):
                raise RuntimeError(
                    f"FFN {name}: {tuple(t.shape)} {t.dtype} {t.device}, want {M} x {size} {dtype} contiguous"
                )
        ws = self.workspace(M)
        io = _lib.SeamIO(
            hidden=HIDDEN, tokens=M, norm_eps=self.norm_eps, flags=_lib.SEAM_GATE_LATER if gate_later else 0,
            a=part.data_ptr(), res=residual.data_ptr(), post=post_mix.data_ptr(), comb=res_mix.data_ptr(),
            pre=pre_mix.data_ptr(), hc_fn=w.hc_ffn_fn.data_ptr(), hc_scale=w.hc_ffn_scale.data_ptr(),
            hc_base=w.hc_ffn_base.data_ptr(), norm_w=w.ffn_norm.data_ptr(), res_out=res_out.data_ptr(),
            normed=normed.data_ptr(), post_out=post_out.data_ptr(), comb_out=comb_out.data_ptr(),
            pre_out=pre_out.data_ptr(),
        )  # fmt: skip
        # the later gate's arguments, and the tensors they point into (kept alive until then)
        self._io = io
        self._keep = (w, part, residual, post_mix, res_mix, pre_mix, outs) if gate_later else None
        rc = self.lib.mkmoe_seam_forward(
            ctypes.byref(io), ws.data_ptr(), ws.numel(), torch.cuda.current_stream(self.device).cuda_stream
        )
        _lib.check(rc, "mkmoe seam forward")
        return outs

    def cancel_gate(self) -> None:
        """Drop a pending ``gate_later`` call's gate: its post_out, comb_out and pre_out stay
        unwritten (for a caller that times or needs the path to ``normed`` alone)."""
        self._io = None
        self._keep = None

    def gate(self) -> None:
        """The gate of the last ``ffn_seam(..., gate_later=True)`` call (its outputs filled in)."""
        io = getattr(self, "_io", None)
        if io is None or not (io.flags & _lib.SEAM_GATE_LATER):
            raise RuntimeError("mkmoe seam gate: no ffn_seam(..., gate_later=True) call to finish")
        ws = self._ws[io.tokens]
        rc = self.lib.mkmoe_seam_gate(
            ctypes.byref(io), ws.data_ptr(), ws.numel(), torch.cuda.current_stream(self.device).cuda_stream
        )
        _lib.check(rc, "mkmoe seam gate")
        self._io = None
        self._keep = None
