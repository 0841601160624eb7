"""The FFN seam's host side without a GPU: the C ABI's argument checks (each returns before
any HIP call, so fake device addresses are safe), its workspace size, and the runner's
weight check."""

import ctypes

import pytest
import torch


def _io(**over):
    from sgl_amd_mono.moe import _lib

    io = _lib.SeamIO(hidden=_lib.SEAM_HIDDEN, tokens=8, norm_eps=1e-20, flags=0)
    for n, _ in _lib.SeamIO._fields_[4:]:
        setattr(io, n, 0x100000)
    for k, v in over.items():
        setattr(io, k, v)
    return io


def test_seam_workspace_bytes():
    from sgl_amd_mono.moe import _lib

    L = _lib.lib()
    n = ctypes.c_size_t()
    assert L.mkmoe_seam_workspace_bytes(5120, 8, ctypes.byref(n)) == 0
    # the collapsed rows (bf16) and 25 partials of each of 160 slices a token, each 256-aligned
    assert n.value == 8 * 5120 * 2 + 8 * 25 * 160 * 4
    assert L.mkmoe_seam_workspace_bytes(4096, 8, ctypes.byref(n)) == -2
    assert L.mkmoe_seam_workspace_bytes(5120, 0, ctypes.byref(n)) == -3
    assert L.mkmoe_seam_workspace_bytes(5120, 65, ctypes.byref(n)) == -3
    assert L.mkmoe_seam_workspace_bytes(5120, 1, None) == -1


@pytest.mark.parametrize(
    "over,code",
    [
        (dict(a=None), -1),
        (dict(pre_out=None), -1),
        (dict(hidden=7168), -2),
        (dict(tokens=0), -3),
        (dict(tokens=65), -3),
        (dict(flags=2), -8),
        (dict(flags=-1), -8),
        (dict(norm_eps=-1.0), -8),
        (dict(norm_eps=float("nan")), -8),
        (dict(res=0x100008), -4),
        (dict(normed=0x100002), -4),
        (dict(comb=0x100002), -4),
    ],
)
def test_seam_forward_rejects_bad_arguments(over, code):
    from sgl_amd_mono.moe import _lib

    L = _lib.lib()
    n = ctypes.c_size_t()
    assert L.mkmoe_seam_workspace_bytes(5120, 8, ctypes.byref(n)) == 0
    io = _io(**over)
    assert L.mkmoe_seam_forward(ctypes.byref(io), 0x200000, n.value, None) == code


def test_seam_forward_rejects_small_workspace_and_null():
    from sgl_amd_mono.moe import _lib

    L = _lib.lib()
    n = ctypes.c_size_t()
    assert L.mkmoe_seam_workspace_bytes(5120, 8, ctypes.byref(n)) == 0
    io = _io()
    assert L.mkmoe_seam_forward(ctypes.byref(io), 0x200000, n.value - 1, None) == -5
    assert L.mkmoe_seam_forward(ctypes.byref(io), 0x200008, n.value, None) == -4
    assert L.mkmoe_seam_forward(ctypes.byref(io), None, n.value, None) == -1
    assert L.mkmoe_seam_forward(None, 0x200000, n.value, None) == -1


def test_seam_gate_needs_the_gate_later_flag():
    from sgl_amd_mono.moe import _lib

    L = _lib.lib()
    n = ctypes.c_size_t()
    assert L.mkmoe_seam_workspace_bytes(5120, 8, ctypes.byref(n)) == 0
    assert L.mkmoe_seam_gate(ctypes.byref(_io(flags=0)), 0x200000, n.value, None) == -8
    assert L.mkmoe_seam_gate(ctypes.byref(_io(flags=1, tokens=0)), 0x200000, n.value, None) == -3
    assert L.mkmoe_seam_gate(ctypes.byref(_io(flags=1)), 0x200000, n.value - 1, None) == -5


def test_seam_weights_check_names_the_tensor():
    from sgl_amd_mono.moe.seam import SeamWeights

    w = SeamWeights(
        hc_ffn_fn=torch.zeros(24, 4 * 5120), hc_ffn_scale=torch.zeros(3), hc_ffn_base=torch.zeros(24),
        ffn_norm=torch.zeros(5120, dtype=torch.bfloat16),
    )  # fmt: skip
    with pytest.raises(RuntimeError, match="hc_ffn_fn"):
        w.check()  # on the CPU
    w.hc_ffn_fn = None
    with pytest.raises(RuntimeError, match="hc_ffn_fn: missing"):
        w.check()


def test_seam_call_refused_while_a_gate_is_pending():
    """A second ffn_seam call while a gate_later call waits for gate() would lose that gate (and,
    at the same token count, overwrite the partials it reads): refused before any launch."""
    from sgl_amd_mono.moe import _lib
    from sgl_amd_mono.moe.seam import SeamRunner

    run = object.__new__(SeamRunner)  # the host checks alone: no device
    run._io = _io(flags=_lib.SEAM_GATE_LATER)
    z = torch.zeros(1)
    with pytest.raises(RuntimeError, match="waits for its gate"):
        run.ffn_seam(None, z, z, z, z, z)
    run.cancel_gate()
    with pytest.raises(Exception) as e:  # no pending gate: on to the argument checks
        run.ffn_seam(None, z, z, z, z, z)
    assert "waits for its gate" not in str(e.value)
