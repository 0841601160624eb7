"""A local stand-in for SGLang's monokernel spec interface (``sglang.srt.monokernels.spec``).

SGLang holds the real interface; it is not installed here. This module keeps
the names and the argument meaning the reference's spec uses
(``sgl_amd_mono/deepseek_v41/spec.py:79-91`` imports them; ``:959-1001``
builds a ``MonoSpec``; ``test/unit/test_deepseek_v41_spec.py:48`` calls
``find_spec``), so that a spec written against SGLang registers, is found and
is checked the same way without it: ``register`` records a lazy path,
``find_spec`` imports it and refuses an ISA the spec has no limits for.
Nothing here runs on the GPU.
"""

from __future__ import annotations

import enum
import importlib
from dataclasses import dataclass, field
from typing import Any, Callable

MONOKERNEL_API_VERSION = 1


class NumericsKind(enum.Enum):
    EXACT = "exact"
    TOLERANCE = "tolerance"


@dataclass(frozen=True)
class Numerics:
    """Per-output bounds of a spec's launches against the normal path."""

    kind: NumericsKind
    bounds: dict = field(default_factory=dict)

    def bound(self, name: str) -> float:
        if self.kind is NumericsKind.EXACT:
            return 0.0
        return self.bounds[name]


class Feature(enum.Enum):
    SPECULATIVE_DECODING = "speculative_decoding"


class StepMetadata(enum.Enum):
    LOW_RATIO_DECODE_SCHEDULE = "low_ratio_decode_schedule"


@dataclass(frozen=True)
class DeviceLimits:
    """What a spec's kernels take on one ISA: the decode row counts (widths), the TP
    sizes and the workgroups that must be resident at once (a persistent grid)."""

    widths: tuple
    tp_sizes: tuple
    resident_blocks: int


@dataclass(frozen=True)
class Requirements:
    dtypes: frozenset = frozenset()
    attention_backends: frozenset = frozenset()
    server_args: dict = field(default_factory=dict)
    hf_config: dict = field(default_factory=dict)
    env: dict = field(default_factory=dict)


@dataclass(frozen=True)
class MonoSpec:
    name: str
    devices: dict
    features: frozenset
    requires: Requirements
    numerics: Numerics
    model_disable_reasons: Callable[..., list]
    build: Callable[..., Any]
    api_version: int = MONOKERNEL_API_VERSION
    config_disable_reasons: Callable[..., list] | None = None
    load_tensor: Callable[..., None] | None = None
    unread_metadata: frozenset = frozenset()


_REGISTRY: dict[tuple[str, str], str] = {}


def register(*, backend: str, architecture: str, path: str) -> None:
    """Record ``path`` ("module:attribute") as ``backend``'s spec for ``architecture``."""
    if ":" not in path:
        raise ValueError(f"spec path {path!r}: want 'module:attribute'")
    _REGISTRY[(backend, architecture)] = path


def registered() -> dict:
    return dict(_REGISTRY)


def find_spec(*, backend: str, architectures, isa: str):
    """-> (spec, "") for the first registered architecture whose spec has limits for
    ``isa``, else (None, the reason)."""
    why = []
    for arch in architectures:
        path = _REGISTRY.get((backend, arch))
        if path is None:
            why.append(f"{arch}: no spec under backend {backend!r}")
            continue
        mod, attr = path.split(":")
        spec = getattr(importlib.import_module(mod), attr)
        if spec.api_version != MONOKERNEL_API_VERSION:
            why.append(f"{arch}: spec API {spec.api_version}, want {MONOKERNEL_API_VERSION}")
            continue
        if isa not in spec.devices:
            why.append(f"{arch}: {spec.name} has no kernels for {isa}")
            continue
        return spec, ""
    return None, "; ".join(why) or "no architectures"
