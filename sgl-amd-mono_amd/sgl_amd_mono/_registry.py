"""Local stand-in of SGLang's monokernel registry, used when SGLang is absent.

SGLang holds the real interface (``sglang.kernels.plugin_kernels.amd.spec``, or the
legacy ``sglang.srt.monokernels.spec``).  This module mirrors the names and the
behaviour this package relies on -- ``register``, ``find_spec``, ``MonoSpec``,
``DeviceLimits``, ``Feature``, ``Numerics``/``NumericsKind``, ``Requirements``,
``ShapeKey`` and ``Plan`` -- as the reference's tests use them
(test/unit/test_glm53_spec.py:52-73, sgl_amd_mono/glm53/spec.py:746-778), so the
plugin surface can be exercised on a machine without SGLang.
"""

from __future__ import annotations

import enum
import importlib
from dataclasses import dataclass, field
from typing import Any, Callable


class Feature(enum.Enum):
    SPECULATIVE_DECODING = "speculative_decoding"


class NumericsKind(enum.Enum):
    EXACT = "exact"
    TOLERANCE = "tolerance"


@dataclass(frozen=True)
class Numerics:
    kind: NumericsKind
    bounds: dict = field(default_factory=dict)


@dataclass(frozen=True)
class DeviceLimits:
    widths: tuple  # decode rows a launch serves
    tp_sizes: tuple
    resident_blocks: int


@dataclass(frozen=True)
class Requirements:
    dtypes: frozenset = frozenset()
    attention_backends: frozenset = frozenset()
    server_args: dict = field(default_factory=dict)
    env: dict = field(default_factory=dict)


@dataclass(frozen=True)
class ShapeKey:
    """The CUDA-graph key SGLang routes a step by."""

    forward_mode: str  # "decode" | "target_verify"
    batch_size: int
    tokens_per_request: int

    @property
    def rows(self) -> int:
        return self.batch_size * self.tokens_per_request


@dataclass
class Plan:
    key: ShapeKey
    state: dict = field(default_factory=dict)


@dataclass(frozen=True)
class MonoSpec:
    name: str
    devices: dict
    features: frozenset
    requires: Requirements
    numerics: Numerics
    model_disable_reasons: Callable[[Any], list]
    build: Callable
    api_version: int = 1
    config_disable_reasons: Callable[[Any], list] | None = None

    def accepts(self, key: ShapeKey, isa: str = "gfx950", tp_size: int = 1) -> tuple[bool, str]:
        """Graph-key routing: whether a step of this shape runs on the spec."""
        lim = self.devices.get(isa)
        if lim is None:
            return False, f"{self.name}: no kernels for {isa}"
        if tp_size not in lim.tp_sizes:
            return False, f"{self.name}: tp_size {tp_size} not in {lim.tp_sizes}"
        if key.forward_mode not in ("decode", "target_verify"):
            return False, f"{self.name}: forward mode {key.forward_mode} is not a decode step"
        if key.forward_mode == "target_verify" and Feature.SPECULATIVE_DECODING not in self.features:
            return False, f"{self.name}: no speculative decoding"
        if key.rows not in lim.widths:
            return False, f"{self.name}: {key.rows} rows not in {lim.widths}"
        return True, ""


# (backend, architecture, model_type) -> "module:ATTR"
_REGISTRY: dict = {}


def register(backend: str, architecture: str, path: str, model_type: str | None = None) -> None:
    _REGISTRY[(backend, architecture, model_type)] = path


def _load(path: str) -> MonoSpec:
    mod, attr = path.split(":")
    return getattr(importlib.import_module(mod), attr)


def find_spec(backend: str, architectures, isa: str, model_type: str | None = None):
    """(spec | None, why): the registered spec of the first matching architecture."""
    for arch in architectures:
        path = _REGISTRY.get((backend, arch, model_type)) or _REGISTRY.get((backend, arch, None))
        if path is None:
            continue
        spec = _load(path)
        if isa not in spec.devices:
            return None, f"{spec.name} has no kernels for {isa}"
        return spec, ""
    return None, f"no {backend} spec for {list(architectures)}"
