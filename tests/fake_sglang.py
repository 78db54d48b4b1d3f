"""A minimal stand-in for SGLang's monokernel registry (SGLang is absent here), with the
names the spec reads: register / find_spec, MonoSpec, DeviceLimits, Requirements,
Numerics(Kind), Feature, ShapeKey, Plan, and runtime_context.get_parallel. Tests install
it into sys.modules; the product code imports SGLang's real modules by the same names."""

import enum
import importlib
import sys
import types
from dataclasses import dataclass, field
from types import SimpleNamespace


class Feature(enum.Enum):
    SPECULATIVE_DECODING = "speculative_decoding"


class NumericsKind(enum.Enum):
    TOLERANCE = "tolerance"
    BITWISE = "bitwise"


@dataclass(frozen=True)
class Numerics:
    kind: NumericsKind
    bounds: dict

    def bound(self, name):
        return self.bounds[name]


@dataclass(frozen=True)
class DeviceLimits:
    widths: tuple
    tp_sizes: tuple
    resident_blocks: int


@dataclass(frozen=True)
class Requirements:
    dtypes: frozenset = frozenset()
    attention_backends: frozenset = frozenset()
    server_args: dict = field(default_factory=dict)
    env: dict = field(default_factory=dict)
    hf_config: dict = field(default_factory=dict)


@dataclass(frozen=True)
class MonoSpec:
    name: str
    devices: dict
    features: frozenset
    requires: Requirements
    numerics: Numerics
    model_disable_reasons: object
    build: object
    api_version: int
    config_disable_reasons: object


@dataclass(frozen=True)
class ShapeKey:
    forward_mode: str
    batch_size: int
    tokens_per_request: int

    @property
    def rows(self):
        return self.batch_size * self.tokens_per_request


@dataclass
class Plan:
    key: ShapeKey
    state: dict = field(default_factory=dict)


_REGISTRY = {}


def register(backend, architecture, path, model_type=None):
    _REGISTRY[(backend, architecture, model_type)] = path


def find_spec(backend, architectures, isa, model_type=None):
    for arch in architectures:
        path = _REGISTRY.get((backend, arch, model_type)) or _REGISTRY.get((backend, arch, None))
        if path is None:
            continue
        mod, attr = path.split(":")
        spec = getattr(importlib.import_module(mod), attr)
        if isa not in spec.devices:
            return None, f"{spec.name} has no kernels for {isa}"
        return spec, ""
    return None, f"no {backend} spec for {architectures}"


PARALLEL = SimpleNamespace(tp_size=1, tp_rank=0)


def install():
    """Put the stand-in modules into sys.modules (idempotent)."""
    if "sglang.kernels.plugin_kernels.amd.spec" in sys.modules:
        return sys.modules["sglang.kernels.plugin_kernels.amd.spec"]
    names = ["sglang", "sglang.kernels", "sglang.kernels.plugin_kernels",
             "sglang.kernels.plugin_kernels.amd", "sglang.kernels.plugin_kernels.amd.spec",
             "sglang.srt", "sglang.srt.runtime_context"]
    mods = {n: types.ModuleType(n) for n in names}
    spec = mods["sglang.kernels.plugin_kernels.amd.spec"]
    for name, obj in dict(Feature=Feature, NumericsKind=NumericsKind, Numerics=Numerics,
                          DeviceLimits=DeviceLimits, Requirements=Requirements,
                          MonoSpec=MonoSpec, ShapeKey=ShapeKey, Plan=Plan,
                          register=register, find_spec=find_spec).items():
        setattr(spec, name, obj)
    mods["sglang.srt.runtime_context"].get_parallel = lambda: PARALLEL
    for n, m in mods.items():
        sys.modules[n] = m
    return spec
