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


# SGLang's layer-boundary residual protocol, as the reference's backbone uses it
# (glm53/spec.py:319-417): a decoder layer returns its output with the residual add still
# pending in the batch's state; the next layer's input norm (or fold) completes it.
def start(fb):
    fb.pending = None
    fb.written = False


def fold(hidden, fb):
    """The full stream: the pending residual added."""
    out = hidden if fb.pending is None else hidden + fb.pending
    fb.pending = None
    return out


def take_output(hidden, fb):
    return hidden


def set_written(hidden, fb):
    fb.written = True
    fb.pending = None
    return hidden


def complete_output(hidden, fb):
    return fold(hidden, fb)


def final_norm(hidden, fb, norm):
    return norm(hidden)


class _TpContext:
    class _Scope:
        def __enter__(self):
            return self

        def __exit__(self, *a):
            return False

    def maybe_input_scattered(self, fb):
        return self._Scope()


class BumpAllocator:
    def __init__(self, buffer_size, dtype, device):
        self.size = buffer_size


def install():
    """Put the stand-in modules into sys.modules (idempotent)."""
    if "sglang.kernels.plugin_kernels.amd.spec" in sys.modules:
        return sys.modules["sglang.kernels.plugin_kernels.amd.spec"]
    names = ["sglang", "sglang.kernels", "sglang.kernels.plugin_kernels",
             "sglang.kernels.plugin_kernels.amd", "sglang.kernels.plugin_kernels.amd.spec",
             "sglang.srt", "sglang.srt.runtime_context", "sglang.srt.layers",
             "sglang.srt.layers.layer_boundary", "sglang.srt.layers.layer_boundary.residual",
             "sglang.srt.layers.layer_boundary.residual.batch", "sglang.srt.utils",
             "sglang.srt.utils.common"]
    mods = {n: types.ModuleType(n) for n in names}
    batch = mods["sglang.srt.layers.layer_boundary.residual.batch"]
    for f in (start, fold, take_output, set_written, complete_output, final_norm):
        setattr(batch, f.__name__, f)
    mods["sglang.srt.layers.layer_boundary"].get_attn_tp_context = lambda: _TpContext()
    mods["sglang.srt.utils.common"].BumpAllocator = BumpAllocator
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
