"""MI355X-native DSA decoder-layer monokernels for SGLang (gfx950).

One GPU's TP=4 share of a DeepSeek-V3.2-geometry decoder layer runs as persistent
gfx950 launches of hand-written HIP kernels (``csrc/``), called through the C ABI of
``include/mono_amd.h`` (``_lib.py``). SGLang loads the package as a general plugin: the
``sglang.srt.plugins`` entry point in ``pyproject.toml`` runs ``register_specs``, which
registers each spec under the monokernel backend ``amd``, the surface of
``sgl_amd_mono/__init__.py:14-54``.
"""

__version__ = "0.1.0"

# the backend name every spec registers under (sgl_amd_mono/__init__.py:15)
BACKEND = "amd"
# each spec by (HF architecture, model type); its module imports only when a server runs
# this backend
SPECS = {
    ("DeepseekV32ForCausalLM", None): "sgl_amd_mono_amd.dsv32.spec:SPEC",
}


def register_specs() -> None:
    """The plugin entry point, which SGLang runs in every process."""
    try:
        from sglang.kernels.plugin_kernels.amd.spec import register
    except ModuleNotFoundError:  # SGLang before sgl-project/sglang#45389
        from sglang.srt.monokernels.spec import register

    for (architecture, model_type), path in SPECS.items():
        register(backend=BACKEND, architecture=architecture, path=path, model_type=model_type)
