"""MI355X-native monokernel plugin for SGLang: the K2 decode layer on gfx950.

SGLang loads this package as a general plugin through the ``sglang.srt.plugins``
entry point (``pyproject.toml``); ``register_specs`` registers the layer's spec
under the monokernel backend ``amd`` -- the same surface as the reference's
sgl_amd_mono/__init__.py:17-72.  The spec's module is imported only when a server
runs the backend.  Without SGLang, the local stand-in registry
(``sgl_amd_mono._registry``) takes the registrations, so the surface can be used and
tested anywhere.
"""

__version__ = "0.1.0"

# the backend name every spec registers under
BACKEND = "amd"

# each spec by (HF architecture, model type); None matches any model type
SPECS = {
    ("GlmMoeDsaForCausalLM", None): "sgl_amd_mono.k2.spec:SPEC",
}


def _registry_module():
    """SGLang's monokernel registry, its legacy location, or the local stand-in."""
    try:
        from sglang.kernels.plugin_kernels.amd import spec as reg  # type: ignore
    except ModuleNotFoundError:
        try:
            from sglang.srt.monokernels import spec as reg  # type: ignore
        except ModuleNotFoundError:
            from . import _registry as reg
    return reg


def register_specs() -> None:
    """The plugin entry point, which SGLang runs in every process."""
    reg = _registry_module()
    for (architecture, model_type), path in SPECS.items():
        reg.register(backend=BACKEND, architecture=architecture, path=path, model_type=model_type)
