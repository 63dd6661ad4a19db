"""MI355X-native monokernel plugin for SGLang: the K2 decode layer on gfx950.

SGLang loads this package as a general plugin through the ``sglang.srt.plugins``
entry point (``pyproject.toml``), whose ``register_specs`` registers the layer's
spec under the monokernel backend ``amd`` -- the same surface as
sgl_amd_mono/__init__.py:17-72 of the reference.
"""

__version__ = "0.1.0"
BACKEND = "amd"
