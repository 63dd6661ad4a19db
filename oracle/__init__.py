"""CPU oracle for the K2 decode path -- TEST INFRASTRUCTURE ONLY.

This package is a plain torch/numpy restatement, on the CPU, of the arithmetic of
sgl-amd-mono's persistent decoder-layer monokernel (the GLM-5.3 launch,
``sgl_amd_mono/glm53/gfx950/kernel.py``) and of the DeepSeek-V4 FP4 indexer it is
measured beside (``sgl_amd_mono/deepseek_v4/gfx950/kernels/stages/indexer.py``).
Every function cites the reference file:line it restates.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker.  The product path (the HIP
library behind ``include/mk2.h`` and the ``sgl_amd_mono`` host package) never
imports, links or calls anything here.

Modules:
  codecs     -- E4M3, E2M1/MXFP4, MXFP8 and E8M0 encoders/decoders, radix keys
  reference  -- index scores, exact top-k, sparse MLA, o_proj, RMSNorm, routers,
                SwiGLU experts, the MoE block and the chained K2 layer

Parity status of each function is listed in the module docstrings; every function
listed there has a pinning test under ``tests/test_oracle*.py``.
"""
