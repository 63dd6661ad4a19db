"""The plugin surface on the CPU: entry point, registration under backend 'amd',
find_spec by architecture and ISA, graph-key routing, refusal reasons (after
test/unit/test_glm53_spec.py:52-73)."""

import tomli as tomllib
import os
from types import SimpleNamespace

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

GLM5_LIKE = SimpleNamespace(
    hidden_size=6144, n_routed_experts=256, num_experts_per_tok=8, moe_intermediate_size=256,
    scoring_func="sigmoid", routed_scaling_factor=2.5, n_shared_experts=1, num_attention_heads=16,
    kv_lora_rank=512, qk_rope_head_dim=64, v_head_dim=128, index_topk=2048, index_n_heads=64,
    index_head_dim=128, rms_norm_eps=1e-6, architectures=["GlmMoeDsaForCausalLM"],
)


def test_entry_point_declared():
    with open(os.path.join(ROOT, "sgl-amd-mono_amd", "pyproject.toml"), "rb") as f:
        meta = tomllib.load(f)
    eps = meta["project"]["entry-points"]["sglang.srt.plugins"]
    assert eps == {"sgl_amd_mono": "sgl_amd_mono:register_specs"}


def test_plugin_registers_the_spec():
    import sgl_amd_mono
    from sgl_amd_mono import _registry as reg
    from sgl_amd_mono.k2 import spec

    sgl_amd_mono.register_specs()
    found, why = reg.find_spec(backend=sgl_amd_mono.BACKEND, architectures=["GlmMoeDsaForCausalLM"],
                               isa="gfx950")
    assert found is spec.SPEC, why
    found, why = reg.find_spec(backend="amd", architectures=["GlmMoeDsaForCausalLM"], isa="gfx942")
    assert found is None and "gfx942" in why
    found, why = reg.find_spec(backend="amd", architectures=["LlamaForCausalLM"], isa="gfx950")
    assert found is None


@pytest.mark.parametrize("mode,bs,tpr,ok", [
    ("decode", 1, 1, True), ("decode", 8, 1, True), ("decode", 32, 1, True),
    ("decode", 3, 1, False), ("decode", 64, 1, False), ("target_verify", 8, 4, True),
    ("target_verify", 16, 4, False), ("extend", 8, 1, False),
])
def test_graph_key_routing(mode, bs, tpr, ok):
    from sgl_amd_mono import _registry as reg
    from sgl_amd_mono.k2 import spec

    got, why = spec.SPEC.accepts(reg.ShapeKey(mode, bs, tpr))
    assert got == ok, why
    assert spec.SPEC.accepts(reg.ShapeKey("decode", 8, 1), tp_size=8)[0] is False


def test_refusal_reasons():
    from sgl_amd_mono.k2 import spec

    assert spec.model_disable_reasons(GLM5_LIKE) == []
    bad = SimpleNamespace(**{**vars(GLM5_LIKE), "n_routed_experts": 300})
    assert spec.model_disable_reasons(bad)
    assert spec.config_disable_reasons(SimpleNamespace(dtype="bfloat16", kv_cache_dtype="fp8_e4m3",
                                                       tp_size=1, page_size=64)) == []
    why = spec.config_disable_reasons(SimpleNamespace(dtype="float16", kv_cache_dtype="bfloat16",
                                                      tp_size=8, page_size=16))
    assert len(why) == 4


def test_config_from_hf_is_configs4():
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import spec

    cfg = spec.config_from_hf(GLM5_LIKE)
    assert cfg.moe == C.C2_MOE
    assert cfg.mla == C.C5_LAYER.mla and cfg.indexer == C.C5_LAYER.indexer


def test_stopped_step_gives_nan_logits_and_raises():
    """A step whose status words (the layers' shared word, each front's) show a stopped
    launch: the logits become NaN on the device, and the host check raises and clears
    every word; clean words leave the logits and pass the check."""
    import torch

    from sgl_amd_mono.k2 import spec

    words = [torch.zeros(1, dtype=torch.int32) for _ in range(3)]
    logits = torch.randn(4, 16)
    want = logits.clone()
    spec.gate_logits(words, logits)
    assert torch.equal(logits, want)
    spec.raise_if_stopped(words)
    words[2][0] = 1  # one front stopped
    spec.gate_logits(words, logits)
    assert bool(torch.isnan(logits).all())
    with pytest.raises(RuntimeError, match="stopped early"):
        spec.raise_if_stopped(words)
    assert all(int(w.item()) == 0 for w in words)
    spec.raise_if_stopped(words)
