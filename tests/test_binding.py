"""The binding of SGLang's model (sgl_amd_mono.k2.binding) on the CPU: what is read in
place, what is copied into the kernels' tiles, and what is refused."""

from dataclasses import replace

import pytest
import torch

import fake_sglang as F


@pytest.fixture(scope="module")
def model():
    return F.make_model(3, torch.device("cpu"), layers=1)


def _cfgs():
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import spec

    cfg = spec.config_from_hf(F.HF)
    cfg = replace(cfg, moe=replace(cfg.moe, expert_fmt=C.FMT_FP8))
    return cfg, spec.front_config_from_hf(F.HF, C.WFMT_FP8_BLOCK)


def test_front_weights_are_read_in_place(model):
    from sgl_amd_mono.k2 import binding

    _, fc = _cfgs()
    L = model.model.layers[0]
    w = binding.bind_front(L, fc)
    attn = L.self_attn
    assert w.w_qkv_a.data_ptr() == attn.fused_qkv_a_proj_with_mqa.weight.data_ptr()
    assert w.s_qkv_a.data_ptr() == attn.fused_qkv_a_proj_with_mqa.weight_scale_inv.data_ptr()
    assert w.w_q_b.data_ptr() == attn.q_b_proj.weight.data_ptr()
    assert w.w_iq.data_ptr() == attn.indexer.wq_b.weight.data_ptr()
    assert w.w_ik.data_ptr() == attn.indexer.wk.weight.data_ptr()
    assert w.w_iw.data_ptr() == attn.indexer.weights_proj.weight.data_ptr()
    # w_kc's memory is already [heads][kv_lora][nope]: a view, no copy
    assert w.w_uk.data_ptr() == attn.w_kc.data_ptr() and w.w_uk.is_contiguous()
    assert torch.equal(w.w_uk, attn.w_kc.transpose(1, 2))
    assert w.g_ik.dtype == torch.float32


def test_shuffled_front_linears_are_read_in_place():
    """Block-FP8 front linears SGLang preshuffled for AITER's GEMM (aiter_bpreshuffled):
    bound in place as WFMT_FP8_AITER16, the same codes as the row-major model's; W_o is
    unshuffled into the same bf16 tiles; a front mixing the two layouts is refused."""
    from sgl_amd_mono.k2 import binding
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2.packing import aiter_unshuffle

    cfg, fc = _cfgs()
    row = F.make_model(3, torch.device("cpu"), layers=1).model.layers[0]
    shf = F.make_model(3, torch.device("cpu"), layers=1, shuffled=True).model.layers[0]
    with pytest.raises(ValueError, match="one format"):
        binding.bind_front(shf, fc)
    a = binding.bind_front(shf, replace(fc, weight_fmt=C.WFMT_FP8_AITER16))
    t = binding.bind_front(row, fc)
    sa = shf.self_attn
    assert a.w_qkv_a.data_ptr() == sa.fused_qkv_a_proj_with_mqa.weight.data_ptr()
    assert a.w_ik.data_ptr() == sa.indexer.wk.weight.data_ptr()
    for n in ("w_qkv_a", "w_q_b", "w_iq", "w_ik"):
        assert torch.equal(aiter_unshuffle(getattr(a, n)), getattr(t, n)), n
    for n in ("s_qkv_a", "s_q_b", "s_iq", "s_ik"):
        assert torch.equal(getattr(a, n), getattr(t, n)), n
    assert torch.equal(binding.bind_mla(shf, cfg.mla, fc.nope).w_o, binding.bind_mla(row, cfg.mla, fc.nope).w_o)
    sa.q_b_proj = row.self_attn.q_b_proj  # one linear row-major, the rest shuffled
    with pytest.raises(ValueError, match="one format"):
        binding.bind_front(shf, replace(fc, weight_fmt=C.WFMT_FP8_AITER16))


def test_mla_and_moe_weights(model):
    from sgl_amd_mono.k2 import binding, synth

    cfg, fc = _cfgs()
    L = model.model.layers[0]
    m = binding.bind_mla(L, cfg.mla, fc.nope)
    assert m.w_uv.data_ptr() == L.self_attn.w_vc.data_ptr()  # [heads][v][kv_lora] memory
    deq = L.self_attn.o_proj.weight.float() * L.self_attn.o_proj.weight_scale_inv.repeat_interleave(
        128, 0).repeat_interleave(128, 1)
    assert torch.equal(m.w_o, deq.to(torch.bfloat16))
    e = binding.bind_moe(L, cfg.moe)
    ex = L.mlp.experts
    E = cfg.moe.n_experts
    # routed experts: the first E physical experts; the fused shared expert is E
    assert torch.equal(e.w13q, ex.w13_weight[:E].view(torch.uint8))
    assert e.w13s.data_ptr() == ex.w13_weight_scale_inv.data_ptr()  # scales in place
    assert torch.equal(e.ws13q, ex.w13_weight[E].view(torch.uint8))
    assert torch.equal(e.ws2s, ex.w2_weight_scale_inv[E])
    assert torch.equal(e.w_router_p, synth.pack_bf16(L.mlp.gate.weight))
    assert e.gamma.data_ptr() == L.post_attention_layernorm.weight.data_ptr()


def test_refusals(model):
    from types import SimpleNamespace

    from sgl_amd_mono.k2 import binding

    cfg, fc = _cfgs()
    L = model.model.layers[0]
    bad = SimpleNamespace(weight=L.self_attn.q_b_proj.weight, weight_scale_inv=L.self_attn.q_b_proj.weight_scale_inv,
                          aiter_bpreshuffled=True)
    with pytest.raises(ValueError, match="shuffled"):
        binding.linear("q_b_proj", bad, bad.weight.shape[0], bad.weight.shape[1], allow_shuffled=False)
    bf = SimpleNamespace(weight=L.self_attn.q_b_proj.weight.float().to(torch.bfloat16), aiter_bpreshuffled=True)
    with pytest.raises(ValueError, match="shuffled bf16"):
        binding.linear("q_b_proj", bf, bf.weight.shape[0], bf.weight.shape[1])
    with pytest.raises(ValueError, match="q_b_proj"):
        binding.linear("q_b_proj", L.self_attn.q_b_proj, 7, 7)
    with pytest.raises(ValueError, match="one format"):
        binding.bind_front(L, replace(fc, weight_fmt=0))
    from sgl_amd_mono.k2 import config as C

    with pytest.raises(ValueError, match="w13_weight"):  # block-FP8 experts bound as MXFP4
        binding.bind_moe(L, replace(cfg.moe, expert_fmt=C.FMT_MXFP4))
    with pytest.raises(ValueError, match="layout"):  # row-major experts bound as AITER's
        binding.bind_moe(L, replace(cfg.moe, weight_layout=C.WLAYOUT_AITER16))


def test_caches_are_views_of_the_pool():
    from sgl_amd_mono.k2 import binding

    pool = F.Pool(1, 8, torch.device("cpu"), 5)
    kv, idx = binding.layer_caches(pool, 0, True)
    assert kv.shape == (8 * 64, 576) and kv.dtype == torch.uint8
    assert kv.data_ptr() == pool.kv[0].data_ptr()
    assert idx.shape == (8, 64, 132) and idx.data_ptr() == pool.idx[0].data_ptr()


def test_shuffled_fp8_experts_are_read_in_place():
    """Block-FP8 experts SGLang rewrote for AITER's MoE (is_shuffled): bound in place,
    routed and the fused shared expert, as views of SGLang's tensors; the row-major
    model's experts are the same codes, copied into tiles."""
    from sgl_amd_mono.k2 import binding
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2.packing import aiter_unshuffle, pack_tiles

    cfg, _ = _cfgs()
    row = F.make_model(3, torch.device("cpu"), layers=1).model.layers[0]
    shf = F.make_model(3, torch.device("cpu"), layers=1, shuffled=True).model.layers[0]
    assert binding.experts_layout(row.mlp.experts) == C.WLAYOUT_TILES
    assert binding.experts_layout(shf.mlp.experts) == C.WLAYOUT_AITER16
    E = cfg.moe.n_experts
    a = binding.bind_moe(shf, replace(cfg.moe, weight_layout=C.WLAYOUT_AITER16))
    ex = shf.mlp.experts
    assert a.w13_p.data_ptr() == ex.w13_weight.data_ptr() and a.w2_p.data_ptr() == ex.w2_weight.data_ptr()
    assert a.ws13_p.data_ptr() == ex.w13_weight[E].data_ptr()
    t = binding.bind_moe(row, cfg.moe)
    assert torch.equal(aiter_unshuffle(a.w13_p), t.w13q) and torch.equal(aiter_unshuffle(a.ws2_p), t.ws2q)
    assert torch.equal(t.w13_p, pack_tiles(t.w13q, 32))


def test_mxfp4_experts_in_both_layouts():
    """MXFP4 experts (E2M1 bytes + E8M0 codes, the shared expert a separate block-FP8
    module): AITER's layout in place -- its bytes are the tiles -- and row-major ones
    copied into tiles, with the same codes; the separate shared expert is brought into
    the experts' layout."""
    from sgl_amd_mono.k2 import binding
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2.packing import aiter_shuffle, e8m0_shuffle, pack_e8m0, pack_tiles

    cfg, _ = _cfgs()
    mc = replace(cfg.moe, expert_fmt=C.FMT_MXFP4)
    row = F.make_model(4, torch.device("cpu"), layers=1, experts="mxfp4").model.layers[0]
    shf = F.make_model(4, torch.device("cpu"), layers=1, experts="mxfp4", shuffled=True).model.layers[0]
    t = binding.bind_moe(row, mc)
    a = binding.bind_moe(shf, replace(mc, weight_layout=C.WLAYOUT_AITER16))
    ex = shf.mlp.experts
    assert a.w13_p.data_ptr() == ex.w13_weight.data_ptr() and a.s2_p.data_ptr() == ex.w2_weight_scale.data_ptr()
    assert torch.equal(t.w13_p.flatten(), a.w13_p.flatten())  # E2M1: the same bytes
    assert torch.equal(e8m0_shuffle(t.w2s), a.s2_p) and torch.equal(pack_e8m0(t.w2s), t.s2_p)
    sh = row.mlp.shared_experts
    assert torch.equal(t.ws13_p, pack_tiles(sh.gate_up_proj.weight.view(torch.uint8), 32))
    # the shuffled model's shared expert is preshuffled already (in place); the
    # row-major one, shuffled, is the same bytes
    assert a.ws13_p.data_ptr() == shf.mlp.shared_experts.gate_up_proj.weight.data_ptr()
    assert torch.equal(a.ws13_p, aiter_shuffle(sh.gate_up_proj.weight.view(torch.uint8)))
    assert t.ws13s.data_ptr() == sh.gate_up_proj.weight_scale_inv.data_ptr()


def test_fp8_uk_uv_need_their_scale():
    """Per-tensor FP8 w_kc / w_vc are widened by the layer's scalar w_scale; without one
    (or with a non-scalar one) binding refuses, as the reference does."""
    from types import SimpleNamespace

    from sgl_amd_mono.k2 import binding

    g = torch.Generator().manual_seed(5)
    kc = (torch.randn(2, 8, 16, generator=g) * 4).to(torch.float8_e4m3fn)
    vc = (torch.randn(2, 16, 8, generator=g) * 4).to(torch.float8_e4m3fn)
    attn = SimpleNamespace(w_kc=kc, w_vc=vc)
    with pytest.raises(ValueError, match="w_scale"):
        binding._uk_uv(attn, 2, 8, 16, 8)
    attn.w_scale = torch.tensor([0.5, 0.5])
    with pytest.raises(ValueError, match="w_scale"):
        binding._uk_uv(attn, 2, 8, 16, 8)
    attn.w_scale = torch.tensor(0.25)
    uk, uv = binding._uk_uv(attn, 2, 8, 16, 8)
    assert torch.equal(uk.float(), (kc.float() * 0.25).bfloat16().float().transpose(1, 2))
    assert torch.equal(uv.float(), (vc.float() * 0.25).bfloat16().float().transpose(1, 2))
