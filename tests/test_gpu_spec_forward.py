"""A routed decode step through the plugin on SGLang's model layout (tests/fake_sglang):
SPEC.build binds the model, forward() runs the step tables, every layer's front and
layer launch on the pool's caches, and the tail; its logits come back through the
logits processor.  Checks: this step's cache rows land at out_cache_loc and nothing
else moves; the last layer, launched again on the bound inputs with its checking
outputs, passes the layer oracle (refs.check_layer); the logits are the tail's of
that layer's output."""

from types import SimpleNamespace

import pytest
import torch

import fake_sglang as F
from refs import check_layer, cpu

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.mark.parametrize("rows", [1, 8])
def test_routed_decode_step(rows):
    from sgl_amd_mono import _registry as reg
    from sgl_amd_mono.k2 import spec
    from sgl_amd_mono.k2.ops import TailOp

    dev = _dev()
    pages = rows * (F.HF.max_context // 64) + 8
    lm = F.make_model(11, dev)
    pool = F.Pool(F.LAYERS, pages, dev, 12)
    st = F.make_step(rows, F.HF.max_context, pages, dev, 13 + rows)
    kv0 = [t.clone() for t in pool.kv]
    idx0 = [t.clone() for t in pool.idx]
    ctx = SimpleNamespace(device=dev, pool_of=lambda fb: pool, page_table_of=lambda fb, n: st.page_table[:n])
    fwd = spec.SPEC.build(lm, F.HF, ctx)
    plan = reg.Plan(key=reg.ShapeKey("decode", rows, 1))
    logits = fwd.forward(plan, st.input_ids, st.positions, st.forward_batch)
    torch.cuda.synchronize()
    assert logits.shape == (rows, F.VOCAB) and bool(torch.isfinite(logits).all())
    # this step's cache rows, and only those
    loc = cpu(st.forward_batch.out_cache_loc)
    for i in range(F.LAYERS):
        kv, kv_before = cpu(pool.kv[i]).view(torch.uint8).view(-1, 576), cpu(kv0[i]).view(torch.uint8).view(-1, 576)
        moved = (kv != kv_before).any(-1).nonzero().flatten()
        assert set(moved.tolist()) <= set(loc.tolist()) and len(moved) >= rows - 1
        ic, ic_before = cpu(pool.idx[i]).view(-1, 64, 132), cpu(idx0[i]).view(-1, 64, 132)
        pages_moved = (ic != ic_before).view(ic.shape[0], -1).any(-1).nonzero().flatten()
        assert set(pages_moved.tolist()) <= set((loc // 64).tolist())
    # the last layer again, with its checking outputs, against the oracle
    li = F.LAYERS - 1
    fo, lo = fwd.ops(li, rows)
    L, cfg = lo.L, lo.cfg
    H, E, K = cfg.mla.hidden, cfg.moe.n_experts, cfg.moe.top_k
    attn = torch.empty(rows, H, dtype=torch.bfloat16, device=dev)
    scores = torch.empty(rows, cfg.indexer.context, dtype=torch.float32, device=dev)
    topk = torch.empty(rows, cfg.indexer.topk, dtype=torch.int32, device=dev)
    lg = torch.empty(rows, E, dtype=torch.float32, device=dev)
    ids = torch.empty(rows, K, dtype=torch.int32, device=dev)
    wts = torch.empty(rows, K, dtype=torch.float32, device=dev)
    out = lo(attn_out=attn, scores=scores, topk=topk, logits=lg, topk_ids=ids, topk_weights=wts)
    torch.cuda.synchronize()
    last = plan.state[("h", li % 2, rows)]
    assert torch.equal(out, last)  # the step's own launch gave the same rows
    stats = check_layer(L, *[cpu(t) for t in (out, attn, scores, topk, lg, ids, wts)])
    print(stats)
    # every row's own new key is in its context and was scored
    for r in range(rows):
        assert int(L.idx.ctx_len[r]) == int(st.positions[r]) + 1
    want, _ = TailOp(fwd.tail_cfg, fwd.g_norm, fwd.w_head, rows, device=dev)(out)
    assert torch.equal(logits, want)


@pytest.mark.parametrize("experts", ["fp8", "mxfp4"])
def test_shuffled_experts_step_matches_row_major(experts):
    """The same model with its experts and block-FP8 linears in AITER's (16, 16)
    layout (read in place; W_o unshuffled into bf16 tiles) and row-major (experts
    copied into tiles): one routed step gives the same logits and caches."""
    from sgl_amd_mono import _registry as reg
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import spec

    dev = _dev()
    rows = 4
    pages = rows * (F.HF.max_context // 64) + 8
    res = []
    for shuffled in (False, True):
        lm = F.make_model(21, dev, experts=experts, shuffled=shuffled)
        pool = F.Pool(F.LAYERS, pages, dev, 22)
        st = F.make_step(rows, F.HF.max_context, pages, dev, 23)
        ctx = SimpleNamespace(device=dev, pool_of=lambda fb, p=pool: p,
                              page_table_of=lambda fb, n, s=st: s.page_table[:n])
        fwd = spec.SPEC.build(lm, F.HF, ctx)
        assert fwd.cfg.moe.weight_layout == (C.WLAYOUT_AITER16 if shuffled else C.WLAYOUT_TILES)
        assert fwd.cfg.moe.expert_fmt == (C.FMT_FP8 if experts == "fp8" else C.FMT_MXFP4)
        assert fwd.front_cfg.weight_fmt == (C.WFMT_FP8_AITER16 if shuffled else C.WFMT_FP8_BLOCK)
        logits = fwd.forward(reg.Plan(key=reg.ShapeKey("decode", rows, 1)), st.input_ids, st.positions,
                             st.forward_batch)
        torch.cuda.synchronize()
        res.append((cpu(logits), [cpu(t) for t in pool.kv]))
    assert torch.equal(res[0][0], res[1][0])
    assert all(torch.equal(a, b) for a, b in zip(res[0][1], res[1][1]))


def test_stopped_layer_gives_no_token():
    """A layer launch that stops early (its dependency waits given a deadline of one
    microsecond, so one gives up from the host's setting and every kernel exits normally) makes
    the step's logits NaN and the eager forward raise; once the words are cleared, the
    next step runs clean on the same ops and workspaces."""
    from sgl_amd_mono import _registry as reg
    from sgl_amd_mono.k2 import spec

    dev = _dev()
    rows = 4
    pages = rows * (F.HF.max_context // 64) + 8
    lm = F.make_model(31, dev)
    pool = F.Pool(F.LAYERS, pages, dev, 32)
    st = F.make_step(rows, F.HF.max_context, pages, dev, 33)
    ctx = SimpleNamespace(device=dev, pool_of=lambda fb: pool, page_table_of=lambda fb, n: st.page_table[:n])
    fwd = spec.SPEC.build(lm, F.HF, ctx)
    plan = reg.Plan(key=reg.ShapeKey("decode", rows, 1))
    fwd.forward(plan, st.input_ids, st.positions, st.forward_batch)  # builds the ops; a clean step
    torch.cuda.synchronize()
    _, lo = fwd.ops(1, rows)
    lo.wait_us = 1
    _, logits = fwd.backbone(plan, st.input_ids, st.positions, st.forward_batch)
    torch.cuda.synchronize()
    assert int(fwd._status.item()) == 1
    assert bool(torch.isnan(logits).all())
    with pytest.raises(RuntimeError, match="stopped early"):
        fwd.check(rows)  # clears the words
    with pytest.raises(RuntimeError, match="stopped early"):
        fwd.forward(plan, st.input_ids, st.positions, st.forward_batch)
    lo.wait_us = 0
    logits = fwd.forward(plan, st.input_ids, st.positions, st.forward_batch)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(logits).all())


def test_fused_front_and_layer_step():
    """A model with C7's front (hidden 6144, q_lora 2048, nope 192, 64 index heads) and
    MXFP4 experts: the library fuses each layer's front with the layer
    (mk2_layer_step_is_fused) and the routed step runs ONE launch a layer
    (LayerStepOp); its logits and caches equal, bit for bit, those of the same step with
    each front and layer launched apart."""
    from sgl_amd_mono import _registry as reg
    from sgl_amd_mono.k2 import spec

    dev = _dev()
    rows = 4
    hf = SimpleNamespace(**{**vars(F.HF), "hidden_size": 6144, "q_lora_rank": 2048, "qk_nope_head_dim": 192,
                            "index_n_heads": 64})
    pages = rows * (hf.max_context // 64) + 8
    res = []
    for fuse in (True, False):
        lm = F.make_model(71, dev, hf=hf, experts="mxfp4")
        pool = F.Pool(F.LAYERS, pages, dev, 72)
        st = F.make_step(rows, hf.max_context, pages, dev, 73)
        ctx = SimpleNamespace(device=dev, pool_of=lambda fb, p=pool: p,
                              page_table_of=lambda fb, n, s=st: s.page_table[:n])
        fwd = spec.SPEC.build(lm, hf, ctx)
        fwd.fuse_front = fuse
        logits = fwd.forward(reg.Plan(key=reg.ShapeKey("decode", rows, 1)), st.input_ids, st.positions,
                             st.forward_batch)
        torch.cuda.synchronize()
        assert all((fwd.fused(li, rows) is not None) == fuse for li in range(F.LAYERS))
        res.append((cpu(logits), [cpu(t) for t in pool.kv], [cpu(t) for t in pool.idx]))
    assert bool(torch.isfinite(res[0][0]).all())
    assert torch.equal(res[0][0], res[1][0])
    assert all(torch.equal(a, b) for a, b in zip(res[0][1], res[1][1]))
    assert all(torch.equal(a, b) for a, b in zip(res[0][2], res[1][2]))
