"""The chained K2 layer on the GPU (indexer -> MLA -> MoE) against the CPU oracle,
checked piecewise (refs.check_layer): exact top-k lists of the kernel's own scores,
scores within 1e-4 of f64, the merged attention (o_latent), the attention term
attn - h and the MoE term out - attn each within rel-L2 1e-2 of the oracle's own
terms, router logits within 1e-4 and expert ids exact on rows with a clear top-8
boundary.  The parity cases draw the residual rows h ~ N(0, (1/128)^2): with h ~ N(0,
1) the bf16 rounding of h + o W_o^T alone would be about 10 % of the attention term,
and a check of attn - h could not see the attention's own errors."""

from types import SimpleNamespace

import pytest
import torch

from refs import check_layer, cpu

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


H_STD = 1.0 / 128


def run_layer(cfg, rows, seed, staged=False, h_std=H_STD, draft=1):
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import LayerOp

    dev = _dev()
    L = synth.make_layer(cfg, rows, seed, dev, h_std=h_std, draft=draft)
    op = LayerOp(cfg, L, rows, device=dev, staged=staged)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    H, E, K = cfg.mla.hidden, cfg.moe.n_experts, cfg.moe.top_k
    attn = torch.empty(rows, H, dtype=torch.bfloat16, device=dev)
    scores = torch.empty(rows, cfg.indexer.context, dtype=torch.float32, device=dev)
    topk = torch.empty(rows, cfg.indexer.topk, dtype=torch.int32, device=dev)
    logits = torch.empty(rows, E, dtype=torch.float32, device=dev)
    ids = torch.empty(rows, K, dtype=torch.int32, device=dev)
    wts = torch.empty(rows, K, dtype=torch.float32, device=dev)
    olat = torch.empty(rows, cfg.mla.heads, cfg.mla.kv_lora, dtype=torch.float32, device=dev)
    out = op(attn_out=attn, scores=scores, topk=topk, logits=logits, topk_ids=ids, topk_weights=wts,
             status=status, o_latent=olat)
    torch.cuda.synchronize()
    if not staged:
        assert int(status.item()) == 0, "a dependency wait of the persistent launch gave up"
    return L, [cpu(t) for t in (out, attn, scores, topk, logits, ids, wts)], cpu(olat)


@pytest.mark.parametrize("staged", [False, True])
@pytest.mark.parametrize("rows", [1, 4, 8])
def test_layer_config5(rows, staged):
    from sgl_amd_mono.k2 import config as C

    L, res, olat = run_layer(C.C5_LAYER, rows, seed=500 + rows, staged=staged)
    stats = check_layer(L, *res, o_latent=olat)
    assert stats["attn_term_checked"] and stats["moe_term_checked"]  # both terms were resolvable and checked
    print(stats)


def test_layer_small_context_32_rows():
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C

    cfg = replace(C.C5_LAYER, mla=replace(C.C5_LAYER.mla, context=8192),
                  indexer=replace(C.C5_LAYER.indexer, context=8192))
    L, res, olat = run_layer(cfg, 32, seed=532)
    stats = check_layer(L, *res, o_latent=olat)
    assert stats["attn_term_checked"] and stats["moe_term_checked"]
    print(stats)


def test_layer_verify_width_full_context():
    """configs[4] at the verify width, 32 rows over the full 65536-position context,
    against the oracle: there the persistent launch runs the top-k selects as tasks of
    their own (32 rows x 32 chunks exceed the workgroups) and each workgroup keeps
    several score chunks in LDS for its slices."""
    from sgl_amd_mono.k2 import config as C

    L, res, olat = run_layer(C.C5_LAYER, 32, seed=533)
    stats = check_layer(L, *res, o_latent=olat)
    assert stats["attn_term_checked"] and stats["moe_term_checked"]
    print(stats)


@pytest.mark.parametrize("staged", [False, True])
def test_layer_verify_draft_layout(staged):
    """configs[4]'s verify step as its config names it: 8 requests x 4 draft tokens
    (32 rows, four a request sharing its index and latent-KV pages, at context lengths
    65533 .. 65536), persistent and staged, against the oracle."""
    from sgl_amd_mono.k2 import config as C

    L, res, olat = run_layer(C.C5_LAYER, 32, seed=534, staged=staged, draft=4)
    assert L.idx.req_ids.tolist() == [r // 4 for r in range(32)]
    stats = check_layer(L, *res, o_latent=olat)
    assert stats["attn_term_checked"] and stats["moe_term_checked"]
    print(stats)


@pytest.mark.parametrize("rows", [8, 32])
def test_layer_fp4_queries(rows):
    """configs[4] with the FP4 x FP4 index scorer (KEYS_FP4_Q4: the queries quantized to
    MXFP4 in the kernel), at the decode and the verify width over the full context,
    against the oracle of the quantized queries."""
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C

    cfg = replace(C.C5_LAYER, indexer=replace(C.C5_LAYER.indexer, keys=C.KEYS_FP4_Q4))
    L, res, olat = run_layer(cfg, rows, seed=560 + rows)
    stats = check_layer(L, *res, o_latent=olat)
    assert stats["attn_term_checked"] and stats["moe_term_checked"]
    print(stats)


@pytest.mark.parametrize("fmt", ["W8A8", "A16W4", "A4W4"])
def test_layer_expert_modes(fmt):
    """The persistent layer with each further expert mode in the MoE stages."""
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C

    cfg = replace(C.C5_LAYER, mla=replace(C.C5_LAYER.mla, context=8192),
                  indexer=replace(C.C5_LAYER.indexer, context=8192),
                  moe=replace(C.C5_LAYER.moe, expert_fmt=getattr(C, "FMT_" + fmt)))
    L, res, olat = run_layer(cfg, 8, seed=540 + cfg.moe.expert_fmt)
    stats = check_layer(L, *res, o_latent=olat)
    assert stats["attn_term_checked"] and stats["moe_term_checked"]
    print(stats)


@pytest.mark.parametrize("staged", [False, True])
def test_layer_fp8_index_cache(staged):
    """The layer reading its index keys from SGLang's FP8 DSA pages [pages, 64, 132]."""
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C

    cfg = replace(C.C5_LAYER, mla=replace(C.C5_LAYER.mla, context=8192),
                  indexer=replace(C.C5_LAYER.indexer, context=8192, keys=C.KEYS_FP8))
    L, res, olat = run_layer(cfg, 8, seed=550, staged=staged)
    assert L.idx.cache_scale is None and L.idx.cache.shape[1:] == (64, 132)
    stats = check_layer(L, *res, o_latent=olat)
    assert stats["attn_term_checked"] and stats["moe_term_checked"]
    print(stats)


@pytest.mark.parametrize("staged", [False, True])
def test_layer_pad_and_short_rows(staged):
    """Row lengths as the step tables give them: a pad row (no keys: no list, zero
    attention, its MoE on h alone), a one-key row, a short row and a full one."""
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C, synth
    from sgl_amd_mono.k2.ops import LayerOp

    dev = _dev()
    cfg = replace(C.C5_LAYER, mla=replace(C.C5_LAYER.mla, context=8192),
                  indexer=replace(C.C5_LAYER.indexer, context=8192))
    rows = 4
    L = synth.make_layer(cfg, rows, 560, dev, h_std=H_STD)
    L.idx.ctx_len.copy_(torch.tensor([8192, 0, 1, 2500], dtype=torch.int32))
    op = LayerOp(cfg, L, rows, device=dev, staged=staged)
    H, E, K = cfg.mla.hidden, cfg.moe.n_experts, cfg.moe.top_k
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    attn = torch.empty(rows, H, dtype=torch.bfloat16, device=dev)
    scores = torch.empty(rows, cfg.indexer.context, dtype=torch.float32, device=dev)
    topk = torch.empty(rows, cfg.indexer.topk, dtype=torch.int32, device=dev)
    logits = torch.empty(rows, E, dtype=torch.float32, device=dev)
    ids = torch.empty(rows, K, dtype=torch.int32, device=dev)
    wts = torch.empty(rows, K, dtype=torch.float32, device=dev)
    olat = torch.empty(rows, cfg.mla.heads, cfg.mla.kv_lora, dtype=torch.float32, device=dev)
    out = op(attn_out=attn, scores=scores, topk=topk, logits=logits, topk_ids=ids, topk_weights=wts,
             status=status, o_latent=olat)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    res = [cpu(t) for t in (out, attn, scores, topk, logits, ids, wts)]
    assert bool((res[3][1] == -1).all()) and res[3][2, 0] == 0 and bool((res[3][2, 1:] == -1).all())
    assert bool((cpu(olat)[1] == 0).all())  # no keys: zero attention
    assert torch.equal(res[1][1], cpu(L.h)[1])  # attn = h + 0
    assert bool(torch.isfinite(res[0]).all())
    stats = check_layer(L, *res, o_latent=cpu(olat))
    print(stats)


@pytest.mark.parametrize("rows", [8, 32])
def test_persistent_layer_repeats_and_matches_staged(rows):
    """Back-to-back persistent launches (counters reset by the launch itself) give the
    same bits each time and the same bits as the stage-by-stage path -- also at the
    verify width, 32 rows over the full 65536-position context, where every workgroup
    runs four score chunks and four slices and the up/gate and down take two column
    groups."""
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import LayerOp

    dev = _dev()
    cfg = C.C5_LAYER
    L = synth.make_layer(cfg, rows, 777, dev)
    p_op = LayerOp(cfg, L, rows, device=dev)
    s_op = LayerOp(cfg, L, rows, device=dev, staged=True)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    outs = [p_op(status=status).clone() for _ in range(3)]
    ref = s_op()
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    for o in outs:
        assert torch.equal(o, outs[0])
    assert torch.equal(outs[0], ref)


def test_persistent_layer_one_workspace_new_inputs():
    """One persistent op (one workspace) over alternating decode inputs (queries, key
    and latent caches, residual rows): every launch gives the stage-by-stage path's
    bits on the same inputs, so nothing a previous launch left in the workspace or in
    the caches is read back."""
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import LayerOp

    dev = _dev()
    cfg = C.C5_LAYER
    A = synth.make_layer(cfg, 8, 777, dev)
    B = synth.make_layer(cfg, 8, 778, dev)
    step = lambda L: [L.idx.q, L.idx.w, L.idx.cache, L.idx.cache_scale, L.mla.q, L.mla.kv, L.mla.kv_scale, L.h]  # noqa: E731
    saved = [t.clone() for t in step(A)]
    p_op = LayerOp(cfg, A, 8, device=dev)
    s_op = LayerOp(cfg, A, 8, device=dev, staged=True)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    outs = []
    for src in (saved, step(B), saved, step(B)):
        for dst, t in zip(step(A), src):
            dst.copy_(t)
        o = p_op(status=status).clone()
        ref = s_op().clone()
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        assert torch.equal(o, ref)
        outs.append(o)
    assert not torch.equal(outs[0], outs[1])
    assert torch.equal(outs[0], outs[2]) and torch.equal(outs[1], outs[3])


def test_persistent_layer_fail_stop():
    """A launch whose dependency waits have a deadline of one microsecond (wait_us=1)
    gives up: every workgroup skips the tasks it has left (fail-stop, as the
    reference's guard stops a launch) and the launch ORs 1 into the op's sticky status
    word, which LayerOp.check() turns into an error.  The stopped launch leaves the
    workspace ready by itself: the next launches, on the same workspace with nothing
    zeroed by the caller, give the staged path's bits, and they leave the status word
    as the stop left it until check() clears it."""
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import LayerOp

    dev = _dev()
    cfg = C.C5_LAYER
    L = synth.make_layer(cfg, 8, 779, dev)
    op = LayerOp(cfg, L, 8, device=dev, wait_us=1)
    ref = LayerOp(cfg, L, 8, device=dev, staged=True)().clone()
    for _ in range(2):  # two stops in a row: the second starts from the first's leftovers
        op.wait_us = 1
        op()
        torch.cuda.synchronize()
        assert int(op.status.item()) == 1
        op.wait_us = 0  # the default deadline, one second
        outs = [op().clone() for _ in range(2)]
        torch.cuda.synchronize()
        assert int(op.status.item()) == 1, "a completed launch must not clear the sticky word"
        with pytest.raises(RuntimeError, match="stopped early"):
            op.check()
        assert int(op.status.item()) == 0
        for o in outs:
            assert torch.equal(o, ref)
    op()
    op.check()  # a clean launch: no error


@pytest.mark.parametrize("rows", [8, 32])
def test_layer_aiter_layout_bits(rows):
    """The persistent layer with its experts in AITER's (16, 16) layout gives the
    tile layout's bits."""
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import LayerOp

    dev = _dev()
    cfg = replace(C.C5_LAYER, mla=replace(C.C5_LAYER.mla, context=8192),
                  indexer=replace(C.C5_LAYER.indexer, context=8192))
    L = synth.make_layer(cfg, rows, 560 + rows, dev)
    La = SimpleNamespace(**vars(L))
    La.moe = synth.moe_in_layout(L.moe, C.WLAYOUT_AITER16)
    cfga = replace(cfg, moe=La.moe.cfg)
    outs = []
    for c, LL in ((cfg, L), (cfga, La)):
        status = torch.zeros(1, dtype=torch.int32, device=dev)
        out = LayerOp(c, LL, rows, device=dev)(status=status)
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        outs.append(cpu(out))
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("staged", [False, True])
def test_layer_without_list_output_same_bits(staged):
    """A launch asked for no top-k output writes only the tagged list its splits read
    (keep_list 0): the layer's output equals, bit for bit, that of the launch that also
    writes the int32 lists for the caller."""
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import LayerOp

    dev = _dev()
    cfg = C.C5_LAYER
    L = synth.make_layer(cfg, 8, 561, dev, h_std=H_STD)
    op = LayerOp(cfg, L, 8, device=dev, staged=staged)
    topk = torch.empty(8, cfg.indexer.topk, dtype=torch.int32, device=dev)
    with_list = op(topk=topk).clone()
    without = op().clone()
    again = op(topk=topk).clone()
    torch.cuda.synchronize()
    op.check()
    assert torch.equal(with_list, without) and torch.equal(with_list, again)
    assert bool((topk >= 0).all())
