"""FP4 indexer + exact top-k on the GPU (64 heads x 128, 65536 keys, top-2048).

Contract, after test/kernels/glm53/check_topk.py:56,116-165:
  * scores within 1e-4 of the row's largest |score| against the f64 oracle;
  * the list is exactly the oracle's radix-select list (12-bit prefix order, lowest
    position first on ties) of the kernel's OWN f32 scores -- bit-exact indices;
  * the selected set equals the oracle's exact top-k of its f64-then-f32 scores on
    rows whose k-th / k+1-th gap is clear of the score tolerance;
  * caches: random, ties (every key identical), zeros, ragged and short contexts.
"""

import pytest
import torch

from oracle import codecs as oc
from oracle import reference as R
from refs import cpu, indexer_oracle_scores

pytestmark = pytest.mark.gpu

SCORE_BOUND = 1e-4


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _run(cfg, rows, seed, ctx_len=None, mode="random"):
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import IndexerOp

    dev = _dev()
    ns = synth.make_indexer(cfg, rows, seed, dev, ctx_len=ctx_len)
    fp8 = ns.cache_scale is None
    if fp8 and mode in ("ties", "recent"):
        _fp8_mode(ns, mode, seed)
    elif mode == "ties":
        # every key = token 0 of page 1 (its chunk-c codes at c * 1024, scale at c * 64)
        v, s = ns.cache.view(-1, 4, 64, 16), ns.cache_scale.view(-1, 4, 64)
        v[:] = v[1, :, :1].clone()
        s[:] = s[1, :, :1].clone()
    elif mode == "zeros":
        ns.cache.zero_()
    elif mode == "recent":  # the last 4096 positions of every row score 16x higher
        for r in range(rows):
            n = int(ns.ctx_len[r])
            pages = ns.page_table[r, (n - 4096) // 64 : n // 64].long()
            sc = ns.cache_scale[pages]
            ns.cache_scale[pages] = (sc.int() + 4).clamp(max=254).to(torch.uint8)
    op = IndexerOp(cfg, rows, ns.page_table.shape[1], device=dev)
    scores, topk = op(ns.q, ns.w, ns.cache, ns.cache_scale, ns.page_table, ns.req_ids, ns.ctx_len)
    torch.cuda.synchronize()
    return ns, cpu(scores), cpu(topk).long()


def _fp8_mode(ns, mode, seed):
    """The FP8 pages' versions of the cases: every key identical ("ties"), or the last
    4096 positions' scales 16x ("recent")."""
    from sgl_amd_mono.k2 import quant, synth

    P = ns.cache.shape[0]
    if mode == "ties":
        key = torch.randn(128, generator=torch.Generator().manual_seed(seed))
        codes, sc = quant.quant_index_fp8(key.expand(P, 64, 128))
        ns.cache.copy_(synth.index_pages_fp8(codes, sc))
        return
    # positive head weights, so that a larger key gives a larger score (with weights of
    # mixed sign most of a row's scores can be negative, and 16x pushes those down)
    ns.w.abs_()
    flat = ns.cache.view(P, 64 * 132)
    for r in range(ns.rows):
        n = int(ns.ctx_len[r])
        for pg in ns.page_table[r, (n - 4096) // 64 : n // 64].long().tolist():
            s = flat[pg, 8192:].view(torch.float32) * 16
            flat[pg, 8192:] = s.view(torch.uint8)


def _check_rows(cfg, ns, scores, topk, expect_clear=True):
    k = cfg.topk
    n_clear = 0
    for r in range(ns.rows):
        n = int(ns.ctx_len[r])
        got = scores[r, :n]
        ref = indexer_oracle_scores(ns, r)
        err = ((got.double() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
        assert err <= SCORE_BOUND, (r, err)
        # the list: exact radix order of the kernel's own scores
        want = R.radix_lists(got, k)
        sel = topk[r]
        m = min(n, k)
        assert torch.equal(sel[:m], want), (r, sel[:8], want[:8])
        assert bool((sel[m:] == -1).all())
        # the set against the oracle's own scores: on every row, within the score
        # tolerance of the oracle's k-th score; exactly where the boundary is clear
        if n > k:
            keys = torch.sort(ref, descending=True).values
            tol = 2 * SCORE_BOUND * ref.abs().max().item()
            picked = torch.zeros(n, dtype=torch.bool)
            picked[sel[:m]] = True
            assert bool((ref[picked] >= keys[k - 1] - tol).all()), r
            assert bool((ref[~picked] <= keys[k - 1] + tol).all()), r
            gap = (keys[k - 1] - keys[k]).item()
            if gap > 2 * SCORE_BOUND * ref.abs().max().item():
                n_clear += 1
                oset = R.exact_topk_set(ref.float(), k)
                assert torch.equal(torch.sort(sel).values, oset), r
    if expect_clear:
        assert n_clear >= 1


def test_indexer_config4_full():
    from sgl_amd_mono.k2 import config as C

    cfg = C.C4_INDEXER
    ns, scores, topk = _run(cfg, 8, seed=41)
    _check_rows(cfg, ns, scores, topk)


def test_indexer_config4_verify_width():
    """configs[3] at the verify width, 32 rows over the full 65536 context: every
    workgroup runs several score chunks and slices of several rows (the standalone
    launch gives slices their tasks in start order by a ticket)."""
    from sgl_amd_mono.k2 import config as C

    cfg = C.C4_INDEXER
    ns, scores, topk = _run(cfg, 32, seed=47)
    # every row's list is the exact top-k of its own scores and within the score
    # tolerance of the oracle's; at 65536 keys a row whose k-th and k+1-th oracle scores
    # lie further apart than that tolerance (where the sets must be equal) is rare, so
    # none is required here (the 8-row case requires one)
    _check_rows(cfg, ns, scores, topk, expect_clear=False)


def test_indexer_ragged_and_short_rows():
    from sgl_amd_mono.k2 import config as C

    cfg = C.IndexerConfig(heads=64, dim=128, topk=2048, context=8192)
    ns, scores, topk = _run(cfg, 5, seed=42, ctx_len=[8192, 5003, 2049, 2048, 100])
    _check_rows(cfg, ns, scores, topk)


def test_indexer_fewer_heads_small_topk():
    from sgl_amd_mono.k2 import config as C

    cfg = C.IndexerConfig(heads=32, dim=128, topk=64, context=4096)
    ns, scores, topk = _run(cfg, 3, seed=43, ctx_len=[4096, 1000, 65])
    _check_rows(cfg, ns, scores, topk)


def test_indexer_ties_take_lowest_positions():
    from sgl_amd_mono.k2 import config as C

    cfg = C.IndexerConfig(heads=64, dim=128, topk=256, context=4096)
    ns, scores, topk = _run(cfg, 2, seed=44, mode="ties")
    for r in range(2):
        assert torch.unique(scores[r]).numel() == 1
        assert torch.equal(topk[r], torch.arange(256))
    _check_rows(cfg, ns, scores, topk, expect_clear=False)


def test_indexer_zero_keys():
    from sgl_amd_mono.k2 import config as C

    cfg = C.IndexerConfig(heads=64, dim=128, topk=128, context=2048)
    ns, scores, topk = _run(cfg, 2, seed=45, mode="zeros")
    assert bool((scores == 0).all())
    assert bool((oc.radix_keys(scores) == (1 << 31)).all())  # +0.0 everywhere, never -0.0
    for r in range(2):
        assert torch.equal(topk[r], torch.arange(128))


def test_indexer_recent_cluster():
    """Top keys clustered at the end of the context (the reference's 'recent' cache,
    check_topk.py:168-189): the sampled bound still holds and the list is exact."""
    from sgl_amd_mono.k2 import config as C

    cfg = C.IndexerConfig(heads=64, dim=128, topk=2048, context=65536)
    ns, scores, topk = _run(cfg, 2, seed=46, mode="recent")
    _check_rows(cfg, ns, scores, topk, expect_clear=False)
    for r in range(2):
        assert int((topk[r] >= 65536 - 4096).sum()) > 1500


# ------------------------------------------------- SGLang's FP8 DSA index cache
def _fp8(cfg):
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C

    return replace(cfg, keys=C.KEYS_FP8)


def test_indexer_fp8_cache_config4_full():
    """configs[3]'s shape with the keys in SGLang's FP8 index pages [pages, 64, 132]."""
    from sgl_amd_mono.k2 import config as C

    cfg = _fp8(C.C4_INDEXER)
    ns, scores, topk = _run(cfg, 8, seed=51)
    assert ns.cache.shape[1:] == (64, 132)
    # FP8 keys leave the 2048th and 2049th of 65536 scores closer than the score
    # tolerance on most rows: the set is checked within the tolerance there
    _check_rows(cfg, ns, scores, topk, expect_clear=False)


def test_indexer_fp8_cache_ragged_rows():
    from sgl_amd_mono.k2 import config as C

    cfg = _fp8(C.IndexerConfig(heads=48, dim=128, topk=2048, context=8192))
    ns, scores, topk = _run(cfg, 5, seed=52, ctx_len=[8192, 5003, 2049, 2048, 100])
    _check_rows(cfg, ns, scores, topk)


def test_indexer_fp8_cache_ties_take_lowest_positions():
    from sgl_amd_mono.k2 import config as C

    cfg = _fp8(C.IndexerConfig(heads=64, dim=128, topk=256, context=4096))
    ns, scores, topk = _run(cfg, 2, seed=53, mode="ties")
    for r in range(2):
        assert torch.unique(scores[r]).numel() == 1
        assert torch.equal(topk[r], torch.arange(256))
    _check_rows(cfg, ns, scores, topk, expect_clear=False)


def test_indexer_fp8_cache_recent_cluster():
    from sgl_amd_mono.k2 import config as C

    cfg = _fp8(C.IndexerConfig(heads=64, dim=128, topk=2048, context=65536))
    ns, scores, topk = _run(cfg, 2, seed=54, mode="recent")
    _check_rows(cfg, ns, scores, topk, expect_clear=False)
    for r in range(2):
        assert int((topk[r] >= 65536 - 4096).sum()) > 1500


# ----------------------------------- FP4 queries: the FP4 x FP4 scaled-MFMA scorer
def _q4(cfg):
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C

    return replace(cfg, keys=C.KEYS_FP4_Q4)


@pytest.mark.parametrize("rows", [8, 32])
def test_indexer_fp4_queries_full_context(rows):
    """configs[3]'s shape with the queries quantized to MXFP4 in the kernel
    (KEYS_FP4_Q4, quantize_fp4_indexer_row's rule) and scored on the FP4 x FP4 scaled
    MFMA: scores within 1e-4 of the f64 oracle of the quantized queries (refs.
    index_queries), the list exactly the radix-select list of the kernel's own scores,
    at the decode and the verify width."""
    from sgl_amd_mono.k2 import config as C

    cfg = _q4(C.C4_INDEXER)
    ns, scores, topk = _run(cfg, rows, seed=60 + rows)
    _check_rows(cfg, ns, scores, topk, expect_clear=False)


def test_indexer_fp4_queries_ragged_rows_fewer_heads():
    """48 heads (the A operands of the absent fourth head group are zero codes) over
    ragged and short rows."""
    from sgl_amd_mono.k2 import config as C

    cfg = _q4(C.IndexerConfig(heads=48, dim=128, topk=2048, context=8192))
    ns, scores, topk = _run(cfg, 5, seed=62, ctx_len=[8192, 5003, 2049, 2048, 100])
    _check_rows(cfg, ns, scores, topk)


def test_indexer_fp4_queries_ties_and_zeros():
    from sgl_amd_mono.k2 import config as C

    cfg = _q4(C.IndexerConfig(heads=64, dim=128, topk=256, context=4096))
    ns, scores, topk = _run(cfg, 2, seed=63, mode="ties")
    for r in range(2):
        assert torch.unique(scores[r]).numel() == 1
        assert torch.equal(topk[r], torch.arange(256))
    _check_rows(cfg, ns, scores, topk, expect_clear=False)
    ns, scores, topk = _run(cfg, 2, seed=64, mode="zeros")
    assert bool((scores == 0).all())
    assert bool((oc.radix_keys(scores) == (1 << 31)).all())
    for r in range(2):
        assert torch.equal(topk[r], torch.arange(256))


def test_indexer_lists_without_score_output():
    """with_scores=False (scores NULL at the C ABI): the launch keeps its scores in LDS
    and writes only the lists, which equal the lists of the launch that writes its
    scores, bit for bit, and the oracle's radix lists of those scores."""
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import IndexerOp

    dev = _dev()
    cfg = C.C4_INDEXER
    ns = synth.make_indexer(cfg, 8, 48, dev)
    op = IndexerOp(cfg, 8, ns.page_table.shape[1], device=dev)
    args = (ns.q, ns.w, ns.cache, ns.cache_scale, ns.page_table, ns.req_ids, ns.ctx_len)
    scores, topk = op(*args)
    none, lists = op(*args, with_scores=False)
    torch.cuda.synchronize()
    assert none is None and op.status() == 0
    assert torch.equal(lists, topk)
    for r in range(8):
        assert torch.equal(cpu(lists)[r].long(), R.radix_lists(cpu(scores)[r], cfg.topk))
