"""MoE block on the GPU against the CPU oracle (the FP8 block and the MXFP4 shard).

Contract (the reference's own checks, test/kernels/glm53/check_layer.py:631-698 and
glm53/gfx950/kernel.py:1967-1999):
  * expert ids: the kernel's picks equal the exact top-k of its own router scores
    (key desc, lower id first), and equal the oracle's where the k-th / k+1-th gap
    exceeds the logit tolerance;
  * router logits within 1e-4 of the largest logit of the row against the oracle (with
    RMSNorm, beyond what the bf16 rounding of near-midpoint normalized elements can
    move them: refs.norm_rounding_slack);
  * bf16 outputs within rel-L2 <= 1e-2 of the oracle (after FP8/FP4 dequant).
"""

import pytest
import torch

from refs import MoEOracle, cpu, logit_error, norm_rounding_slack
from oracle import reference as R
from oracle import codecs as oc

pytestmark = pytest.mark.gpu

REL_L2 = 1e-2
LOGIT_TOL = 1e-4
SIG_ULPS = 8  # the hardware sigmoid's distance from torch.sigmoid, in ulps of the row's largest score


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _run(cfg, rows, seed, norm=False, residual=False):
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import MoEOp

    dev = _dev()
    w = synth.make_moe(cfg, rows, seed, dev, norm=norm)
    op = MoEOp(cfg, w, rows, norm=norm, residual=residual, eps=1e-6)
    logits = torch.empty(rows, cfg.n_experts, dtype=torch.float32, device=dev)
    ids = torch.empty(rows, cfg.top_k, dtype=torch.int32, device=dev)
    wts = torch.empty(rows, cfg.top_k, dtype=torch.float32, device=dev)
    out = op(w.x, logits=logits, topk_ids=ids, topk_weights=wts)
    torch.cuda.synchronize()
    return w, cpu(out).float(), cpu(logits), cpu(ids).long(), cpu(wts)


def _check(cfg, w, out, logits, ids, wts, norm=False, residual=False):
    from sgl_amd_mono.k2 import config as C

    orc = MoEOracle(w)
    ref, rids, rw, rlogits = orc(w.x, norm=norm, residual=residual, eps=1e-6)
    # logits against the oracle
    slack = norm_rounding_slack(w.x.float(), orc.gamma, 1e-6) if norm else None
    assert logit_error(logits, rlogits, orc.w_router, slack) <= LOGIT_TOL
    # ids: exact top-k of the kernel's own scores.  The sigmoid router scores with the
    # hardware exp2 and rcp (as the reference kernel does, glm53/gfx950/kernel.py:
    # 5635-5639), within SIG_ULPS ulps of torch's sigmoid of the same logit: rows whose
    # k-th and k+1-th own scores lie that close may pick either, and there the picks
    # must be a top-k of the own scores up to that slack.
    if cfg.router == C.ROUTER_SIGMOID_BIAS:
        own_score = torch.sigmoid(logits) + orc.bias
        slack = SIG_ULPS * torch.finfo(torch.float32).eps * own_score.abs().amax(-1, keepdim=True)
        ref_keys = torch.sigmoid(rlogits) + orc.bias
    else:
        own_score = logits
        slack = torch.zeros(logits.shape[0], 1)
        ref_keys = rlogits
    own_keys = oc.radix_keys(own_score)
    own = torch.sort(own_keys, dim=-1, descending=True, stable=True).indices[:, : cfg.top_k]
    srt_own = torch.sort(own_score, dim=-1, descending=True).values
    own_clear = (srt_own[:, cfg.top_k - 1] - srt_own[:, cfg.top_k]) > 2 * slack[:, 0]
    assert torch.equal(ids[own_clear], own[own_clear]), (ids, own)
    for r in (~own_clear).nonzero().flatten().tolist():
        kth = srt_own[r, cfg.top_k - 1]
        picked = torch.zeros(own_score.shape[1], dtype=torch.bool)
        picked[ids[r]] = True
        assert len(set(ids[r].tolist())) == cfg.top_k
        assert bool((own_score[r][picked] >= kth - 2 * slack[r]).all())
        assert bool((own_score[r][~picked] <= kth + 2 * slack[r]).all())
    # ids: equal to the oracle's wherever the selection boundary is not a near tie
    srt = torch.sort(ref_keys, dim=-1, descending=True).values
    gap = srt[:, cfg.top_k - 1] - srt[:, cfg.top_k]
    clear = gap > 1e-4 * ref_keys.abs().amax(-1)
    assert clear.any()
    assert torch.equal(ids[clear], rids[clear])
    assert torch.allclose(wts[clear], rw[clear], rtol=1e-4, atol=1e-6)
    err = R.rel_l2(out, ref)
    assert err <= REL_L2, err
    return err


@pytest.mark.parametrize("rows", [1, 4, 8])
def test_moe_fp8_config1(rows):
    from sgl_amd_mono.k2 import config as C

    cfg = C.C1_MOE
    w, out, logits, ids, wts = _run(cfg, rows, seed=100 + rows)
    _check(cfg, w, out, logits, ids, wts)


@pytest.mark.parametrize("rows", [1, 8, 32])
def test_moe_mxfp4_config2(rows):
    from sgl_amd_mono.k2 import config as C

    cfg = C.C2_MOE
    w, out, logits, ids, wts = _run(cfg, rows, seed=200 + rows)
    _check(cfg, w, out, logits, ids, wts)


@pytest.mark.parametrize("hidden", [2048, 7168])
def test_moe_mxfp4_down_tiles(hidden):
    """Down tasks of 32 hidden rows (hidden not a multiple of 48; 6144 takes 24-row
    tasks), with the norm and the residual."""
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C

    cfg = replace(C.C2_MOE, hidden=hidden, n_experts=64)
    w, out, logits, ids, wts = _run(cfg, 8, seed=hidden, norm=True, residual=True)
    _check(cfg, w, out, logits, ids, wts, norm=True, residual=True)


def test_moe_mxfp4_norm_residual():
    from sgl_amd_mono.k2 import config as C

    cfg = C.C2_MOE
    w, out, logits, ids, wts = _run(cfg, 8, seed=7, norm=True, residual=True)
    _check(cfg, w, out, logits, ids, wts, norm=True, residual=True)


def test_selftest_mfma_layouts():
    """The three matrix-core operand modes against torch on one 16x16 tile."""
    import ctypes  # noqa: F401

    from sgl_amd_mono import _lib
    from sgl_amd_mono.k2.quant import quant_mxfp4

    dev = _dev()
    g = torch.Generator().manual_seed(3)
    a = torch.randn(16, 128, generator=g)
    b = torch.randn(16, 128, generator=g)
    d = torch.empty(16, 16, device=dev)
    L = _lib.lib()
    st = _lib.stream_handle(dev)

    def run(mode, a_, sa_, b_, sb_):
        keep = [t.to(dev).contiguous() if t is not None else None for t in (a_, sa_, b_, sb_)]
        ptrs = [t.data_ptr() if t is not None else None for t in keep]
        _lib.check(L.mk2_selftest_mfma(mode, ptrs[0], ptrs[1], ptrs[2], ptrs[3], d.data_ptr(), st))
        torch.cuda.synchronize()
        return cpu(d).clone()

    # mode 0: bf16 x bf16
    ab, bb = a.bfloat16(), b.bfloat16()
    got = run(0, ab, None, bb, None)
    assert torch.allclose(got, ab.float() @ bb.float().T, rtol=1e-5, atol=1e-4)
    # mode 2: E4M3 widened x bf16
    a8 = oc.e4m3_encode(a * 10)
    got = run(2, a8, None, bb, None)
    assert torch.allclose(got, oc.e4m3_decode(a8) @ bb.float().T, rtol=1e-5, atol=1e-3)
    # mode 2 again, every finite E4M3 code exactly: A holds code (128 i + k) mod 256
    # (NaN codes as zero), B picks one column k per output column, so d[i][j] is the
    # widened value of A[i][k_j] itself
    codes = torch.arange(16 * 128, dtype=torch.int64) % 256
    codes[(codes & 0x7F) == 0x7F] = 0
    a_all = codes.to(torch.uint8).view(16, 128)
    want = oc.e4m3_decode(a_all)
    for k0 in range(0, 128, 16):
        sel = torch.zeros(16, 128)
        sel[torch.arange(16), k0 + torch.arange(16)] = 1.0
        got = run(2, a_all, None, sel.bfloat16(), None)
        assert torch.equal(got, want[:, k0:k0 + 16].float()), k0
    # mode 1: E2M1 x E4M3 with E8M0 scales
    aq, asc = quant_mxfp4(a)
    bq, bsc = oc.mxfp8_quant(b)
    got = run(1, aq, asc, bq, bsc)
    ref = oc.mxfp4_dequant(aq, asc) @ oc.mxfp8_dequant(bq, bsc).T
    assert torch.allclose(got, ref, rtol=1e-4, atol=2e-3), (got - ref).abs().max()


@pytest.mark.parametrize("rows", [1, 8])
def test_moe_w8a8_config1(rows):
    """E4M3 weights with E4M3 activations, one f32 scale per 128 (the reference's W8A8
    MoeMode): the C1 shape with its FP8 block-scaled weights."""
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C

    cfg = replace(C.C1_MOE, expert_fmt=C.FMT_W8A8)
    w, out, logits, ids, wts = _run(cfg, rows, seed=300 + rows)
    _check(cfg, w, out, logits, ids, wts)


@pytest.mark.parametrize("fmt", ["A16W4", "A4W4"])
@pytest.mark.parametrize("rows", [1, 8, 32])
def test_moe_fp4_weight_modes_config2(fmt, rows):
    """E2M1 weights against bf16 activations (A16W4) and MXFP4 activations (A4W4), on
    the C2 shape."""
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C

    cfg = replace(C.C2_MOE, expert_fmt=getattr(C, "FMT_" + fmt))
    w, out, logits, ids, wts = _run(cfg, rows, seed=400 + rows + 7 * cfg.expert_fmt)
    _check(cfg, w, out, logits, ids, wts)


@pytest.mark.parametrize("fmt", ["W8A8", "A16W4", "A4W4"])
def test_moe_modes_norm_residual(fmt):
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C

    base = C.C1_MOE if fmt == "W8A8" else C.C2_MOE
    cfg = replace(base, expert_fmt=getattr(C, "FMT_" + fmt))
    w, out, logits, ids, wts = _run(cfg, 8, seed=11 + cfg.expert_fmt, norm=True, residual=True)
    _check(cfg, w, out, logits, ids, wts, norm=True, residual=True)


@pytest.mark.parametrize("fmt,rows", [("FP8", 4), ("W8A8", 8), ("MXFP4", 8), ("A16W4", 8), ("A4W4", 8),
                                      ("MXFP4", 32), ("FP8", 32)])
def test_moe_aiter_layout_bits(fmt, rows):
    """The experts (routed and shared) read in place in AITER's (16, 16) layout, as
    SGLang leaves them for AITER's MoE, give the same bits as the tile layout: the
    layouts change only where the kernels load a lane's bytes and scale codes."""
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import MoEOp

    dev = _dev()
    f = getattr(C, "FMT_" + fmt)
    cfg = replace(C.C2_MOE if f in C.FP4_WEIGHT_FMTS else C.C1_MOE, expert_fmt=f)
    w = synth.make_moe(cfg, rows, 720 + 10 * f + rows, dev, norm=True)
    wa = synth.moe_in_layout(w, C.WLAYOUT_AITER16)
    assert not torch.equal(wa.ws13_p, w.ws13_p)  # the shared expert is re-laid too
    outs = []
    for c, ww in ((cfg, w), (wa.cfg, wa)):
        ids = torch.empty(rows, cfg.top_k, dtype=torch.int32, device=dev)
        out = MoEOp(c, ww, rows, norm=True, residual=True, eps=1e-6)(w.x, topk_ids=ids)
        outs.append((cpu(out), cpu(ids)))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][0], outs[1][0])
