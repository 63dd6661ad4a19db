"""The layer parity checker (refs.check_layer) on the CPU: fed the oracle's own stage
outputs it passes; an error of a few percent planted in the attention term, in the
merged attention or in the MoE term (on the CPU, in the oracle's outputs) fails it.
With residual rows ~ N(0, 1) the attention term would drown in the bf16 rounding of
h + o W_o^T, which the checker reports as a rounding floor above its resolution."""

from dataclasses import replace

import pytest
import torch

from oracle import codecs as oc
from oracle import reference as R
from refs import MoEOracle, check_layer, indexer_oracle_scores, mla_oracle


def _cfg():
    from sgl_amd_mono.k2 import config as C

    moe = replace(C.C2_MOE, hidden=2048, n_experts=64)
    return replace(C.C5_LAYER, mla=replace(C.C5_LAYER.mla, hidden=2048, context=4096),
                   indexer=replace(C.C5_LAYER.indexer, context=4096), moe=moe)


def _oracle_outputs(L, attn_scale=1.0, olat_scale=1.0, moe_scale=1.0):
    """The oracle's stage outputs of layer L, in the kernel's output formats, with the
    attention term, o_latent or the MoE term scaled (a planted error)."""
    cfg = L.cfg
    rows, k = L.rows, cfg.indexer.topk
    scores = torch.zeros(rows, cfg.indexer.context)
    topk = torch.full((rows, k), -1, dtype=torch.int64)
    for r in range(rows):
        s = indexer_oracle_scores(L.idx, r).float()
        scores[r, : s.numel()] = s
        lst = R.radix_lists(s, k)
        topk[r, : lst.numel()] = lst
    olat, _, y = mla_oracle(L.mla, sel=topk, h=L.h, parts=True)
    attn = oc.bf16_round((L.h.double() + attn_scale * y).float())
    orc = MoEOracle(L.moe)
    _, ids, wts, logits, ymoe = orc(attn, norm=True, residual=True, eps=cfg.eps, parts=True)
    out = oc.bf16_round((attn.double() + moe_scale * ymoe).float())
    return [out, attn, scores, topk.int(), logits, ids.int(), wts], olat * olat_scale


@pytest.fixture(scope="module")
def layer_small_h():
    from sgl_amd_mono.k2 import synth

    return synth.make_layer(_cfg(), 2, 91, "cpu", h_std=1.0 / 128)


def test_check_layer_passes_the_oracle(layer_small_h):
    res, olat = _oracle_outputs(layer_small_h)
    stats = check_layer(layer_small_h, *res, o_latent=olat)
    assert stats["attn_term_checked"] and stats["moe_term_checked"]
    # the oracle against itself: only the bf16 rounding of the sums remains
    assert stats["attn_term_rel_l2"] <= 2 * stats["attn_term_floor"]
    assert stats["moe_term_rel_l2"] <= 2 * stats["moe_term_floor"]


@pytest.mark.parametrize("plant", [dict(attn_scale=1.05), dict(olat_scale=1.05), dict(moe_scale=1.05)])
def test_check_layer_catches_a_planted_five_percent_error(layer_small_h, plant):
    res, olat = _oracle_outputs(layer_small_h, **plant)
    with pytest.raises(AssertionError):
        check_layer(layer_small_h, *res, o_latent=olat)


def test_a_unit_residual_hides_the_attention_term():
    """With h ~ N(0, 1) the total attention output passes even with a 5 % error in the
    attention term (the dilution the small residual avoids), and the checker reports
    the term as unresolvable (floor > 3e-3) instead of claiming to have checked it."""
    from sgl_amd_mono.k2 import synth

    L = synth.make_layer(_cfg(), 2, 92, "cpu", h_std=1.0)
    res, olat = _oracle_outputs(L, attn_scale=1.05)
    out, attn = res[0], res[1]
    _, ref_attn = mla_oracle(L.mla, sel=res[3], h=L.h)
    assert R.rel_l2(attn, ref_attn) <= 1e-2  # diluted: the old check passed this
    stats = check_layer(L, *res)
    assert not stats["attn_term_checked"] and stats["attn_term_floor"] > 3e-3
