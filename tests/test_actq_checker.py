"""The byte checks of tests/test_gpu_act_quant.py on the CPU: fed an f32 evaluation of
the MoE block's activations quantized by the oracle's own rules (what a correct
kernel leaves, up to its f32 sum order) they pass in every expert mode; fed the same
with a planted mistake -- an E8M0 rounded down instead of up, E4M3 codes truncated
instead of rounded to nearest even, E2M1 ties rounded away from even -- they fail."""

from dataclasses import replace

import pytest
import torch

import test_gpu_act_quant as T
from oracle import codecs as oc
from oracle import reference as R
from refs import MoEOracle


def _fake(fmt, base, rows=8, plant=None):
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth

    # the configs' formats on a smaller block (64 experts, hidden 2048): the checks do
    # not depend on the size, and the CPU suite stays short
    cfg = replace(getattr(C, base), expert_fmt=fmt, n_experts=64, hidden=2048)
    w = synth.make_moe(cfg, rows, 5, "cpu", norm=True)
    orc = MoEOracle(w)
    xn = R.rmsnorm(w.x.float(), w.gamma, T.EPS)
    a = dict(xn=xn.bfloat16(), xq=None, xs=None, xsf=None, mid_q=None, mid_s=None, mid_sf=None, mid_b=None,
             mid_sh=None, compact=False)
    if fmt == C.FMT_MXFP4:
        a["xq"], a["xs"] = oc.mxfp8_quant(xn)
    elif fmt == C.FMT_A4W4:
        a["xq"], a["xs"] = oc.mxfp4_act_quant(xn)
    elif fmt == C.FMT_W8A8:
        a["xq"], a["xsf"] = oc.fp8_block_act_quant(xn)
    xd = T._act_dequant(fmt, a)
    logits = xn @ orc.w_router.T
    if cfg.router == C.ROUTER_SIGMOID_BIAS:
        ids, _ = R.route_sigmoid_bias(logits, orc.bias, cfg.top_k, cfg.route_scale)
    else:
        ids, _ = R.route_softmax(logits, cfg.top_k)
    act = sorted(set(ids.flatten().tolist()))
    a["act"] = torch.tensor(act)
    inter = cfg.inter
    mids = []
    for e in act:
        w13, _ = orc.expert_weights(e)
        gu = xd.float() @ w13.float().T  # f32, in torch's order
        mids.append(R.swiglu(gu[:, :inter], gu[:, inter:]))
    mid = torch.stack(mids)
    if fmt in (C.FMT_FP8, C.FMT_A16W4):
        a["mid_b"] = mid.bfloat16()
    elif fmt == C.FMT_MXFP4:
        a["mid_q"], a["mid_s"] = oc.mxfp8_quant(mid)
        if plant == "scale_down":
            a["mid_s"] = a["mid_s"] - 1
        if plant == "truncate":
            v = mid * torch.exp2(127.0 - a["mid_s"].float()).repeat_interleave(32, -1)
            c = oc.e4m3_encode(v)
            over = oc.e4m3_decode(c).abs() > v.abs()
            a["mid_q"] = torch.where(over & ((c & 0x7F) > 0), c - 1, c).to(torch.uint8)
    elif fmt == C.FMT_A4W4:
        a["mid_q"], a["mid_s"] = oc.mxfp4_act_quant(mid)
        if plant == "scale_down":
            a["mid_s"] = a["mid_s"] - 1
        if plant == "ties_away":
            v = (mid * torch.exp2(127.0 - a["mid_s"].float()).repeat_interleave(32, -1)).clamp(-6, 6)
            # round half away from zero on the E2M1 grid: a tie takes the larger magnitude
            m = v.abs()
            c = ((m >= 0.25).to(torch.uint8) + (m >= 0.75).to(torch.uint8) + (m >= 1.25).to(torch.uint8)
                 + (m >= 1.75).to(torch.uint8) + (m >= 2.5).to(torch.uint8) + (m >= 3.5).to(torch.uint8)
                 + (m >= 5.0).to(torch.uint8)) | (torch.signbit(v).to(torch.uint8) << 3)
            a["mid_q"] = oc.fp4_pack(c)
    else:
        a["mid_q"], a["mid_sf"] = oc.fp8_block_act_quant(mid)
    if cfg.n_shared:
        sw13, _ = orc.shared
        gu = xn.float() @ sw13.float().T
        a["mid_sh"] = R.swiglu(gu[:, :cfg.shared_inter], gu[:, cfg.shared_inter:]).bfloat16()
    return w, a, ids, orc


@pytest.mark.parametrize("fmt,base", T.MODES)
def test_checker_passes_a_correct_evaluation(fmt, base):
    from sgl_amd_mono.k2 import config as C

    f = getattr(C, "FMT_" + fmt)
    w, a, ids, orc = _fake(f, base)
    T.check_rows_quant(f, a, w.x, w.gamma)
    T.check_mid_quant(f, a, orc, ids)


@pytest.mark.parametrize("fmt,plant", [("MXFP4", "scale_down"), ("MXFP4", "truncate"), ("A4W4", "scale_down")])
def test_checker_catches_planted_mistakes(fmt, plant):
    from sgl_amd_mono.k2 import config as C

    f = getattr(C, "FMT_" + fmt)
    w, a, ids, orc = _fake(f, "C2_MOE", plant=plant)
    with pytest.raises(AssertionError):
        T.check_mid_quant(f, a, orc, ids)


def test_checker_catches_rows_quant_ties():
    """The normalized rows are bf16 values, so E2M1 ties are common there: rounding them
    away from even instead of to even fails the bit-exact row check."""
    from sgl_amd_mono.k2 import config as C

    w, a, ids, orc = _fake(C.FMT_A4W4, "C2_MOE")
    xn = a["xn"].float()
    blocks = xn.view(xn.shape[0], -1, 32)
    code = oc.mxfp4_act_code(blocks.abs().amax(-1))
    v = (blocks / torch.exp2(code.float() - 127.0)[..., None]).clamp(-6, 6).reshape(xn.shape)
    m = v.abs()
    c = ((m >= 0.25).to(torch.uint8) + (m >= 0.75).to(torch.uint8) + (m >= 1.25).to(torch.uint8)
         + (m >= 1.75).to(torch.uint8) + (m >= 2.5).to(torch.uint8) + (m >= 3.5).to(torch.uint8)
         + (m >= 5.0).to(torch.uint8)) | (torch.signbit(v).to(torch.uint8) << 3)
    a["xq"] = oc.fp4_pack(c)
    with pytest.raises(AssertionError, match="MXFP4 row codes"):
        T.check_rows_quant(C.FMT_A4W4, a)
