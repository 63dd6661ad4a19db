"""The expert activation quantizers on the GPU, byte for byte against the oracle.

The MoE block quantizes two activations on the device, per expert mode: the
normalized rows (by the router tasks; the reference's quant_scaled / quant_mxfp8 /
quant_mx4, glm53/gfx950/kernel.py:1740-1777,5563-5614) and the SwiGLU mid (by the
up/gate tasks, kernel.py:6955-6985,7032-7060).  The reference pins its MXFP4 quant
bit for bit (test/kernels/glm53/check_mxfp4.py:40-60).  Here every launch's codes
and scales are read back from the workspace (mk2_moe_workspace_layout) and compared
with the oracle's quantizers (oracle/codecs.py):

  * normalized rows: xn equals the oracle's bf16(x * rstd * gamma) on every element
    outside refs.norm_rounding_slack (there within its one ulp); the codes and scales
    equal the oracle's quantizer applied to the kernel's own xn on EVERY element;
  * SwiGLU mid: the oracle forms mid = silu(g) * u in f64 from the kernel's own
    quantized rows and the dequantized expert weights.  The kernel's g and u are f32
    sums (MFMA partial sums, block scales, cross-wave adds) whose error is bounded by
    ACC_REL * sum_k |x_k w_k|; carried through silu(g) * u (and the hardware exp /
    rcp, MID_REL of mid) that gives each element an interval [mid - b, mid + b].
    Every kernel scale must be the oracle's rule applied to some amax in its block's
    interval, every code the oracle's quantization (on the kernel's scale) of some
    value in its element's interval, and at least 99 % of the codes (and scales) must
    equal the oracle's of mid itself.  A wrong rounding or scale rule moves whole
    blocks outside these intervals; cancellation near zero is what they admit.
"""

import pytest
import torch

from oracle import codecs as oc
from oracle import reference as R
from refs import MoEOracle, cpu, norm_rounding_slack

pytestmark = pytest.mark.gpu

EPS = 1e-6
MID_AGREE = 0.99


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _magnitude_order(codes, fmt):
    """Signed position of each code on its format's value grid (monotone in the value):
    E4M3 bytes, E2M1 nibbles or bf16 bit patterns."""
    c = codes.to(torch.int64)
    if fmt == "e4m3":
        sign, mag = (c >> 7) & 1, c & 0x7F
    elif fmt == "e2m1":
        sign, mag = (c >> 3) & 1, c & 0x7
    else:  # bf16 bits as int16
        c = c & 0xFFFF
        sign, mag = (c >> 15) & 1, c & 0x7FFF
    return torch.where(sign == 1, -mag, mag)


ACC_REL = 2.0**-19  # f32 sums of up to 6144 products: 32 eps of the absolute sum
MID_REL = 4e-6       # silu's hardware exp and reciprocal


def _codes_within(got, want, lo, hi, fmt, what):
    """Every code within [lo, hi] on its grid; >= MID_AGREE equal to `want`."""
    g = _magnitude_order(got, fmt)
    a, b = _magnitude_order(lo, fmt), _magnitude_order(hi, fmt)
    bad = (g < torch.minimum(a, b)) | (g > torch.maximum(a, b))
    assert not bool(bad.any()), (what, "codes outside their error interval", int(bad.sum()))
    agree = float((g == _magnitude_order(want, fmt)).double().mean())
    assert agree >= MID_AGREE, (what, agree)
    return agree


def _mid_interval(xq, w13, rows, inter):
    """(mid, b): the f64 SwiGLU mid of the given rows and the bound b of each element's
    f32 evaluation error."""
    gu = xq[rows] @ w13.double().T
    absum = xq[rows].abs() @ w13.double().abs().T
    g, u = gu[:, :inter], gu[:, inter:]
    sg = torch.sigmoid(g)
    mid = g * sg * u
    dmid_dg = u * sg * (1.0 + g * (1.0 - sg))
    b = ACC_REL * (absum[:, :inter] * dmid_dg.abs() + absum[:, inter:] * (g * sg).abs()) + MID_REL * mid.abs()
    return mid, b


def _nibbles(packed):
    """[..., n] bytes -> [..., 2n] E2M1 codes, the lower element in the low nibble."""
    return oc.fp4_unpack(packed)


def _act_dequant(fmt, a):
    """The kernel's own quantized rows as f32 (what its experts multiply)."""
    from sgl_amd_mono.k2 import config as C

    if fmt == C.FMT_MXFP4:
        return oc.mxfp8_dequant(cpu(a["xq"]), cpu(a["xs"]))
    if fmt == C.FMT_A4W4:
        return oc.mxfp4_dequant(cpu(a["xq"]), cpu(a["xs"]))
    if fmt == C.FMT_W8A8:
        return oc.fp8_block_act_dequant(cpu(a["xq"]), cpu(a["xsf"]))
    return cpu(a["xn"]).float()


def check_rows_quant(fmt, a, x=None, gamma=None, eps=EPS):
    """D2: the kernel's normalized rows (against the oracle's RMSNorm of x when given)
    and their codes and scales against the oracle's quantizer of those rows."""
    from sgl_amd_mono.k2 import config as C

    xn = cpu(a["xn"]).float()
    if x is not None:
        ref = R.rmsnorm(cpu(x).float(), cpu(gamma), eps)
        slack = norm_rounding_slack(cpu(x).float(), cpu(gamma), eps)
        d = (xn - ref).abs()
        assert bool((d[slack == 0] == 0).all()), "normalized rows off the oracle's bf16"
        assert bool((d <= slack).all()), "normalized rows off by more than their rounding slack"
    if fmt == C.FMT_MXFP4:
        q, s = oc.mxfp8_quant(xn)
        assert torch.equal(cpu(a["xs"]), s), "MXFP8 row scales"
        assert torch.equal(cpu(a["xq"]), q), "MXFP8 row codes"
    elif fmt == C.FMT_A4W4:
        q, s = oc.mxfp4_act_quant(xn)
        assert torch.equal(cpu(a["xs"]), s), "MXFP4 row scales"
        assert torch.equal(cpu(a["xq"]), q), "MXFP4 row codes"
    elif fmt == C.FMT_W8A8:
        q, s = oc.fp8_block_act_quant(xn)
        assert torch.equal(cpu(a["xsf"]), s), "FP8 per-128 row scales"
        assert torch.equal(cpu(a["xq"]), q), "FP8 per-128 row codes"
    else:
        assert a["xq"] is None and a["xs"] is None and a["xsf"] is None


def check_mid_quant(fmt, a, orc, ids):
    """E3: every routed slot's mid (and the shared expert's) against the oracle's mid of
    the kernel's own quantized rows.  Returns the code agreement of each part."""
    from sgl_amd_mono.k2 import config as C

    act = a["act"].tolist()
    ids = cpu(ids).long()
    want_experts = sorted(set(ids.flatten().tolist()))
    assert act == want_experts, ("distinct-expert list", act, want_experts)
    xq = _act_dequant(fmt, a).double()
    M = xq.shape[0]
    inter = orc.cfg.inter
    agree = {}
    for j, e in enumerate(act):
        rows = [r for r in range(M) if e in ids[r].tolist()] if a["compact"] else list(range(M))
        w13, _ = orc.expert_weights(e)
        mid, b = _mid_interval(xq, w13, rows, inter)
        n = len(rows)
        what = f"slot {j} (expert {e})"
        bf = lambda v: v.float().bfloat16().view(torch.int16)  # noqa: E731
        if fmt in (C.FMT_FP8, C.FMT_A16W4):
            got = cpu(a["mid_b"][j, :n]).contiguous().view(torch.int16)
            agree[j] = _codes_within(got, bf(mid), bf(mid - b), bf(mid + b), "bf16", what)
            continue
        if fmt == C.FMT_W8A8:
            blocks, bb = mid.view(n, inter // 128, 128), b.view(n, inter // 128, 128)
            amax, slack = blocks.abs().amax(-1), bb.amax(-1)
            got_s = cpu(a["mid_sf"][j, :n]).double()
            nz = amax > 0
            assert bool(((got_s * 448.0 - amax).abs() <= slack + 1e-6 * amax)[nz].all()), (what, "f32 scales")
            # codes of the oracle's mid on the kernel's own scales
            enc = lambda v: oc.e4m3_encode((v / got_s[..., None]).float()).view(n, inter)  # noqa: E731
            agree[j] = _codes_within(cpu(a["mid_q"][j, :n]), enc(blocks), enc(blocks - bb), enc(blocks + bb),
                                     "e4m3", what)
            continue
        # E8M0-scaled blocks of 32: MXFP8 (A8W4) or MXFP4 (A4W4)
        blocks, bb = mid.view(n, inter // 32, 32), b.view(n, inter // 32, 32)
        amax, slack = blocks.abs().amax(-1), bb.amax(-1)
        rule = oc.mxfp8_scale_code if fmt == C.FMT_MXFP4 else oc.mxfp4_act_code
        got_s = cpu(a["mid_s"][j, :n]).long()
        lo_s, hi_s = rule((amax - slack).clamp_min(0).float()), rule((amax + slack).float())
        assert bool(((got_s >= lo_s) & (got_s <= hi_s)).all()), (what, "E8M0 scales")
        assert float((got_s == rule(amax.float())).double().mean()) >= MID_AGREE, (what, "E8M0 scales")
        inv = torch.exp2(127.0 - got_s.double())[..., None]
        if fmt == C.FMT_MXFP4:
            enc = lambda v: oc.e4m3_encode((v * inv).float()).view(n, inter)  # noqa: E731
            agree[j] = _codes_within(cpu(a["mid_q"][j, :n]), enc(blocks), enc(blocks - bb), enc(blocks + bb),
                                     "e4m3", what)
        else:
            enc = lambda v: oc.e2m1_encode((v * inv).float().clamp(-6.0, 6.0)).view(n, inter)  # noqa: E731
            agree[j] = _codes_within(_nibbles(cpu(a["mid_q"][j, :n])), enc(blocks), enc(blocks - bb),
                                     enc(blocks + bb), "e2m1", what)
    if a["mid_sh"] is not None and orc.shared is not None:
        sw13, _ = orc.shared
        mid, b = _mid_interval(cpu(a["xn"]).double(), sw13, list(range(M)), sw13.shape[0] // 2)
        bf = lambda v: v.float().bfloat16().view(torch.int16)  # noqa: E731
        agree["shared"] = _codes_within(cpu(a["mid_sh"]).contiguous().view(torch.int16), bf(mid), bf(mid - b),
                                        bf(mid + b), "bf16", "shared mid")
    return agree


def _run_block(cfg, rows, seed, norm=True):
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import MoEOp

    dev = _dev()
    w = synth.make_moe(cfg, rows, seed, dev, norm=norm)
    op = MoEOp(cfg, w, rows, norm=norm, residual=True, eps=EPS)
    ids = torch.empty(rows, cfg.top_k, dtype=torch.int32, device=dev)
    op(w.x, topk_ids=ids)
    torch.cuda.synchronize()
    a = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in op.activations().items()}
    return w, a, ids


MODES = [("FP8", "C1_MOE"), ("MXFP4", "C2_MOE"), ("W8A8", "C1_MOE"), ("A16W4", "C2_MOE"), ("A4W4", "C2_MOE")]


@pytest.mark.parametrize("fmt,base", MODES)
@pytest.mark.parametrize("rows", [8, 32])
def test_moe_activation_bytes(fmt, base, rows):
    """Each expert mode, the MoE block alone with its RMSNorm, at 8 rows and at the
    verify width 32 (compacted expert rows for A8W4 and A4W4)."""
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C

    f = getattr(C, "FMT_" + fmt)
    cfg = replace(getattr(C, base), expert_fmt=f)
    w, a, ids = _run_block(cfg, rows, seed=900 + 10 * f + rows)
    assert a["compact"] == (rows > 16 and f in (C.FMT_MXFP4, C.FMT_A4W4))
    check_rows_quant(f, a, w.x, w.gamma)
    agree = check_mid_quant(f, a, MoEOracle(w), ids)
    print(fmt, rows, "mid code agreement: min", min(agree.values()))


def test_moe_activation_bytes_without_norm():
    """norm=0: the rows the quantizer reads are x itself."""
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C

    cfg = replace(C.C2_MOE, expert_fmt=C.FMT_A4W4)
    w, a, ids = _run_block(cfg, 8, seed=77, norm=False)
    assert torch.equal(cpu(a["xn"]), cpu(w.x))
    check_rows_quant(C.FMT_A4W4, a)
    check_mid_quant(C.FMT_A4W4, a, MoEOracle(w), ids)


@pytest.mark.parametrize("fmt", ["MXFP4", "W8A8"])
def test_layer_activation_bytes(fmt):
    """Inside the persistent layer launch (configs[4] at 8 rows, a shorter context): the
    router tasks normalize the attention output the launch produced itself."""
    from dataclasses import replace

    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import LayerOp

    dev = _dev()
    f = getattr(C, "FMT_" + fmt)
    cfg = replace(C.C5_LAYER, mla=replace(C.C5_LAYER.mla, context=8192),
                  indexer=replace(C.C5_LAYER.indexer, context=8192),
                  moe=replace(C.C5_LAYER.moe, expert_fmt=f))
    L = synth.make_layer(cfg, 8, seed=31 + f, device=dev)
    op = LayerOp(cfg, L, 8)
    attn = torch.empty(8, cfg.mla.hidden, dtype=torch.bfloat16, device=dev)
    ids = torch.empty(8, cfg.moe.top_k, dtype=torch.int32, device=dev)
    op(attn_out=attn, topk_ids=ids)
    torch.cuda.synchronize()
    op.check()
    a = op.moe_activations()
    check_rows_quant(f, a, attn, L.moe.gamma, cfg.eps)
    check_mid_quant(f, a, MoEOracle(L.moe), ids)
