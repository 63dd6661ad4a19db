"""Closed-form pins of the oracle functions that the layer's parity rests on:
expert_mxfp4, expert_fp8, expert_a4w4, expert_w8a8, mla_output, o_proj, moe_mix,
fp8_row_dequant and the MXFP4 / FP8 per-128 activation rules.

Every input is chosen so the exact answer can be written down by hand: weights that
E2M1 x E8M0 (or E4M3) represent exactly, activations whose MXFP8 blocks have a known
E8M0 and elements on E4M3 rounding ties, values on bf16 rounding ties, permutation
matrices (not involutions, so a transposed operand shows).  The expected numbers are
literals derived in the comments, not recomputed by the oracle's own formula.  Each
pin also runs a copy of the function with one planted mistake (a dropped rounding or
quantization step, a transposed operand, a wrong broadcast) and checks that the pin
catches it (after test/kernels/glm53/check_topk.py:150-165).

Reference points: MXFP8 activations and A8W4 experts glm53/gfx950/kernel.py:1284-1307,
1752-1766, 7032-7060; bf16 hand-offs of o_lat and W_UV kernel.py:5340-5385; W_o +
residual kernel.py:5391-5469; E4M3 rows with a per-token scale (the latent cache).
"""

import math

import pytest
import torch

from oracle import codecs as oc
from oracle import reference as R


def _exact(got, want):
    got, want = torch.as_tensor(got, dtype=torch.float64), torch.as_tensor(want, dtype=torch.float64)
    return got.shape == want.shape and bool(torch.equal(got, want))


# --------------------------------------------------------------------------- experts
def _mxfp4_expert_case():
    """H = 64 (two 32-blocks), inter = 32 (one mid block).  Returns x [1, 64], w13
    [64, 64] (gate rows 0..31, up rows 32..63), w2 [64, 32], the expected y [64].

    x block A = x[0:32]: amax 50, 50 * f32(1/448) = 0.1116 -> ceil-pow2 2^-3 (E8M0 124);
      q = x * 8:  400 -> tie of 384 (mant 100) and 416 (101) -> 384 -> xq 48
                   68 -> tie of 64 (000) and 72 (001)     -> 64  -> xq 8
                   76 -> tie of 72 (001) and 80 (010)     -> 80  -> xq 10
    x block B = x[32:64]: amax 3 -> 0.0067 -> 2^-7 (E8M0 120); q = x * 128:
                  384 exact -> xq 3;  68 -> 64 -> xq 0.5;  76 -> 80 -> xq 0.625;
                   56 exact -> xq 0.4375
    gate (row i, one weight on one column) and up give g, u, mid = silu(g) * u; silu(g)
    = g exactly in f32 for g >= 18 (exp(-g) < half an ulp of 1):
      i=0: 3.0 * xq[0] = 144,   2.0 * xq[32] = 6      -> mid 864
      i=1: 1.5 * xq[0] = 72,    1.5 * xq[33] = 0.75   -> mid 54
      i=2: 1.0 * xq[0] = 48,    2.0 * xq[35] = 0.875  -> mid 42
      i=3: 0.375 * xq[0] = 18, -1.0 * xq[34] = -0.625 -> mid -11.25
      i=4: -0.5 * xq[0] = -24,  1.0 * xq[32] = 3      -> mid ~ -2.7e-9
      i=5: 3.0 * xq[1] = 24,    1.0 * xq[33] = 0.5    -> mid 12
      i=6: 2.0 * xq[2] = 20,    1.0 * xq[32] = 3      -> mid 60
    mid block: amax 864 -> 1.93 -> 2 (E8M0 128); q = mid / 2:
      432 -> tie of 416 (101) and 448 (110) -> 448 -> 896
       27 -> tie of 26 (101) and 28 (110)   -> 28  -> 56
       21 -> tie of 20 (010) and 22 (011)   -> 20  -> 40
      -5.625 -> nearest -5.5                       -> -11
      -1.4e-9 -> -0                                -> -0
        6 -> 12;   30 -> 60
    down: w2[h, h] = 1 (h < 32), w2[32 + i, i] = 0.5.
    """
    x = torch.zeros(1, 64)
    x[0, 0], x[0, 1], x[0, 2] = 50.0, 8.5, 9.5
    x[0, 32], x[0, 33], x[0, 34], x[0, 35] = 3.0, 0.53125, 0.59375, 0.4375
    w13 = torch.zeros(64, 64)
    for i, (gc, gw, uc, uw) in enumerate([(0, 3.0, 32, 2.0), (0, 1.5, 33, 1.5), (0, 1.0, 35, 2.0),
                                          (0, 0.375, 34, -1.0), (0, -0.5, 32, 1.0), (1, 3.0, 33, 1.0),
                                          (2, 2.0, 32, 1.0)]):
        w13[i, gc] = gw
        w13[32 + i, uc] = uw
    w2 = torch.zeros(64, 32)
    for i in range(32):
        w2[i, i] = 1.0
        w2[32 + i, i] = 0.5
    mq = torch.zeros(32)
    mq[:7] = torch.tensor([896.0, 56.0, 40.0, -11.0, -0.0, 12.0, 60.0])
    y = torch.cat([mq, 0.5 * mq])
    return x, w13, w2, y


def test_expert_mxfp4_weights_are_exact_mxfp4():
    _, w13, w2, _ = _mxfp4_expert_case()
    for w in (w13, w2):
        assert torch.equal(oc.mxfp4_dequant(*oc.mxfp4_quant(w)), w)


def test_expert_mxfp4_closed_form():
    x, w13, w2, y = _mxfp4_expert_case()
    assert _exact(R.expert_mxfp4(x, w13, w2)[0], y)


def _planted_mxfp4(x, w13, w2, quant_x=True, quant_mid=True, ties_up=False):
    """expert_mxfp4 with one step dropped or altered (the negative controls)."""
    def q8(v):
        if ties_up:  # E4M3 ties rounded away from zero instead of to even
            codes, sc = oc.mxfp8_quant(v)
            inv = torch.exp2(127.0 - sc.float()).repeat_interleave(32, -1)
            return oc.mxfp8_dequant(oc.e4m3_encode(v * inv * (1 + 2.0**-20)), sc)
        return oc.mxfp8_dequant(*oc.mxfp8_quant(v))
    inter = w13.shape[0] // 2
    xq = q8(x) if quant_x else x
    gu = xq @ w13.T
    mid = R.swiglu(gu[..., :inter], gu[..., inter:])
    mq = q8(mid) if quant_mid else mid
    return mq @ w2.T


@pytest.mark.parametrize("plant", [dict(quant_x=False), dict(quant_mid=False), dict(ties_up=True)])
def test_expert_mxfp4_pin_catches_planted_mistakes(plant):
    x, w13, w2, y = _mxfp4_expert_case()
    assert _exact(_planted_mxfp4(x, w13, w2), y[None])  # the unplanted copy agrees
    assert not _exact(_planted_mxfp4(x, w13, w2, **plant), y[None])


def test_expert_fp8_mid_rounds_to_bf16_on_ties():
    """gate = 32 * x0 (silu(32) = 32 in f32); up = x0 + x1 with x1 = 2^-8 or 3 * 2^-8,
    so mid = 32 + 2^-3 (tie of 32 and 32.25 -> 32) or 32 + 0.375 (tie of 32.25 and 32.5
    -> 32.5); W2 = identity.  Without mid's bf16 rounding the answer is 32.125 / 32.375."""
    x = torch.tensor([[1.0, 2.0**-8], [1.0, 3 * 2.0**-8]])
    w13 = torch.tensor([[32.0, 0.0], [1.0, 1.0]])  # gate row, up row (E4M3 values)
    w2 = torch.tensor([[1.0]])
    y = R.expert_fp8(x, w13, w2)
    assert _exact(y[:, 0], [32.0, 32.5])
    gu = x @ w13.T
    planted = R.swiglu(gu[:, :1], gu[:, 1:]) @ w2.T  # mid not rounded
    assert not _exact(planted[:, 0], [32.0, 32.5])


def test_moe_mix_is_the_route_weighted_sum():
    """Experts that scale their input by (e + 1) and a shared expert that adds 100:
    y = sum_k w_k (id_k + 1) x + 100, exactly (powers-of-two weights)."""
    x = torch.tensor([[1.0, -2.0], [0.5, 4.0]])
    ids = torch.tensor([[3, 0], [1, 2]])
    w = torch.tensor([[0.5, 0.25], [2.0, 0.125]])
    y = R.moe_mix(x, ids, w, lambda e, xr: (e + 1) * xr, lambda xr: torch.full_like(xr, 100.0))
    want = torch.stack([(0.5 * 4 + 0.25 * 1) * x[0], (2.0 * 2 + 0.125 * 3) * x[1]]) + 100.0
    assert _exact(y, want)
    planted = R.moe_mix(x, ids, w.flip(-1), lambda e, xr: (e + 1) * xr, lambda xr: torch.full_like(xr, 100.0))
    assert not _exact(planted, want)  # weights paired with the wrong slots


# ------------------------------------------------------------------ W_UV and W_o
E8, E7, E6 = 2.0**-8, 2.0**-7, 2.0**-6


def _mla_output_case():
    """2 heads, v_dim 4, kv_lora 8.  o_lat and W_UV, with the expected bf16 o.

    bf16(o_lat[0]) = [1, 1 + 2^-6, 2, -1, 0.5, 0.25, 3, 0]   (ties: 1 + 2^-8 -> 1,
      1 + 3 * 2^-8 -> 1 + 2^-6, 2 + 2^-7 -> 2, 0.25 + 2^-10 -> 0.25)
    bf16(o_lat[1]) = [1, 5, 0.75, -2, 1.5, 6, 0.125, 2^-8]
    head 0 rows pick columns 1, 3, 5 and 2 * column 2: [1 + 2^-6, -1, 0.25, 4]
    head 1: v0 = c0 + c7 = 1 + 2^-8 -> tie -> 1;  v1 = 0.5 * c1 = 2.5;
            v2 = -c3 + c6 = 2.125;  v3 = c4 + 3 * c7 = 1.51171875 -> tie of 1.5078125 and
            1.515625 -> 1.515625
    """
    o_lat = torch.tensor([
        [1 + E8, 1 + 3 * E8, 2 + E7, -(1 + E8), 0.5, 0.25 + 2.0**-10, 3.0, 0.0],
        [1 + E8, 5.0, 0.75, -2.0, 1.5, 6.0, 0.125, E8],
    ])
    w_uv = torch.zeros(2, 4, 8)
    w_uv[0, 0, 1] = 1.0
    w_uv[0, 1, 3] = 1.0
    w_uv[0, 2, 5] = 1.0
    w_uv[0, 3, 2] = 2.0
    w_uv[1, 0, 0] = w_uv[1, 0, 7] = 1.0
    w_uv[1, 1, 1] = 0.5
    w_uv[1, 2, 3], w_uv[1, 2, 6] = -1.0, 1.0
    w_uv[1, 3, 4], w_uv[1, 3, 7] = 1.0, 3.0
    want = [1 + E6, -1.0, 0.25, 4.0, 1.0, 2.5, 2.125, 1.515625]
    return o_lat, w_uv, want


def test_mla_output_closed_form():
    o_lat, w_uv, want = _mla_output_case()
    assert _exact(R.mla_output(o_lat, w_uv), want)


@pytest.mark.parametrize("plant", ["no_lat_round", "no_out_round", "transposed_uv"])
def test_mla_output_pin_catches_planted_mistakes(plant):
    o_lat, w_uv, want = _mla_output_case()
    ol = o_lat if plant == "no_lat_round" else oc.bf16_round(o_lat)
    w = w_uv[:, :, :4].transpose(1, 2) if plant == "transposed_uv" else w_uv[:, :, :]
    if plant == "transposed_uv":  # W_UV read as [c][v] (the first 4 latent dims only)
        o = torch.einsum("hcv,hc->hv", w, ol[:, :4])
    else:
        o = torch.einsum("hvc,hc->hv", w, ol)
    o = o if plant == "no_out_round" else oc.bf16_round(o)
    assert not _exact(o.flatten(), want)


def _o_proj_case():
    """W_o = the permutation n <- k = perm[n], perm = [2, 0, 3, 1] (not an involution).
    y = o W_o^T: row 0 [0.5, 1 + 2^-7, -2, 3], row 1 [2^-8, 1, 10, 1 + 2^-7].
    With h: row 0: 0.5 + 2^-9 -> tie -> 0.5;  1 + 3 * 2^-8 -> tie -> 1 + 2^-6;
                   -2 + 2^-7 = -1.9921875 (exact);  3 + 2^-6 (exact)
            row 1: 1 + 2^-8 -> tie -> 1 (twice);  10 + 2^-5 -> tie of 10 and 10.0625 -> 10;
                   1 + 5 * 2^-8 -> tie of 1.015625 and 1.0234375 -> 1.015625"""
    o = torch.tensor([[1 + E7, 3.0, 0.5, -2.0], [1.0, 1 + E7, E8, 10.0]])
    perm = [2, 0, 3, 1]
    w_o = torch.zeros(4, 4)
    for n, k in enumerate(perm):
        w_o[n, k] = 1.0
    h = torch.tensor([[2.0**-9, E8, E7, E6], [1.0, E8, 2.0**-5, 3 * E8]])
    want_h = [[0.5, 1 + E6, -1.9921875, 3.015625], [1.0, 1.0, 10.0, 1.015625]]
    want_0 = [[0.5, 1 + E7, -2.0, 3.0], [E8, 1.0, 10.0, 1 + E7]]
    return o, w_o, h, want_h, want_0


def test_o_proj_closed_form():
    o, w_o, h, want_h, want_0 = _o_proj_case()
    assert _exact(R.o_proj(o, w_o, h), want_h)
    assert _exact(R.o_proj(o, w_o, None), want_0)


def test_o_proj_pin_catches_planted_mistakes():
    o, w_o, h, want_h, want_0 = _o_proj_case()
    assert not _exact(oc.bf16_round(h + o @ w_o), want_h)  # W_o not transposed
    assert not _exact(h + o @ w_o.T, want_h)  # no bf16 rounding of the sum


# ----------------------------------------------------------- E4M3 rows with a scale
def _e4m3_from_bits(b: int) -> float:
    """E4M3 (fn) from its bit fields: sign, 4-bit exponent (bias 7), 3-bit mantissa;
    exponent 0 is subnormal (m / 8 * 2^-6); 0x7F / 0xFF are NaN."""
    s, e, m = b >> 7, (b >> 3) & 15, b & 7
    if e == 15 and m == 7:
        return math.nan
    v = (m / 8.0) * 2.0**-6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
    return -v if s else v


def test_fp8_row_dequant_all_codes_and_scales():
    codes = torch.arange(256, dtype=torch.int64).to(torch.uint8)
    table = torch.tensor([_e4m3_from_bits(b) for b in range(256)], dtype=torch.float64)
    finite = ~torch.isnan(table)
    scales = torch.tensor([1.0, 0.5, 3.0, 2.0**-20, 448.0])
    rows = codes[None].repeat(len(scales), 1)
    got = oc.fp8_row_dequant(rows, scales).double()
    want = table[None] * scales.double()[:, None]
    assert torch.equal(got[:, finite], want[:, finite])
    assert bool(torch.isnan(got[:, ~finite]).all())
    # planted: the scale broadcast along the row instead of per row
    sq = rows[:, :5]
    planted = oc.e4m3_decode(sq) * scales[None, :]
    assert not torch.equal(planted.double(), table[None, :5] * scales.double()[:, None])


# ------------------------------------------------------ MXFP4 and FP8 per-128 activations
def test_mxfp4_act_code_closed_form():
    """ceil-pow2 of amax/6 through the f32 bits: 6 -> 1 (127), 6.1 -> 2 (128), 3 -> 1/2
    (126), 24 -> 4 (129), 0 -> 0; f32(1/6) rounds up, so 6 * f32(1/6) is exactly 1."""
    amax = torch.tensor([6.0, 6.1, 3.0, 24.0, 0.0, 12.0, 12.0001])
    assert oc.mxfp4_act_code(amax).tolist() == [127, 128, 126, 129, 0, 128, 129]


def test_mxfp4_act_quant_ties_to_even():
    """A block of amax 24 (scale 4): x/4 = 6, 2.5 (tie of 2 and 3 -> 2), 3.5 (tie of 3
    and 4 -> 4), 0.25 (tie of 0 and 0.5 -> 0), 0.75 (tie of 0.5 and 1 -> 1), 1.25 (tie of
    1 and 1.5 -> 1), 1.75 (tie of 1.5 and 2 -> 2), -5 (tie of -4 and -6 -> -4)."""
    x = torch.zeros(32)
    x[:8] = torch.tensor([24.0, 10.0, 14.0, 1.0, 3.0, 5.0, 7.0, -20.0])
    b, s = oc.mxfp4_act_quant(x)
    assert s.tolist() == [129]
    want = torch.zeros(32)
    want[:8] = torch.tensor([24.0, 8.0, 16.0, 0.0, 4.0, 4.0, 8.0, -16.0])
    assert _exact(oc.mxfp4_dequant(b, s), want)
    # planted: ties rounded away from zero
    q = x / 4.0
    planted = torch.sign(q) * torch.tensor([oc.E2M1_VALUES[min(range(8), key=lambda c: (abs(abs(v) - oc.E2M1_VALUES[c]), -c))]
                                            for v in q.tolist()]) * 4.0
    assert not _exact(planted, want)


def test_fp8_block_act_quant_closed_form():
    """Block 0: amax 448 -> scale 1 (448 * f32(1/448) rounds to 1), q = x: 1.0625 -> 1
    (tie, even), 1.1875 -> 1.25 (tie, even).  Block 1: amax 7 -> scale 1/64, x * 64:
    1.0625 -> 1, 1.1875 -> 1.25, 0.0625 exact.  Block 2: all zero -> scale 1, codes 0."""
    x = torch.zeros(384)
    x[0], x[1], x[2] = 448.0, 1.0625, 1.1875
    x[128], x[129], x[130], x[131] = 7.0, 1.0625 / 64, 1.1875 / 64, 0.0625 / 64
    b, s = oc.fp8_block_act_quant(x)
    assert s.tolist() == [1.0, 1.0 / 64, 1.0]
    want = torch.zeros(384)
    want[0], want[1], want[2] = 448.0, 1.0, 1.25
    want[128], want[129], want[130], want[131] = 7.0, 1.0 / 64, 1.25 / 64, 0.0625 / 64
    assert _exact(oc.fp8_block_act_dequant(b, s), want)
    # planted: one scale for the whole row (amax 448): 2^-10 is half the smallest E4M3
    # subnormal and rounds to 0 (even)
    bp = oc.e4m3_encode(x)
    assert not _exact(oc.e4m3_decode(bp), want)


def _a4w4_case():
    """H = 64, inter = 32.  x block A (amax 24, scale 4): 24 -> 24, 10 -> 8 (2.5 -> 2),
    14 -> 16 (3.5 -> 4); block B (amax 3, scale 1/2): 3 -> 3, 0.625 -> 0.5 (1.25 -> 1),
    0.875 -> 1 (1.75 -> 2).  g = 24 for every row (silu(24) = 24 in f32):
    i=0: 1.0 * x0, up 1.0 * x32 = 3 -> mid 72;  i=1: 3.0 * x1, up 1.0 * x33 = 0.5 -> 12;
    i=2: 1.5 * x2, up 1.0 * x34 = 1 -> 24;  i=3: 1.0 * x0, up -1.5 * x33 = -0.75 -> -18.
    mid block: amax 72 -> 72/6 = 12 -> scale 16: 4.5 -> 4 (nearest) -> 64, 0.75 -> 1 (tie,
    even) -> 16, 1.5 -> 24, -1.125 -> -1 -> -16.  down: w2[h, h] = 1, w2[32 + i, i] = 0.5."""
    x = torch.zeros(1, 64)
    x[0, 0], x[0, 1], x[0, 2] = 24.0, 10.0, 14.0
    x[0, 32], x[0, 33], x[0, 34] = 3.0, 0.625, 0.875
    w13 = torch.zeros(64, 64)
    for i, (gc, gw, uc, uw) in enumerate([(0, 1.0, 32, 1.0), (1, 3.0, 33, 1.0), (2, 1.5, 34, 1.0), (0, 1.0, 33, -1.5)]):
        w13[i, gc] = gw
        w13[32 + i, uc] = uw
    w2 = torch.zeros(64, 32)
    for i in range(32):
        w2[i, i] = 1.0
        w2[32 + i, i] = 0.5
    mq = torch.zeros(32)
    mq[:4] = torch.tensor([64.0, 16.0, 24.0, -16.0])
    return x, w13, w2, torch.cat([mq, 0.5 * mq])


def test_expert_a4w4_closed_form():
    x, w13, w2, y = _a4w4_case()
    assert _exact(R.expert_a4w4(x, w13, w2)[0], y)
    # planted: the mid not quantized (72 instead of 64), then x not quantized
    gu = oc.mxfp4_dequant(*oc.mxfp4_act_quant(x)) @ w13.T
    assert not _exact((R.swiglu(gu[:, :32], gu[:, 32:]) @ w2.T)[0], y)
    gu = x @ w13.T
    mid = R.swiglu(gu[:, :32], gu[:, 32:])
    assert not _exact((oc.mxfp4_dequant(*oc.mxfp4_act_quant(mid)) @ w2.T)[0], y)


def _w8a8_case():
    """H = 256, inter = 128.  x block A: amax 448 (scale 1): 448, 1.0625 -> 1, 1.1875 ->
    1.25; block B: amax 7 (scale 1/64): 7, 1.0625/64 -> 1/64, 1.1875/64 -> 1.25/64.
    i=0: g = 0.25 * 448 = 112, u = 256 / 64 = 4 -> mid 448;  i=1: g = 32 * 1, u = 64 / 64
    = 1 -> 32;  i=2: g = 16 * 1.25 = 20, u = 64 * 1.25/64 -> 25.  mid block: amax 448 ->
    scale 1, q = mid: 448, 32, 25 -> 24 (tie of 24 and 26, even).  down: w2[h, h] = 1,
    w2[128 + i, i] = 0.5."""
    x = torch.zeros(1, 256)
    x[0, 0], x[0, 1], x[0, 2] = 448.0, 1.0625, 1.1875
    x[0, 128], x[0, 129], x[0, 130] = 7.0, 1.0625 / 64, 1.1875 / 64
    w13 = torch.zeros(256, 256)
    for i, (gc, gw, uc, uw) in enumerate([(0, 0.25, 129, 256.0), (1, 32.0, 129, 64.0), (2, 16.0, 130, 64.0)]):
        w13[i, gc] = gw
        w13[128 + i, uc] = uw
    w2 = torch.zeros(256, 128)
    for i in range(128):
        w2[i, i] = 1.0
        w2[128 + i, i] = 0.5
    mq = torch.zeros(128)
    mq[:3] = torch.tensor([448.0, 32.0, 24.0])
    return x, w13, w2, torch.cat([mq, 0.5 * mq])


def test_expert_w8a8_closed_form():
    x, w13, w2, y = _w8a8_case()
    assert _exact(R.expert_w8a8(x, w13, w2)[0], y)
    gu = oc.fp8_block_act_dequant(*oc.fp8_block_act_quant(x)) @ w13.T
    assert not _exact((R.swiglu(gu[:, :128], gu[:, 128:]) @ w2.T)[0], y)  # mid not quantized
    gu = x @ w13.T
    mid = R.swiglu(gu[:, :128], gu[:, 128:])
    assert not _exact((oc.fp8_block_act_dequant(*oc.fp8_block_act_quant(mid)) @ w2.T)[0], y)  # x not quantized


# ------------------------------------------------------------------------- tail
def _tail_case():
    """H = 8, V = 5.  Row 0 = +-2 (mean square 4: rstd 1/2 exactly at eps 0), row 1 =
    0.25 everywhere (rstd 4); g = (1, 1, .5, 2, 1, 1, 1, 1), so normed row 0 = (1, -1,
    .5, -2, 1, -1, 1, -1) and row 1 = g.  LM-head rows: e0, e3, all ones, 3 e2 - e7, and
    e0 + 2^-9 e1, whose logits 1 -+ 2^-9 round to bf16 1."""
    x = torch.tensor([[2.0, -2, 2, -2, 2, -2, 2, -2], [0.25] * 8])
    g = torch.tensor([1.0, 1, 0.5, 2, 1, 1, 1, 1])
    w = torch.zeros(5, 8)
    w[0, 0] = 1
    w[1, 3] = 1
    w[2] = 1
    w[3, 2], w[3, 7] = 3, -1
    w[4, 0], w[4, 1] = 1, 2.0**-9
    normed = torch.tensor([[1.0, -1, 0.5, -2, 1, -1, 1, -1], [1.0, 1, 0.5, 2, 1, 1, 1, 1]])
    logits = torch.tensor([[1.0, -2, -1.5, 2.5, 1 - 2.0**-9], [1.0, 2, 8.5, 0.5, 1]])
    return x, g, w, normed, logits


def test_tail_closed_form():
    x, g, w, normed, logits = _tail_case()
    got_l, got_n = R.tail(x, g, w, 0.0)
    assert torch.equal(got_n, normed)
    # row 0's last logit 1 - 2^-9 is below half an ulp of 1 away from 1: bf16 rounds it to 1
    logits[0, 4] = 1.0
    assert torch.equal(got_l, logits)


@pytest.mark.parametrize("plant", ["no_gamma", "no_round", "transposed"])
def test_tail_pin_catches_planted_mistakes(plant):
    x, g, w, normed, logits = _tail_case()
    logits[0, 4] = 1.0
    if plant == "no_gamma":
        got, _ = R.tail(x, torch.ones(8), w, 0.0)
    elif plant == "no_round":
        n = R.rmsnorm(x, g, 0.0)
        got = (n.double() @ w.double().t()).float()
    else:
        got, _ = R.tail(x, g, w.flip(1), 0.0)  # the LM-head rows read with k reversed
    assert not torch.equal(got, logits)
