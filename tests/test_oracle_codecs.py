"""Pins the oracle's number formats (CPU only).

Each check is chosen so a plausible slip fails it: brute force over every code
(no formula retyped), the tie cases of round-to-nearest-even, saturation, and the
power-of-two scale rules at their boundaries.
"""

import itertools
import math

import pytest
import torch

from oracle import codecs as oc

E2M1_MAG = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def _nearest_even_code(x: float) -> int:
    """Brute force: the E2M1 code nearest to x (ties -> even code), saturating."""
    m = min(abs(x), 6.0)
    best = min(range(8), key=lambda c: (abs(E2M1_MAG[c] - m), c % 2))
    return best | (8 if math.copysign(1.0, x) < 0 else 0)


def test_e2m1_decode_table():
    codes = torch.arange(16, dtype=torch.uint8)
    v = oc.e2m1_decode(codes)
    assert v[:8].tolist() == E2M1_MAG
    assert v[8:].tolist() == [-m for m in E2M1_MAG]


@pytest.mark.parametrize("x,code", [(0.25, 0), (0.75, 2), (1.25, 2), (1.75, 4), (2.5, 4),
                                    (3.5, 6), (5.0, 6), (7.0, 7), (1e9, 7), (-0.25, 8),
                                    (-2.5, 12), (-5.0, 14), (0.2499, 0), (0.2501, 1)])
def test_e2m1_ties_to_even_and_saturation(x, code):
    assert int(oc.e2m1_encode(torch.tensor([x]))[0]) == code


def test_e2m1_encode_matches_brute_force():
    xs = torch.linspace(-7, 7, 2801)
    got = oc.e2m1_encode(xs).tolist()
    want = [_nearest_even_code(float(x)) for x in xs]
    assert got == want


def test_fp4_pack_nibble_order():
    codes = torch.tensor([1, 2, 3, 4], dtype=torch.uint8)
    b = oc.fp4_pack(codes)
    assert b.tolist() == [0x21, 0x43]  # even element in the low nibble
    assert torch.equal(oc.fp4_unpack(b), codes)


def test_e4m3_encode_is_nearest_even_over_all_codes():
    # every finite E4M3 value, and midpoints between neighbours
    codes = torch.arange(256, dtype=torch.uint8)
    vals = oc.e4m3_decode(codes)
    fin = vals[torch.isfinite(vals)]
    pos = torch.unique(fin[fin >= 0]).sort().values
    assert float(pos[-1]) == 448.0
    assert torch.equal(oc.e4m3_decode(oc.e4m3_encode(pos)), pos)
    mids = (pos[:-1] + pos[1:]) / 2
    got = oc.e4m3_decode(oc.e4m3_encode(mids))
    # a midpoint rounds to the neighbour whose code is even
    lo_codes = oc.e4m3_encode(pos[:-1]).long()
    want = torch.where(lo_codes % 2 == 0, pos[:-1], pos[1:])
    assert torch.equal(got, want)
    assert float(oc.e4m3_decode(oc.e4m3_encode(torch.tensor([1e6])))[0]) == 448.0  # clamp


def test_mxfp4_scale_rule_boundaries():
    # amax = 6 * 2^k exactly -> scale 2^k; a hair above -> 2^(k+1)
    for k in (-8, -3, 0, 2, 5):
        amax = torch.tensor([6.0 * 2.0**k])
        assert int(oc.mxfp4_scale_code(amax)[0]) == 127 + k
        above = torch.nextafter(amax, torch.tensor([1e30]))
        assert int(oc.mxfp4_scale_code(above)[0]) == 127 + k + 1
    # floor at 6 * 2^-126: the code never drops below 1
    assert int(oc.mxfp4_scale_code(torch.tensor([0.0]))[0]) == 1


def test_mxfp8_scale_rule_boundaries():
    for k in (-10, -2, 0, 3):
        amax = torch.tensor([448.0 * 2.0**k])
        assert int(oc.mxfp8_scale_code(amax)[0]) == 127 + k
        above = torch.nextafter(amax, torch.tensor([1e30]))
        assert int(oc.mxfp8_scale_code(above)[0]) == 127 + k + 1
    assert int(oc.mxfp8_scale_code(torch.tensor([0.0]))[0]) == 1  # clamped to [1, 254]


def test_mx_roundtrip_error_bounds():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 256, generator=g)
    b, s = oc.mxfp4_quant(x)
    y = oc.mxfp4_dequant(b, s)
    blocks = x.view(64, 8, 32)
    amax = blocks.abs().amax(-1, keepdim=True)
    # E2M1 spacing near the top is 2 (4 -> 6) in units of the scale, so the error is
    # at most scale = pow2ceil(amax / 6) <= amax / 3
    err = (y.view(64, 8, 32) - blocks).abs()
    assert bool((err <= amax / 3 + 1e-7).all())
    q, sc = oc.mxfp8_quant(x)
    y8 = oc.mxfp8_dequant(q, sc)
    rel = ((y8 - x).abs() / x.abs().clamp_min(1e-3)).view(-1)
    assert float(rel[x.abs().view(-1) > 0.1].max()) <= 2.0**-3 + 1e-6  # 3 mantissa bits


def test_fp8_block_dequant_layout():
    codes = oc.e4m3_encode(torch.ones(256, 256))
    scales = torch.tensor([[1.0, 2.0], [3.0, 4.0]])
    v = oc.fp8_block_dequant(codes, scales)
    assert float(v[0, 0]) == 1.0 and float(v[0, 200]) == 2.0
    assert float(v[200, 0]) == 3.0 and float(v[200, 200]) == 4.0


def test_radix_keys_order_matches_float_order():
    vals = torch.tensor([-math.inf, -3.5, -1e-30, -0.0, 0.0, 1e-30, 2.0, math.inf])
    keys = oc.radix_keys(vals)
    assert keys.tolist() == sorted(keys.tolist())
    assert int(keys[3]) < int(keys[4])  # -0.0 ranks below +0.0
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1000, generator=g)
    assert torch.equal(torch.argsort(oc.radix_keys(x), stable=True), torch.argsort(x, stable=True))


def test_bf16_round_is_nearest_even():
    # 1 + 2^-8 is a bf16 tie between 1 and 1 + 2^-7: rounds to the even mantissa (1)
    assert float(oc.bf16_round(torch.tensor([1.0 + 2.0**-8]))[0]) == 1.0
    assert float(oc.bf16_round(torch.tensor([1.0 + 3 * 2.0**-8]))[0]) == 1.0 + 2.0**-6


def test_negative_control_planted_rounding_slip_is_caught():
    """A planted mistake in the oracle (ties rounded up instead of to even) fails the
    brute-force check above."""
    def bad_encode(q):
        m = q.abs()
        c = sum((m >= t).to(torch.uint8) for t in (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0))
        return c | (torch.signbit(q).to(torch.uint8) << 3)

    xs = torch.tensor([0.25, 1.25, 2.5, 5.0])
    assert bad_encode(xs).tolist() != oc.e2m1_encode(xs).tolist()
    assert bad_encode(xs).tolist() != [_nearest_even_code(float(x)) for x in xs]


def test_product_quantizers_agree_with_oracle():
    """The package's weight encoders (product code) against the oracle's restatement."""
    from sgl_amd_mono.k2 import quant

    g = torch.Generator().manual_seed(2)
    w = torch.randn(48, 256, generator=g) * 0.02
    b1, s1 = quant.quant_mxfp4(w)
    b2, s2 = oc.mxfp4_quant(w)
    assert torch.equal(b1, b2) and torch.equal(s1, s2)
    # ties exactly on E2M1 boundaries after scaling
    ties = torch.tensor([[0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0] * 4]) * 2.0**-3
    assert torch.equal(quant.quant_mxfp4(ties)[0], oc.mxfp4_quant(ties)[0])
    codes, scales = quant.quant_fp8_block(w)
    deq = oc.fp8_block_dequant(codes, scales)
    assert float((deq - w).abs().max()) <= float(w.abs().max()) * 2.0**-3


def test_all_e2m1_pairs_decode():
    for a, b in itertools.product(range(16), repeat=2):
        byte = torch.tensor([a | (b << 4)], dtype=torch.uint8)
        v = oc.e2m1_decode(oc.fp4_unpack(byte))
        assert v.tolist() == [oc.e2m1_decode(torch.tensor([a], dtype=torch.uint8))[0].item(),
                              oc.e2m1_decode(torch.tensor([b], dtype=torch.uint8))[0].item()]


# ------------------------------------------------------------- DSA FP8 index cache
@pytest.mark.parametrize("amax, field", [
    (448.0, 127),            # 448 / 448 = 1 exactly: scale 1
    (448.00003, 128),        # the next f32 above: scale 2
    (224.0, 126),            # 0.5 exactly
    (1.0, 127 - 8),          # 1/448 = 0.00223 lies in (2^-9, 2^-8]
    (0.0, 127 - 22),         # floor 1e-4: 2.23e-7 lies in (2^-23, 2^-22]
    (3.0e-5, 127 - 22),      # below the floor: the floor's scale
])
def test_index_key_scale_rule_closed_form(amax, field):
    assert int(oc.index_key_scale_code(torch.tensor(amax))) == field


def test_index_key_quant_is_exact_on_representable_keys():
    """A key of E4M3 values times a power of two comes back exactly, and its scale puts
    the largest magnitude at 448 * 2^-k for the smallest such k."""
    vals = torch.tensor([448.0, -1.0, 0.5, 3.25, 0.0] + [0.0] * 123)
    for e in (-12, 0, 5):
        k = vals * 2.0**e
        codes, scale = oc.index_key_quant(k)
        assert float(scale) == 2.0**e
        assert torch.equal(oc.e4m3_decode(codes) * scale, k)


def test_index_page_single_byte_placement():
    """One nonzero value byte: token 21, dim 37 sits at byte (21 // 16) * 2048 + (37 // 16)
    * 256 + (21 % 16) * 16 + 37 % 16 = 2645 of the page; its scale at 8192 + 4 * 21."""
    page = torch.zeros(1, oc.INDEX_PAGE_BYTES, dtype=torch.uint8)
    page[0, 2645] = int(oc.e4m3_encode(torch.tensor(3.0)))
    page[0, 8192 + 4 * 21 : 8192 + 4 * 22] = torch.tensor([0.25], dtype=torch.float32).view(torch.uint8)
    keys = oc.index_page_decode(page)
    assert float(keys[0, 21, 37]) == 0.75
    assert int((keys != 0).sum()) == 1


def _token_major_decode(pages):
    """A planted mistake: the values read token-major (byte t * 128 + d)."""
    pg = pages.reshape(-1, oc.INDEX_PAGE_BYTES)
    vals = oc.e4m3_decode(pg[:, : oc.INDEX_VALUE_BYTES].contiguous()).view(-1, 64, 128)
    return vals * pg[:, oc.INDEX_VALUE_BYTES :].contiguous().view(torch.float32)[..., None]


def test_index_pages_writer_and_reader_agree():
    """The package's page writer (the kernel's byte formula, glm53/gfx950/kernel.py:698-705)
    against the oracle's reader (the check's, glm53/check.py:75-82): the round trip
    returns every key; the planted token-major reader does not."""
    from sgl_amd_mono.k2 import quant, synth

    g = torch.Generator().manual_seed(9)
    k = torch.randn(3, 64, 128, generator=g) * torch.logspace(-3, 2, 64).view(1, 64, 1)
    codes, scales = quant.quant_index_fp8(k)
    c2, s2 = oc.index_key_quant(k)
    assert torch.equal(codes, c2) and torch.equal(scales, s2)  # product encoder == oracle rule
    pages = synth.index_pages_fp8(codes, scales)
    assert pages.shape == (3, 64, 132) and pages.dtype == torch.uint8
    want = oc.e4m3_decode(codes) * scales[..., None]
    assert torch.equal(oc.index_page_decode(pages), want)
    assert not torch.equal(_token_major_decode(pages), want)
    assert float((want - k).abs().max() / k.abs().amax()) < 2.0**-3


def test_fp4_query_scale_rule():
    """quantize_fp4_indexer_row's E8M0 (index_query.py:286-291): the ceil power of two
    of f32(amax / 6), floored at f32(1e-4), clamped to [1, 254]."""
    for k in (-8, -3, 0, 2, 5):
        amax = torch.tensor([6.0 * 2.0**k])
        assert int(oc.fp4_query_scale_code(amax)[0]) == 127 + k
        above = torch.nextafter(amax, torch.tensor([1e30]))
        assert int(oc.fp4_query_scale_code(above)[0]) == 127 + k + 1
    # the floor: f32(1e-4) lies in (2^-14, 2^-13], so a zero or tiny group gets 2^-13
    assert 2.0**-14 < float(torch.tensor(1e-4, dtype=torch.float32)) <= 2.0**-13
    for amax in (0.0, 1e-30, 6e-4 * 0.5):
        assert int(oc.fp4_query_scale_code(torch.tensor([amax]))[0]) == 127 - 13
    # the keys' MXFP4 rule floors at 6 * 2^-126 instead: a plant of that rule differs
    assert int(oc.mxfp4_scale_code(torch.tensor([0.0]))[0]) == 1
    # the largest f32 group: 3.4e38 / 6 < 2^126, so finite inputs stay below the clamp
    assert int(oc.fp4_query_scale_code(torch.tensor([torch.finfo(torch.float32).max]))[0]) == 253


def test_fp4_query_quant_codes():
    """Values on the grid come back exactly; a tie goes to the even code; beyond 6
    saturates; a negative value that rounds to zero gets code 0, not 8
    (_e2m1_code, index_query.py:217-227)."""
    grid = torch.tensor(oc.E2M1_VALUES)
    # a group of 32 with amax 6 (scale 2^0): every grid value and its negative exactly
    x = torch.cat([grid, -grid, torch.tensor([6.0] * 16)])
    b, s = oc.fp4_query_quant(x)
    assert int(s[0]) == 127
    assert torch.equal(oc.mxfp4_dequant(b, s), x)
    # ties (midpoints of the grid) to the even code, and tiny negatives to +0
    mids = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    want = torch.tensor([0.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0])
    x = torch.cat([mids, -mids, torch.tensor([-0.1, -0.2, 6.0] + [0.0] * 15)])
    b, s = oc.fp4_query_quant(x)
    codes = oc.fp4_unpack(b)
    assert torch.equal(oc.mxfp4_dequant(b, s)[:14], torch.cat([want, -want]))
    assert int(codes[14]) == 0 and int(codes[15]) == 0  # no -0 code
    # the scaled group: amax 6 * 2^3 -> scale 2^3, values quantized at that scale
    x = torch.linspace(-48.0, 48.0, 32)
    b, s = oc.fp4_query_quant(x)
    assert int(s[0]) == 130
    y = oc.mxfp4_dequant(b, s)
    assert float((y - x).abs().max()) <= 8.0 * 1.0 + 1e-6  # half of the widest step (2) at 2^3


def test_fp4_query_quant_matches_brute_force():
    """Each code is the nearest grid value to x / 2^(e - 127), ties to the even code,
    checked against an exhaustive nearest search in f64."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(64, 128, generator=g) * torch.exp2(torch.randint(-6, 6, (64, 1), generator=g).float())
    b, s = oc.fp4_query_quant(x)
    y = oc.mxfp4_dequant(b, s).double()
    sc = oc.e8m0_value(s).double().repeat_interleave(32, -1)
    v = (x.double() / sc).clamp(-6, 6)
    grid = torch.tensor(oc.E2M1_VALUES, dtype=torch.float64)
    d = (v.abs()[..., None] - grid).abs()
    best = d.min(-1).values
    # the kernel's value is one of the nearest grid points
    got = (y / sc).abs()
    assert torch.allclose((got - v.abs()).abs(), best, atol=0, rtol=0)
