"""The expert weights' two layouts: this build's tiles and AITER's (16, 16) shuffle.

AITER is a dependency of the reference that this image does not hold; its layouts are
pinned here by what the reference states of them: the weight bytes as
[N/16, K/32, 2, 16 rows, 16 B] (glm53/check.py:383-389, ``unshuffle``), and the E8M0
codes by e8m0_shuffle's byte formula (qwen38_a95b_mxfp4/gfx950/layout.py:84-91,
``scale_index``), each checked on single bytes placed by hand, and by the kernels'
own addressing (restated from csrc/moe_stages.h ``fp8_half``, ``e8m0_word``,
``e8m0_shift``) on every lane of small matrices.
"""

import pytest
import torch

from dataclasses import replace

from sgl_amd_mono.k2 import config as C
from sgl_amd_mono.k2.packing import aiter_shuffle, aiter_unshuffle, e8m0_shuffle, e8m0_unshuffle, pack_e8m0, pack_tiles


def _bytes(*shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 256, shape, generator=g, dtype=torch.uint8)


def test_aiter_shuffle_places_one_byte():
    """Row 21, byte 77 of a [32, 256] matrix: 16-row group 1, row 5 in it; 32-byte
    column 2, half 0, byte 13 -> ((1 * 8 + 2) * 2 + 0) * 256 + 5 * 16 + 13 = 5213."""
    w = torch.zeros(32, 256, dtype=torch.uint8)
    w[21, 77] = 9
    assert (aiter_shuffle(w).flatten() == 9).nonzero().flatten().tolist() == [5213]


def test_e8m0_shuffle_places_one_code():
    """Expert 1, row 19, code 13 of [2, 32, 16]: global row 51 (row/32 = 1, row/16 % 2 =
    1, row % 16 = 3), col 13 (col/8 = 1, col/4 % 2 = 1, col % 4 = 1), C/8 = 2 ->
    ((((1 * 2 + 1) * 4 + 1) * 16 + 3) * 2 + 1) * 2 + 1 = 847."""
    s = torch.zeros(2, 32, 16, dtype=torch.uint8)
    s[1, 19, 13] = 7
    assert (e8m0_shuffle(s).flatten() == 7).nonzero().flatten().tolist() == [847]


def test_round_trips():
    w = _bytes(3, 64, 512)
    assert torch.equal(aiter_unshuffle(aiter_shuffle(w)), w)
    s = _bytes(2, 64, 16, seed=1)
    assert torch.equal(e8m0_unshuffle(e8m0_shuffle(s)), s)
    with pytest.raises(ValueError):
        aiter_shuffle(_bytes(24, 64))
    with pytest.raises(ValueError):
        e8m0_shuffle(_bytes(32, 12))


def test_e2m1_tiles_are_aiter_bytes():
    """E2M1 pairs: the tile packing ([N/16][K/128][64 lanes][16 B], lane = 16 g + row)
    and AITER's (16, 16) layout are the same bytes, so the kernels read either."""
    w = _bytes(2, 64, 384, seed=2)
    assert torch.equal(pack_tiles(w, 16).reshape(2, 64, 384), aiter_shuffle(w))


def _fp8_half(aiter: bool, lane: int, h: int) -> int:
    return (lane >> 4) * 512 + h * 256 + (lane & 15) * 16 if aiter else lane * 32 + h * 16


@pytest.mark.parametrize("aiter", [False, True])
def test_e4m3_block_addressing(aiter):
    """Every lane's two 16-byte halves of every 16 x 128 block, at the kernels'
    offsets, hold row c16's k 32 g + 16 h .. + 15 of that block (tiles and AITER)."""
    N, K = 32, 256
    w = _bytes(N, K, seed=3)
    lay = aiter_shuffle(w) if aiter else pack_tiles(w, 32).reshape(N, K)
    flat = lay.flatten()
    for nt in range(N // 16):
        for kb in range(K // 128):
            blk = (nt * (K // 128) + kb) * 2048
            for lane in range(64):
                g, c16 = lane >> 4, lane & 15
                for h in range(2):
                    got = flat[blk + _fp8_half(aiter, lane, h):][:16]
                    want = w[16 * nt + c16, 128 * kb + 32 * g + 16 * h:][:16]
                    assert torch.equal(got, want), (nt, kb, lane, h)


def _e8m0_word(aiter: bool, s_e: torch.Tensor, K: int, t: int, kb: int, lane: int) -> int:
    if aiter:
        w = ((t >> 1) * (K // 256) + (kb >> 1)) * 64 + lane
    else:
        w = (t * ((K // 128 + 3) // 4) + (kb >> 2)) * 64 + lane
    b = s_e[4 * w:4 * w + 4].tolist()
    return b[0] | b[1] << 8 | b[2] << 16 | b[3] << 24


def _e8m0_shift(aiter: bool, t: int, kb: int) -> int:
    return 8 * (2 * (kb & 1) + (t & 1)) if aiter else 8 * (kb & 3)


@pytest.mark.parametrize("aiter", [False, True])
def test_e8m0_word_addressing(aiter):
    """The kernels' E8M0 word and byte for (tile t, k-block kb, lane) hold the code of
    row 16 t + c16, 32-block 4 kb + g, for every expert of [2, 64, K/32] (tiles and
    AITER, whose rows run across the experts)."""
    E, N, K = 2, 64, 512
    s = _bytes(E, N, K // 32, seed=4)
    lay = (e8m0_shuffle(s) if aiter else pack_e8m0(s)).flatten()
    per = N * (K // 32) if aiter else (N // 16) * ((K // 128 + 3) // 4) * 256
    for e in range(E):
        s_e = lay[e * per:(e + 1) * per]
        for t in range(N // 16):
            for kb in range(K // 128):
                for lane in range(64):
                    code = (_e8m0_word(aiter, s_e, K, t, kb, lane) >> _e8m0_shift(aiter, t, kb)) & 0xFF
                    assert code == s[e, 16 * t + (lane & 15), 4 * kb + (lane >> 4)].item(), (e, t, kb, lane)


def test_config_layout_rules():
    replace(C.C2_MOE, weight_layout=C.WLAYOUT_AITER16).validate(8)
    with pytest.raises(ValueError):
        replace(C.C2_MOE, weight_layout=2).validate(8)
    with pytest.raises(ValueError):  # E2M1 rows: the E8M0 layout needs inter % 256
        replace(C.C2_MOE, inter=384, weight_layout=C.WLAYOUT_AITER16).validate(8)
    replace(C.C1_MOE, inter=384, weight_layout=C.WLAYOUT_AITER16).validate(4)
