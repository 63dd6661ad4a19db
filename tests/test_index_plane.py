"""SGLang's FP4 index plane (score_fp4.py:9-12): the packer the synthetic caches use
and the oracle's reader agree, and both put bytes where the reference's addressing
(`_keys`, score_fp4.py:212-241) looks for them."""

import torch

from oracle import codecs as oc
from refs import index_keys_f32


def _token_major(pages, seed):
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 256, (pages, 64, 64), generator=g, dtype=torch.uint8)
    scales = torch.randint(100, 140, (pages, 64, 4), generator=g, dtype=torch.uint8)
    return codes, scales


def test_plane_addresses():
    from sgl_amd_mono.k2.synth import index_plane

    codes, scales = _token_major(2, 1)
    plane, sp = index_plane(codes, scales)
    assert plane.shape == (2, 4096) and sp.shape == (2, 256)
    for p, t, c in [(0, 0, 0), (1, 17, 2), (1, 63, 3), (0, 40, 1)]:
        # payload [chunk][token][16 B]; scales [chunk][(token % 16) * 4 + token // 16]
        assert torch.equal(plane[p, c * 1024 + t * 16 : c * 1024 + t * 16 + 16], codes[p, t, 16 * c : 16 * c + 16])
        assert int(sp[p, c * 64 + (t % 16) * 4 + t // 16]) == int(scales[p, t, c])


def test_plane_round_trip_through_page_table():
    from sgl_amd_mono.k2.synth import index_plane

    codes, scales = _token_major(5, 2)
    plane, sp = index_plane(codes, scales)
    pt = torch.tensor([[3, 0, 4]], dtype=torch.int32)  # logical pages 0..2 of request 0
    n = 150
    got = index_keys_f32(plane, sp, pt, 0, n)
    want = oc.mxfp4_dequant(codes[[3, 0, 4]], scales[[3, 0, 4]]).reshape(-1, 128)[:n]
    assert torch.equal(got, want)
