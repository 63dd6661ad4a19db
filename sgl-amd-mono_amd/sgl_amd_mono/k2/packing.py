"""Weight tile packing for the matrix-core GEMVs (build time, once).

Every weight the kernels stream is cut into tiles of 16 rows x 128 k.  In a tile,
lane ``l`` of a 64-lane wavefront owns row ``l % 16`` and the 32 consecutive k
``32 * (l // 16) .. + 32`` -- exactly one MFMA operand per lane for the
16x16x128 f8f6f4 instruction, and four 16x16x32 bf16 operands -- so one wave
load of a whole tile is one contiguous 1 KiB (E2M1), 2 KiB (E4M3) or 4 KiB
(bf16) run of HBM.  Tiles are stored k-block-major inside a 16-row group:
``[N / 16][K / 128][64 lanes][chunk bytes]``.

MXFP4's E8M0 scales follow the same lane order, four consecutive k-blocks a
32-bit word: ``[N / 16][ceil(K / 512)][64 lanes][4 bytes]``; the kernel selects
the byte of the k-block with the MFMA's scale byte-select.

The reference packs for the same reason with its own permutations
(glm53/gfx950/packing.py:29-133, AITER's (16, 16) shuffle glm53/check.py:383-389).

The experts can also be read in AITER's layouts, as SGLang leaves them for AITER's MoE
(``aiter_shuffle``, ``e8m0_shuffle`` below): for E2M1 bytes that layout is byte for
byte the tile packing; E4M3 tiles keep a lane's two 16-byte halves 256 bytes apart.
"""

from __future__ import annotations

import torch


def pack_tiles(w: torch.Tensor, chunk: int) -> torch.Tensor:
    """Row-major bytes [..., N, K_bytes] -> [..., N/16, K_bytes/(4*chunk), 64, chunk].

    ``chunk`` is the bytes one lane holds per 128-k block: 16 (E2M1), 32 (E4M3),
    64 (bf16)."""
    b = w.contiguous().view(torch.uint8)
    *lead, n, kbytes = b.shape
    if n % 16 or kbytes % (4 * chunk):
        raise ValueError(f"cannot tile [{n}, {kbytes}] bytes with chunk {chunk}")
    t = b.reshape(*lead, n // 16, 16, kbytes // (4 * chunk), 4, chunk)
    # [.., nt, row16, kb, g, c] -> [.., nt, kb, g, row16, c]; lane = g * 16 + row16
    t = t.movedim(-4, -2)  # row16 next to chunk
    return t.reshape(*lead, n // 16, kbytes // (4 * chunk), 64, chunk).contiguous()


def unpack_tiles(p: torch.Tensor, dtype=torch.uint8) -> torch.Tensor:
    """Inverse of pack_tiles: [..., N/16, KB, 64, chunk] -> [..., N, KB*4*chunk]."""
    *lead, nt, kb, lanes, chunk = p.shape
    t = p.reshape(*lead, nt, kb, 4, 16, chunk).movedim(-2, -4)
    return t.reshape(*lead, nt * 16, kb * 4 * chunk).contiguous().view(dtype)


def pack_e8m0(s: torch.Tensor) -> torch.Tensor:
    """E8M0 [..., N, K/32] -> [..., N/16, ceil(K/512), 64, 4] (pad code 127 = 1.0).

    Lane l, byte j of word G holds row 16*nt + l%16, 32-block 4*(4*G + j) + l//16."""
    *lead, n, k32 = s.shape
    kb = k32 // 4
    groups = -(-kb // 4)
    pad = torch.full((*lead, n, groups * 16), 127, dtype=torch.uint8, device=s.device)
    pad[..., :k32] = s
    t = pad.reshape(*lead, n // 16, 16, groups, 4, 4)  # nt, row16, G, j, g
    t = t.permute(*range(len(lead)), -5, -3, -1, -4, -2)  # nt, G, g, row16, j
    return t.reshape(*lead, n // 16, groups, 64, 4).contiguous()


def unpack_e8m0(p: torch.Tensor, k32: int) -> torch.Tensor:
    *lead, nt, groups, lanes, four = p.shape
    t = p.reshape(*lead, nt, groups, 4, 16, 4)  # nt, G, g, row16, j
    t = t.permute(*range(len(lead)), -5, -2, -4, -1, -3)  # nt, row16, G, j, g
    return t.reshape(*lead, nt * 16, groups * 16)[..., :k32].contiguous()


def aiter_shuffle(w: torch.Tensor) -> torch.Tensor:
    """Row-major bytes [..., N, K_bytes] in AITER's (16, 16) layout, as its
    shuffle_weight(w, (16, 16)) leaves 1-byte elements (E4M3, or E2M1 pairs):
    [..., N/16, K_bytes/32, 2, 16 rows, 16 B], the inverse of the reference's unshuffle
    (glm53/check.py:383-389)."""
    b = w.contiguous().view(torch.uint8)
    *lead, n, kb = b.shape
    if n % 16 or kb % 32:
        raise ValueError(f"cannot shuffle [{n}, {kb}] bytes in (16, 16) blocks")
    d = len(lead)
    t = b.reshape(*lead, n // 16, 16, kb // 32, 2, 16)  # [.., nt, row, c, h, byte]
    t = t.permute(*range(d), d, d + 2, d + 3, d + 1, d + 4)  # [.., nt, c, h, row, byte]
    return t.reshape(*lead, n, kb).contiguous()


def aiter_unshuffle(w: torch.Tensor) -> torch.Tensor:
    """Inverse of aiter_shuffle: AITER's (16, 16) bytes -> row-major [..., N, K_bytes]."""
    b = w.contiguous().view(torch.uint8)
    *lead, n, kb = b.shape
    d = len(lead)
    t = b.reshape(*lead, n // 16, kb // 32, 2, 16, 16)  # [.., nt, c, h, row, byte]
    t = t.permute(*range(d), d, d + 3, d + 1, d + 2, d + 4)  # [.., nt, row, c, h, byte]
    return t.reshape(*lead, n, kb).contiguous()


def e8m0_shuffle(s: torch.Tensor) -> torch.Tensor:
    """E8M0 codes [..., N, K/32] in the order of AITER's e8m0_shuffle, its rows counted
    across the leading dims (as SGLang shuffles an [E, N, K/32] tensor flattened to
    [E * N, K/32]): view(rows/32, 2, 16, C/8, 2, 4).permute(0, 3, 5, 2, 4, 1) with C =
    K/32 (qwen38_a95b_mxfp4/gfx950/layout.py:84-91), so that code (row, col) sits at
    ((((row/32 * C/8 + col/8) * 4 + col%4) * 16 + row%16) * 2 + col/4%2) * 2 + row/16%2.
    Needs the rows a multiple of 32 and C of 8."""
    *lead, n, c = s.shape
    rows = n
    for x in lead:
        rows *= x
    if rows % 32 or c % 8:
        raise ValueError(f"e8m0_shuffle needs rows % 32 == 0 and K/32 % 8 == 0, got {rows} x {c}")
    t = s.contiguous().view(torch.uint8).reshape(rows // 32, 2, 16, c // 8, 2, 4)
    return t.permute(0, 3, 5, 2, 4, 1).reshape(*lead, n, c).contiguous()


def e8m0_unshuffle(s: torch.Tensor) -> torch.Tensor:
    """Inverse of e8m0_shuffle."""
    *lead, n, c = s.shape
    rows = n
    for x in lead:
        rows *= x
    t = s.contiguous().view(torch.uint8).reshape(rows // 32, c // 8, 4, 16, 2, 2)  # r32, c8, f, b, d, a
    return t.permute(0, 5, 3, 1, 4, 2).reshape(*lead, n, c).contiguous()
