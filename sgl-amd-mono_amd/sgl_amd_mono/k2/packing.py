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
