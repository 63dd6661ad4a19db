"""Weight and cache encoders (build time, any torch device).

These write the byte formats the kernels read:
  * MXFP4 weights / FP4 index keys: E2M1 codes, two a byte (even element in the low
    nibble), one E8M0 per 32 elements = the smallest power of two >= amax / 6
    (the rule of deepseek_v4/gfx950/kernels/stages/indexer.py:143-151).
  * FP8 weights: E4M3 codes with one f32 scale per 128 x 128 block, scale = amax / 448
    (the layout glm53/check.py:427-432 reads).
  * FP8 latent-KV rows: E4M3 codes with one f32 scale per token, scale = amax / 448.
  * FP8 index keys (SGLang's DSA index cache): E4M3 codes with one power-of-two f32
    scale per key, 2^ceil(log2(max(amax, 1e-4) / 448)) (glm53/gfx950/kernel.py:3134-3147).
Activations are quantized on the GPU by the kernels themselves.
"""

from __future__ import annotations

import torch

FP8_MAX = 448.0


def _pow2_ceil_exponent(v: torch.Tensor) -> torch.Tensor:
    """Unbiased exponent e of the smallest 2^e >= v (v > 0, f32), via the bit fields."""
    bits = v.float().contiguous().view(torch.int32)
    field = (bits >> 23) & 0xFF
    frac = bits & 0x7FFFFF
    return (field - 127) + (frac != 0).to(torch.int32)


def quant_mxfp4(w: torch.Tensor):
    """[..., K] -> (uint8 [..., K/2], uint8 E8M0 [..., K/32])."""
    w = w.float()
    shp = w.shape
    if shp[-1] % 32:
        raise ValueError("MXFP4 needs K % 32 == 0")
    b = w.reshape(*shp[:-1], shp[-1] // 32, 32)
    amax = b.abs().amax(-1).clamp_min(6.0 * 2.0**-126)
    e = _pow2_ceil_exponent(amax * torch.tensor(1.0 / 6.0, dtype=torch.float32))
    e = e.clamp(max=127)
    q = (b * torch.exp2(-e.float())[..., None]).clamp(-6.0, 6.0)
    mag = q.abs()
    # E2M1 magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6; nearest, ties to the even code
    edges_up = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], device=w.device)
    code = torch.bucketize(mag, edges_up, right=False)  # counts edges strictly below mag
    # a value exactly on an edge whose upper neighbour has the even code rounds up
    on_edge_up = (mag == 0.75) | (mag == 1.75) | (mag == 3.5)
    code = code + on_edge_up.to(code.dtype)
    code = code.to(torch.uint8) | (torch.signbit(q).to(torch.uint8) << 3)
    code = code.reshape(shp)
    packed = code[..., 0::2] | (code[..., 1::2] << 4)
    return packed.contiguous(), (e + 127).to(torch.uint8).contiguous()


def _e4m3(x: torch.Tensor) -> torch.Tensor:
    return x.clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn).view(torch.uint8)


def quant_fp8_block(w: torch.Tensor, block: int = 128):
    """[..., N, K] -> (E4M3 uint8 [..., N, K], f32 scales [..., ceil(N/128), ceil(K/128)])."""
    w = w.float()
    *lead, n, k = w.shape
    nb, kb = -(-n // block), -(-k // block)
    pad = torch.zeros(*lead, nb * block, kb * block, device=w.device)
    pad[..., :n, :k] = w
    t = pad.reshape(*lead, nb, block, kb, block)
    amax = t.abs().amax(dim=(-3, -1))
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = t / scale[..., :, None, :, None]
    codes = _e4m3(q).reshape(*lead, nb * block, kb * block)[..., :n, :k]
    return codes.contiguous(), scale.float().contiguous()


def quant_fp8_rows(v: torch.Tensor):
    """[..., D] -> (E4M3 uint8 [..., D], f32 scale [...]) with scale = amax / 448."""
    v = v.float()
    amax = v.abs().amax(-1)
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    return _e4m3(v / scale[..., None]).contiguous(), scale.contiguous()


def quant_index_fp8(k: torch.Tensor):
    """Index keys [..., 128] -> (E4M3 uint8 [..., 128], f32 power-of-two scales [...])."""
    k = k.float()
    e = _pow2_ceil_exponent(k.abs().amax(-1).clamp_min(1e-4) / FP8_MAX)
    return _e4m3(k * torch.exp2(-e.float())[..., None]).contiguous(), torch.exp2(e.float()).contiguous()
