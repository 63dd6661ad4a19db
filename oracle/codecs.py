"""Number formats of the K2 path, restated on the CPU (test infrastructure only).

Formats (all little-endian bytes):
  * E4M3 (OCP FP8, "fn": no inf, max 448): torch.float8_e4m3fn bits.  Encoding clamps
    to +-448 first and rounds to nearest even, as the kernel clamps before its
    convert (glm53/gfx950/kernel.py:1740-1750, common/mx.py:21-23).
  * E2M1 (FP4): codes 0..7 = {0, .5, 1, 1.5, 2, 3, 4, 6}, bit 3 = sign, two codes
    a byte, the even element in the low nibble (glm53/check.py:435-444).
  * E8M0: a biased power-of-two exponent byte, value 2^(code - 127).
  * MXFP4: E2M1 codes with one E8M0 per 32 consecutive elements; the scale is the
    smallest power of two >= max(amax, 6 * 2^-126) * f32(1/6)
    (deepseek_v4/gfx950/kernels/stages/indexer.py:143-151, kernels/common.py:86-99).
  * MXFP8 (activations): E4M3 codes with one E8M0 per 32; the E8M0 is the
    ceil-power-of-two exponent of amax * f32(1/448), clamped to [1, 254]
    (glm53/gfx950/kernel.py:1752-1766, common/mx.py:26-37).
  * MXFP4 activations: E2M1 codes with one E8M0 per 32; the E8M0 is AITER's round-up
    rule, the smallest power of two >= amax * f32(1/6), at most 254 (common/mx.py:40-45,
    kernel.py:354,1768-1777).
  * FP8 per-128 activations: E4M3 codes with an f32 scale amax * f32(1/448) per 128;
    q = clamp(x * 448/amax, +-448) (kernel.py:1740-1750, whose multiplier is the
    hardware reciprocal: here, as in this build's kernels, the IEEE quotient).
  * DSA index keys (SGLang's FP8 index cache, uint8 [pages, 64, 132]): per key, E4M3
    values times one power-of-two f32 scale 2^ceil(log2(max(amax, 1e-4) / 448))
    (kernel.py:3134-3147); a page holds 64 x 128 values in 16 x 16 tiles -- byte b is
    token (b // 2048) * 16 + (b % 256) // 16 (glm53/check.py:75-82), dim
    ((b % 2048) // 256) * 16 + b % 16 -- then the 64 keys' f32 scales.
  * MXFP4 index queries (the FP4 x FP4 scorer's): E2M1 codes with one E8M0 per 32
    dims; the E8M0 is the ceil-power-of-two exponent of max(f32(amax / 6), f32(1e-4)),
    clamped to [1, 254], and a value that rounds to zero keeps no sign
    (deepseek_v41/gfx950/attention/index_query.py:217-227,283-293).
  * radix key: the order-preserving u32 of f32 score bits (glm53/check.py:111-114).

Every function here is pinned by tests/test_oracle_codecs.py (closed forms, brute
force over all codes, tie cases).
"""

from __future__ import annotations

import torch

FP8_MAX = 448.0
FP4_MAX = 6.0
E2M1_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)  # glm53/check.py:435


def _f32(x) -> torch.Tensor:
    return torch.as_tensor(x).to(torch.float32)


# ----------------------------------------------------------------------------- E4M3
def e4m3_encode(x: torch.Tensor) -> torch.Tensor:
    """f32 -> E4M3 bytes (uint8): clamp to +-448, round to nearest even
    (glm53/gfx950/kernel.py:1748-1749 clamps, the convert rounds RNE)."""
    x = _f32(x).clamp(-FP8_MAX, FP8_MAX)
    return x.to(torch.float8_e4m3fn).view(torch.uint8)


def e4m3_decode(b: torch.Tensor) -> torch.Tensor:
    """E4M3 bytes -> f32 (exact)."""
    return b.contiguous().view(torch.float8_e4m3fn).to(torch.float32)


# ----------------------------------------------------------------------------- E2M1
def e2m1_encode(q: torch.Tensor) -> torch.Tensor:
    """Pre-scaled f32 -> E2M1 codes (uint8, one per element): saturate at 6, round to
    nearest, ties to the even code (common/mx.py:55-66 rounds as AITER's quants).
    A tie sits half way between two table values; the even code wins."""
    q = _f32(q)
    m = q.abs()
    # code boundaries: > for a tie that rounds down, >= for a tie that rounds up
    c = (
        (m > 0.25).to(torch.uint8)
        + (m >= 0.75).to(torch.uint8)
        + (m > 1.25).to(torch.uint8)
        + (m >= 1.75).to(torch.uint8)
        + (m > 2.5).to(torch.uint8)
        + (m >= 3.5).to(torch.uint8)
        + (m > 5.0).to(torch.uint8)
    )
    sign = (torch.signbit(q)).to(torch.uint8) << 3
    return c | sign


def e2m1_decode(codes: torch.Tensor) -> torch.Tensor:
    """E2M1 codes (uint8 0..15) -> f32 (glm53/check.py:438-444)."""
    table = torch.tensor(E2M1_VALUES, dtype=torch.float32)
    c = codes.long()
    v = table[c & 7]
    return torch.where((c & 8) != 0, -v, v)


def fp4_pack(codes: torch.Tensor) -> torch.Tensor:
    """[..., K] codes -> [..., K/2] bytes, the even element in the low nibble."""
    c = codes.to(torch.uint8)
    return c[..., 0::2] | (c[..., 1::2] << 4)


def fp4_unpack(b: torch.Tensor) -> torch.Tensor:
    """[..., K/2] bytes -> [..., K] codes."""
    return torch.stack([b & 0xF, b >> 4], -1).flatten(-2)


# ----------------------------------------------------------------------------- E8M0
def e8m0_value(code: torch.Tensor) -> torch.Tensor:
    """E8M0 byte -> f32 2^(code - 127)."""
    return torch.exp2(code.to(torch.float32) - 127.0)


def _ceil_pow2_code(v: torch.Tensor) -> torch.Tensor:
    """Biased exponent of the smallest power of two >= v (v > 0 normal or subnormal,
    f32): the exponent field, plus one when any mantissa bit is set
    (common/mx.py:26-31)."""
    bits = _f32(v).view(torch.int32).to(torch.int64)
    e = (bits >> 23) & 0xFF
    return e + ((bits & 0x7FFFFF) != 0).to(torch.int64)


def mxfp4_scale_code(amax: torch.Tensor) -> torch.Tensor:
    """E8M0 of an MXFP4 block: pow2_ceil(max(amax, 6 * 2^-126) * f32(1/6))
    (deepseek_v4/gfx950/kernels/stages/indexer.py:147), at most 254."""
    v = torch.maximum(_f32(amax), torch.tensor(FP4_MAX * 2.0**-126, dtype=torch.float32))
    v = v * torch.tensor(1.0 / FP4_MAX, dtype=torch.float32)
    return _ceil_pow2_code(v).clamp(max=254)


def mxfp4_quant(x: torch.Tensor):
    """[..., K] f32 -> (bytes [..., K/2], E8M0 [..., K/32]); K % 32 == 0
    (indexer.py:143-151: q = clamp(v * rcp(sc), +-6), E2M1 RNE)."""
    x = _f32(x)
    shp = x.shape
    blocks = x.reshape(*shp[:-1], shp[-1] // 32, 32)
    code = mxfp4_scale_code(blocks.abs().amax(-1))
    inv = torch.exp2(127.0 - code.to(torch.float32))  # exact reciprocal of a power of two
    q = (blocks * inv[..., None]).clamp(-FP4_MAX, FP4_MAX)
    codes = e2m1_encode(q).reshape(shp)
    return fp4_pack(codes), code.to(torch.uint8)


def fp4_query_scale_code(amax: torch.Tensor) -> torch.Tensor:
    """E8M0 of a 32-dim group of index queries: the smallest power of two >=
    max(f32(amax / 6), f32(1e-4)) -- the IEEE quotient, not a product with f32(1/6) --
    clamped to [1, 254] (index_query.py:286-291)."""
    v = _f32(amax) / torch.tensor(FP4_MAX, dtype=torch.float32)
    v = torch.maximum(v, torch.tensor(1.0e-4, dtype=torch.float32))
    return _ceil_pow2_code(v).clamp(1, 254)


def fp4_query_quant(x: torch.Tensor):
    """[..., K] f32 -> (bytes [..., K/2], E8M0 [..., K/32]), K % 32 == 0:
    quantize_fp4_indexer_row (index_query.py:283-293).  Codes are the E2M1 of
    x * 2^(127 - e), saturating at 6, ties to the even code (_e2m1_code,
    index_query.py:217-227), and a value that rounds to zero gets code 0."""
    x = _f32(x)
    shp = x.shape
    blocks = x.reshape(*shp[:-1], shp[-1] // 32, 32)
    code = fp4_query_scale_code(blocks.abs().amax(-1))
    inv = torch.exp2(127.0 - code.to(torch.float32))  # exact: a power of two
    c = e2m1_encode((blocks * inv[..., None]).clamp(-FP4_MAX, FP4_MAX))
    c = torch.where((c & 7) == 0, torch.zeros_like(c), c).reshape(shp)
    return fp4_pack(c), code.to(torch.uint8)


def mxfp4_dequant(b: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """(bytes [..., K/2], E8M0 [..., K/32]) -> f32 [..., K] (glm53/check.py:438-444)."""
    v = e2m1_decode(fp4_unpack(b))
    return v * e8m0_value(scales).repeat_interleave(32, -1)


# ----------------------------------------------------------------------------- MXFP8
def mxfp8_scale_code(amax: torch.Tensor) -> torch.Tensor:
    """E8M0 of an MXFP8 activation block: ceil-pow2 exponent of amax * f32(1/448),
    clamped to [1, 254] (glm53/gfx950/kernel.py:1752-1762)."""
    v = _f32(amax) * torch.tensor(1.0 / FP8_MAX, dtype=torch.float32)
    return _ceil_pow2_code(v).clamp(1, 254)


def mxfp8_quant(x: torch.Tensor):
    """[..., K] f32 -> (E4M3 bytes [..., K], E8M0 [..., K/32]); q = clamp(x * 2^-e,
    +-448) rounded RNE (glm53/gfx950/kernel.py:1763-1766)."""
    x = _f32(x)
    shp = x.shape
    blocks = x.reshape(*shp[:-1], shp[-1] // 32, 32)
    code = mxfp8_scale_code(blocks.abs().amax(-1))
    inv = torch.exp2(127.0 - code.to(torch.float32))
    q = blocks * inv[..., None]
    return e4m3_encode(q).reshape(shp), code.to(torch.uint8)


def mxfp8_dequant(b: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    return e4m3_decode(b) * e8m0_value(scales).repeat_interleave(32, -1)


# ----------------------------------------------------------------- MXFP4 activations
def mxfp4_act_code(amax: torch.Tensor) -> torch.Tensor:
    """E8M0 of an MXFP4 activation block: ((bits of amax * f32(1/6)) + 0x7FFFFF) >> 23,
    at most 254 -- the code of the smallest power of two >= amax / 6, 0 for amax = 0
    (common/mx.py:40-45)."""
    v = _f32(amax) * torch.tensor(1.0 / FP4_MAX, dtype=torch.float32)
    bits = v.contiguous().view(torch.int32).to(torch.int64)
    return (((bits + 0x7FFFFF) >> 23) & 0xFF).clamp(max=254)


def mxfp4_act_quant(x: torch.Tensor):
    """[..., K] f32 -> (bytes [..., K/2], E8M0 [..., K/32]): E2M1 of x / 2^(code - 127),
    round to nearest even, saturating at 6 (common/mx.py:55-66, kernel.py:1768-1777)."""
    x = _f32(x)
    shp = x.shape
    blocks = x.reshape(*shp[:-1], shp[-1] // 32, 32)
    code = mxfp4_act_code(blocks.abs().amax(-1))
    q = (blocks / torch.exp2(code.to(torch.float32) - 127.0)[..., None]).clamp(-FP4_MAX, FP4_MAX)
    return fp4_pack(e2m1_encode(q).reshape(shp)), code.to(torch.uint8)


# --------------------------------------------------------------- FP8 per-128 activations
def fp8_block_act_quant(x: torch.Tensor):
    """[..., K] f32 -> (E4M3 bytes [..., K], f32 scales [..., K/128]): per 128 values,
    scale = amax * f32(1/448) and q = E4M3(clamp(x * (448 / amax), +-448)), RNE; an
    all-zero block has scale 1 (kernel.py:1740-1750)."""
    x = _f32(x)
    shp = x.shape
    blocks = x.reshape(*shp[:-1], shp[-1] // 128, 128)
    amax = blocks.abs().amax(-1)
    nz = amax > 0
    one = torch.ones_like(amax)
    scale = torch.where(nz, amax * torch.tensor(1.0 / FP8_MAX, dtype=torch.float32), one)
    inv = torch.where(nz, torch.tensor(FP8_MAX, dtype=torch.float32) / torch.where(nz, amax, one), one)
    return e4m3_encode(blocks * inv[..., None]).reshape(shp), scale


def fp8_block_act_dequant(b: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return e4m3_decode(b) * scale.float().repeat_interleave(128, -1)


# ------------------------------------------------------------ FP8 with f32 block scales
def fp8_block_dequant(codes: torch.Tensor, scales: torch.Tensor, block: int = 128) -> torch.Tensor:
    """E4M3 [N, K] with f32 scales [ceil(N/128), ceil(K/128)] -> f32 [N, K]
    (glm53/check.py:427-432)."""
    n, k = codes.shape[-2:]
    s = scales.float().repeat_interleave(block, -2).repeat_interleave(block, -1)
    return e4m3_decode(codes) * s[..., :n, :k]


def fp8_row_dequant(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """E4M3 rows [..., D] with one f32 scale per row [...] -> f32."""
    return e4m3_decode(codes) * scales.float()[..., None]


# ------------------------------------------------------------- DSA FP8 index cache
INDEX_PAGE = 64
INDEX_DIM = 128
INDEX_VALUE_BYTES = INDEX_PAGE * INDEX_DIM  # 8192; the f32 scales follow
INDEX_PAGE_BYTES = INDEX_PAGE * (INDEX_DIM + 4)  # 8448 (glm53/gfx950/runner.py:28-31)


def index_key_scale_code(amax: torch.Tensor) -> torch.Tensor:
    """The f32 exponent field of an FP8 index key's scale: ceil-pow2 of
    max(amax, f32(1e-4)) / 448, the IEEE quotient (glm53/gfx950/kernel.py:3134-3144)."""
    v = torch.maximum(_f32(amax), _f32(1.0e-4)) / _f32(FP8_MAX)
    return _ceil_pow2_code(v)


def index_key_quant(k: torch.Tensor):
    """Index keys [..., 128] -> (E4M3 uint8 [..., 128], f32 scales [...]): the values
    times 2^(127 - field), exactly the inverse power of two (kernel.py:3145-3147)."""
    field = index_key_scale_code(_f32(k).abs().amax(-1))
    scale = torch.exp2((field - 127).to(torch.float32))
    inv = torch.exp2((127 - field).to(torch.float32))
    return e4m3_encode(_f32(k) * inv[..., None]), scale


def index_page_decode(pages: torch.Tensor) -> torch.Tensor:
    """uint8 index pages [P, 64, 132] (or [P, 8448]) -> f32 keys [P, 64, 128], each
    value times its key's scale, by the byte -> (token, dim) map of the 16 x 16 tiles
    (glm53/check.py:75-82)."""
    pg = pages.reshape(-1, INDEX_PAGE_BYTES)
    b = torch.arange(INDEX_VALUE_BYTES)
    token = (b // 2048) * 16 + (b % 256) // 16
    dim = ((b % 2048) // 256) * 16 + b % 16
    vals = e4m3_decode(pg[:, :INDEX_VALUE_BYTES].contiguous())
    scales = pg[:, INDEX_VALUE_BYTES:].contiguous().view(torch.float32)  # [P, 64]
    keys = torch.empty(pg.shape[0], INDEX_PAGE, INDEX_DIM, dtype=torch.float32)
    keys[:, token, dim] = vals * scales[:, token]
    return keys


# ----------------------------------------------------------------------------- bf16
def bf16_round(x: torch.Tensor) -> torch.Tensor:
    """f32 -> nearest-even bf16, returned as f32."""
    return _f32(x).to(torch.bfloat16).to(torch.float32)


# ------------------------------------------------------------------------ radix keys
def radix_keys(scores: torch.Tensor) -> torch.Tensor:
    """f32 scores -> int64 keys in [0, 2^32) whose order is the f32 order, larger keys
    ranking first (glm53/check.py:111-114: b >= 0 -> b + 2^31, else ~b & 0xFFFFFFFF)."""
    b = _f32(scores).contiguous().view(torch.int32).to(torch.int64)
    return torch.where(b >= 0, b + (1 << 31), (~b) & 0xFFFFFFFF)

