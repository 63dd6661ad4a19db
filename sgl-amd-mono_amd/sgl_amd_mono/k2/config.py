"""Geometry of the K2 decode layer (one GPU's share) and the five benchmark shapes.

The reference fixes one geometry per model in ``glm53/gfx950/config.py:184-197``
(hidden 6144, kv_lora 512, rope 64, 256 experts, top-8, inter 256 a rank, route
scale 2.5).  Here each piece of the layer is a frozen dataclass so the same
kernels serve the FP8 MoE block, the MXFP4 MoE shard,
sparse MLA, the FP4 indexer and the chained layer
(configs[4]).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field, replace

PAGE = 64  # tokens a KV / index page (glm53/gfx950/config.py page size 64)

ROUTER_SOFTMAX = 0  # softmax over the picked logits (qwen38 style)
ROUTER_SIGMOID_BIAS = 1  # sigmoid, picked by sigmoid + bias, * route_scale (glm53)
# expert modes (the reference's MoE modes, glm53/gfx950/config.py:88-93, and MXFP4 rows)
FMT_FP8 = 0  # W8A16: E4M3 weights, f32 128 x 128 block scales, bf16 activations
FMT_MXFP4 = 1  # A8W4: E2M1 weights, E8M0 per 32, MXFP8 activations
FMT_W8A8 = 2  # E4M3 weights, E4M3 activations with an f32 scale per 128
FMT_A16W4 = 3  # E2M1 weights, bf16 activations
FMT_A4W4 = 4  # E2M1 weights, MXFP4 activations
FP4_WEIGHT_FMTS = (FMT_MXFP4, FMT_A16W4, FMT_A4W4)
# index cache formats (MK2_KEYS_*)
KEYS_FP4 = 0  # SGLang's FP4 index plane: E2M1 codes + E8M0 per 32 dims, two tensors
KEYS_FP8 = 1  # SGLang's DSA index cache: uint8 [pages, 64, 132], E4M3 + f32 scale a key
# the FP4 plane scored against the queries quantized to MXFP4 in the kernel, on the
# FP4 x FP4 scaled MFMA (the verify-width scorer; its scores are the quantized queries')
KEYS_FP4_Q4 = 2
# the expert weights' layouts (MK2_WLAYOUT_*)
WLAYOUT_TILES = 0  # this build's tile packing (k2/packing.py pack_tiles / pack_e8m0)
WLAYOUT_AITER16 = 1  # AITER's (16, 16) shuffle + e8m0_shuffle, as SGLang leaves them for AITER

MAX_ROWS = 32  # decode rows a launch serves (verify: 8 requests x 4 draft tokens)


@dataclass(frozen=True)
class MoEConfig:
    hidden: int
    n_experts: int
    top_k: int
    inter: int
    router: int
    route_scale: float
    expert_fmt: int
    n_shared: int
    shared_inter: int
    weight_layout: int = WLAYOUT_TILES

    def validate(self, rows: int) -> None:
        """The rules of the C side (mk2_moe_workspace_bytes), checked before any call."""
        if not 1 <= rows <= MAX_ROWS:
            raise ValueError(f"rows must be in [1, {MAX_ROWS}], got {rows}")
        if self.hidden < 512 or self.hidden % 512:
            raise ValueError(f"hidden must be a positive multiple of 512, got {self.hidden}")
        if self.n_experts not in (64, 128, 192, 256):
            raise ValueError(f"n_experts must be 64, 128, 192 or 256, got {self.n_experts}")
        if not 1 <= self.top_k <= 8:
            raise ValueError(f"top_k must be in [1, 8], got {self.top_k}")
        if self.router not in (ROUTER_SOFTMAX, ROUTER_SIGMOID_BIAS):
            raise ValueError(f"unknown router {self.router}")
        if self.expert_fmt not in (FMT_FP8, FMT_MXFP4, FMT_W8A8, FMT_A16W4, FMT_A4W4):
            raise ValueError(f"unknown expert mode {self.expert_fmt}")
        imax = 4096 if self.expert_fmt in FP4_WEIGHT_FMTS else 1024
        if self.inter < 128 or self.inter % 128 or self.inter > imax:
            raise ValueError(f"inter must be a multiple of 128 in [128, {imax}] for this format, got {self.inter}")
        if self.n_shared not in (0, 1):
            raise ValueError("at most one shared expert")
        if self.n_shared and (self.shared_inter < 128 or self.shared_inter % 128 or self.shared_inter > 4096):
            raise ValueError(f"shared_inter must be a multiple of 128 in [128, 4096], got {self.shared_inter}")
        if self.weight_layout not in (WLAYOUT_TILES, WLAYOUT_AITER16):
            raise ValueError(f"unknown weight_layout {self.weight_layout}")
        if self.weight_layout == WLAYOUT_AITER16 and self.expert_fmt in FP4_WEIGHT_FMTS and self.inter % 256:
            raise ValueError(f"AITER's E8M0 layout needs inter a multiple of 256, got {self.inter}")


@dataclass(frozen=True)
class MlaConfig:
    heads: int = 16
    kv_lora: int = 512
    rope: int = 64
    v_dim: int = 128
    hidden: int = 6144
    topk: int = 2048
    context: int = 32768

    @property
    def qk_dim(self) -> int:
        return self.kv_lora + self.rope

    @property
    def sm_scale(self) -> float:
        return 1.0 / math.sqrt(self.qk_dim)

    def validate(self, rows: int) -> None:
        """The rules of the C side (mk2_mla_workspace_bytes)."""
        if (self.heads, self.kv_lora, self.rope) != (16, 512, 64):
            raise ValueError("the MLA kernels serve 16 heads of 512 + 64 latent dims")
        if self.v_dim < 16 or self.v_dim % 16 or self.v_dim > 512 or (self.heads * self.v_dim) % 128:
            raise ValueError("v_dim must be a multiple of 16 in [16, 512] with heads * v_dim a multiple of 128")
        if self.hidden < 16 or self.hidden % 16:
            raise ValueError("hidden must be a positive multiple of 16")
        if self.topk < 64 or self.topk % 64 or self.topk > 65536:
            raise ValueError("topk must be a multiple of 64 in [64, 65536]")
        if self.context < 64 or self.context % PAGE:
            raise ValueError("context must be a positive multiple of 64")
        if not 1 <= rows <= MAX_ROWS:
            raise ValueError(f"rows must be in [1, {MAX_ROWS}]")


@dataclass(frozen=True)
class IndexerConfig:
    heads: int = 64
    dim: int = 128
    topk: int = 2048
    context: int = 65536
    keys: int = KEYS_FP4

    def validate(self, rows: int) -> None:
        if self.dim != 128:
            raise ValueError("index keys are 128 dims")
        if self.keys not in (KEYS_FP4, KEYS_FP8, KEYS_FP4_Q4):
            raise ValueError(f"unknown index cache format {self.keys}")
        if self.heads % 16 or not 16 <= self.heads <= 64:
            raise ValueError("index heads must be a multiple of 16 in [16, 64]")
        if not 64 <= self.context <= 65536 or self.context % PAGE:
            raise ValueError("context must be a multiple of 64 in [64, 65536]")
        if self.topk % 64 or not 64 <= self.topk <= 4096:
            raise ValueError("topk must be a multiple of 64 in [64, 4096]")
        if not 1 <= rows <= MAX_ROWS:
            raise ValueError(f"rows must be in [1, {MAX_ROWS}]")


@dataclass(frozen=True)
class K2Config:
    mla: MlaConfig = field(default_factory=MlaConfig)
    indexer: IndexerConfig = field(default_factory=IndexerConfig)
    moe: MoEConfig = None  # type: ignore[assignment]
    eps: float = 1e-6

    def validate(self, rows: int) -> None:
        self.mla.validate(rows)
        self.indexer.validate(rows)
        self.moe.validate(rows)
        if self.mla.hidden != self.moe.hidden:
            raise ValueError("attention and MoE hidden sizes differ")
        if self.mla.topk != self.indexer.topk:
            raise ValueError("the attention attends the indexer's top-k")
        if self.mla.context != self.indexer.context:
            raise ValueError("the indexer and the attention share one context")


WFMT_BF16 = 0  # attention weights as loaded in bf16
WFMT_FP8_BLOCK = 1  # E4M3 with f32 128 x 128 block scales
WFMT_FP8_AITER16 = 2  # the same, the bytes in AITER's (16, 16) layout (SGLang's preshuffled linears)
_ENGINE_K = (1024, 2048, 3072, 4096, 6144, 7168, 8192)


@dataclass(frozen=True)
class FrontConfig:
    """The layer's front (the reference's K1) on one GPU's heads."""

    hidden: int = 6144
    q_lora: int = 2048
    kv_lora: int = 512
    rope: int = 64
    nope: int = 192
    heads: int = 16
    index_heads: int = 64  # 0: no indexer
    weight_fmt: int = WFMT_FP8_BLOCK
    keys: int = KEYS_FP4
    kv_scaled: bool = True
    max_position: int = 65535
    eps: float = 1e-6
    index_eps: float = 1e-6

    def validate(self, rows: int) -> None:
        """The rules of the C side (mk2_front_workspace_bytes)."""
        if not 1 <= rows <= MAX_ROWS:
            raise ValueError(f"rows must be in [1, {MAX_ROWS}], got {rows}")
        if self.hidden not in _ENGINE_K or self.q_lora not in _ENGINE_K:
            raise ValueError(f"hidden and q_lora must be among {_ENGINE_K}")
        if self.kv_lora != 512 or self.rope != 64:
            raise ValueError("kv_lora must be 512 and rope 64")
        if self.nope not in (128, 192, 256):
            raise ValueError("nope must be 128, 192 or 256")
        if not 1 <= self.heads <= 128:
            raise ValueError("heads must be in [1, 128]")
        if self.index_heads and (self.index_heads % 16 or self.index_heads > 64):
            raise ValueError("index_heads must be 0 or a multiple of 16 up to 64")
        if self.weight_fmt not in (WFMT_BF16, WFMT_FP8_BLOCK, WFMT_FP8_AITER16):
            raise ValueError(f"unknown weight format {self.weight_fmt}")
        if self.keys not in (KEYS_FP4, KEYS_FP8):
            raise ValueError(f"unknown index cache format {self.keys}")
        if self.max_position < 0 or not (self.eps > 0 and self.index_eps > 0):
            raise ValueError("max_position must be >= 0 and the eps positive")


@dataclass(frozen=True)
class TailConfig:
    """The tail after the last layer: final RMSNorm, then this GPU's LM-head rows."""

    hidden: int = 6144
    vocab_rows: int = 19360  # GLM-5.3's 154880-token vocabulary over 8 GPUs
    eps: float = 1e-5

    def validate(self, rows: int) -> None:
        """The rules of the C side (mk2_tail_launch)."""
        if not 1 <= rows <= MAX_ROWS:
            raise ValueError(f"rows must be in [1, {MAX_ROWS}], got {rows}")
        if self.hidden % 1024 or not 2048 <= self.hidden <= 8192:
            raise ValueError(f"hidden must be a multiple of 1024 in [2048, 8192], got {self.hidden}")
        if self.vocab_rows < 1:
            raise ValueError(f"vocab_rows must be positive, got {self.vocab_rows}")
        if not self.eps > 0:
            raise ValueError("eps must be positive")


# FP8 MoE block, CPU-runnable
C1_MOE = MoEConfig(
    hidden=2048, n_experts=64, top_k=8, inter=768, router=ROUTER_SOFTMAX,
    route_scale=1.0, expert_fmt=FMT_FP8, n_shared=1, shared_inter=768,
)
# MXFP4 MoE decode shard (one GPU's share: inter 2048 / 8)
C2_MOE = MoEConfig(
    hidden=6144, n_experts=256, top_k=8, inter=256, router=ROUTER_SIGMOID_BIAS,
    route_scale=2.5, expert_fmt=FMT_MXFP4, n_shared=1, shared_inter=256,
)
# sparse-MLA decode attention + o_proj
C3_MLA = MlaConfig(context=32768)
# FP4 indexer + exact top-2048
C4_INDEXER = IndexerConfig(context=65536)
# the chained layer (3 + 4 + 2), one context for indexer and attention
C5_LAYER = K2Config(
    mla=replace(C3_MLA, context=65536), indexer=C4_INDEXER, moe=C2_MOE, eps=1e-6
)
# the tail after the layer stack (one GPU's share of the LM head)
C6_TAIL = TailConfig()
# the layer's front ahead of configs[4] (GLM-5 geometry on one GPU's 16 heads)
C7_FRONT = FrontConfig()
