"""Seeded synthetic layers in the kernels' formats (tests and the benchmark).

There are no checkpoints offline, so every benchmark and parity case runs on
random-init weights of the right architecture: weights ~ N(0, 0.02) before
quantization, activations ~ N(0, 1), shuffled page tables whose page 0 is never
used, and selected positions drawn uniformly without replacement (the input
conventions of test/kernels/glm53/check_layer.py:69-101,248-261).

Each ``make_*`` returns a plain namespace holding the canonical (row-major)
quantized tensors -- what an oracle dequantizes -- and the packed tensors the
kernels stream.  Generation runs on ``device`` with a torch.Generator seeded there.
"""

from __future__ import annotations

from dataclasses import replace
from types import SimpleNamespace

import torch

from . import config as C
from .packing import aiter_shuffle, e8m0_shuffle, pack_e8m0, pack_tiles
from .quant import quant_fp8_block, quant_fp8_rows, quant_index_fp8, quant_mxfp4

WEIGHT_STD = 0.02


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn(g, *shape, device, std=1.0):
    return torch.randn(*shape, generator=g, device=device) * std


def pack_bf16(w: torch.Tensor) -> torch.Tensor:
    """bf16 [..., N, K] -> tiles of 64 B a lane."""
    return pack_tiles(w.contiguous().view(torch.uint8), 64)


def make_moe(cfg: C.MoEConfig, rows: int, seed: int, device, norm: bool = False):
    """Router, routed experts (FP8 or MXFP4), one FP8 shared expert, input rows."""
    g = _gen(seed, device)
    H, E, I, SI = cfg.hidden, cfg.n_experts, cfg.inter, cfg.shared_inter
    ns = SimpleNamespace(cfg=cfg, rows=rows)
    ns.x = _randn(g, rows, H, device=device).to(torch.bfloat16)
    ns.gamma = (1.0 + _randn(g, H, device=device, std=0.1)).to(torch.bfloat16) if norm else None
    ns.w_router = _randn(g, E, H, device=device, std=WEIGHT_STD).to(torch.bfloat16)
    ns.bias = (
        _randn(g, E, device=device, std=0.05).float()
        if cfg.router == C.ROUTER_SIGMOID_BIAS
        else None
    )
    ns.w_router_p = pack_bf16(ns.w_router)
    if cfg.expert_fmt in C.FP4_WEIGHT_FMTS:
        w13q = torch.empty(E, 2 * I, H // 2, dtype=torch.uint8, device=device)
        w13s = torch.empty(E, 2 * I, H // 32, dtype=torch.uint8, device=device)
        w2q = torch.empty(E, H, I // 2, dtype=torch.uint8, device=device)
        w2s = torch.empty(E, H, I // 32, dtype=torch.uint8, device=device)
        for e in range(E):
            w13q[e], w13s[e] = quant_mxfp4(_randn(g, 2 * I, H, device=device, std=WEIGHT_STD))
            w2q[e], w2s[e] = quant_mxfp4(_randn(g, H, I, device=device, std=WEIGHT_STD))
        ns.w13_p, ns.s13_p = pack_tiles(w13q, 16), pack_e8m0(w13s)
        ns.w2_p, ns.s2_p = pack_tiles(w2q, 16), pack_e8m0(w2s)
    else:
        w13q = torch.empty(E, 2 * I, H, dtype=torch.uint8, device=device)
        w13s = torch.empty(E, 2 * I // 128, H // 128, dtype=torch.float32, device=device)
        w2q = torch.empty(E, H, I, dtype=torch.uint8, device=device)
        w2s = torch.empty(E, H // 128, I // 128, dtype=torch.float32, device=device)
        for e in range(E):
            w13q[e], w13s[e] = quant_fp8_block(_randn(g, 2 * I, H, device=device, std=WEIGHT_STD))
            w2q[e], w2s[e] = quant_fp8_block(_randn(g, H, I, device=device, std=WEIGHT_STD))
        ns.w13_p, ns.s13_p = pack_tiles(w13q, 32), w13s
        ns.w2_p, ns.s2_p = pack_tiles(w2q, 32), w2s
    ns.w13q, ns.w13s, ns.w2q, ns.w2s = w13q, w13s, w2q, w2s
    if cfg.n_shared:
        ns.ws13q, ns.ws13s = quant_fp8_block(_randn(g, 2 * SI, H, device=device, std=WEIGHT_STD))
        ns.ws2q, ns.ws2s = quant_fp8_block(_randn(g, H, SI, device=device, std=WEIGHT_STD))
        ns.ws13_p, ns.ws2_p = pack_tiles(ns.ws13q, 32), pack_tiles(ns.ws2q, 32)
    else:
        ns.ws13q = ns.ws13s = ns.ws2q = ns.ws2s = ns.ws13_p = ns.ws2_p = None
    return ns


def moe_in_layout(ns, layout: int):
    """make_moe's weights (routed and shared experts) in another layout (C.WLAYOUT_*):
    the same codes and scales re-laid; the router and the rows are shared."""
    if layout == C.WLAYOUT_TILES:
        return ns
    if layout != C.WLAYOUT_AITER16:
        raise ValueError(f"unknown layout {layout}")
    out = SimpleNamespace(**vars(ns))
    out.w13_p, out.w2_p = aiter_shuffle(ns.w13q), aiter_shuffle(ns.w2q)
    if ns.cfg.expert_fmt in C.FP4_WEIGHT_FMTS:
        out.s13_p, out.s2_p = e8m0_shuffle(ns.w13s), e8m0_shuffle(ns.w2s)
    if ns.ws13q is not None:
        out.ws13_p, out.ws2_p = aiter_shuffle(ns.ws13q), aiter_shuffle(ns.ws2q)
    out.cfg = replace(ns.cfg, weight_layout=layout)
    return out


def _page_table(g, requests: int, pages_per_req: int, device) -> torch.Tensor:
    """Shuffled physical pages 1 .. requests * pages_per_req (page 0 never used)."""
    perm = torch.randperm(requests * pages_per_req, generator=g, device=device) + 1
    return perm.view(requests, pages_per_req).to(torch.int32).contiguous()


def index_plane(codes: torch.Tensor, scales: torch.Tensor):
    """Token-major FP4 keys (codes [P, 64, 64], E8M0 [P, 64, 4]) -> SGLang's FP4 index
    plane: codes [P, 4 chunks, 64 tokens, 16 B] and scales [P, 4 chunks, 64] with token
    t's byte at (t % 16) * 4 + t // 16 (score_fp4.py:9-12, the deepseek_v4 memory pool)."""
    P = codes.shape[0]
    plane = codes.view(P, 64, 4, 16).permute(0, 2, 1, 3).reshape(P, 4096).contiguous()
    sc = scales.view(P, 4, 16, 4).permute(0, 3, 2, 1).reshape(P, 256).contiguous()
    return plane, sc


def index_pages_fp8(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Token-major FP8 keys (E4M3 codes [P, 64, 128], f32 scales [P, 64]) -> SGLang's DSA
    index pages, uint8 [P, 64, 132]: token t's dim d at byte (t // 16) * 2048 + (d // 16)
    * 256 + (t % 16) * 16 + d % 16 (glm53/gfx950/kernel.py:698-705), then the 64 scales."""
    P = codes.shape[0]
    tiles = codes.view(P, 4, 16, 8, 16).permute(0, 1, 3, 2, 4).reshape(P, 64 * 128)
    sc = scales.float().contiguous().view(torch.uint8).view(P, 256)
    return torch.cat([tiles, sc], dim=1).view(P, 64, 132).contiguous()


def make_indexer(cfg: C.IndexerConfig, rows: int, seed: int, device, ctx_len=None, draft: int = 1):
    """Index-key pages in the config's format (FP4: E2M1 codes + E8M0 per 32 dims in the
    FP4 plane; FP8: the DSA pages, cache_scale None), bf16 queries and head weights ~
    N(0, 1).  One request a row, or with draft > 1 a speculative verify step: rows
    draft * i .. draft * i + draft - 1 are request i's draft tokens, at the context's
    last draft positions (context lengths context - draft + 1 .. context), sharing the
    request's pages."""
    if draft < 1 or rows % draft:
        raise ValueError(f"rows {rows} must be a multiple of draft {draft}")
    g = _gen(seed, device)
    ctx = cfg.context
    ppr = ctx // C.PAGE
    reqs = rows // draft
    ns = SimpleNamespace(cfg=cfg, rows=rows)
    ns.q = _randn(g, rows, cfg.heads, cfg.dim, device=device).to(torch.bfloat16)
    ns.w = _randn(g, rows, cfg.heads, device=device).to(torch.bfloat16)
    ns.page_table = _page_table(g, reqs, ppr, device)
    n_pages = reqs * ppr + 1
    keys = _randn(g, n_pages, C.PAGE, cfg.dim, device=device)
    if cfg.keys == C.KEYS_FP8:
        ns.cache, ns.cache_scale = index_pages_fp8(*quant_index_fp8(keys)), None
    else:
        codes, scales = quant_mxfp4(keys)  # [P, 64, 64], [P, 64, 4]
        ns.cache, ns.cache_scale = index_plane(codes, scales)
    ns.req_ids = torch.arange(rows, dtype=torch.int32, device=device) // draft
    if ctx_len is None:
        ctx_len = [ctx - draft + 1 + r % draft for r in range(rows)]
    ns.ctx_len = torch.tensor(ctx_len, dtype=torch.int32, device=device)
    return ns


def make_mla(cfg: C.MlaConfig, rows: int, seed: int, device, residual: bool = True, h_std: float = 1.0):
    """FP8 latent-KV pages with per-token f32 scales, absorbed bf16 queries,
    selected positions, W_UV and W_o (bf16, ~ N(0, 0.02)), residual rows ~ N(0,
    h_std^2).  A small h_std keeps the attention term o W_o^T above the bf16 rounding
    of h + o W_o^T, so a check of the sum minus h sees the attention's own error."""
    g = _gen(seed, device)
    ctx = cfg.context
    ppr = ctx // C.PAGE
    ns = SimpleNamespace(cfg=cfg, rows=rows)
    ns.q = _randn(g, rows, cfg.heads, cfg.qk_dim, device=device).to(torch.bfloat16)
    ns.page_table = _page_table(g, rows, ppr, device)
    n_pages = rows * ppr + 1
    kv = _randn(g, n_pages, C.PAGE, cfg.qk_dim, device=device)
    ns.kv, ns.kv_scale = quant_fp8_rows(kv)
    ns.req_ids = torch.arange(rows, dtype=torch.int32, device=device)
    ns.sel = torch.stack(
        [torch.randperm(ctx, generator=g, device=device)[: cfg.topk] for _ in range(rows)]
    ).to(torch.int32).contiguous()
    ns.w_uv = _randn(g, cfg.heads, cfg.v_dim, cfg.kv_lora, device=device, std=WEIGHT_STD).to(
        torch.bfloat16
    )
    ns.w_o = _randn(g, cfg.hidden, cfg.heads * cfg.v_dim, device=device, std=WEIGHT_STD).to(
        torch.bfloat16
    )
    ns.w_o_p = pack_bf16(ns.w_o)
    ns.h = _randn(g, rows, cfg.hidden, device=device, std=h_std).to(torch.bfloat16) if residual else None
    return ns


def rope_cos_sin(max_position: int, rope: int, device, theta: float = 10000.0) -> torch.Tensor:
    """SGLang's cos_sin_cache layout, f32 [max_position + 1][rope]: cos of position * f_i
    in the first half, sin in the second, f_i = theta^(-2i / rope)."""
    inv = theta ** (-torch.arange(0, rope, 2, dtype=torch.float64) / rope)
    ang = torch.arange(max_position + 1, dtype=torch.float64)[:, None] * inv[None, :]
    return torch.cat([ang.cos(), ang.sin()], dim=1).float().to(device).contiguous()


def _front_weight(g, rows, cols, fmt, device, std=WEIGHT_STD):
    w = _randn(g, rows, cols, device=device, std=std)
    if fmt == C.WFMT_FP8_BLOCK:
        return quant_fp8_block(w)
    return w.to(torch.bfloat16).contiguous(), None


def front_in_layout(ns, fmt: int):
    """make_front's block-FP8 weights (W_qkv_a, W_q_b, W_iq, W_ik) in AITER's (16, 16)
    layout (C.WFMT_FP8_AITER16): the same codes and scales re-laid."""
    if fmt != C.WFMT_FP8_AITER16 or ns.cfg.weight_fmt != C.WFMT_FP8_BLOCK:
        raise ValueError("re-lays block-FP8 front weights into AITER's layout")
    out = SimpleNamespace(**vars(ns))
    for name in ("w_qkv_a", "w_q_b", "w_iq", "w_ik"):
        if getattr(ns, name) is not None:
            setattr(out, name, aiter_shuffle(getattr(ns, name)))
    out.cfg = replace(ns.cfg, weight_fmt=fmt)
    return out


def make_front(cfg: C.FrontConfig, rows: int, seed: int, device, n_pages: int = 64):
    """The front's weights in SGLang's formats (row-major bf16 or E4M3 + 128 x 128 f32
    block scales, w_kc as [heads][kv_lora][nope]), residual rows x ~ N(0, 1), distinct
    cache slots in n_pages 64-token pages, random positions, and empty caches of both
    the latent rows and the configured index format."""
    g = _gen(seed, device)
    ns = SimpleNamespace(cfg=cfg, rows=rows)
    H, QL, NA = cfg.hidden, cfg.q_lora, cfg.q_lora + cfg.kv_lora + cfg.rope
    ns.x = _randn(g, rows, H, device=device).to(torch.bfloat16)
    norm = lambda n: (1.0 + _randn(g, n, device=device, std=0.1)).to(torch.bfloat16)  # noqa: E731
    ns.g_in, ns.g_q_a, ns.g_kv_a = norm(H), norm(QL), norm(cfg.kv_lora)
    ns.w_qkv_a, ns.s_qkv_a = _front_weight(g, NA, H, cfg.weight_fmt, device)
    ns.w_q_b, ns.s_q_b = _front_weight(g, cfg.heads * (cfg.nope + cfg.rope), QL, cfg.weight_fmt, device)
    ns.w_uk = _randn(g, cfg.heads, cfg.kv_lora, cfg.nope, device=device, std=0.05).to(torch.bfloat16)
    ih = cfg.index_heads
    if ih:
        ns.w_iq, ns.s_iq = _front_weight(g, ih * 128, QL, cfg.weight_fmt, device)
        ns.w_ik, ns.s_ik = _front_weight(g, 128, H, cfg.weight_fmt, device)
        ns.g_ik = 1.0 + _randn(g, 128, device=device, std=0.1)
        ns.b_ik = _randn(g, 128, device=device, std=0.1)
        ns.w_iw = _randn(g, ih, H, device=device, std=WEIGHT_STD).to(torch.bfloat16)
    else:
        ns.w_iq = ns.s_iq = ns.w_ik = ns.s_ik = ns.g_ik = ns.b_ik = ns.w_iw = None
    ns.rope_cos_sin = rope_cos_sin(cfg.max_position, cfg.rope, device)
    ns.positions = torch.randint(0, cfg.max_position + 1, (rows,), generator=g, device=device).to(torch.int64)
    ns.slots = torch.randperm(n_pages * C.PAGE, generator=g, device=device)[:rows].to(torch.int64)
    ns.kv_cache = torch.zeros(n_pages * C.PAGE, cfg.kv_lora + cfg.rope, dtype=torch.uint8, device=device)
    ns.kv_scale = torch.zeros(n_pages * C.PAGE, dtype=torch.float32, device=device) if cfg.kv_scaled else None
    if cfg.keys == C.KEYS_FP8:
        ns.index_cache = torch.zeros(n_pages, C.PAGE, 132, dtype=torch.uint8, device=device)
        ns.index_scale = None
    else:
        ns.index_cache = torch.zeros(n_pages, 4096, dtype=torch.uint8, device=device)
        ns.index_scale = torch.zeros(n_pages, 256, dtype=torch.uint8, device=device)
    return ns


def make_tail(cfg: C.TailConfig, rows: int, seed: int, device):
    """The last layer's rows x ~ N(0, 1) (bf16), the final norm's weight 1 + N(0,
    0.1^2) and LM-head rows ~ N(0, 1/hidden) in SGLang's bf16 [vocab_rows, hidden]."""
    g = _gen(seed, device)
    ns = SimpleNamespace(cfg=cfg, rows=rows)
    ns.x = _randn(g, rows, cfg.hidden, device=device).to(torch.bfloat16)
    ns.g_norm = (1.0 + _randn(g, cfg.hidden, device=device, std=0.1)).to(torch.bfloat16)
    ns.w_head = _randn(g, cfg.vocab_rows, cfg.hidden, device=device, std=cfg.hidden**-0.5).to(torch.bfloat16)
    return ns


def make_layer(cfg: C.K2Config, rows: int, seed: int, device, h_std: float = 1.0, draft: int = 1):
    """One chained layer: indexer keys and queries, latent-KV pages sharing the
    indexer's page table, attention weights, residual rows ~ N(0, h_std^2), MoE
    weights with the post-attention RMSNorm weight.  draft > 1: a verify step of
    rows / draft requests with draft tokens each (make_indexer)."""
    idx = make_indexer(cfg.indexer, rows, seed, device, draft=draft)
    mla = make_mla(cfg.mla, rows, seed + 1, device, residual=True, h_std=h_std)
    mla.page_table = idx.page_table
    mla.req_ids = idx.req_ids
    mla.sel = None  # the chain supplies the indexer's selection
    moe = make_moe(cfg.moe, rows, seed + 2, device, norm=True)
    return SimpleNamespace(cfg=cfg, rows=rows, idx=idx, mla=mla, moe=moe, h=mla.h)


def view_rows(L, rows: int):
    """The first `rows` decode rows of a layer built for more (weights, caches and page
    tables shared; the per-row inputs sliced, still contiguous)."""
    if not 1 <= rows <= L.rows:
        raise ValueError(f"rows must be in [1, {L.rows}]")
    idx = SimpleNamespace(**vars(L.idx))
    mla = SimpleNamespace(**vars(L.mla))
    for ns, names in ((idx, ("q", "w", "req_ids", "ctx_len")), (mla, ("q", "req_ids", "h"))):
        for n in names:
            t = getattr(ns, n)
            if t is not None:
                setattr(ns, n, t[:rows])
        ns.rows = rows
    return SimpleNamespace(cfg=L.cfg, rows=rows, idx=idx, mla=mla, moe=L.moe, h=mla.h)
