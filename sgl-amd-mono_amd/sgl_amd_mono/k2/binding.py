"""Binding SGLang's DeepSeek-V3.2 / GLM-5 model to the kernels.

Mirrors the reference's weight binding and per-step cache binding
(glm53/gfx950/weights.py:214-731 ``_linear``, ``_uk_uv``, ``_indexer``,
``_fp8_experts``, ``layer_weights``; glm53/spec.py:527-556 ``_bind``):

- Read in place wherever the kernels read SGLang's layout as it is:
  - the front's block-FP8 (row-major, or preshuffled by SGLang into AITER's (16, 16)
    layout) or bf16 linears: ``fused_qkv_a_proj_with_mqa``, ``q_b_proj``, and the
    indexer's ``wq_b`` and ``wk``;
  - the norms, the indexer's ``weights_proj``, and ``w_kc`` / ``w_vc``;
  - the experts' block scales and the rotary table;
  - the caches from SGLang's token-to-KV pool: the unscaled E4M3 latent rows
    [slots, 576] and the FP8 index pages [pages, 64, 132].
  - the experts (block FP8 or MXFP4, routed and shared) when SGLang left them in
    AITER's (16, 16) layout for AITER's MoE, which the expert kernels read as it is.
- Copied once, at bind time, where a kernel takes its own tile layout:
  - the router (bf16 tiles);
  - W_o (dequantized to bf16 tiles);
  - row-major experts (into E4M3 / E2M1 tiles), with the fused shared expert
    (SGLang's physical expert n_experts) split out as the shared expert.
"""

from __future__ import annotations

from types import SimpleNamespace

import torch

from . import config as C
from .packing import aiter_shuffle, aiter_unshuffle, pack_e8m0, pack_tiles
from .synth import pack_bf16


def _need(name: str, t, shape, dtypes) -> torch.Tensor:
    if t is None:
        raise ValueError(f"needs {name}")
    if tuple(t.shape) != tuple(shape) or t.dtype not in dtypes:
        raise ValueError(f"needs {name} {list(shape)} of {[str(d) for d in dtypes]}, got {list(t.shape)} {t.dtype}")
    return t


def _fp8_bytes(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint8)


def _block_dequant(w: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """E4M3 [N, K] with f32 [ceil(N/128), ceil(K/128)] block scales -> f32."""
    n, k = w.shape
    sc = s.float().repeat_interleave(128, 0).repeat_interleave(128, 1)[:n, :k]
    return w.view(torch.float8_e4m3fn).float() * sc


def _linear_shuffled(lin) -> bool:
    # SGLang marks a linear it rewrote into AITER's (16, 16) layout (weights.py:142-147)
    return bool(getattr(lin, "aiter_bpreshuffled", False) or getattr(lin.weight, "is_shuffled", False))


def linear(name: str, lin, rows: int, cols: int, allow_shuffled: bool = True):
    """(weight bytes or bf16, f32 block scales or None, weight format C.WFMT_*) of a
    linear as SGLang keeps it after loading (the reference's _linear,
    weights.py:214-224), read in place: bf16, block FP8 row-major, or block FP8 that
    SGLang preshuffled into AITER's (16, 16) layout (WFMT_FP8_AITER16; refused with
    `allow_shuffled` False).  A shuffled bf16 linear is refused."""
    shuffled = _linear_shuffled(lin)
    w = lin.weight
    if w.dtype == torch.float8_e4m3fn:
        if shuffled and not allow_shuffled:
            raise ValueError(f"needs {name} row-major (not AITER's shuffled layout)")
        _need(name, w, (rows, cols), (torch.float8_e4m3fn,))
        s = _need(f"{name}.weight_scale_inv", getattr(lin, "weight_scale_inv", None),
                  ((rows + 127) // 128, (cols + 127) // 128), (torch.float32,))
        return _fp8_bytes(w), s, C.WFMT_FP8_AITER16 if shuffled else C.WFMT_FP8_BLOCK
    if shuffled:
        raise ValueError(f"needs {name} row-major or block FP8 (a shuffled bf16 linear)")
    _need(name, w, (rows, cols), (torch.bfloat16,))
    return w, None, C.WFMT_BF16


def _bf16_of(name: str, lin, rows: int, cols: int) -> torch.Tensor:
    """A linear's weight as bf16 (dequantized from block FP8, unshuffled from AITER's
    layout): a copy for a kernel that takes bf16 tiles."""
    w, s, fmt = linear(name, lin, rows, cols)
    if fmt == C.WFMT_FP8_AITER16:
        w, fmt = aiter_unshuffle(w), C.WFMT_FP8_BLOCK
    return (_block_dequant(w, s) if fmt == C.WFMT_FP8_BLOCK else w.float()).to(torch.bfloat16)


def _uk_uv(attn, heads: int, nope: int, kv_lora: int, v_dim: int):
    """W_UK as the front reads it, bf16 [heads][kv_lora][nope], and W_UV as the
    attention reads it, bf16 [heads][v][kv_lora]: SGLang's w_kc [heads, nope, kv_lora]
    and w_vc [heads, kv_lora, v] transposed -- views of its memory when that is
    already this order, else copies.  Per-tensor FP8 needs its scalar w_scale, as the
    reference requires (weights.py:347-393), and is widened to bf16(e4m3 * w_scale)
    once at bind time: the attention's MFMAs run on bf16 W_UK / W_UV, so each weight
    carries one bf16 rounding the reference's FP8 path does not (within the layer's
    rel-L2 tolerance; not pinned against an FP8-weight reference)."""
    w_kc, w_vc = attn.w_kc, attn.w_vc
    _need("w_kc", w_kc, (heads, nope, kv_lora), (torch.bfloat16, torch.float8_e4m3fn))
    _need("w_vc", w_vc, (heads, kv_lora, v_dim), (torch.bfloat16, torch.float8_e4m3fn))
    out = []
    for t in (w_kc.transpose(1, 2), w_vc.transpose(1, 2)):
        if t.dtype == torch.float8_e4m3fn:
            ws = getattr(attn, "w_scale", None)
            if not torch.is_tensor(ws) or ws.numel() != 1:
                raise ValueError("FP8 w_kc / w_vc need the layer's w_scale as a 1-element tensor")
            t = (t.float() * ws.float().reshape(())).to(torch.bfloat16)
        out.append(t if t.is_contiguous() else t.contiguous())
    return out


def bind_front(layer, cfg: C.FrontConfig) -> SimpleNamespace:
    """A layer's front weights (sgl_amd_mono.k2.ops.FrontOp's fields) from its module."""
    attn = layer.self_attn
    H, QL, NA = cfg.hidden, cfg.q_lora, cfg.q_lora + cfg.kv_lora + cfg.rope
    bf = (torch.bfloat16,)
    ns = SimpleNamespace(cfg=cfg)
    ns.g_in = _need("input_layernorm", layer.input_layernorm.weight, (H,), bf)
    ns.g_q_a = _need("q_a_layernorm", attn.q_a_layernorm.weight, (QL,), bf)
    ns.g_kv_a = _need("kv_a_layernorm", attn.kv_a_layernorm.weight, (cfg.kv_lora,), bf)
    ns.w_qkv_a, ns.s_qkv_a, f0 = linear("fused_qkv_a_proj_with_mqa", attn.fused_qkv_a_proj_with_mqa, NA, H)
    ns.w_q_b, ns.s_q_b, f1 = linear("q_b_proj", attn.q_b_proj, cfg.heads * (cfg.nope + cfg.rope), QL)
    fmts = {f0, f1}
    ns.w_uk, _ = _uk_uv(attn, cfg.heads, cfg.nope, cfg.kv_lora, attn.w_vc.shape[-1])
    ind = getattr(attn, "indexer", None)
    if cfg.index_heads:
        if ind is None:
            raise ValueError("the config has an indexer, the layer none")
        ns.w_iq, ns.s_iq, f2 = linear("indexer.wq_b", ind.wq_b, cfg.index_heads * 128, QL)
        ns.w_ik, ns.s_ik, f3 = linear("indexer.wk", ind.wk, 128, H)
        fmts |= {f2, f3}
        ns.w_iw = _need("indexer.weights_proj", ind.weights_proj.weight, (cfg.index_heads, H), bf)
        ns.g_ik = ind.k_norm.weight.detach().float().contiguous()
        ns.b_ik = ind.k_norm.bias.detach().float().contiguous()
    else:
        ns.w_iq = ns.s_iq = ns.w_ik = ns.s_ik = ns.w_iw = ns.g_ik = ns.b_ik = None
    if fmts != {cfg.weight_fmt}:
        raise ValueError(f"needs the front's linears in one format ({cfg.weight_fmt}), got {sorted(fmts)}")
    return ns


def bind_mla(layer, cfg: C.MlaConfig, nope: int) -> SimpleNamespace:
    """The attention's output weights: W_UV (in place when SGLang's w_vc memory is
    [heads][v][kv_lora]) and W_o as bf16 tiles (a copy; dequantized from block FP8)."""
    attn = layer.self_attn
    ns = SimpleNamespace(cfg=cfg)
    _, ns.w_uv = _uk_uv(attn, cfg.heads, nope, cfg.kv_lora, cfg.v_dim)
    ns.w_o = _bf16_of("o_proj", attn.o_proj, cfg.hidden, cfg.heads * cfg.v_dim)
    ns.w_o_p = pack_bf16(ns.w_o)
    return ns


def experts_layout(experts) -> int:
    """The experts' weight layout as SGLang leaves them: AITER's (16, 16) shuffle when
    it rewrote them for AITER's MoE (it marks the tensor ``is_shuffled``, as the
    reference checks, glm53/gfx950/weights.py:142-147,310-322), else row-major."""
    return C.WLAYOUT_AITER16 if getattr(experts.w13_weight, "is_shuffled", False) else C.WLAYOUT_TILES


def _shared_fp8(mlp, cfg: C.MoEConfig, ns) -> None:
    """A separate ``shared_experts`` module's block-FP8 linears in the experts' layout:
    in place when they are in it already, else a copy."""
    sh = mlp.shared_experts
    H, SI = cfg.hidden, cfg.shared_inter
    out = []
    for name, lin, rows, cols in (("gate_up_proj", sh.gate_up_proj, 2 * SI, H), ("down_proj", sh.down_proj, H, SI)):
        w, s, f = linear("shared_experts." + name, lin, rows, cols)
        if f not in (C.WFMT_FP8_BLOCK, C.WFMT_FP8_AITER16):
            raise ValueError("needs the shared expert in block FP8")
        shuffled = f == C.WFMT_FP8_AITER16
        if cfg.weight_layout == C.WLAYOUT_AITER16:
            out.append((w if shuffled else aiter_shuffle(w), s))
        else:
            out.append((pack_tiles(aiter_unshuffle(w) if shuffled else w, 32), s))
    (ns.ws13_p, ns.ws13s), (ns.ws2_p, ns.ws2s) = out


def bind_moe(layer, cfg: C.MoEConfig) -> SimpleNamespace:
    """The MoE weights (sgl_amd_mono.k2.ops.MoEOp's fields): the post-attention norm in
    place, the router as bf16 tiles, and the experts -- block FP8 (W8A16 / W8A8 modes)
    or MXFP4 (A8W4 / A16W4 / A4W4) -- in place when SGLang left them in AITER's
    (16, 16) layout (cfg.weight_layout AITER16), else copied once into tiles; the
    shared expert (block FP8) from SGLang's fused physical expert n_experts or from a
    separate ``shared_experts`` module (the reference's _fp8_experts / _mxfp4_experts,
    glm53/gfx950/weights.py:510-560)."""
    mlp = layer.mlp
    H, E, I = cfg.hidden, cfg.n_experts, cfg.inter
    ns = SimpleNamespace(cfg=cfg)
    ns.gamma = _need("post_attention_layernorm", layer.post_attention_layernorm.weight, (H,), (torch.bfloat16,))
    router = _need("gate", mlp.gate.weight, (E, H), (torch.bfloat16, torch.float32))
    if router.dtype != torch.bfloat16 and not torch.equal(router.to(torch.bfloat16).float(), router):
        raise ValueError("needs router weights exactly representable in bf16")
    ns.w_router = router.to(torch.bfloat16)
    ns.w_router_p = pack_bf16(ns.w_router)
    ns.bias = None
    if cfg.router == C.ROUTER_SIGMOID_BIAS:
        ns.bias = _need("e_score_correction_bias", mlp.gate.e_score_correction_bias, (E,), (torch.float32,))
    ex = mlp.experts
    if experts_layout(ex) != cfg.weight_layout:
        raise ValueError(f"the experts' layout {experts_layout(ex)} differs from the config's {cfg.weight_layout}")
    aiter = cfg.weight_layout == C.WLAYOUT_AITER16
    phys = ex.w13_weight.shape[0]
    fused_shared = phys == E + 1
    if phys not in (E, E + 1):
        raise ValueError(f"needs {E} routed experts (+1 fused shared), got {phys}")
    if cfg.expert_fmt in C.FP4_WEIGHT_FMTS:
        u8 = (torch.uint8,)
        w13 = _need("w13_weight", ex.w13_weight, (phys, 2 * I, H // 2), u8)
        s13 = _need("w13_weight_scale", ex.w13_weight_scale.view(torch.uint8), (phys, 2 * I, H // 32), u8)
        w2 = _need("w2_weight", ex.w2_weight, (phys, H, I // 2), u8)
        s2 = _need("w2_weight_scale", ex.w2_weight_scale.view(torch.uint8), (phys, H, I // 32), u8)
        if fused_shared:
            raise ValueError("MXFP4 experts with the shared expert fused in: the shared expert runs in block FP8")
        if aiter:  # in place: AITER's E2M1 bytes are the tiles; its E8M0 order is read as it is
            ns.w13_p, ns.s13_p, ns.w2_p, ns.s2_p = w13, s13, w2, s2
        else:
            ns.w13_p, ns.s13_p = pack_tiles(w13, 16), pack_e8m0(s13)
            ns.w2_p, ns.s2_p = pack_tiles(w2, 16), pack_e8m0(s2)
        ns.w13q, ns.w13s, ns.w2q, ns.w2s = w13, s13, w2, s2
    else:
        if cfg.expert_fmt not in (C.FMT_FP8, C.FMT_W8A8):
            raise ValueError(f"unknown expert mode {cfg.expert_fmt}")
        w13 = _need("w13_weight", ex.w13_weight, (phys, 2 * I, H), (torch.float8_e4m3fn,))
        s13 = _need("w13_weight_scale_inv", ex.w13_weight_scale_inv, (phys, 2 * I // 128, H // 128), (torch.float32,))
        w2 = _need("w2_weight", ex.w2_weight, (phys, H, I), (torch.float8_e4m3fn,))
        s2 = _need("w2_weight_scale_inv", ex.w2_weight_scale_inv, (phys, H // 128, I // 128), (torch.float32,))
        ns.w13q, ns.w2q = _fp8_bytes(w13[:E]), _fp8_bytes(w2[:E])
        ns.w13s, ns.w2s = s13[:E], s2[:E]
        ns.s13_p, ns.s2_p = ns.w13s, ns.w2s
        if aiter:  # in place (views of the first E experts)
            ns.w13_p, ns.w2_p = ns.w13q, ns.w2q
        else:
            ns.w13_p, ns.w2_p = pack_tiles(ns.w13q, 32), pack_tiles(ns.w2q, 32)
    if cfg.n_shared:
        if fused_shared:
            ns.ws13q, ns.ws13s = _fp8_bytes(w13[E]), s13[E]
            ns.ws2q, ns.ws2s = _fp8_bytes(w2[E]), s2[E]
            ns.ws13_p = ns.ws13q if aiter else pack_tiles(ns.ws13q, 32)
            ns.ws2_p = ns.ws2q if aiter else pack_tiles(ns.ws2q, 32)
        else:
            _shared_fp8(mlp, cfg, ns)
    else:
        ns.ws13s = ns.ws2s = ns.ws13_p = ns.ws2_p = None
    return ns


def layer_caches(pool, i: int, index: bool):
    """(latent rows uint8 [slots, 576], FP8 index pages uint8 [pages, 64, 132] or None)
    from SGLang's token-to-KV pool, in place (the reference's _bind, spec.py:527-556:
    SGLang's HIP DSA cache is E4M3 rows without scales)."""
    kv = pool.get_key_buffer(i)
    if kv.dtype not in (torch.float8_e4m3fn, torch.uint8) or kv.shape[-1] != 576 or not kv.is_contiguous():
        raise RuntimeError(f"layer {i}: MLA cache {kv.dtype} {tuple(kv.shape)}; needs contiguous E4M3 [slots, 1, 576]")
    kv = kv.view(torch.uint8).view(-1, 576)
    if not index:
        return kv, None
    idx = pool.get_index_k_with_scale_buffer(i)
    if idx.dtype != torch.uint8 or not idx.is_contiguous() or idx.numel() % (64 * 132):
        raise RuntimeError(f"layer {i}: index cache {idx.dtype} {tuple(idx.shape)}; needs contiguous uint8 pages")
    return kv, idx.view(-1, 64, 132)
