"""A small model in SGLang's own module layout, for the binding tests (no SGLang here).

The attribute names, dtypes and memory layouts are those the reference binds
(glm53/gfx950/weights.py:214-731, glm53/spec.py:527-556):
- block-FP8 linears carry ``weight`` (E4M3) and ``weight_scale_inv``;
- ``w_kc`` / ``w_vc`` are transposed views of [heads][kv_lora][nope] and
  [heads][v][kv_lora] memory;
- the experts hold the shared expert fused as physical expert n_experts (block FP8),
  or are MXFP4 (E2M1 bytes + E8M0 codes) beside a block-FP8 ``shared_experts``
  module; with ``shuffled`` they are in AITER's (16, 16) layout with e8m0_shuffle'd
  codes and marked ``is_shuffled``, as SGLang leaves them for AITER's MoE, and the
  block-FP8 linears are preshuffled into the same layout and marked
  ``aiter_bpreshuffled`` (their scales unchanged), as SGLang leaves them for AITER's
  preshuffled GEMM;
- the token-to-KV pool gives E4M3 rows [slots, 1, 576] and FP8 index pages.
The caches are filled with a random history, so a step's rows have context.
"""

from __future__ import annotations

from types import SimpleNamespace

import torch

HF = SimpleNamespace(
    hidden_size=2048, q_lora_rank=1024, kv_lora_rank=512, qk_rope_head_dim=64, qk_nope_head_dim=128,
    v_head_dim=128, num_attention_heads=16, index_n_heads=16, index_head_dim=128, index_topk=256,
    n_routed_experts=64, num_experts_per_tok=8, moe_intermediate_size=256, n_shared_experts=1,
    scoring_func="sigmoid", routed_scaling_factor=2.5, rms_norm_eps=1e-6, max_context=2048,
    architectures=["GlmMoeDsaForCausalLM"],
)
VOCAB = 1000
LAYERS = 2


def _gen(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _fp8_linear(g, rows, cols, device, std=0.02, shuffled=False):
    from sgl_amd_mono.k2.packing import aiter_shuffle
    from sgl_amd_mono.k2.quant import quant_fp8_block

    q, s = quant_fp8_block(torch.randn(rows, cols, generator=g, device=device) * std)
    if shuffled:
        return SimpleNamespace(weight=aiter_shuffle(q).view(torch.float8_e4m3fn), weight_scale_inv=s,
                               aiter_bpreshuffled=True)
    return SimpleNamespace(weight=q.view(torch.float8_e4m3fn), weight_scale_inv=s)


def _norm(g, n, device):
    return SimpleNamespace(weight=(1 + 0.1 * torch.randn(n, generator=g, device=device)).to(torch.bfloat16))


def _mark(t: torch.Tensor) -> torch.Tensor:
    t.is_shuffled = True  # what AITER's shuffle_weight sets on the tensor it returns
    return t


def _experts(g, hf, device, experts: str, shuffled: bool):
    """SGLang's fused-MoE parameters: block FP8 with the shared expert fused as expert
    E, or MXFP4 (then the shared expert is a separate module, returned second)."""
    from sgl_amd_mono.k2.packing import aiter_shuffle, e8m0_shuffle
    from sgl_amd_mono.k2.quant import quant_mxfp4

    H, E, I = hf.hidden_size, hf.n_routed_experts, hf.moe_intermediate_size
    if experts == "fp8":
        w13 = torch.empty(E + 1, 2 * I, H, dtype=torch.uint8, device=device)
        s13 = torch.empty(E + 1, 2 * I // 128, H // 128, device=device)
        w2 = torch.empty(E + 1, H, I, dtype=torch.uint8, device=device)
        s2 = torch.empty(E + 1, H // 128, I // 128, device=device)
        for e in range(E + 1):
            a, b = _fp8_linear(g, 2 * I, H, device), _fp8_linear(g, H, I, device)
            w13[e], s13[e] = a.weight.view(torch.uint8), a.weight_scale_inv
            w2[e], s2[e] = b.weight.view(torch.uint8), b.weight_scale_inv
        if shuffled:
            w13, w2 = aiter_shuffle(w13), aiter_shuffle(w2)
        w13, w2 = w13.view(torch.float8_e4m3fn), w2.view(torch.float8_e4m3fn)
        if shuffled:
            w13, w2 = _mark(w13), _mark(w2)
        return SimpleNamespace(w13_weight=w13, w13_weight_scale_inv=s13, w2_weight=w2, w2_weight_scale_inv=s2), None
    w13 = torch.empty(E, 2 * I, H // 2, dtype=torch.uint8, device=device)
    s13 = torch.empty(E, 2 * I, H // 32, dtype=torch.uint8, device=device)
    w2 = torch.empty(E, H, I // 2, dtype=torch.uint8, device=device)
    s2 = torch.empty(E, H, I // 32, dtype=torch.uint8, device=device)
    for e in range(E):
        w13[e], s13[e] = quant_mxfp4(0.02 * torch.randn(2 * I, H, generator=g, device=device))
        w2[e], s2[e] = quant_mxfp4(0.02 * torch.randn(H, I, generator=g, device=device))
    if shuffled:
        w13, s13, w2, s2 = _mark(aiter_shuffle(w13)), e8m0_shuffle(s13), _mark(aiter_shuffle(w2)), e8m0_shuffle(s2)
    SI = I * hf.n_shared_experts
    shared = SimpleNamespace(gate_up_proj=_fp8_linear(g, 2 * SI, H, device, shuffled=shuffled),
                             down_proj=_fp8_linear(g, H, SI, device, shuffled=shuffled))
    return SimpleNamespace(w13_weight=w13, w13_weight_scale=s13, w2_weight=w2, w2_weight_scale=s2), shared


def make_model(seed: int, device, hf=HF, vocab=VOCAB, layers=LAYERS, experts: str = "fp8", shuffled: bool = False):
    from sgl_amd_mono.k2 import synth

    g = _gen(seed, device)
    H, QL, KV, R, NO, V = (hf.hidden_size, hf.q_lora_rank, hf.kv_lora_rank, hf.qk_rope_head_dim,
                           hf.qk_nope_head_dim, hf.v_head_dim)
    NH, IH, E, I = hf.num_attention_heads, hf.index_n_heads, hf.n_routed_experts, hf.moe_intermediate_size
    rope = synth.rope_cos_sin(hf.max_context - 1, R, device)
    mods = []
    for _ in range(layers):
        attn = SimpleNamespace(
            fused_qkv_a_proj_with_mqa=_fp8_linear(g, QL + KV + R, H, device, shuffled=shuffled),
            q_a_layernorm=_norm(g, QL, device), kv_a_layernorm=_norm(g, KV, device),
            q_b_proj=_fp8_linear(g, NH * (NO + R), QL, device, shuffled=shuffled),
            o_proj=_fp8_linear(g, H, NH * V, device, shuffled=shuffled),
            # SGLang's memory order, seen through the logical shapes it keeps
            w_kc=(0.05 * torch.randn(NH, KV, NO, generator=g, device=device)).to(torch.bfloat16).transpose(1, 2),
            w_vc=(0.02 * torch.randn(NH, V, KV, generator=g, device=device)).to(torch.bfloat16).transpose(1, 2),
            rotary_emb=SimpleNamespace(cos_sin_cache=rope),
            indexer=SimpleNamespace(
                wq_b=_fp8_linear(g, IH * 128, QL, device, shuffled=shuffled),
                wk=_fp8_linear(g, 128, H, device, shuffled=shuffled),
                k_norm=SimpleNamespace(weight=1 + 0.1 * torch.randn(128, generator=g, device=device),
                                       bias=0.1 * torch.randn(128, generator=g, device=device)),
                weights_proj=SimpleNamespace(
                    weight=(0.02 * torch.randn(IH, H, generator=g, device=device)).to(torch.bfloat16)),
            ),
        )
        ex, shared = _experts(g, hf, device, experts, shuffled)
        mlp = SimpleNamespace(
            gate=SimpleNamespace(weight=(0.02 * torch.randn(E, H, generator=g, device=device)).to(torch.bfloat16),
                                 e_score_correction_bias=0.05 * torch.randn(E, generator=g, device=device)),
            experts=ex,
        )
        if shared is not None:
            mlp.shared_experts = shared
        mods.append(SimpleNamespace(self_attn=attn, mlp=mlp, input_layernorm=_norm(g, H, device),
                                    post_attention_layernorm=_norm(g, H, device)))
    emb = torch.randn(vocab, H, generator=g, device=device).to(torch.bfloat16)
    model = SimpleNamespace(layers=mods, embed_tokens=SimpleNamespace(weight=emb), norm=_norm(g, H, device))
    lm_head = SimpleNamespace(weight=(H ** -0.5 * torch.randn(vocab, H, generator=g, device=device)).to(torch.bfloat16))
    return SimpleNamespace(model=model, lm_head=lm_head, logits_processor=LogitsProcessor())


class LogitsProcessor:
    """SGLang's logits processor as the forward uses it: called with the final
    norm's rows, it returns the logits of _get_logits."""

    def _get_logits(self, hidden_states, lm_head, logits_metadata, *args, **kwargs):
        return hidden_states.float() @ lm_head.weight.float().t()

    def __call__(self, input_ids, hidden_states, lm_head, forward_batch, aux=None):
        return self._get_logits(hidden_states, lm_head, None)


class Pool:
    """SGLang's token-to-KV pool: per layer E4M3 latent rows and FP8 index pages."""

    def __init__(self, layers, pages, device, seed):
        from sgl_amd_mono.k2 import quant, synth

        g = _gen(seed, device)
        self.kv, self.idx = [], []
        for _ in range(layers):
            lat = torch.randn(pages * 64, 576, generator=g, device=device).clamp(-400, 400)
            self.kv.append(lat.to(torch.float8_e4m3fn).view(pages * 64, 1, 576))
            keys = torch.randn(pages, 64, 128, generator=g, device=device)
            self.idx.append(synth.index_pages_fp8(*quant.quant_index_fp8(keys)).view(pages, 64 * 132))

    def get_key_buffer(self, i):
        return self.kv[i]

    def get_index_k_with_scale_buffer(self, i):
        return self.idx[i]


def make_step(rows: int, context: int, pages: int, device, seed: int):
    """A decode step: each row a request with its own pages, a position in the context,
    out_cache_loc the slot of that position through the page table."""
    g = _gen(seed, device)
    ppr = context // 64
    pt = (torch.randperm(pages - 1, generator=g, device=device)[: rows * ppr] + 1).view(rows, ppr).to(torch.int32)
    pos = torch.randint(64, context, (rows,), generator=g, device=device).to(torch.int64)
    loc = pt[torch.arange(rows, device=device), (pos // 64).long()].long() * 64 + pos % 64
    ids = torch.randint(0, VOCAB, (rows,), generator=g, device=device).to(torch.int64)
    return SimpleNamespace(page_table=pt.contiguous(), positions=pos, input_ids=ids,
                           forward_batch=SimpleNamespace(out_cache_loc=loc))
