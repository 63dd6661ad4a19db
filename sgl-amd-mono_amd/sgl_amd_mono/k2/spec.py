"""The K2 monokernel spec: registry entry, refusal reasons, build and forward.

Mirrors the reference's per-model spec (sgl_amd_mono/glm53/spec.py:588-778): SGLang
routes a decode (or speculative-verify) step to the spec by its CUDA-graph key
``ShapeKey(forward_mode, batch_size, tokens_per_request)`` against
``DeviceLimits.widths``; ``build(model, hf_config, ctx)`` binds the model's layers and
returns an object whose ``forward(plan, ...)`` runs one K2 launch a layer.

This build serves one GPU's share of the layer (TP size 1: the reference's TP
all-reduces are not part of it).  A routed step runs, on SGLang's own tensors
(sgl_amd_mono.k2.binding): the step tables, the embedding rows, then per layer the
front (the reference's K1: norms, projections, RoPE, this step's cache rows) and the
K2 layer launch, then the tail (final norm, LM head), whose logits SGLang's logits
processor returns -- the reference's _Built.forward / _backbone / _layer
(glm53/spec.py:395-556).
"""

from __future__ import annotations

from types import SimpleNamespace

import torch

from .. import _registry_module
from . import config as C

_local = _registry_module()  # SGLang's registry classes, or the local stand-in


ROWS = (1, 2, 4, 8, 16, 32)  # decode rows a launch serves (verify: batch x draft tokens)
TP_SIZES = (1,)
RESIDENT_BLOCKS = 256  # one workgroup per MI355X CU

NUMERICS = _local.Numerics(
    _local.NumericsKind.TOLERANCE,
    {
        "layer_out_rel_l2": 1e-2,  # bf16 outputs against the oracle
        "index_score_rel_max": 1e-4,  # index scores against f64, of the row's max
        "topk": "exact",  # the radix list of the launch's own scores
        "expert_ids": "exact",  # top-k of the launch's own router keys, lower id on ties
    },
)


def config_disable_reasons(server_args) -> list:
    """Why a server configuration cannot use the spec (empty: it can)."""
    why = []
    dtype = getattr(server_args, "dtype", "bfloat16")
    if dtype not in ("bfloat16", "auto"):
        why.append(f"dtype {dtype}: the kernels take bf16 activations")
    kv = getattr(server_args, "kv_cache_dtype", "fp8_e4m3")
    if kv not in ("fp8_e4m3", "auto"):
        why.append(f"kv_cache_dtype {kv}: the latent cache is FP8 E4M3 with per-token scales")
    tp = getattr(server_args, "tp_size", 1)
    if tp not in TP_SIZES:
        why.append(f"tp_size {tp}: this build runs one GPU's share (no TP reduce)")
    page = getattr(server_args, "page_size", C.PAGE) or C.PAGE
    if page != C.PAGE:
        why.append(f"page_size {page}: the caches use {C.PAGE}-token pages")
    return why


def config_from_hf(hf) -> C.K2Config:
    """The layer geometry of an HF config (DeepSeek-V3.2 / GLM-5 field names)."""
    moe = C.MoEConfig(
        hidden=hf.hidden_size,
        n_experts=hf.n_routed_experts,
        top_k=hf.num_experts_per_tok,
        inter=hf.moe_intermediate_size,
        router=C.ROUTER_SIGMOID_BIAS if getattr(hf, "scoring_func", "sigmoid") == "sigmoid" else C.ROUTER_SOFTMAX,
        route_scale=float(getattr(hf, "routed_scaling_factor", 1.0)),
        expert_fmt=C.FMT_MXFP4 if getattr(hf, "expert_format", "mxfp4") == "mxfp4" else C.FMT_FP8,
        n_shared=int(getattr(hf, "n_shared_experts", 1) > 0),
        shared_inter=hf.moe_intermediate_size * max(1, getattr(hf, "n_shared_experts", 1)),
    )
    mla = C.MlaConfig(
        heads=hf.num_attention_heads,
        kv_lora=hf.kv_lora_rank,
        rope=hf.qk_rope_head_dim,
        v_dim=hf.v_head_dim,
        hidden=hf.hidden_size,
        topk=hf.index_topk,
        context=getattr(hf, "max_context", 65536),
    )
    idx = C.IndexerConfig(heads=hf.index_n_heads, dim=hf.index_head_dim, topk=hf.index_topk,
                          context=mla.context)
    return C.K2Config(mla=mla, indexer=idx, moe=moe, eps=float(getattr(hf, "rms_norm_eps", 1e-6)))


def model_disable_reasons(hf) -> list:
    """Why a model cannot run on the spec (empty: it can)."""
    try:
        cfg = config_from_hf(hf)
        cfg.validate(max(ROWS))
    except (AttributeError, ValueError) as e:
        return [str(e)]
    return []


def front_config_from_hf(hf, weight_fmt: int = C.WFMT_FP8_BLOCK) -> C.FrontConfig:
    """The front's geometry of an HF config: SGLang's DSA caches (FP8 index pages,
    unscaled E4M3 latent rows)."""
    return C.FrontConfig(
        hidden=hf.hidden_size, q_lora=hf.q_lora_rank, kv_lora=hf.kv_lora_rank, rope=hf.qk_rope_head_dim,
        nope=hf.qk_nope_head_dim, heads=hf.num_attention_heads, index_heads=hf.index_n_heads,
        weight_fmt=weight_fmt, keys=C.KEYS_FP8, kv_scaled=False,
        max_position=getattr(hf, "max_context", 65536) - 1, eps=float(getattr(hf, "rms_norm_eps", 1e-6)),
    )


class K2Forward:
    """What build() returns: a routed step on SGLang's model (the reference's _Built,
    glm53/spec.py:395-556).  pool_of(forward_batch) and page_table_of(forward_batch,
    rows) give SGLang's token-to-KV pool and the rows' int32 page table; by default from
    SGLang's forward context and attention backend."""

    def __init__(self, lm, cfg: C.K2Config, front_cfg: C.FrontConfig, tail_cfg: C.TailConfig, device,
                 *, pool_of=None, page_table_of=None):
        from . import binding

        self.lm, self.cfg, self.front_cfg, self.tail_cfg, self.device = lm, cfg, front_cfg, tail_cfg, device
        layers = lm.model.layers
        self.fronts = [binding.bind_front(L, front_cfg) for L in layers]
        self.mlas = [binding.bind_mla(L, cfg.mla, front_cfg.nope) for L in layers]
        self.moes = [binding.bind_moe(L, cfg.moe) for L in layers]
        self.emb = lm.model.embed_tokens.weight
        self.g_norm = lm.model.norm.weight
        self.w_head = lm.lm_head.weight
        cs = layers[0].self_attn.rotary_emb.cos_sin_cache
        self.cos_sin = cs.float().contiguous()[: front_cfg.max_position + 1]
        self.max_position = front_cfg.max_position
        self.pool_of = pool_of or _sglang_pool
        self.page_table_of = page_table_of or _sglang_page_table
        self._ops, self._steps, self._tails, self._tables, self._fused = {}, {}, {}, {}, {}
        # each layer's front and layer as ONE persistent launch where the library
        # instantiates the front shape with these experts (mk2_layer_step_is_fused), as
        # the reference's K2 launch carries its front; else two launches a layer
        self.fuse_front = True
        # one sticky status word for every layer launch of a step (a persistent launch
        # whose dependency wait gave up ORs 1 into it; the fronts keep theirs in their
        # workspaces): a stopped launch's outputs are undefined, so a step with any
        # word set returns NaN logits and, on the eager path, raises (the reference's
        # guard stops visibly, common/guard.py:91-97,211-227)
        self._status = torch.zeros(1, dtype=torch.int32, device=device)
        # the logits processor returns the tail's logits on a routed step (the reference
        # hooks _get_logits the same way, glm53/spec.py:423-441)
        lp = getattr(lm, "logits_processor", None)
        self._logits = None
        if lp is not None and hasattr(lp, "_get_logits"):
            self._own_logits = lp._get_logits
            lp._get_logits = self._get_logits

    def _get_logits(self, hidden_states, lm_head, logits_metadata, *args, **kwargs):
        if self._logits is None:
            return self._own_logits(hidden_states, lm_head, logits_metadata, *args, **kwargs)
        return self._logits[: hidden_states.shape[0]]

    def tables(self, rows: int):
        """The row tables every layer op of width `rows` reads: one page table of the
        widest context (max_position + 1 tokens), into which a step copies SGLang's
        rows once; req_ids and ctx_len are the step rows' own tensors (filled in place
        by the step-table launch).  Shared by all layers, so a step copies nothing per
        layer and the ops do not depend on the width of SGLang's table."""
        if rows not in self._tables:
            st = self.step_rows(rows)
            pages = (self.max_position + 64) // 64
            pt = torch.zeros(rows, pages, dtype=torch.int32, device=self.device)
            self._tables[rows] = SimpleNamespace(page_table=pt, req_ids=st.req_ids, ctx_len=st.ctx_len)
        return self._tables[rows]

    def ops(self, li: int, rows: int, kv=None, icache=None):
        """(FrontOp, LayerOp) of layer li at `rows` rows, created on first use with the
        layer's caches (kv, icache) and the shared row tables; the layer's input tensors
        are rebound every step."""
        from .ops import FrontOp, LayerOp, LayerStepOp

        key = (li, rows)
        if key not in self._ops:
            dev, cfg, fc = self.device, self.cfg, self.front_cfg
            tab = self.tables(rows)
            idx = SimpleNamespace(
                cfg=cfg.indexer, rows=rows,
                q=torch.empty(rows, fc.index_heads, 128, dtype=torch.bfloat16, device=dev),
                w=torch.empty(rows, fc.index_heads, dtype=torch.bfloat16, device=dev),
                cache=icache, cache_scale=None, page_table=tab.page_table, req_ids=tab.req_ids,
                ctx_len=tab.ctx_len)
            mla = SimpleNamespace(**vars(self.mlas[li]))
            mla.rows = rows
            mla.q = torch.empty(rows, fc.heads, fc.kv_lora + fc.rope, dtype=torch.bfloat16, device=dev)
            mla.kv, mla.kv_scale, mla.page_table, mla.req_ids = kv, None, tab.page_table, tab.req_ids
            L = SimpleNamespace(cfg=cfg, rows=rows, idx=idx, mla=mla, moe=self.moes[li],
                                h=torch.empty(rows, cfg.mla.hidden, dtype=torch.bfloat16, device=dev))
            fo, lo = FrontOp(fc, self.fronts[li], rows, device=dev), LayerOp(cfg, L, rows, device=dev)
            self._ops[key] = (fo, lo)
            if fo.fuses_with(cfg.moe.expert_fmt):
                self._fused[key] = LayerStepOp(fo, lo)
        return self._ops[key]

    def fused(self, li: int, rows: int):
        """The LayerStepOp (front and layer in one launch) of layer li at `rows` rows,
        or None where the library has no such instance (or fuse_front is off)."""
        return self._fused.get((li, rows)) if self.fuse_front else None

    def step_rows(self, rows: int):
        from .ops import StepRows

        if rows not in self._steps:
            self._steps[rows] = StepRows(rows, self.cfg.indexer.topk, device=self.device)
        return self._steps[rows]

    def tail(self, rows: int):
        from .ops import TailOp

        if rows not in self._tails:
            self._tails[rows] = TailOp(self.tail_cfg, self.g_norm, self.w_head, rows, device=self.device)
        return self._tails[rows]

    def status_words(self, rows: int) -> list:
        """The device status words of a step at `rows` rows: the layers' shared word and
        every front's (a 1-element int32 view each)."""
        return [self._status] + [self._ops[(li, rows)][0].status_word() for li in range(len(self.fronts))
                                 if (li, rows) in self._ops]

    def backbone(self, plan, input_ids, positions, forward_batch):
        """Every layer one front-and-layer launch (or a front and a layer launch where
        the library does not fuse the shape), then the tail: (normed rows, logits).
        The logits are NaN when any launch of the step stopped early (gate_logits)."""
        accepts = getattr(SPEC, "accepts", None)  # SGLang routes by the spec itself
        if accepts is not None:
            ok, why = accepts(plan.key)
            if not ok:
                raise ValueError(why)
        S = plan.key.batch_size * plan.key.tokens_per_request
        st = self.step_rows(S)(forward_batch.out_cache_loc, positions, S, self.max_position, ids_in=input_ids)
        pt = self.page_table_of(forward_batch, S)
        tab = self.tables(S)
        w = min(pt.shape[1], tab.page_table.shape[1])
        tab.page_table[:, :w].copy_(pt[:S, :w])  # once a step, for every layer
        pool = self.pool_of(forward_batch)
        from . import binding

        h = torch.nn.functional.embedding(input_ids[:S].long(), self.emb)
        for li in range(len(self.fronts)):
            kv, icache = binding.layer_caches(pool, li, self.front_cfg.index_heads > 0)
            fo, lo = self.ops(li, S, kv, icache)
            L = lo.L
            L.idx.cache, L.mla.kv, L.h = icache, kv, h
            out = plan.state.setdefault(("h", li % 2, S), torch.empty_like(h))
            step = self.fused(li, S)
            if step is not None:
                h = step(st.positions, st.slots, self.cos_sin, out=out, status=self._status)
            else:
                fo(h, st.positions, st.slots, self.cos_sin, kv, None, icache, None,
                   mla_q=L.mla.q, index_q=L.idx.q, index_w=L.idx.w)
                h = lo(out=out, status=self._status)
        logits, normed = self.tail(S)(h)
        gate_logits(self.status_words(S), logits)
        return normed, logits

    def check(self, rows: int) -> None:
        """Raises RuntimeError when a launch of a step at `rows` rows stopped early since
        the last check, and clears the words (synchronizes; raise_if_stopped)."""
        raise_if_stopped(self.status_words(rows))

    def forward(self, plan, input_ids, positions, forward_batch, input_embeds=None, pp_proxy_tensors=None):
        """DeepseekV2ForCausalLM.forward for a routed decode or verify step; with input
        embeddings, SGLang's own forward (as the reference, glm53/spec.py:443-461).  On
        the eager path a step whose launch stopped early raises instead of returning
        logits; under graph capture its logits are NaN (no host read is possible)."""
        lm = self.lm
        if input_embeds is not None:
            return type(lm).forward(lm, input_ids, positions, forward_batch, input_embeds, pp_proxy_tensors)
        normed, self._logits = self.backbone(plan, input_ids, positions, forward_batch)
        try:
            if not torch.cuda.is_current_stream_capturing():
                self.check(plan.key.batch_size * plan.key.tokens_per_request)
            return lm.logits_processor(input_ids, normed, lm.lm_head, forward_batch, None)
        finally:
            self._logits = None


def gate_logits(status_words, logits) -> None:
    """logits := NaN where any status word is nonzero, on the device (no host read, so a
    captured step carries it too): a stopped launch's output never becomes a token."""
    bad = torch.stack([w.reshape(()) for w in status_words]).ne(0).any()
    logits.masked_fill_(bad, float("nan"))


def raise_if_stopped(status_words) -> None:
    """Reads the status words (a host read); if any is set, clears them all and raises
    RuntimeError: a launch of the step stopped early and its outputs are undefined."""
    vals = [int(w.reshape(()).item()) for w in status_words]
    if any(vals):
        for w in status_words:
            w.zero_()
        raise RuntimeError(f"K2 step: a persistent launch stopped early (a dependency wait gave up; status words "
                           f"{vals}); its outputs are not valid")


def _sglang_pool(forward_batch):
    from sglang.srt.model_executor.forward_context import get_token_to_kv_pool  # type: ignore

    return get_token_to_kv_pool()


def _sglang_page_table(forward_batch, rows: int):
    from sglang.srt.model_executor.forward_context import get_attn_backend  # type: ignore

    return get_attn_backend().forward_metadata.real_page_table[:rows]


def _build(model, hf_config, ctx):
    """Binds SGLang's model (``model`` is its DeepseekV2ForCausalLM / GLM-5 module
    tree) and returns the forward; ``ctx`` may carry pool_of / page_table_of."""
    from dataclasses import replace

    from .binding import experts_layout, linear

    cfg = config_from_hf(hf_config)
    layer0 = model.model.layers[0]
    qkv = layer0.self_attn.fused_qkv_a_proj_with_mqa
    first = qkv.weight
    # the front's format (bf16, block FP8, or block FP8 SGLang preshuffled for AITER)
    _, _, wfmt = linear("fused_qkv_a_proj_with_mqa", qkv, first.shape[0], first.shape[1])
    # SGLang's DSA index cache holds FP8 pages; its experts' dtype names their mode
    efmt = C.FMT_FP8 if layer0.mlp.experts.w13_weight.dtype == torch.float8_e4m3fn else C.FMT_MXFP4
    # experts SGLang rewrote for AITER's MoE are read in place in that layout
    layout = experts_layout(layer0.mlp.experts)
    cfg = replace(cfg, moe=replace(cfg.moe, expert_fmt=efmt, weight_layout=layout),
                  indexer=replace(cfg.indexer, keys=C.KEYS_FP8))
    rows = layer0.self_attn.rotary_emb.cos_sin_cache.shape[0]
    front = front_config_from_hf(hf_config, wfmt)
    front = replace(front, max_position=min(front.max_position, rows - 1))
    tail = C.TailConfig(hidden=hf_config.hidden_size, vocab_rows=model.lm_head.weight.shape[0],
                        eps=float(getattr(hf_config, "rms_norm_eps", 1e-6)))
    device = getattr(ctx, "device", None) or first.device
    return K2Forward(model, cfg, front, tail, device, pool_of=getattr(ctx, "pool_of", None),
                     page_table_of=getattr(ctx, "page_table_of", None))


SPEC = _local.MonoSpec(
    name="k2_gfx950",
    devices={"gfx950": _local.DeviceLimits(widths=ROWS, tp_sizes=TP_SIZES, resident_blocks=RESIDENT_BLOCKS)},
    features=frozenset({_local.Feature.SPECULATIVE_DECODING}),
    requires=_local.Requirements(
        dtypes=frozenset({"bfloat16"}),
        attention_backends=frozenset({"dsa"}),
        server_args={"kv_cache_dtype": frozenset({"auto", "fp8_e4m3"}), "tp_size": frozenset(TP_SIZES)},
        env={},
    ),
    numerics=NUMERICS,
    model_disable_reasons=model_disable_reasons,
    build=_build,
    api_version=1,
    config_disable_reasons=config_disable_reasons,
)
