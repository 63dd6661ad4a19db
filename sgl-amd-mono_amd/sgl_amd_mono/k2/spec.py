"""The K2 monokernel spec: registry entry, refusal reasons, build and forward.

Mirrors the reference's per-model spec (sgl_amd_mono/glm53/spec.py:588-778): SGLang
routes a decode (or speculative-verify) step to the spec by its CUDA-graph key
``ShapeKey(forward_mode, batch_size, tokens_per_request)`` against
``DeviceLimits.widths``; ``build(model, hf_config, ctx)`` binds the model's layers and
returns an object whose ``forward(plan, ...)`` runs one K2 launch a layer.

This build serves one GPU's share of the layer (TP size 1: the reference's TP
all-reduces are not part of it).  The layer's front (input RMSNorm, q/kv
projections, RoPE, cache writes: the reference's K1) is outside the path; the
forward receives its products -- index queries and head weights, absorbed MLA
queries -- with the step.
"""

from __future__ import annotations

from types import SimpleNamespace

from .. import _registry as _local
from . import config as C


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


class K2Forward:
    """What build() returns: one chained-layer launch a layer, per routed step."""

    def __init__(self, cfg: C.K2Config, layers, device):
        self.cfg, self.layers, self.device = cfg, layers, device
        self._ops = {}  # (layer, rows) -> LayerOp

    def op(self, li: int, rows: int):
        from .ops import LayerOp

        key = (li, rows)
        if key not in self._ops:
            L = self.layers[li]
            if L.rows != rows:
                L = replace_rows(L, rows)
            self._ops[key] = LayerOp(self.cfg, L, rows, device=self.device)
        return self._ops[key]

    def forward(self, plan, input_ids=None, positions=None, forward_batch=None, input_embeds=None,
                pp_proxy_tensors=None):
        """Runs every layer on the step's rows; returns the last hidden rows (bf16)."""
        ok, why = SPEC.accepts(plan.key)
        if not ok:
            raise ValueError(why)
        rows = plan.key.rows
        fb = forward_batch
        h = fb.hidden
        if tuple(h.shape) != (rows, self.cfg.mla.hidden):
            raise ValueError(f"hidden rows {tuple(h.shape)} do not match the plan's {rows} rows")
        for li in range(len(self.layers)):
            op = self.op(li, rows)
            L = op.L
            L.h = h
            L.idx.q, L.idx.w, L.mla.q = fb.index_q[li], fb.index_w[li], fb.mla_q[li]
            L.idx.ctx_len = L.mla.ctx_len = fb.ctx_len
            h = op(out=plan.state.setdefault(("out", li % 2), h.new_empty(h.shape)))
        return h


def replace_rows(L, rows):
    """A layer namespace viewed for a different row count (weights shared)."""
    return SimpleNamespace(**{**vars(L), "rows": rows})


def _build(model, hf_config, ctx):
    """Binds a model's layers (namespaces in the kernels' formats, one a layer, as
    sgl_amd_mono.k2.synth builds them) and returns the forward."""
    cfg = config_from_hf(hf_config)
    layers = list(model.k2_layers)
    device = getattr(ctx, "device", None) or layers[0].h.device
    return K2Forward(cfg, layers, device)


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
