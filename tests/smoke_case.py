"""The case __graft_entry__.smoke() runs: one persistent launch of the chained K2 layer
(configs[4] geometry, context cut to 4096 positions) over 2 decode rows, checked
piecewise against the CPU oracle (refs.check_layer: top-k lists exact, scores within
1e-4 of f64, the merged attention, the attention term and the MoE term within rel-L2
1e-2 of the oracle's, expert ids exact; residual rows ~ N(0, (1/128)^2) so that the
attention term is resolvable above the bf16 rounding of the residual sum)."""

from dataclasses import replace

import torch

from refs import check_layer, cpu


def run(dev):
    from sgl_amd_mono.k2 import config as C, synth
    from sgl_amd_mono.k2.ops import LayerOp

    base = C.C5_LAYER
    cfg = replace(base, mla=replace(base.mla, context=4096), indexer=replace(base.indexer, context=4096))
    rows = 2
    L = synth.make_layer(cfg, rows, 4242, dev, h_std=1.0 / 128)
    op = LayerOp(cfg, L, rows, device=dev)
    H, E, K = cfg.mla.hidden, cfg.moe.n_experts, cfg.moe.top_k
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    attn = torch.empty(rows, H, dtype=torch.bfloat16, device=dev)
    scores = torch.empty(rows, cfg.indexer.context, dtype=torch.float32, device=dev)
    topk = torch.empty(rows, cfg.indexer.topk, dtype=torch.int32, device=dev)
    logits = torch.empty(rows, E, dtype=torch.float32, device=dev)
    ids = torch.empty(rows, K, dtype=torch.int32, device=dev)
    wts = torch.empty(rows, K, dtype=torch.float32, device=dev)
    olat = torch.empty(rows, cfg.mla.heads, cfg.mla.kv_lora, dtype=torch.float32, device=dev)
    out = op(attn_out=attn, scores=scores, topk=topk, logits=logits, topk_ids=ids, topk_weights=wts,
             status=status, o_latent=olat)
    torch.cuda.synchronize()
    if int(status.item()) != 0:
        raise AssertionError("smoke: a dependency wait of the persistent launch gave up")
    stats = check_layer(L, *[cpu(t) for t in (out, attn, scores, topk, logits, ids, wts)], o_latent=cpu(olat))
    if not (stats["attn_term_checked"] and stats["moe_term_checked"]):
        raise AssertionError(f"smoke: the attention term was not resolvable: {stats}")
    print("smoke:", stats)
