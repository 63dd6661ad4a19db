"""The case __graft_entry__.smoke() runs: one persistent launch of the chained K2 layer
(configs[4] geometry, context cut to 4096 positions) over 2 decode rows, checked
piecewise against the CPU oracle (refs.check_layer: top-k lists exact, scores within
1e-4 of f64, attention and layer outputs within rel-L2 1e-2, expert ids exact)."""

from dataclasses import replace

import torch

from refs import check_layer, cpu


def run(dev):
    from sgl_amd_mono.k2 import config as C, synth
    from sgl_amd_mono.k2.ops import LayerOp

    base = C.C5_LAYER
    cfg = replace(base, mla=replace(base.mla, context=4096), indexer=replace(base.indexer, context=4096))
    rows = 2
    L = synth.make_layer(cfg, rows, 4242, dev)
    op = LayerOp(cfg, L, rows, device=dev)
    H, E, K = cfg.mla.hidden, cfg.moe.n_experts, cfg.moe.top_k
    status = torch.full((1,), -1, dtype=torch.int32, device=dev)
    attn = torch.empty(rows, H, dtype=torch.bfloat16, device=dev)
    scores = torch.empty(rows, cfg.indexer.context, dtype=torch.float32, device=dev)
    topk = torch.empty(rows, cfg.indexer.topk, dtype=torch.int32, device=dev)
    logits = torch.empty(rows, E, dtype=torch.float32, device=dev)
    ids = torch.empty(rows, K, dtype=torch.int32, device=dev)
    wts = torch.empty(rows, K, dtype=torch.float32, device=dev)
    out = op(attn_out=attn, scores=scores, topk=topk, logits=logits, topk_ids=ids, topk_weights=wts,
             status=status)
    torch.cuda.synchronize()
    if int(status.item()) != 0:
        raise AssertionError("smoke: a dependency wait of the persistent launch gave up")
    stats = check_layer(L, *[cpu(t) for t in (out, attn, scores, topk, logits, ids, wts)])
    print("smoke:", stats)
