"""The HIP kernels against the committed golden vectors (inputs regenerated on the
CPU from the fixture's seed, digests checked, then copied to the GPU).  Bar: ids and
top-k lists exact (the fixtures have no near ties at the boundary), floats within
the parity tolerances of the other GPU tests."""

import json
import os

import numpy as np
import pytest
import torch

import golden_cases as G
from oracle import reference as R

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _load(name):
    z = np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    return meta, {k: torch.from_numpy(z[k]) for k in z.files if k != "meta"}


@pytest.mark.parametrize("name", ["moe_fp8_small", "moe_mxfp4_small"])
def test_gpu_golden_moe(name):
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2.ops import MoEOp

    dev = _dev()
    meta, exp = _load(name)
    w0 = G.regenerate(meta, "cpu")
    assert G.digests(w0) == meta["sha256"]
    w = G.to_device(w0, dev)
    cfg, rows, norm = C.MoEConfig(**meta["cfg"]), meta["rows"], meta["norm"]
    op = MoEOp(cfg, w, rows, norm=norm, residual=norm, eps=1e-6)
    ids = torch.empty(rows, cfg.top_k, dtype=torch.int32, device=dev)
    lg = torch.empty(rows, cfg.n_experts, dtype=torch.float32, device=dev)
    out = op(w.x, logits=lg, topk_ids=ids)
    torch.cuda.synchronize()
    assert torch.equal(ids.cpu(), exp["ids"])
    assert ((lg.cpu() - exp["logits"]).abs() / exp["logits"].abs().amax(-1, keepdim=True)).max() <= 1e-4
    assert R.rel_l2(out.cpu().float(), exp["out"]) <= 1e-2


def test_gpu_golden_indexer():
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2.ops import IndexerOp

    dev = _dev()
    meta, exp = _load("indexer_small")
    ns0 = G.regenerate(meta, "cpu")
    assert G.digests(ns0) == meta["sha256"]
    ns = G.to_device(ns0, dev)
    cfg = C.IndexerConfig(**meta["cfg"])
    op = IndexerOp(cfg, len(meta["ctx_len"]), ns.page_table.shape[1], device=dev)
    scores, topk = op(ns.q, ns.w, ns.cache, ns.cache_scale, ns.page_table, ns.req_ids, ns.ctx_len)
    torch.cuda.synchronize()
    for r, n in enumerate(meta["ctx_len"]):
        ref = exp["scores"][r, :n].double()
        got = scores[r, :n].cpu().double()
        assert ((got - ref).abs().max() / ref.abs().max()) <= 1e-4
        assert torch.equal(topk[r].cpu(), exp["topk"][r])


def test_gpu_golden_mla():
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2.ops import SparseMlaOp

    dev = _dev()
    meta, exp = _load("mla_small")
    ns0 = G.regenerate(meta, "cpu")
    assert G.digests(ns0) == meta["sha256"]
    ns = G.to_device(ns0, dev)
    cfg = C.MlaConfig(**meta["cfg"])
    rows = meta["rows"]
    op = SparseMlaOp(cfg, ns, rows, ns.page_table.shape[1], device=dev)
    olat = torch.empty(rows, cfg.heads, cfg.kv_lora, dtype=torch.float32, device=dev)
    out = op(ns.q, ns.kv, ns.kv_scale, ns.page_table, ns.req_ids, ns.sel, h=ns.h, o_latent=olat)
    torch.cuda.synchronize()
    assert R.rel_l2(olat.cpu(), exp["o_latent"]) <= 1e-2
    assert R.rel_l2(out.cpu().float(), exp["out"]) <= 1e-2
