#!/usr/bin/env python3
"""Writes the golden vectors under tests/golden/ (run from the repo root).

The reference ships no data files (its checks seed their inputs at run time), so
the vectors are this repo's own: small seeded cases of every piece of the layer,
generated on the CPU by sgl_amd_mono.k2.synth, with the oracle's outputs.  To keep
the files small, each fixture stores its inputs as (config, seed, SHA-256 of every
generated tensor) -- a test regenerates them and checks the digests before use --
and its expected outputs as arrays.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "sgl-amd-mono_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

from sgl_amd_mono.k2 import config as C  # noqa: E402
from sgl_amd_mono.k2 import synth  # noqa: E402


from golden_cases import digests  # noqa: E402


# ------------------------------------------------------------------- the cases
MOE_FP8 = C.MoEConfig(hidden=512, n_experts=64, top_k=8, inter=128, router=C.ROUTER_SOFTMAX,
                      route_scale=1.0, expert_fmt=C.FMT_FP8, n_shared=1, shared_inter=128)
MOE_MXFP4 = C.MoEConfig(hidden=512, n_experts=64, top_k=8, inter=128, router=C.ROUTER_SIGMOID_BIAS,
                        route_scale=2.5, expert_fmt=C.FMT_MXFP4, n_shared=1, shared_inter=128)
INDEXER = C.IndexerConfig(heads=16, dim=128, topk=128, context=1024)
INDEXER_CTX = [1024, 700, 129]
MLA = C.MlaConfig(hidden=256, v_dim=16, topk=128, context=1024)


def case_moe(name, cfg, rows, seed, norm):
    from refs import MoEOracle

    w = synth.make_moe(cfg, rows, seed, "cpu", norm=norm)
    out, ids, wts, logits = MoEOracle(w)(w.x, norm=norm, residual=norm, eps=1e-6)
    meta = {"kind": "moe", "cfg": vars(cfg), "rows": rows, "seed": seed, "norm": norm,
            "sha256": digests(w)}
    return meta, {"out": out.numpy(), "ids": ids.numpy().astype(np.int32), "weights": wts.numpy(),
                  "logits": logits.numpy()}


def case_indexer(seed):
    from oracle import reference as R
    from refs import indexer_oracle_scores

    ns = synth.make_indexer(INDEXER, len(INDEXER_CTX), seed, "cpu", ctx_len=INDEXER_CTX)
    scores = np.zeros((ns.rows, INDEXER.context), dtype=np.float32)
    topk = np.full((ns.rows, INDEXER.topk), -1, dtype=np.int32)
    for r in range(ns.rows):
        s = indexer_oracle_scores(ns, r).float()
        scores[r, : s.numel()] = s.numpy()
        lst = R.radix_lists(s, INDEXER.topk).numpy()
        topk[r, : lst.size] = lst
    meta = {"kind": "indexer", "cfg": vars(INDEXER), "ctx_len": INDEXER_CTX, "seed": seed,
            "sha256": digests(ns)}
    return meta, {"scores": scores, "topk": topk}


def case_mla(rows, seed):
    from refs import mla_oracle

    ns = synth.make_mla(MLA, rows, seed, "cpu", residual=True)
    ns.sel[0, -40:] = -1  # unused slots
    olat, out = mla_oracle(ns)
    meta = {"kind": "mla", "cfg": vars(MLA), "rows": rows, "seed": seed, "sha256": digests(ns),
            "unused_tail": 40}
    return meta, {"o_latent": olat.numpy(), "out": out.numpy()}


CASES = {
    "moe_fp8_small": lambda: case_moe("moe_fp8_small", MOE_FP8, 4, 7001, False),
    "moe_mxfp4_small": lambda: case_moe("moe_mxfp4_small", MOE_MXFP4, 5, 7002, True),
    "indexer_small": lambda: case_indexer(7003),
    "mla_small": lambda: case_mla(3, 7004),
}


def write(name: str) -> str:
    meta, arrays = CASES[name]()
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, meta=np.array(json.dumps(meta)), **arrays)
    return path


if __name__ == "__main__":
    torch.set_num_threads(max(1, (os.cpu_count() or 2) // 2))
    for n in sys.argv[1:] or CASES:
        print("wrote", write(n))
