"""The oracle against the committed golden vectors (CPU).

Each fixture regenerates its inputs from (config, seed), checks their SHA-256
digests, recomputes the oracle and compares: indices and expert ids exactly,
floats to 1e-6 relative (the same code on the same inputs, up to BLAS order)."""

import json
import os

import numpy as np
import pytest
import torch

import golden_cases as G

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    z = np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False)
    return json.loads(str(z["meta"])), {k: z[k] for k in z.files if k != "meta"}


@pytest.mark.parametrize("name", ["moe_fp8_small", "moe_mxfp4_small", "indexer_small", "mla_small"])
def test_golden_inputs_regenerate_bit_exactly(name):
    meta, _ = _load(name)
    ns = G.regenerate(meta, "cpu")
    assert G.digests(ns) == meta["sha256"]


@pytest.mark.parametrize("name", ["moe_fp8_small", "moe_mxfp4_small"])
def test_golden_moe(name):
    from refs import MoEOracle

    meta, exp = _load(name)
    w = G.regenerate(meta, "cpu")
    out, ids, wts, logits = MoEOracle(w)(w.x, norm=meta["norm"], residual=meta["norm"], eps=1e-6)
    assert np.array_equal(ids.numpy(), exp["ids"])
    np.testing.assert_allclose(wts.numpy(), exp["weights"], rtol=1e-6)
    np.testing.assert_allclose(logits.numpy(), exp["logits"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out.numpy(), exp["out"], rtol=1e-2, atol=1e-3)


def test_golden_indexer():
    from oracle import reference as R
    from refs import indexer_oracle_scores

    meta, exp = _load("indexer_small")
    ns = G.regenerate(meta, "cpu")
    for r, n in enumerate(meta["ctx_len"]):
        s = indexer_oracle_scores(ns, r).float()
        np.testing.assert_allclose(s.numpy(), exp["scores"][r, :n], rtol=1e-6, atol=1e-6)
        lst = R.radix_lists(torch.from_numpy(exp["scores"][r, :n]), meta["cfg"]["topk"])
        assert np.array_equal(lst.numpy(), exp["topk"][r, : lst.numel()])


def test_golden_mla():
    from refs import mla_oracle

    meta, exp = _load("mla_small")
    ns = G.regenerate(meta, "cpu")
    olat, out = mla_oracle(ns)
    np.testing.assert_allclose(olat.numpy(), exp["o_latent"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out.numpy(), exp["out"], rtol=1e-2, atol=1e-2)
