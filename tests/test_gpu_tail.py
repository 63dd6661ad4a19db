"""The tail launch (final RMSNorm + this GPU's LM-head rows) on the GPU against the
oracle, with the reference's own bounds (test/kernels/glm53/check_layer.py:744-773,
glm53/spec.py:200-201):
  * logits within rel-L2 1.7e-3 of the oracle's bf16 tail and 7.5e-3 of an f32 tail;
  * the normed rows equal the oracle's bf16 rows up to one bf16 ulp where the two rstd
    evaluations fall on either side of a rounding point;
  * the top-1 token equals the oracle's on rows whose top-2 gap is clear;
  * a planted mistake in the oracle (the final norm's weight x1.01) fails the bound.
"""

import pytest
import torch

from oracle import reference as R
from refs import cpu

pytestmark = pytest.mark.gpu

LOGITS_REL = 1.7e-3
LOGITS_VS_F32 = 7.5e-3


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _run(cfg, rows, seed):
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import TailOp

    dev = _dev()
    ns = synth.make_tail(cfg, rows, seed, dev)
    op = TailOp(cfg, ns.g_norm, ns.w_head, rows, device=dev)
    logits, normed = op(ns.x)
    torch.cuda.synchronize()
    return ns, cpu(logits), cpu(normed).float()


def _check(cfg, ns, logits, normed):
    x, g, w = cpu(ns.x), cpu(ns.g_norm), cpu(ns.w_head)
    ref, ref_n = R.tail(x, g, w, cfg.eps)
    # normed: equal, or one bf16 ulp apart on a few elements
    d = (normed - ref_n).abs()
    ulp = torch.pow(2.0, torch.floor(torch.log2(ref_n.abs().clamp_min(1e-30))) - 7)
    assert bool((d <= ulp).all()), float((d / ulp).max())
    assert float((d > 0).double().mean()) < 1e-3
    # logits against the oracle's bf16 tail and against an f32 tail
    xf = x.float()
    f32 = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + cfg.eps) * g.float()) @ w.float().t()
    err, err32 = R.rel_l2(logits, ref), R.rel_l2(logits, f32)
    assert err <= LOGITS_REL, err
    assert err32 <= LOGITS_VS_F32, err32
    # top-1 on rows with a clear gap
    top2 = torch.topk(ref, 2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 4 * LOGITS_REL * ref.abs().amax(-1)
    assert torch.equal(logits.argmax(-1)[clear], ref.argmax(-1)[clear])
    # planted: the oracle's final norm weight x1.01 must fail the bound
    bad, _ = R.tail(x, g.float() * 1.01, w, cfg.eps)
    assert R.rel_l2(logits, bad) > LOGITS_REL
    return err, err32


@pytest.mark.parametrize("rows", [1, 4, 8, 16, 32])
def test_tail_config6(rows):
    from sgl_amd_mono.k2 import config as C

    cfg = C.C6_TAIL
    ns, logits, normed = _run(cfg, rows, seed=600 + rows)
    print(_check(cfg, ns, logits, normed))


@pytest.mark.parametrize("hidden, vocab_rows, rows", [(2048, 4096, 3), (7168, 16, 17), (8192, 1040, 8),
                                                      (4096, 1001, 5), (3072, 5, 2), (6144, 151552 // 8, 8),
                                                      (2048, 40000, 4)])
def test_tail_other_shapes(hidden, vocab_rows, rows):
    """Other hidden sizes (their own k-step counts); vocab rows fewer than the CUs (one a
    workgroup), not a multiple of 16 (partial tiles), another vocabulary's shard and more
    than 128 a workgroup (several chunks of tiles); a second 16-row pass of one row."""
    from sgl_amd_mono.k2 import config as C

    cfg = C.TailConfig(hidden=hidden, vocab_rows=vocab_rows)
    ns, logits, normed = _run(cfg, rows, seed=hidden + rows)
    _check(cfg, ns, logits, normed)


def test_tail_repeats_bit_identical():
    from sgl_amd_mono.k2 import config as C, synth
    from sgl_amd_mono.k2.ops import TailOp

    dev = _dev()
    cfg = C.C6_TAIL
    ns = synth.make_tail(cfg, 8, 77, dev)
    op = TailOp(cfg, ns.g_norm, ns.w_head, 8, device=dev)
    a = [t.clone() for t in op(ns.x)]
    for _ in range(3):
        b = op(ns.x)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_tail_logits_round_to_nearest_even():
    """Rows of ones normalize to exactly 1 in bf16 (rstd = 1/sqrt(1 + 1e-5) rounds back
    to 1), so each logit is the exact sum of its LM-head row, rounded once to bf16:
    1 + 2^-8 (a tie: to 1, the even neighbour), 1 + 3 2^-8 (a tie: up to 1 + 2^-6),
    1 + 2^-8 + 2^-12 (past the tie: up to 1 + 2^-7), -(1 + 3 2^-8) (to -(1 + 2^-6)),
    and 3 (exact)."""
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2.ops import TailOp

    dev = _dev()
    cfg = C.TailConfig(hidden=2048, vocab_rows=5)
    x = torch.ones(2, cfg.hidden, dtype=torch.bfloat16, device=dev)
    g = torch.ones(cfg.hidden, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(cfg.vocab_rows, cfg.hidden)
    w[0, 0], w[0, 1] = 1, 2.0**-8
    w[1, 0], w[1, 5], w[1, 1000] = 1, 2.0**-7, 2.0**-8
    w[2, 0], w[2, 7], w[2, 2047] = 1, 2.0**-8, 2.0**-12
    w[3, 3], w[3, 4], w[3, 9] = -1, -(2.0**-7), -(2.0**-8)
    w[4, 10], w[4, 11], w[4, 12] = 1, 1, 1
    w = w.to(torch.bfloat16).to(dev)
    logits, normed = TailOp(cfg, g, w, 2, device=dev)(x)
    torch.cuda.synchronize()
    assert bool((cpu(normed).float() == 1).all())
    want = torch.tensor([1.0, 1 + 2.0**-6, 1 + 2.0**-7, -(1 + 2.0**-6), 3.0])
    assert torch.equal(cpu(logits), want.expand(2, 5)), cpu(logits)
