"""Pins the oracle's layer arithmetic (CPU only) against independent statements of
the same mathematics: explicit loops, torch library routines, brute force on tiny
inputs, invariants -- and negative controls that plant a slip in a copy of the
oracle and see the check fail (after test/kernels/glm53/check_topk.py:150-165)."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import codecs as oc
from oracle import reference as R


def test_index_scores_explicit_loops():
    g = torch.Generator().manual_seed(0)
    q, w, keys = torch.randn(4, 8, generator=g), torch.randn(4, generator=g), torch.randn(5, 8, generator=g)
    got = R.index_scores(q, w, keys)
    for c in range(5):
        want = sum(
            max(0.0, sum(float(q[h, d]) * float(keys[c, d]) for d in range(8))) * float(w[h])
            for h in range(4)
        )
        assert abs(float(got[c]) - want) < 1e-9


def test_index_scores_never_negative_zero():
    q = torch.zeros(2, 4)
    w = torch.tensor([-1.0, -2.0])
    s = R.index_scores(q, w, torch.ones(3, 4)).float()
    assert bool((oc.radix_keys(s) == (1 << 31)).all())


def _brute_topk_set(x, k):
    order = sorted(range(len(x)), key=lambda i: (-float(x[i]), i))
    return sorted(order[:k])


@pytest.mark.parametrize("seed", range(5))
def test_radix_lists_set_is_exact_topk(seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(300, generator=g)
    x[::7] = x[3]  # ties
    k = 37
    lst = R.radix_lists(x, k)
    assert sorted(lst.tolist()) == _brute_topk_set(x, k)
    assert lst.numel() == k and len(set(lst.tolist())) == k
    # the set equals torch.topk's values (torch leaves tie order open)
    assert torch.equal(torch.sort(x[lst]).values, torch.sort(torch.topk(x, k).values).values)
    assert torch.equal(R.exact_topk_set(x, k), torch.tensor(_brute_topk_set(x, k)))


def test_radix_lists_order():
    # keys in three 12-bit-prefix groups: above, same prefix above kth, ties
    x = torch.tensor([1.0, 100.0, 1.0001, 1.0, 50.0, 1.0, 0.5])
    lst = R.radix_lists(x, 5).tolist()
    # above the k-th's 12-bit prefix: 100 (pos 1), 50 (pos 4) in position order; then
    # same prefix as 1.0 and above it: 1.0001 (pos 2); then ties at 1.0: pos 0, 3
    assert lst == [1, 4, 2, 0, 3]


def test_radix_lists_short_rows_keep_all():
    assert R.radix_lists(torch.randn(10), 16).tolist() == list(range(10))


def test_sparse_mla_brute_force():
    g = torch.Generator().manual_seed(1)
    q = torch.randn(3, 6, generator=g)
    kv = torch.randn(5, 6, generator=g)
    got = R.sparse_mla(q, kv, 0.3, 4)
    for h in range(3):
        s = [0.3 * float(q[h] @ kv[j]) for j in range(5)]
        m = max(s)
        e = [math.exp(v - m) for v in s]
        z = sum(e)
        want = [sum(e[j] / z * float(kv[j, c]) for j in range(5)) for c in range(4)]
        assert torch.allclose(got[h], torch.tensor(want), atol=1e-6)


def test_sparse_mla_key_order_invariant_and_split_merge():
    g = torch.Generator().manual_seed(2)
    q, kv = torch.randn(16, 576, generator=g), torch.randn(256, 576, generator=g)
    a = R.sparse_mla(q, kv, 576**-0.5, 512)
    perm = torch.randperm(256, generator=g)
    assert torch.allclose(a, R.sparse_mla(q, kv[perm], 576**-0.5, 512), atol=1e-6)
    # the split-softmax merge the kernel does equals one softmax
    s = (q.double() @ kv.double().T) * 576**-0.5
    parts = []
    for c in range(4):
        sc = s[:, 64 * c : 64 * c + 64]
        m = sc.amax(-1, keepdim=True)
        p = torch.exp(sc - m)
        parts.append((m, p.sum(-1, keepdim=True), p @ kv[64 * c : 64 * c + 64, :512].double()))
    M = torch.stack([m for m, _, _ in parts]).amax(0)
    L = sum(l * torch.exp(m - M) for m, l, _ in parts)
    O = sum(o * torch.exp(m - M) for m, _, o in parts) / L
    assert torch.allclose(a.double(), O, atol=1e-6)


def test_rmsnorm_matches_torch():
    g = torch.Generator().manual_seed(3)
    a, gamma = torch.randn(4, 512, generator=g), torch.randn(512, generator=g)
    want = F.rms_norm(a, (512,), gamma, eps=1e-6)
    assert torch.allclose(R.rmsnorm(a, gamma, 1e-6), oc.bf16_round(want), atol=1e-2, rtol=1e-2)


def test_route_softmax_matches_softmax_topk_renormalize():
    g = torch.Generator().manual_seed(4)
    lg = torch.randn(6, 64, generator=g)
    ids, w = R.route_softmax(lg, 8)
    p = torch.softmax(lg.double(), -1)
    top = torch.topk(p, 8)
    assert torch.equal(torch.sort(ids, -1).values, torch.sort(top.indices, -1).values)
    assert torch.allclose(w.double(), top.values / top.values.sum(-1, keepdim=True), atol=1e-6)


def test_route_ties_take_lower_ids():
    lg = torch.zeros(1, 64)
    ids, w = R.route_softmax(lg, 8)
    assert ids[0].tolist() == list(range(8))
    s_ids, _ = R.route_sigmoid_bias(torch.zeros(1, 64), torch.zeros(64), 8, 2.5)
    assert s_ids[0].tolist() == list(range(8))


def test_route_sigmoid_bias_selects_by_biased_key_weights_by_sigmoid():
    lg = torch.tensor([[0.0, 1.0, 2.0, -1.0]])
    bias = torch.tensor([10.0, 0.0, 0.0, 20.0])
    ids, w = R.route_sigmoid_bias(lg, bias, 2, 2.5)
    assert ids[0].tolist() == [3, 0]  # bias decides the picks
    s = torch.sigmoid(torch.tensor([-1.0, 0.0]))
    assert torch.allclose(w[0], s / s.sum() * 2.5)  # weights use the unbiased sigmoid


def test_swiglu_matches_silu():
    g = torch.Generator().manual_seed(5)
    a, b = torch.randn(100, generator=g), torch.randn(100, generator=g)
    assert torch.allclose(R.swiglu(a, b), F.silu(a) * b, atol=1e-6)


def test_moe_block_single_expert_and_linearity():
    """One expert with hand-built weights: gate = up = x, down = identity, so
    y = silu(x) * x exactly (before the bf16 rounding of mid)."""
    H = 8
    x = torch.linspace(-2, 2, H)[None]
    w13 = torch.cat([torch.eye(H), torch.eye(H)])
    w2 = torch.eye(H)
    y = R.expert_fp8(x, w13, w2)
    assert torch.allclose(y, oc.bf16_round(F.silu(x) * x), atol=1e-6)
    out, ids, w, _ = R.moe_block(
        x, lambda v: torch.tensor([[5.0, 0.0, 0.0]]), lambda lg: R.route_softmax(lg, 1),
        lambda e, xr: (e + 1) * xr.float(), None,
    )
    assert ids.tolist() == [[0]] and torch.allclose(out, oc.bf16_round(x))


def test_negative_controls_fail_the_topk_checks():
    """A wrong slot, two entries swapped and a flipped score bit each fail
    (check_topk.py:150-165)."""
    g = torch.Generator().manual_seed(6)
    x = torch.randn(500, generator=g)
    k = 50
    good = R.radix_lists(x, k)
    bad = good.clone()
    bad[0] = int(torch.sort(oc.radix_keys(x), descending=True, stable=True).indices[k])
    assert sorted(bad.tolist()) != _brute_topk_set(x, k)
    swapped = good.clone()
    swapped[[0, 1]] = swapped[[1, 0]]
    assert not torch.equal(swapped, R.radix_lists(x, k))
    flipped = x.clone()
    i = int(good[0])
    flipped[i] = -abs(flipped[i]) - 10  # the top score pushed to the bottom
    assert i not in R.radix_lists(flipped, k).tolist()
