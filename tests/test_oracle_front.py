"""Pins the oracle's layer front (the reference's K1) on the CPU: each piece against
mathematics or a library routine, and the composed front on a case worked by hand,
with planted mistakes that must fail."""

import math
from types import SimpleNamespace

import pytest
import scipy.linalg
import torch

from oracle import reference as R


def test_rope_pairs_rotates_each_pair():
    x = torch.tensor([[1.0, 0.0, 0.0, 2.0]])
    th = torch.tensor([[0.3, 1.1]])
    y = R.rope_pairs(x, th.cos(), th.sin())
    assert torch.allclose(y, torch.tensor([[math.cos(0.3), math.sin(0.3), -2 * math.sin(1.1), 2 * math.cos(1.1)]]))
    # the inverse rotation returns the input; norms are kept
    z = R.rope_pairs(y, th.cos(), -th.sin())
    assert torch.allclose(z, x, atol=1e-6)


def test_hadamard_is_sylvester_and_orthonormal():
    h = R.hadamard(128)
    assert torch.equal(h, torch.from_numpy(scipy.linalg.hadamard(128)).double())
    x = torch.randn(3, 128, generator=torch.Generator().manual_seed(1))
    assert torch.allclose(R.fwht128(R.fwht128(x)), x, atol=1e-5)
    e0 = torch.zeros(128)
    e0[0] = 1
    assert torch.allclose(R.fwht128(e0), torch.full((128,), 128 ** -0.5))


def test_layernorm_is_torchs():
    g = torch.Generator().manual_seed(2)
    x, w, b = torch.randn(4, 128, generator=g), torch.randn(128, generator=g), torch.randn(128, generator=g)
    ref = torch.nn.functional.layer_norm(x, (128,), w, b, eps=1e-6)
    assert torch.allclose(R.layernorm(x, w, b, 1e-6), ref, atol=1e-5)


def _hand_front():
    """hidden 4, q_lora 2, kv_lora 2, rope 2, nope 2, one head; position 1 rotates by 90
    degrees (cos 0, sin 1); eps 0.  x = (2, -2, 2, -2) normalizes to (1, -1, 1, -1);
    q_a = (x0, x1) = (1, -1) -> q_an (1, -1); kv_a = 2 (x2, x3) = (2, -2) -> (1, -1);
    k_pe = (x0, x2) = (1, 1) -> rotated (-1, 1); q_b = (q0, q1, q0, 0): q_nope (1, -1),
    q_pe (1, 0) -> (0, 1); W_UK rows c: (1, 0), (1, 1): q_lat = (1, 0)."""
    w = SimpleNamespace(
        g_in=torch.ones(4), g_q_a=torch.ones(2), g_kv_a=torch.ones(2),
        w_qkv_a=torch.tensor([[1.0, 0, 0, 0], [0, 1, 0, 0], [0, 0, 2, 0], [0, 0, 0, 2], [1, 0, 0, 0],
                              [0, 0, 1, 0]]),
        w_q_b=torch.tensor([[1.0, 0], [0, 1], [1, 0], [0, 0]]),
        w_uk=torch.tensor([[[1.0, 0], [1, 1]]]),
    )
    cs = torch.tensor([[1.0, 0.0], [0.0, 1.0]])  # positions 0, 1: cos | sin
    x = torch.tensor([[2.0, -2, 2, -2]])
    return x, w, cs


def _run(x, w, cs):
    return R.front(x, w, torch.tensor([1]), cs, eps=0.0, index_eps=0.0, nope=2, heads=1, index_heads=0,
                   kv_lora=2, rope=2)


def test_front_worked_by_hand():
    out = _run(*_hand_front())
    assert torch.equal(out["mla_q"], torch.tensor([[[1.0, 0, 0, 1]]]))
    assert torch.equal(out["kv_row"], torch.tensor([[1.0, -1, -1, 1]]))
    assert torch.equal(out["q_an"], torch.tensor([[1.0, -1]]))


@pytest.mark.parametrize("plant", ["w_uk_transposed", "q_b_rows_swapped", "no_q_norm"])
def test_front_pin_catches_planted_mistakes(plant):
    x, w, cs = _hand_front()
    if plant == "w_uk_transposed":
        w.w_uk = w.w_uk.transpose(1, 2).contiguous()
    elif plant == "q_b_rows_swapped":
        w.w_q_b = w.w_q_b.flip(0)
    else:
        w.g_q_a = torch.full((2,), 2.0)  # a norm scale the hand case does not have
    assert not torch.equal(_run(x, w, cs)["mla_q"], torch.tensor([[[1.0, 0, 0, 1]]]))


def test_front_index_key_order_of_steps():
    """The index key is LayerNorm, then RoPE on the first 64 dims only, then the
    Hadamard transform: with a +-1 key (mean 0, variance 1: LayerNorm is the identity at
    eps 0) and a 90-degree rotation, the key is fwht of the rotated vector; rotating all
    128 dims, or not rotating, gives another."""
    k = torch.tensor([1.0, -1.0] * 64)
    w = SimpleNamespace(
        g_in=torch.ones(128), g_q_a=torch.ones(128), g_kv_a=torch.ones(512),
        w_qkv_a=torch.zeros(128 + 512 + 64, 128), w_q_b=torch.zeros(1 * (128 + 64), 128),
        w_uk=torch.zeros(1, 512, 128), w_iq=torch.zeros(16 * 128, 128), w_ik=torch.diag(k),
        g_ik=torch.ones(128), b_ik=torch.zeros(128), w_iw=torch.zeros(16, 128),
    )
    cs = torch.zeros(2, 64)
    cs[1, 32:] = 1.0  # position 1: cos 0, sin 1 on all 32 pairs
    x = torch.ones(1, 128)  # normalizes to ones; ik = diag(k) . 1 = k
    out = R.front(x, w, torch.tensor([1]), cs, eps=0.0, index_eps=0.0, nope=128, heads=1, index_heads=16)
    rot = k.clone()
    rot[0:64:2], rot[1:64:2] = -k[1:64:2], k[0:64:2]
    assert torch.allclose(out["index_key"][0], R.fwht128(rot), atol=1e-6)
    all_rot = torch.stack([-k[1::2], k[0::2]], dim=1).reshape(-1)
    assert not torch.allclose(out["index_key"][0], R.fwht128(all_rot), atol=1e-3)
    assert not torch.allclose(out["index_key"][0], R.fwht128(k), atol=1e-3)
