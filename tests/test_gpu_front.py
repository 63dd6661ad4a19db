"""The layer's front (the reference's K1) on the GPU against the oracle.

Bounds: the absorbed MLA queries, the index queries and head weights within rel-L2
1e-2 of the oracle's (bf16 outputs after FP8 weights, as the layer's own bound); the
cache rows it writes equal the oracle's quantization of the oracle's pre-quant values
on >= 99 % of the bytes (the rest: values on a rounding boundary that two f32
evaluation orders put either side), with the same scales, dequantized within rel-L2
1e-2; pad rows (slot -1) and every other slot untouched.
"""

from dataclasses import replace
from types import SimpleNamespace

import pytest
import torch

from oracle import codecs as oc
from oracle import reference as R
from refs import cpu

pytestmark = pytest.mark.gpu

REL_L2 = 1e-2


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _dequant(w, s, fmt):
    from sgl_amd_mono.k2 import config as C

    w = cpu(w)
    return oc.fp8_block_dequant(w, cpu(s)) if fmt == C.WFMT_FP8_BLOCK else w.float()


def _oracle(cfg, ns):
    fmt = cfg.weight_fmt
    w = SimpleNamespace(
        g_in=cpu(ns.g_in), g_q_a=cpu(ns.g_q_a), g_kv_a=cpu(ns.g_kv_a),
        w_qkv_a=_dequant(ns.w_qkv_a, ns.s_qkv_a, fmt), w_q_b=_dequant(ns.w_q_b, ns.s_q_b, fmt),
        w_uk=cpu(ns.w_uk).float(),
    )
    if cfg.index_heads:
        w.w_iq, w.w_ik = _dequant(ns.w_iq, ns.s_iq, fmt), _dequant(ns.w_ik, ns.s_ik, fmt)
        w.g_ik, w.b_ik, w.w_iw = cpu(ns.g_ik), cpu(ns.b_ik), cpu(ns.w_iw).float()
    pos = cpu(ns.positions).clamp(max=cfg.max_position)
    return R.front(cpu(ns.x).float(), w, pos, cpu(ns.rope_cos_sin), eps=cfg.eps, index_eps=cfg.index_eps,
                   nope=cfg.nope, heads=cfg.heads, index_heads=cfg.index_heads)


def _run(cfg, rows, seed, pad_rows=()):
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import FrontOp

    dev = _dev()
    ns = synth.make_front(cfg, rows, seed, dev)
    for r in pad_rows:
        ns.slots[r] = -1
    op = FrontOp(cfg, ns, rows, device=dev)
    mla_q, index_q, index_w = op(ns.x, ns.positions, ns.slots, ns.rope_cos_sin, ns.kv_cache, ns.kv_scale,
                                 ns.index_cache, ns.index_scale)
    torch.cuda.synchronize()
    return ns, cpu(mla_q).float(), None if index_q is None else cpu(index_q).float(), \
        None if index_w is None else cpu(index_w).float()


def _byte_agreement(a, b):
    return float((a == b).double().mean())


def _check(cfg, ns, mla_q, index_q, index_w, pad_rows=()):
    from sgl_amd_mono.k2 import config as C

    ref = _oracle(cfg, ns)
    stats = {"mla_q": R.rel_l2(mla_q, ref["mla_q"])}
    assert stats["mla_q"] <= REL_L2, stats
    if cfg.index_heads:
        stats["index_q"] = R.rel_l2(index_q, ref["index_q"])
        stats["index_w"] = R.rel_l2(index_w, ref["index_w"])
        assert stats["index_q"] <= REL_L2 and stats["index_w"] <= REL_L2, stats
    slots = cpu(ns.slots)
    live = [r for r in range(ns.rows) if r not in pad_rows]
    kv = cpu(ns.kv_cache)
    # the latent rows: the oracle's E4M3 of the oracle's values (over their scale)
    for r in live:
        row = ref["kv_row"][r]
        if cfg.kv_scaled:
            sc = float(row.abs().max()) / 448.0
            got_sc = float(cpu(ns.kv_scale)[slots[r]])
            assert abs(got_sc - sc) <= 1e-6 * sc, (r, got_sc, sc)
            want = oc.e4m3_encode(row / torch.tensor(sc, dtype=torch.float32))
            deq = oc.e4m3_decode(kv[slots[r]]) * got_sc
        else:
            want = oc.e4m3_encode(row)
            deq = oc.e4m3_decode(kv[slots[r]])
        assert _byte_agreement(kv[slots[r]], want) >= 0.99, r
        assert R.rel_l2(deq, row) <= 0.05, r  # E4M3 keeps 3 mantissa bits
    # nothing else written
    written = torch.zeros(kv.shape[0], dtype=torch.bool)
    written[slots[live]] = True
    assert int(kv[~written].abs().sum()) == 0
    # the index keys
    if cfg.index_heads:
        key = ref["index_key"]
        ic = cpu(ns.index_cache)
        for r in live:
            page, t = int(slots[r]) // 64, int(slots[r]) % 64
            if cfg.keys == C.KEYS_FP8:
                codes, scale = oc.index_key_quant(key[r])
                got = oc.index_page_decode(ic[page : page + 1])[0, t]
                assert float(got.abs().max()) > 0
                pg = ic[page].reshape(-1)
                got_scale = pg[8192 + 4 * t : 8192 + 4 * t + 4].view(torch.float32)
                assert float(got_scale) == float(scale), r
                want = oc.e4m3_decode(codes) * scale
                assert float((got == want).double().mean()) >= 0.99, r
            else:
                codes, scales = oc.mxfp4_quant(key[r][None])
                plane = ic[page].view(4, 64, 16)[:, t]  # [4 chunks][16 B]
                sp = cpu(ns.index_scale)[page].view(4, 64)
                got_sc = torch.stack([sp[c, (t % 16) * 4 + t // 16] for c in range(4)])
                assert _byte_agreement(got_sc, scales[0]) == 1.0, r
                assert _byte_agreement(plane.reshape(-1), codes[0]) >= 0.97, r
            want_key = key[r]
            assert float(want_key.abs().max()) > 0
        # pad rows and untouched pages: nothing written there
        pages = {int(slots[r]) // 64 for r in live}
        for p in range(ic.shape[0]):
            if p not in pages:
                assert int(ic[p].abs().sum()) == 0
    return stats


@pytest.mark.parametrize("rows", [1, 8, 32])
def test_front_config7(rows):
    """FP8 block weights, the FP4 index plane, scaled latent rows (the layer's defaults)."""
    from sgl_amd_mono.k2 import config as C

    cfg = C.C7_FRONT
    ns, *out = _run(cfg, rows, seed=700 + rows)
    print(_check(cfg, ns, *out))


def test_front_bf16_weights_fp8_index_unscaled_cache():
    """bf16 weights, SGLang's FP8 index pages and its unscaled latent cache, nope 128."""
    from sgl_amd_mono.k2 import config as C

    cfg = replace(C.C7_FRONT, weight_fmt=C.WFMT_BF16, keys=C.KEYS_FP8, kv_scaled=False, nope=128)
    ns, *out = _run(cfg, 8, seed=711)
    print(_check(cfg, ns, *out))


def test_front_pad_rows_and_no_indexer():
    """Pad rows write no cache rows; a front without the indexer (a layer reusing the
    previous selection); other sizes (hidden 7168, q_lora 1024, 32 index heads)."""
    from sgl_amd_mono.k2 import config as C

    cfg = replace(C.C7_FRONT, hidden=7168, q_lora=1024, index_heads=32, keys=C.KEYS_FP8)
    ns, *out = _run(cfg, 5, seed=712, pad_rows=(1, 3))
    print(_check(cfg, ns, *out, pad_rows=(1, 3)))
    cfg0 = replace(C.C7_FRONT, index_heads=0)
    ns0, *out0 = _run(cfg0, 4, seed=713)
    assert out0[1] is None and out0[2] is None
    print(_check(cfg0, ns0, *out0))


@pytest.mark.parametrize("rows", [8, 32])
def test_front_aiter_layout_bits(rows):
    """Block-FP8 weights SGLang preshuffled into AITER's (16, 16) layout
    (WFMT_FP8_AITER16), read in place: the same codes as the row-major weights give
    the same bits -- queries, head weights and both caches."""
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import FrontOp

    dev = _dev()
    cfg = C.C7_FRONT
    ns = synth.make_front(cfg, rows, 720 + rows, dev)
    sh = synth.front_in_layout(ns, C.WFMT_FP8_AITER16)
    res = []
    for n in (ns, sh):
        kv, ic = ns.kv_cache.clone(), ns.index_cache.clone()
        ks = None if ns.kv_scale is None else ns.kv_scale.clone()
        isc = None if ns.index_scale is None else ns.index_scale.clone()
        out = FrontOp(n.cfg, n, rows, device=dev)(ns.x, ns.positions, ns.slots, ns.rope_cos_sin, kv, ks, ic, isc)
        torch.cuda.synchronize()
        res.append([cpu(t) for t in (*out, kv, ic, ks, isc) if t is not None])
    assert len(res[0]) == len(res[1]) >= 5
    for a, b in zip(*res):
        assert torch.equal(a, b)


def _front_outputs(cfg, ns, rows, staged, repeats=1):
    """The front's outputs and both caches (fresh copies of ns's) from `repeats`
    launches of one op (the persistent launch resets its own counters)."""
    from sgl_amd_mono.k2.ops import FrontOp

    dev = _dev()
    op = FrontOp(cfg, ns, rows, device=dev, staged=staged)
    res = []
    for _ in range(repeats):
        kv, ic = ns.kv_cache.clone(), ns.index_cache.clone()
        ks = None if ns.kv_scale is None else ns.kv_scale.clone()
        isc = None if ns.index_scale is None else ns.index_scale.clone()
        out = op(ns.x, ns.positions, ns.slots, ns.rope_cos_sin, kv, ks, ic, isc)
        torch.cuda.synchronize()
        res.append([cpu(t) for t in (*out, kv, ic, ks, isc) if t is not None])
    return op, res


@pytest.mark.parametrize("case", ["c7-1", "c7-8", "c7-32", "bf16-nope128", "aiter", "h7168-no-indexer"])
def test_front_persistent_matches_staged(case):
    """The persistent front (one launch, counters between its stages) gives the six
    stage launches' bits -- outputs, latent and index cache rows and scales -- on
    back-to-back launches (its counters reset by the launch itself), at 1, 8 and 32
    rows (two GEMV passes), bf16 weights, AITER's layout, hidden 7168 without the
    indexer; its status word stays 0."""
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth

    dev = _dev()
    rows = {"c7-1": 1, "c7-32": 32}.get(case, 8)
    cfg = {
        "bf16-nope128": replace(C.C7_FRONT, weight_fmt=C.WFMT_BF16, nope=128),
        "h7168-no-indexer": replace(C.C7_FRONT, hidden=7168, q_lora=1024, index_heads=0, keys=C.KEYS_FP8),
    }.get(case, C.C7_FRONT)
    ns = synth.make_front(cfg, rows, 730 + rows, dev)
    if case == "aiter":
        ns = synth.front_in_layout(ns, C.WFMT_FP8_AITER16)
        cfg = ns.cfg
    p_op, p = _front_outputs(cfg, ns, rows, staged=False, repeats=3)
    assert p_op.persistent, case
    _, s = _front_outputs(cfg, ns, rows, staged=True)
    assert p_op.status() == 0
    for launch in p:
        assert len(launch) == len(s[0])
        for a, b in zip(launch, s[0]):
            assert torch.equal(a, b)


def test_front_persistent_new_inputs_each_launch():
    """One persistent front op over alternating steps (residual rows, positions, slots,
    the cache contents): each launch gives the stage launches' bits on its own inputs,
    so nothing a previous launch left in the workspace is read back."""
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import FrontOp

    dev = _dev()
    cfg, rows = C.C7_FRONT, 8
    A = synth.make_front(cfg, rows, 741, dev)
    B = synth.make_front(cfg, rows, 742, dev)
    p_op = FrontOp(cfg, A, rows, device=dev)  # the weights are A's; B gives the step inputs
    s_op = FrontOp(cfg, A, rows, device=dev, staged=True)
    assert p_op.persistent
    outs = []
    for src in (A, B, A, B):
        res = []
        for op in (p_op, s_op):
            kv, ic = src.kv_cache.clone(), src.index_cache.clone()
            ks = None if src.kv_scale is None else src.kv_scale.clone()
            isc = None if src.index_scale is None else src.index_scale.clone()
            out = op(src.x, src.positions, src.slots, src.rope_cos_sin, kv, ks, ic, isc)
            torch.cuda.synchronize()
            res.append([cpu(t) for t in (*out, kv, ic, ks, isc) if t is not None])
        for a, b in zip(*res):
            assert torch.equal(a, b)
        outs.append(res[0][0])
    assert p_op.status() == 0
    assert not torch.equal(outs[0], outs[1])
    assert torch.equal(outs[0], outs[2]) and torch.equal(outs[1], outs[3])
