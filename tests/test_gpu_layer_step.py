"""The front and the K2 layer in one persistent launch (mk2_layer_step_launch) against
the front's launch followed by the layer's: the same bits in the layer's output, the
front's outputs (the layer's queries and head weights) and both caches."""

from dataclasses import replace

import pytest
import torch

from refs import cpu

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _step_inputs(L, rows, seed, dev, max_position):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    pages = L.mla.kv.shape[0]
    slots = torch.randperm(pages * 64, generator=g, device=dev)[:rows].to(torch.int64)
    positions = torch.randint(0, max_position + 1, (rows,), generator=g, device=dev).to(torch.int64)
    return positions, slots


def _state(L):
    return [cpu(t) for t in (L.mla.q, L.idx.q, L.idx.w, L.mla.kv, L.mla.kv_scale, L.idx.cache, L.idx.cache_scale)]


@pytest.mark.parametrize("aiter", [False, True])
@pytest.mark.parametrize("rows", [8, 32])
def test_layer_step_matches_front_then_layer(rows, aiter):
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import FrontOp, LayerOp, LayerStepOp

    dev = _dev()
    cfg = C.C5_LAYER
    fc = C.C7_FRONT
    fw = synth.make_front(fc, rows, 950 + rows, dev)
    if aiter:
        fw = synth.front_in_layout(fw, C.WFMT_FP8_AITER16)
        fc = fw.cfg
    res = []
    for fused in (False, True):
        L = synth.make_layer(cfg, rows, 960 + rows, dev)  # the same layer (and caches) for both
        positions, slots = _step_inputs(L, rows, 970 + rows, dev, fc.max_position)
        fop = FrontOp(fc, fw, rows, device=dev)
        lop = LayerOp(cfg, L, rows, device=dev)
        outs = []
        for _ in range(2):  # back to back: both launches' counters reset themselves
            if fused:
                out = LayerStepOp(fop, lop)(positions, slots, fw.rope_cos_sin)
            else:
                fop(L.h, positions, slots, fw.rope_cos_sin, L.mla.kv, L.mla.kv_scale, L.idx.cache,
                    L.idx.cache_scale, L.mla.q, L.idx.q, L.idx.w)
                out = lop()
            torch.cuda.synchronize()
            outs.append(cpu(out))
        assert torch.equal(outs[0], outs[1])
        assert int(lop.status.item()) == 0 and fop.status() == 0
        res.append([outs[0]] + _state(L))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_layer_step_refusals():
    """A front shape the launch does not instance is refused (the two launches serve it)."""
    from sgl_amd_mono import _lib
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import FrontOp, LayerOp, LayerStepOp

    dev = _dev()
    rows = 8
    L = synth.make_layer(C.C5_LAYER, rows, 990, dev)
    fw = synth.make_front(C.C7_FRONT, rows, 991, dev)
    positions, slots = _step_inputs(L, rows, 992, dev, C.C7_FRONT.max_position)
    del fw
    bf = replace(C.C7_FRONT, weight_fmt=C.WFMT_BF16)
    fb = synth.make_front(bf, rows, 993, dev)
    step = LayerStepOp(FrontOp(bf, fb, rows, device=dev), LayerOp(C.C5_LAYER, L, rows, device=dev))
    with pytest.raises(_lib.Mk2Error, match="no instance"):
        step(positions, slots, fb.rope_cos_sin)
