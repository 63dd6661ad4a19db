"""The allocation-free layer entry point, mk2_layer_launch_static (its scratch is the
library's own device array), against the workspace entry point mk2_layer_launch on the
same inputs: identical bits for the layer output, the attention output, the top-k
lists and the expert ids.  Two calls in a row, the second with a smaller input (fewer
rows, shorter context: a different scratch layout over the same array, which the call
must clear itself), then a HIP graph of the static launch replayed with eager work in
between, every replay checked against the eager result.  On the CPU: a shape whose
scratch exceeds the array is refused with MK2_ENOSPACE before anything is enqueued."""

from dataclasses import replace

import pytest
import torch



def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _outputs(cfg, rows, dev):
    H, K = cfg.mla.hidden, cfg.moe.top_k
    return (torch.empty(rows, H, dtype=torch.bfloat16, device=dev),
            torch.empty(rows, H, dtype=torch.bfloat16, device=dev),
            torch.empty(rows, cfg.indexer.topk, dtype=torch.int32, device=dev),
            torch.empty(rows, K, dtype=torch.int32, device=dev))


def _launch(op, outs):
    out, attn, topk, ids = outs
    op(out, attn_out=attn, topk=topk, topk_ids=ids)


def _small(C):
    return replace(C.C5_LAYER, mla=replace(C.C5_LAYER.mla, context=8192),
                   indexer=replace(C.C5_LAYER.indexer, context=8192))


@pytest.mark.gpu
@pytest.mark.parametrize("staged", [False, True])
def test_static_scratch_matches_workspace_entry(staged):
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import LayerOp

    dev = _dev()
    for cfg, rows, seed in ((C.C5_LAYER, 8, 901), (_small(C), 4, 902)):
        print(f"static scratch: rows {rows} context {cfg.indexer.context} staged {staged}", flush=True)
        L = synth.make_layer(cfg, rows, seed, dev)
        ws_op = LayerOp(cfg, L, rows, device=dev, staged=staged)
        st_op = LayerOp(cfg, L, rows, device=dev, staged=staged, static_scratch=True)
        assert st_op.workspace is None
        ref, got = _outputs(cfg, rows, dev), _outputs(cfg, rows, dev)
        _launch(ws_op, ref)
        _launch(st_op, got)
        torch.cuda.synchronize()
        ws_op.check()
        st_op.check()
        for a, b in zip(got, ref):
            assert torch.equal(a, b)


@pytest.mark.gpu
def test_static_scratch_graph_replays():
    from sgl_amd_mono.k2 import config as C
    from sgl_amd_mono.k2 import synth
    from sgl_amd_mono.k2.ops import LayerOp

    dev = _dev()
    cfg, rows = C.C5_LAYER, 8
    L = synth.make_layer(cfg, rows, 903, dev)
    st_op = LayerOp(cfg, L, rows, device=dev, static_scratch=True)
    ref, got = _outputs(cfg, rows, dev), _outputs(cfg, rows, dev)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        _launch(st_op, ref)  # eager, on the capture stream (also takes the array's address)
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            _launch(st_op, got)
    torch.cuda.synchronize()
    other = synth.make_layer(_small(C), 4, 904, dev)
    other_op = LayerOp(_small(C), other, 4, device=dev, static_scratch=True)
    other_outs = _outputs(_small(C), 4, dev)
    for i in range(3):
        with torch.cuda.stream(stream):  # the clear and the replay ordered on one stream
            for t in got:
                t.zero_()
            g.replay()
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(a, b), f"replay {i}"
        _launch(other_op, other_outs)  # eager work of another shape on the same array
        torch.cuda.synchronize()
    st_op.check()
    other_op.check()


def test_static_scratch_refuses_an_oversized_shape():
    """32 rows with top-k 4096 of 65536 keys and an expert inter of 1024 need more
    scratch than the 64 MiB array (about 68 MiB: the split partials are 32 x 64 splits
    x 16 x 512 x 2 B = 32 MiB, the rows' scores and bin candidates 24 MiB, the
    experts' mid rows the rest): MK2_ENOSPACE, with the sizes in the message, and no
    GPU call (this runs without a GPU)."""
    import ctypes

    from sgl_amd_mono import _lib
    from sgl_amd_mono.k2 import config as C

    if not _lib.LIB_PATH.exists():
        pytest.skip("libmk2.so not built")
    L = _lib.lib()
    cfg = C.C5_LAYER
    ic, mc, ec = cfg.indexer, cfg.mla, cfg.moe
    rows, topk = 32, 4096
    ia = _lib.IndexerArgs(_lib.IndexerShape(rows, ic.heads, ic.dim, topk, ic.context, ic.context // 64),
                          *([1] * 7), None, None, None, 0)
    ma = _lib.MlaArgs(_lib.MlaShape(rows, 16, 512, 64, 128, mc.hidden, topk, mc.context // 64, mc.sm_scale),
                      *([1] * 5), None, 1, 1, 1, None, None, 0, None)
    ea = _lib.MoeArgs(_lib.MoeShape(rows, ec.hidden, ec.n_experts, ec.top_k, 1024, ec.router, ec.expert_fmt,
                                    ec.n_shared, ec.shared_inter, 1, 1, ec.route_scale, 1e-6),
                      _lib.MoeWeights(*([1] * 11)), None, None, None, 0, None, None, None)
    la = _lib.LayerArgs(ia, ma, ea, None, 2, None, 0, 0, 0, None, None)
    need = ctypes.c_size_t()
    assert L.mk2_layer_workspace_bytes(ctypes.byref(la), ctypes.byref(need)) == _lib.MK2_OK
    assert need.value > 64 << 20
    assert L.mk2_layer_launch_static(ctypes.byref(la), None) == _lib.MK2_ENOSPACE
    msg = L.mk2_last_error().decode()
    assert "static" in msg and str(need.value) in msg
