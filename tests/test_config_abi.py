"""The Python configs and the C side accept the same shapes: for a grid of MoE, MLA and
indexer configurations, ``validate()`` passes exactly when the library's workspace
query (which runs the C argument checks, no GPU needed) returns MK2_OK.  A config the
C side rejects must never get past ``validate()`` to fail at the launch."""

import ctypes
import itertools
from dataclasses import replace

import pytest

from sgl_amd_mono.k2 import config as C


def _lib():
    from sgl_amd_mono import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libmk2.so not built (run __graft_entry__.build())")
    return _lib, _lib.lib()


def _py_ok(cfg, rows):
    try:
        cfg.validate(rows)
        return True
    except ValueError:
        return False


def _moe_c_ok(_l, L, cfg, rows):
    s = _l.MoeShape(rows, cfg.hidden, cfg.n_experts, cfg.top_k, cfg.inter, cfg.router, cfg.expert_fmt,
                    cfg.n_shared, cfg.shared_inter, 1, 1, cfg.route_scale, 1e-6, cfg.weight_layout)
    n = ctypes.c_size_t()
    return L.mk2_moe_workspace_bytes(ctypes.byref(s), ctypes.byref(n)) == 0


def test_moe_validate_matches_c():
    _l, L = _lib()
    seen = {True: 0, False: 0}
    for hidden, E, k, inter, fmt, ns, si, rows, wl in itertools.product(
        (256, 512, 2048, 6144, 7168 + 256), (16, 48, 64, 96, 192, 256, 320), (0, 1, 8, 9),
        (32, 96, 128, 256, 768, 1024, 2048, 4096, 8192), (C.FMT_FP8, C.FMT_MXFP4), (0, 1),
        (32, 128, 768, 4224), (1, 8, 32, 33), (C.WLAYOUT_TILES, C.WLAYOUT_AITER16, 2),
    ):
        cfg = replace(C.C2_MOE, hidden=hidden, n_experts=E, top_k=k, inter=inter, expert_fmt=fmt,
                      n_shared=ns, shared_inter=si, weight_layout=wl)
        py, c = _py_ok(cfg, rows), _moe_c_ok(_l, L, cfg, rows)
        assert py == c, (cfg, rows, py, c, L.mk2_last_error())
        seen[py] += 1
    assert seen[True] > 100 and seen[False] > 100


def test_mla_validate_matches_c():
    _l, L = _lib()
    seen = {True: 0, False: 0}
    for v_dim, hidden, topk, rows in itertools.product(
        (8, 16, 64, 128, 512, 528), (8, 16, 6144, 7000), (32, 64, 2048, 65536, 65600), (1, 32, 33),
    ):
        cfg = replace(C.C3_MLA, v_dim=v_dim, hidden=hidden, topk=topk)
        s = _l.MlaShape(rows, cfg.heads, cfg.kv_lora, cfg.rope, cfg.v_dim, cfg.hidden, cfg.topk,
                        cfg.context // C.PAGE, cfg.sm_scale)
        n = ctypes.c_size_t()
        c = L.mk2_mla_workspace_bytes(ctypes.byref(s), ctypes.byref(n)) == 0
        py = _py_ok(cfg, rows)
        assert py == c, (cfg, rows, py, c, L.mk2_last_error())
        seen[py] += 1
    assert seen[True] and seen[False]


def test_indexer_validate_matches_c():
    _l, L = _lib()
    seen = {True: 0, False: 0}
    for heads, topk, ctx, rows, keys in itertools.product(
        (8, 16, 48, 64, 80), (32, 64, 2048, 4096, 4160), (32, 64, 8192, 65536, 65600, 131072), (1, 32, 33),
        (C.KEYS_FP4, C.KEYS_FP8, C.KEYS_FP4_Q4, 3),
    ):
        cfg = replace(C.C4_INDEXER, heads=heads, topk=topk, context=ctx, keys=keys)
        s = _l.IndexerShape(rows, cfg.heads, cfg.dim, cfg.topk, cfg.context, max(1, cfg.context // C.PAGE), cfg.keys)
        n = ctypes.c_size_t()
        c = L.mk2_indexer_workspace_bytes(ctypes.byref(s), ctypes.byref(n)) == 0
        py = _py_ok(cfg, rows)
        assert py == c, (cfg, rows, py, c, L.mk2_last_error())
        seen[py] += 1
    assert seen[True] and seen[False]


def test_a_config_the_c_side_rejects_fails_validate():
    """48 experts and inter 96 are multiples of 16 and 32 but outside the C limits
    (multiples of 64 and 128): validate() refuses them before any launch."""
    _l, L = _lib()
    cfg = replace(C.C1_MOE, n_experts=48, inter=96)
    assert not _moe_c_ok(_l, L, cfg, 4)
    with pytest.raises(ValueError):
        cfg.validate(4)


def test_tail_validate_matches_c():
    """The tail's argument checks (mk2_tail_launch) against TailConfig.validate().  The C
    side validates before it touches the device; on this CPU-only host an accepted call
    then fails to query the CU count (MK2_ELAUNCH), a refused one returns MK2_EINVAL.
    The pointers are never dereferenced, so the check runs only where no GPU exists."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("accepted calls would launch on the fake pointers")
    _l, L = _lib()
    fake = 0x1000
    seen = {True: 0, False: 0}
    for hidden, vocab_rows, rows in itertools.product((1024, 2048, 6144, 6000, 8192, 9216), (0, 16, 19360, 19361),
                                                      (0, 1, 32, 33)):
        cfg = C.TailConfig(hidden=hidden, vocab_rows=vocab_rows)
        a = _l.TailArgs(rows, hidden, vocab_rows, cfg.eps, fake, fake, fake, fake, None)
        rc = L.mk2_tail_launch(ctypes.byref(a), None)
        c = rc != _l.MK2_EINVAL
        py = _py_ok(cfg, rows)
        assert py == c, (cfg, rows, py, rc, L.mk2_last_error())
        seen[py] += 1
    assert seen[True] and seen[False]


def test_front_validate_matches_c():
    """FrontConfig.validate() against mk2_front_workspace_bytes over a grid of shapes."""
    from dataclasses import replace as rep

    _l, L = _lib()
    seen = {True: 0, False: 0}
    for hidden, q_lora, nope, ih, rows, fmt in itertools.product(
        (1024, 1536, 6144, 7168, 9216), (1536, 2048), (128, 160, 192), (0, 16, 48, 80), (1, 32, 33), (0, 1, 2, 3),
    ):
        cfg = rep(C.C7_FRONT, hidden=hidden, q_lora=q_lora, nope=nope, index_heads=ih, weight_fmt=fmt)
        s = _l.FrontShape(rows, cfg.hidden, cfg.q_lora, cfg.kv_lora, cfg.rope, cfg.nope, cfg.heads, cfg.index_heads,
                          cfg.weight_fmt, cfg.keys, int(cfg.kv_scaled), cfg.max_position, cfg.eps, cfg.index_eps)
        n = ctypes.c_size_t()
        c = L.mk2_front_workspace_bytes(ctypes.byref(s), ctypes.byref(n)) == 0
        py = _py_ok(cfg, rows)
        assert py == c, (cfg, rows, py, c, L.mk2_last_error())
        seen[py] += 1
    assert seen[True] and seen[False]
