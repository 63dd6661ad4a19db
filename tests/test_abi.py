"""The C-ABI library on the CPU: it loads, exports every entry point include/mk2.h
declares, its ctypes mirrors have the C layouts, and argument errors come back as
codes with a message before anything reaches the GPU."""

import ctypes
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mk2.h")


def _declared():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(mk2_\w+)\s*\(", src, re.M)))


def _lib():
    from sgl_amd_mono import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libmk2.so not built (run __graft_entry__.build())")
    return _lib, _lib.lib()


def test_every_declared_symbol_is_exported():
    _l, L = _lib()
    names = _declared()
    assert len(names) >= 10
    for n in names:
        assert hasattr(L, n), n
    assert L.mk2_abi_version() == _l.ABI_VERSION == 4


def test_ctypes_layouts_match_the_header():
    _l, _ = _lib()
    prog = r'''
#include <stdio.h>
#include <stddef.h>
#include "mk2.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(mk2_moe_shape), sizeof(mk2_moe_weights),
         sizeof(mk2_moe_args), sizeof(mk2_indexer_shape), sizeof(mk2_indexer_args),
         sizeof(mk2_mla_shape), sizeof(mk2_mla_args), sizeof(mk2_layer_args), sizeof(mk2_tail_args),
         sizeof(mk2_step_args), sizeof(mk2_front_shape), sizeof(mk2_front_weights), sizeof(mk2_front_args));
  printf("%zu %zu %zu %zu %zu %zu %zu %zu\n", offsetof(mk2_moe_args, logits), offsetof(mk2_mla_args, o_latent),
         offsetof(mk2_layer_args, workspace_bytes), offsetof(mk2_indexer_shape, key_fmt),
         offsetof(mk2_tail_args, normed), offsetof(mk2_step_args, ids_in_bytes), offsetof(mk2_step_args, ctx_len),
         offsetof(mk2_layer_args, wait_us));
  printf("%d %d %d\n", MK2_MAX_WAIT_US, MK2_BLOCK_STATUS_OFFSET, MK2_FRONT_STATUS_OFFSET);
  return 0;
}
'''
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "t.c"), os.path.join(d, "t")
        open(c, "w").write(prog)
        subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), c, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    sizes = [int(x) for x in out[0].split()]
    offs = [int(x) for x in out[1].split()]
    mine = [ctypes.sizeof(t) for t in (_l.MoeShape, _l.MoeWeights, _l.MoeArgs, _l.IndexerShape,
                                       _l.IndexerArgs, _l.MlaShape, _l.MlaArgs, _l.LayerArgs, _l.TailArgs,
                                       _l.StepArgs, _l.FrontShape, _l.FrontWeights, _l.FrontArgs)]
    assert sizes == mine
    assert offs == [_l.MoeArgs.logits.offset, _l.MlaArgs.o_latent.offset,
                    _l.LayerArgs.workspace_bytes.offset, _l.IndexerShape.key_fmt.offset,
                    _l.TailArgs.normed.offset, _l.StepArgs.ids_in_bytes.offset, _l.StepArgs.ctx_len.offset,
                    _l.LayerArgs.wait_us.offset]
    consts = [int(x) for x in out[2].split()]
    assert consts == [_l.MK2_MAX_WAIT_US, _l.MK2_BLOCK_STATUS_OFFSET, _l.MK2_FRONT_STATUS_OFFSET]


def _moe_shape(_l, **kw):
    base = dict(rows=8, hidden=6144, n_experts=256, top_k=8, inter=256, router=1, expert_fmt=1,
                n_shared=1, shared_inter=256, norm=0, residual=0, route_scale=2.5, eps=1e-6)
    base.update(kw)
    return _l.MoeShape(**base)


def test_workspace_queries_and_shape_errors():
    _l, L = _lib()
    n = ctypes.c_size_t()
    assert L.mk2_moe_workspace_bytes(ctypes.byref(_moe_shape(_l)), ctypes.byref(n)) == 0
    assert n.value > 0
    for bad in (dict(rows=0), dict(rows=33), dict(hidden=1000), dict(n_experts=100), dict(top_k=9),
                dict(router=5), dict(expert_fmt=7), dict(inter=100), dict(weight_layout=2),
                dict(weight_layout=1, inter=128)):
        rc = L.mk2_moe_workspace_bytes(ctypes.byref(_moe_shape(_l, **bad)), ctypes.byref(n))
        assert rc == _l.MK2_EINVAL, bad
        assert L.mk2_last_error().decode().startswith("moe:"), bad
    ish = _l.IndexerShape(8, 64, 128, 2048, 65536, 1024)
    assert L.mk2_indexer_workspace_bytes(ctypes.byref(ish), ctypes.byref(n)) == 0
    assert L.mk2_indexer_workspace_bytes(ctypes.byref(_l.IndexerShape(8, 64, 128, 2048, 131072, 2048)),
                                         ctypes.byref(n)) == _l.MK2_EINVAL
    msh = _l.MlaShape(8, 16, 512, 64, 128, 6144, 2048, 512, 576**-0.5)
    assert L.mk2_mla_workspace_bytes(ctypes.byref(msh), ctypes.byref(n)) == 0
    assert L.mk2_mla_workspace_bytes(ctypes.byref(_l.MlaShape(8, 8, 512, 64, 128, 6144, 2048, 512, 0.1)),
                                     ctypes.byref(n)) == _l.MK2_EINVAL


def test_launch_argument_errors_never_reach_the_device():
    _l, L = _lib()
    assert L.mk2_moe_launch(None, None) == _l.MK2_EINVAL
    args = _l.MoeArgs(_moe_shape(_l), _l.MoeWeights(), None, None, None, 0, None, None, None)
    assert L.mk2_moe_launch(ctypes.byref(args), None) == _l.MK2_EINVAL
    assert "NULL" in L.mk2_last_error().decode()
    assert L.mk2_sparse_mla_launch(None, None) == _l.MK2_EINVAL
    assert L.mk2_indexer_topk_launch(None, None) == _l.MK2_EINVAL
    # the FP4 index plane's scales are required (pointers below are never dereferenced:
    # the arguments are rejected first)
    fake = 0x1000
    ia = _l.IndexerArgs(_l.IndexerShape(8, 64, 128, 2048, 65536, 1024), fake, fake, fake, None, fake, fake,
                        fake, None, None, fake, 1 << 30)
    assert L.mk2_indexer_topk_launch(ctypes.byref(ia), None) == _l.MK2_EINVAL
    assert "cache_scale" in L.mk2_last_error().decode()
    # the FP8 index cache carries its scales: a separate scale plane is refused, and an
    # unknown key format is refused by the shape check
    ia.shape.key_fmt, ia.cache_scale = _l.MK2_KEYS_FP8, fake
    assert L.mk2_indexer_topk_launch(ctypes.byref(ia), None) == _l.MK2_EINVAL
    assert "cache_scale must be NULL" in L.mk2_last_error().decode()
    ia.shape.key_fmt = 3
    assert L.mk2_indexer_topk_launch(ctypes.byref(ia), None) == _l.MK2_EINVAL
    assert "key_fmt" in L.mk2_last_error().decode()
    # FP4 queries score the FP4 plane: its scales are required as for MK2_KEYS_FP4
    ia.shape.key_fmt, ia.cache_scale = _l.MK2_KEYS_FP4_Q4, None
    assert L.mk2_indexer_topk_launch(ctypes.byref(ia), None) == _l.MK2_EINVAL
    assert "cache_scale" in L.mk2_last_error().decode()
    assert L.mk2_layer_launch(None, None) == _l.MK2_EINVAL
    assert L.mk2_step_rows_launch(None, None) == _l.MK2_EINVAL
    sa = _l.StepArgs(width=33, rows=1, topk=2048)
    assert L.mk2_step_rows_launch(ctypes.byref(sa), None) == _l.MK2_EINVAL
    assert "width" in L.mk2_last_error().decode()
    sa = _l.StepArgs(width=4, rows=5, topk=2048)
    assert L.mk2_step_rows_launch(ctypes.byref(sa), None) == _l.MK2_EINVAL
    assert L.mk2_write_seed_launch(None, None, None, 0, None, 1, 2048, None) == _l.MK2_EINVAL
    assert L.mk2_front_launch(None, None) == _l.MK2_EINVAL
    fs = _l.FrontShape(8, 6144, 2048, 512, 64, 160, 16, 64, 1, 0, 1, 65535, 1e-6, 1e-6)
    n = ctypes.c_size_t()
    assert L.mk2_front_workspace_bytes(ctypes.byref(fs), ctypes.byref(n)) == _l.MK2_EINVAL
    assert "nope" in L.mk2_last_error().decode()
    assert L.mk2_front_is_persistent(ctypes.byref(fs)) == -_l.MK2_EINVAL
    assert L.mk2_layer_step_is_fused(ctypes.byref(fs), 1) == -_l.MK2_EINVAL
    assert L.mk2_front_launch_staged(None, None) == _l.MK2_EINVAL
    fs.nope = 192
    assert L.mk2_front_workspace_bytes(ctypes.byref(fs), ctypes.byref(n)) == _l.MK2_OK and n.value > 0
    # the persistent front: its counters and status word lead the workspace
    assert n.value > _l.MK2_FRONT_STATUS_OFFSET
    assert L.mk2_front_is_persistent(ctypes.byref(fs)) == 1  # C7: hidden 6144, q_lora 2048, nope 192
    # the front-and-layer launch: C7's front with A8W4 (MXFP4) experts only
    assert L.mk2_layer_step_is_fused(ctypes.byref(fs), 1) == 1
    assert [L.mk2_layer_step_is_fused(ctypes.byref(fs), f) for f in (0, 2, 3, 4)] == [0, 0, 0, 0]
    fs.weight_fmt = 2  # block FP8 in AITER's layout: instanced too
    assert L.mk2_layer_step_is_fused(ctypes.byref(fs), 1) == 1
    fs.weight_fmt = 0  # bf16 front weights: not
    assert L.mk2_layer_step_is_fused(ctypes.byref(fs), 1) == 0
    fs.weight_fmt = 1
    fs.hidden = 4096  # K steps the persistent launch does not instantiate: the stage launches
    assert L.mk2_front_is_persistent(ctypes.byref(fs)) == 0
    assert L.mk2_layer_step_is_fused(ctypes.byref(fs), 1) == 0
    assert L.mk2_tail_launch(None, None) == _l.MK2_EINVAL
    ta = _l.TailArgs(8, 6144, 0, 1e-5, fake, fake, fake, fake, None)
    assert L.mk2_tail_launch(ctypes.byref(ta), None) == _l.MK2_EINVAL
    assert "vocab_rows" in L.mk2_last_error().decode()
    ta.vocab_rows, ta.hidden = 19360, 6000
    assert L.mk2_tail_launch(ctypes.byref(ta), None) == _l.MK2_EINVAL
    assert "hidden" in L.mk2_last_error().decode()
    ta.hidden, ta.normed = 6144, fake
    assert L.mk2_tail_launch(ctypes.byref(ta), None) == _l.MK2_EINVAL
    assert "alias" in L.mk2_last_error().decode()
    assert L.mk2_selftest_mfma(9, None, None, None, None, None, None) == _l.MK2_EINVAL
