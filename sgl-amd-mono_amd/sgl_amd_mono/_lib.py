"""ctypes binding of ``libmk2.so`` (the C ABI in ``include/mk2.h``).

The structures below mirror the C structs field for field.  torch is imported
first on purpose: its ROCm wheel ships the HIP runtime under the same SONAME
(``libamdhip64.so.7``) that libmk2 links against, so loading libmk2 after torch
binds both to one runtime -- one device context, one set of streams.  The loader
checks that only one HIP runtime is mapped and refuses otherwise.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see the module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libmk2.so"

MK2_OK, MK2_EINVAL, MK2_ELAUNCH, MK2_ENOSPACE = 0, 1, 2, 3
ABI_VERSION = 4  # MK2_ABI_VERSION of the header these structures mirror
MK2_MAX_WAIT_US = 40_000_000  # the longest dependency-wait deadline (mk2.h)
MK2_KEYS_FP4, MK2_KEYS_FP8, MK2_KEYS_FP4_Q4 = 0, 1, 2
MK2_WLAYOUT_TILES, MK2_WLAYOUT_AITER16 = 0, 1


class Mk2Error(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"mk2 error {code}: {msg}")
        self.code = code


class MoeShape(ctypes.Structure):
    _fields_ = [
        ("rows", c_int), ("hidden", c_int), ("n_experts", c_int), ("top_k", c_int),
        ("inter", c_int), ("router", c_int), ("expert_fmt", c_int), ("n_shared", c_int),
        ("shared_inter", c_int), ("norm", c_int), ("residual", c_int),
        ("route_scale", c_float), ("eps", c_float), ("weight_layout", c_int),
    ]


class MoeWeights(ctypes.Structure):
    _fields_ = [
        ("gamma", c_void_p), ("w_router", c_void_p), ("router_bias", c_void_p),
        ("w13", c_void_p), ("s13", c_void_p), ("w2", c_void_p), ("s2", c_void_p),
        ("ws13", c_void_p), ("ss13", c_void_p), ("ws2", c_void_p), ("ss2", c_void_p),
    ]


class MoeArgs(ctypes.Structure):
    _fields_ = [
        ("shape", MoeShape), ("w", MoeWeights), ("x", c_void_p), ("out", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("logits", c_void_p), ("topk_ids", c_void_p), ("topk_weights", c_void_p),
    ]


class MoeWsLayout(ctypes.Structure):
    _fields_ = [
        ("xn", c_int64), ("xq", c_int64), ("xs", c_int64), ("xsf", c_int64), ("act", c_int64),
        ("mid_q", c_int64), ("mid_s", c_int64), ("mid_sf", c_int64), ("mid_b", c_int64), ("mid_sh", c_int64),
        ("dmax", c_int), ("compact", c_int),
    ]


class IndexerShape(ctypes.Structure):
    _fields_ = [
        ("rows", c_int), ("heads", c_int), ("dim", c_int), ("topk", c_int),
        ("max_ctx", c_int), ("table_stride", c_int), ("key_fmt", c_int),
    ]


class IndexerArgs(ctypes.Structure):
    _fields_ = [
        ("shape", IndexerShape), ("q", c_void_p), ("w", c_void_p), ("cache", c_void_p), ("cache_scale", c_void_p),
        ("page_table", c_void_p), ("req_ids", c_void_p), ("ctx_len", c_void_p),
        ("scores", c_void_p), ("topk", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
    ]


class MlaShape(ctypes.Structure):
    _fields_ = [
        ("rows", c_int), ("heads", c_int), ("kv_lora", c_int), ("rope", c_int),
        ("v_dim", c_int), ("hidden", c_int), ("topk", c_int), ("table_stride", c_int),
        ("sm_scale", c_float),
    ]


class MlaArgs(ctypes.Structure):
    _fields_ = [
        ("shape", MlaShape), ("q", c_void_p), ("kv", c_void_p), ("kv_scale", c_void_p),
        ("page_table", c_void_p), ("req_ids", c_void_p), ("sel", c_void_p),
        ("w_uv", c_void_p), ("w_o", c_void_p), ("h", c_void_p), ("out", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t), ("o_latent", c_void_p),
    ]


MK2_LAYER_PERSISTENT, MK2_LAYER_STAGED = 0, 1


class LayerArgs(ctypes.Structure):
    _fields_ = [
        ("indexer", IndexerArgs), ("mla", MlaArgs), ("moe", MoeArgs),
        ("attn_out", c_void_p), ("out", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("mode", c_int), ("wait_us", c_int), ("status", c_void_p), ("timeline", c_void_p),
    ]


MK2_WFMT_BF16, MK2_WFMT_FP8_BLOCK, MK2_WFMT_FP8_AITER16 = 0, 1, 2
MK2_FRONT_STATUS_OFFSET = 6528  # bytes into the front's workspace: the persistent launch's status word
MK2_BLOCK_STATUS_OFFSET = 26624  # bytes into a block entry point's workspace: its status word


class FrontShape(ctypes.Structure):
    _fields_ = [
        ("rows", c_int), ("hidden", c_int), ("q_lora", c_int), ("kv_lora", c_int), ("rope", c_int),
        ("nope", c_int), ("heads", c_int), ("index_heads", c_int), ("weight_fmt", c_int), ("key_fmt", c_int),
        ("kv_scaled", c_int), ("max_position", c_int), ("eps", c_float), ("index_eps", c_float),
    ]


class FrontWeights(ctypes.Structure):
    _fields_ = [
        ("g_in", c_void_p), ("w_qkv_a", c_void_p), ("s_qkv_a", c_void_p), ("g_q_a", c_void_p),
        ("g_kv_a", c_void_p), ("w_q_b", c_void_p), ("s_q_b", c_void_p), ("w_uk", c_void_p),
        ("w_iq", c_void_p), ("s_iq", c_void_p), ("w_ik", c_void_p), ("s_ik", c_void_p),
        ("g_ik", c_void_p), ("b_ik", c_void_p), ("w_iw", c_void_p),
    ]


class FrontArgs(ctypes.Structure):
    _fields_ = [
        ("shape", FrontShape), ("weights", FrontWeights), ("x", c_void_p), ("positions", c_void_p),
        ("slots", c_void_p), ("rope_cos_sin", c_void_p), ("kv_cache", c_void_p), ("kv_scale", c_void_p),
        ("index_cache", c_void_p), ("index_scale", c_void_p), ("mla_q", c_void_p), ("index_q", c_void_p),
        ("index_w", c_void_p), ("workspace", c_void_p), ("workspace_bytes", c_size_t),
    ]


class TailArgs(ctypes.Structure):
    _fields_ = [
        ("rows", c_int), ("hidden", c_int), ("vocab_rows", c_int), ("eps", c_float),
        ("x", c_void_p), ("g_norm", c_void_p), ("w_head", c_void_p), ("logits", c_void_p), ("normed", c_void_p),
    ]


class StepArgs(ctypes.Structure):
    _fields_ = [
        ("width", c_int), ("rows", c_int), ("topk", c_int), ("seed_by_position", c_int),
        ("max_position", c_int64),
        ("out_cache_loc", c_void_p), ("loc_stride", c_int64),
        ("positions", c_void_p), ("pos_stride", c_int64),
        ("ids_in", c_void_p), ("ids_stride", c_int64), ("ids_in_bytes", c_int),
        ("seed", c_void_p), ("seed_stride", c_int64),
        ("slots", c_void_p), ("positions_out", c_void_p), ("indptr", c_void_p), ("req_ids", c_void_p),
        ("topk_out", c_void_p), ("ids", c_void_p), ("ctx_len", c_void_p),
    ]


# entry point -> (argtypes); every one returns int
SIGNATURES = {
    "mk2_moe_workspace_bytes": [POINTER(MoeShape), POINTER(c_size_t)],
    "mk2_moe_launch": [POINTER(MoeArgs), c_void_p],
    "mk2_moe_workspace_layout": [POINTER(MoeShape), POINTER(MoeWsLayout)],
    "mk2_indexer_workspace_bytes": [POINTER(IndexerShape), POINTER(c_size_t)],
    "mk2_indexer_topk_launch": [POINTER(IndexerArgs), c_void_p],
    "mk2_mla_workspace_bytes": [POINTER(MlaShape), POINTER(c_size_t)],
    "mk2_sparse_mla_launch": [POINTER(MlaArgs), c_void_p],
    "mk2_layer_workspace_bytes": [POINTER(LayerArgs), POINTER(c_size_t)],
    "mk2_layer_launch": [POINTER(LayerArgs), c_void_p],
    "mk2_layer_workspace_layout": [POINTER(LayerArgs), POINTER(c_int64)],
    "mk2_layer_launch_static": [POINTER(LayerArgs), c_void_p],
    "mk2_tail_launch": [POINTER(TailArgs), c_void_p],
    "mk2_front_workspace_bytes": [POINTER(FrontShape), POINTER(c_size_t)],
    "mk2_front_launch": [POINTER(FrontArgs), c_void_p],
    "mk2_front_launch_staged": [POINTER(FrontArgs), c_void_p],
    "mk2_front_is_persistent": [POINTER(FrontShape)],
    "mk2_layer_step_launch": [POINTER(FrontArgs), POINTER(LayerArgs), c_void_p],
    "mk2_layer_step_is_fused": [POINTER(FrontShape), c_int],
    "mk2_step_rows_launch": [POINTER(StepArgs), c_void_p],
    "mk2_write_seed_launch": [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int, c_int, c_void_p],
    "mk2_abi_version": [],
    "mk2_selftest_mfma": [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    "mk2_probe_stream_read": [c_void_p, c_size_t, c_void_p, c_void_p],
    "mk2_probe_handoff_bytes": [c_int, POINTER(c_size_t), POINTER(c_size_t)],
    "mk2_probe_handoff": [c_int, c_void_p, c_size_t, c_void_p, c_size_t, c_void_p, c_int, c_int, c_void_p],
}

_LIB = None


def _hip_runtimes_mapped() -> set:
    try:
        with open("/proc/self/maps") as f:
            return {ln.split()[-1] for ln in f if "libamdhip64" in ln}
    except OSError:
        return set()


def lib(required_symbols=None):
    """Load libmk2.so once; raise if it is missing (there is no fallback path)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built: run `python __graft_entry__.py build` "
            "(or sgl_amd_mono._build.build()) first; the K2 ops have no CPU fallback"
        )
    handle = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
    for name, argtypes in SIGNATURES.items():
        if not hasattr(handle, name):
            continue  # tests/test_abi.py requires every symbol; callers fail at use
        fn = getattr(handle, name)
        fn.argtypes = argtypes
        fn.restype = c_int
    if hasattr(handle, "mk2_probe_stream_unit"):
        handle.mk2_probe_stream_unit.argtypes = []
        handle.mk2_probe_stream_unit.restype = c_size_t
    handle.mk2_last_error.argtypes = []
    handle.mk2_last_error.restype = c_char_p
    if handle.mk2_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH} has ABI {handle.mk2_abi_version()}, these bindings mirror {ABI_VERSION}: rebuild it")
    runtimes = _hip_runtimes_mapped()
    if len(runtimes) > 1:
        raise RuntimeError(f"two HIP runtimes are mapped ({sorted(runtimes)}); import torch first")
    _LIB = handle
    return handle


def check(rc: int) -> None:
    if rc != MK2_OK:
        raise Mk2Error(rc, lib().mk2_last_error().decode())


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_handle(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream
