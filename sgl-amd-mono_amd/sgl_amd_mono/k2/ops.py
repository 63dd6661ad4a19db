"""Host wrappers of the C ABI: argument structs, workspace, launch on the current
stream.  Shapes and dtypes are validated here before anything is enqueued, as the
reference's runner does (glm53/gfx950/runner.py:312-318,388-421); the library
validates again on its side of the boundary.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib
from . import config as C


def _need(t, name, dtype=None, shape=None):
    if t is None:
        raise ValueError(f"{name} is required")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    return t


def _p(t):
    return None if t is None else t.data_ptr()


def moe_activation_views(shape, workspace, base: int = 0) -> dict:
    """Views of what the last launch on `workspace` left of the MoE block's activations
    (mk2_moe_workspace_layout; the MoE workspace starts `base` bytes in): xn bf16
    [M, H]; the mode's xq / xs / xsf codes and scales; act (the distinct experts, by
    slot); mid_q / mid_s / mid_sf or mid_b [dmax, M, ...] and mid_sh.  For checking the
    device quantizers; the views alias the workspace (clone before the next launch)."""
    lay = _lib.MoeWsLayout()
    _lib.check(_lib.lib().mk2_moe_workspace_layout(ctypes.byref(shape), ctypes.byref(lay)))
    M, H, I, SI, D = shape.rows, shape.hidden, shape.inter, shape.shared_inter, lay.dmax
    fp4 = shape.expert_fmt == C.FMT_A4W4

    def view(off, dtype, shp):
        if off < 0:
            return None
        n = 1
        for d in shp:
            n *= d
        nb = n * torch.empty((), dtype=dtype).element_size()
        return workspace[base + off: base + off + nb].view(dtype).view(*shp)

    out = {
        "xn": view(lay.xn, torch.bfloat16, (M, H)),
        "xq": view(lay.xq, torch.uint8, (M, H // 2 if fp4 else H)),
        "xs": view(lay.xs, torch.uint8, (M, H // 32)),
        "xsf": view(lay.xsf, torch.float32, (M, H // 128)),
        "mid_q": view(lay.mid_q, torch.uint8, (D, M, I // 2 if fp4 else I)),
        "mid_s": view(lay.mid_s, torch.uint8, (D, M, I // 32)),
        "mid_sf": view(lay.mid_sf, torch.float32, (D, M, I // 128)),
        "mid_b": view(lay.mid_b, torch.bfloat16, (D, M, I)),
        "mid_sh": view(lay.mid_sh, torch.bfloat16, (M, SI)) if shape.n_shared else None,
        "compact": bool(lay.compact),
    }
    act = view(lay.act, torch.int64, (1 + D,)).cpu() & 0xFFFFFFFF
    out["act"] = act[1: 1 + int(act[0])].clone()
    return out


def _block_status(workspace) -> int:
    """A block launch's sticky status word (nonzero: a dependency wait of a persistent
    launch passed its deadline; that launch's outputs are undefined).  Syncs."""
    off = _lib.MK2_BLOCK_STATUS_OFFSET
    return int(workspace[off:off + 4].view(torch.int32).item())


class MoEOp:
    """The MoE block of one layer (router -> top-k -> routed + shared experts)."""

    def __init__(self, cfg: C.MoEConfig, w, rows: int, *, norm: bool = False,
                 residual: bool = False, eps: float = 1e-6, device=None):
        cfg.validate(rows)
        self.cfg, self.rows, self.w = cfg, rows, w
        self.device = torch.device(device or w.w13_p.device)
        self.shape = _lib.MoeShape(
            rows, cfg.hidden, cfg.n_experts, cfg.top_k, cfg.inter, cfg.router,
            cfg.expert_fmt, cfg.n_shared, cfg.shared_inter, int(norm), int(residual),
            cfg.route_scale, eps, cfg.weight_layout,
        )
        if norm:
            _need(w.gamma, "gamma", torch.bfloat16, (cfg.hidden,))
        self.weights = _lib.MoeWeights(
            _p(w.gamma), _p(w.w_router_p), _p(w.bias), _p(w.w13_p), _p(w.s13_p),
            _p(w.w2_p), _p(w.s2_p), _p(w.ws13_p), _p(w.ws13s), _p(w.ws2_p), _p(w.ws2s),
        )
        nbytes = ctypes.c_size_t()
        _lib.check(_lib.lib().mk2_moe_workspace_bytes(ctypes.byref(self.shape), ctypes.byref(nbytes)))
        # zero-filled: the persistent launch's counters start at zero, and each launch
        # leaves them so
        self.workspace = torch.zeros(nbytes.value, dtype=torch.uint8, device=self.device)

    def status(self) -> int:
        """The launches' sticky status word (_block_status)."""
        return _block_status(self.workspace)

    def __call__(self, x, out=None, *, logits=None, topk_ids=None, topk_weights=None):
        H = self.cfg.hidden
        _need(x, "x", torch.bfloat16, (self.rows, H))
        if out is None:
            out = torch.empty_like(x)
        _need(out, "out", torch.bfloat16, (self.rows, H))
        args = _lib.MoeArgs(
            self.shape, self.weights, _p(x), _p(out), _p(self.workspace),
            self.workspace.numel(), _p(logits), _p(topk_ids), _p(topk_weights),
        )
        _lib.check(_lib.lib().mk2_moe_launch(ctypes.byref(args), _lib.stream_handle(self.device)))
        return out

    def activations(self) -> dict:
        """What the last launch left of the activations (moe_activation_views)."""
        return moe_activation_views(self.shape, self.workspace)


class IndexerOp:
    """Index-key scores (FP4 plane or FP8 DSA pages) and the exact top-k of every row."""

    def __init__(self, cfg: C.IndexerConfig, rows: int, table_stride: int, device=None):
        cfg.validate(rows)
        self.cfg, self.rows = cfg, rows
        self.device = torch.device(device or "cuda")
        self.shape = _lib.IndexerShape(rows, cfg.heads, cfg.dim, cfg.topk, cfg.context, table_stride, cfg.keys)
        nbytes = ctypes.c_size_t()
        _lib.check(_lib.lib().mk2_indexer_workspace_bytes(ctypes.byref(self.shape), ctypes.byref(nbytes)))
        # zero-filled: the persistent launch's counters start at zero, and each launch
        # leaves them so
        self.workspace = torch.zeros(nbytes.value, dtype=torch.uint8, device=self.device)

    def status(self) -> int:
        """The launches' sticky status word (_block_status)."""
        return _block_status(self.workspace)

    def __call__(self, q, w, cache, cache_scale, page_table, req_ids, ctx_len, scores=None, topk=None,
                 with_scores: bool = True):
        """(scores, topk).  with_scores=False: the launch keeps the scores to itself (in
        LDS, as the layer does; `scores` must be None and None is returned for it) and
        writes only the lists."""
        cfg, rows = self.cfg, self.rows
        _need(q, "q", torch.bfloat16, (rows, cfg.heads, cfg.dim))
        _need(w, "w", torch.bfloat16, (rows, cfg.heads))
        _need(cache, "cache", torch.uint8)
        if cfg.keys == C.KEYS_FP8:
            if cache_scale is not None:
                raise ValueError("the FP8 index cache holds its scales: cache_scale must be None")
            if cache.dim() != 3 or tuple(cache.shape[1:]) != (64, 132):
                raise ValueError(f"the FP8 index cache must be uint8 [pages, 64, 132], got {tuple(cache.shape)}")
        else:
            _need(cache_scale, "cache_scale", torch.uint8)
        _need(page_table, "page_table", torch.int32)
        if page_table.shape[1] != self.shape.table_stride:
            raise ValueError("page_table row stride differs from the op's table_stride")
        _need(req_ids, "req_ids", torch.int32, (rows,))
        _need(ctx_len, "ctx_len", torch.int32, (rows,))
        if not with_scores:
            if scores is not None:
                raise ValueError("with_scores=False takes no scores tensor")
        elif scores is None:
            scores = torch.empty(rows, cfg.context, dtype=torch.float32, device=self.device)
        if topk is None:
            topk = torch.empty(rows, cfg.topk, dtype=torch.int32, device=self.device)
        if scores is not None:
            _need(scores, "scores", torch.float32, (rows, cfg.context))
        _need(topk, "topk", torch.int32, (rows, cfg.topk))
        args = _lib.IndexerArgs(
            self.shape, _p(q), _p(w), _p(cache), _p(cache_scale), _p(page_table), _p(req_ids), _p(ctx_len),
            _p(scores), _p(topk), _p(self.workspace), self.workspace.numel(),
        )
        _lib.check(_lib.lib().mk2_indexer_topk_launch(ctypes.byref(args), _lib.stream_handle(self.device)))
        return scores, topk


class FrontOp:
    """The layer's front (the reference's K1): residual rows in; the absorbed MLA
    queries, index queries and head weights out, and this step's cache rows written.
    `w` holds SGLang's tensors as loaded (see sgl_amd_mono.k2.synth.make_front).  One
    persistent launch where the library instantiates the shape (`persistent`), else
    (or with staged=True) the six stage launches; both give the same bits."""

    def __init__(self, cfg: C.FrontConfig, w, rows: int, device=None, staged: bool = False):
        cfg.validate(rows)
        self.cfg, self.w, self.rows, self.staged = cfg, w, rows, staged
        self.device = torch.device(device or w.w_qkv_a.device)
        self.shape = _lib.FrontShape(rows, cfg.hidden, cfg.q_lora, cfg.kv_lora, cfg.rope, cfg.nope, cfg.heads,
                                     cfg.index_heads, cfg.weight_fmt, cfg.keys, int(cfg.kv_scaled),
                                     cfg.max_position, cfg.eps, cfg.index_eps)
        wdt = torch.bfloat16 if cfg.weight_fmt == C.WFMT_BF16 else torch.uint8
        NA = cfg.q_lora + cfg.kv_lora + cfg.rope
        _need(w.g_in, "g_in", torch.bfloat16, (cfg.hidden,))
        _need(w.w_qkv_a, "w_qkv_a", wdt, (NA, cfg.hidden))
        _need(w.w_q_b, "w_q_b", wdt, (cfg.heads * (cfg.nope + cfg.rope), cfg.q_lora))
        _need(w.w_uk, "w_uk", torch.bfloat16, (cfg.heads, cfg.kv_lora, cfg.nope))
        if cfg.index_heads:
            _need(w.w_iq, "w_iq", wdt, (cfg.index_heads * 128, cfg.q_lora))
            _need(w.w_ik, "w_ik", wdt, (128, cfg.hidden))
            _need(w.w_iw, "w_iw", torch.bfloat16, (cfg.index_heads, cfg.hidden))
            _need(w.g_ik, "g_ik", torch.float32, (128,))
            _need(w.b_ik, "b_ik", torch.float32, (128,))
        g = lambda n: getattr(w, n, None)  # noqa: E731
        self.weights = _lib.FrontWeights(
            _p(w.g_in), _p(w.w_qkv_a), _p(g("s_qkv_a")), _p(w.g_q_a), _p(w.g_kv_a), _p(w.w_q_b), _p(g("s_q_b")),
            _p(w.w_uk), _p(g("w_iq")), _p(g("s_iq")), _p(g("w_ik")), _p(g("s_ik")), _p(g("g_ik")), _p(g("b_ik")),
            _p(g("w_iw")),
        )
        nbytes = ctypes.c_size_t()
        _lib.check(_lib.lib().mk2_front_workspace_bytes(ctypes.byref(self.shape), ctypes.byref(nbytes)))
        # zero-filled: the persistent launch's counters start at zero and each launch
        # leaves them so
        self.workspace = torch.zeros(nbytes.value, dtype=torch.uint8, device=self.device)
        rc = _lib.lib().mk2_front_is_persistent(ctypes.byref(self.shape))
        _lib.check(-rc if rc < 0 else _lib.MK2_OK)
        self.persistent = rc == 1 and not staged

    def fuses_with(self, expert_fmt: int) -> bool:
        """Whether the library runs this front and a layer with experts of expert_fmt
        (C.FMT_*) as one launch (mk2_layer_step_is_fused; LayerStepOp)."""
        rc = _lib.lib().mk2_layer_step_is_fused(ctypes.byref(self.shape), expert_fmt)
        _lib.check(-rc if rc < 0 else _lib.MK2_OK)
        return rc == 1 and self.persistent

    def status(self) -> int:
        """The persistent launches' sticky status word (nonzero: a dependency wait passed
        its deadline; that launch's outputs are undefined).  Synchronizes."""
        return int(self.status_word().item())

    def status_word(self):
        """The persistent launches' sticky status word, a device view (int32 [1]) into
        the workspace: read it without a host sync, or clear it with zero_()."""
        off = _lib.MK2_FRONT_STATUS_OFFSET
        return self.workspace[off:off + 4].view(torch.int32)

    def _make_args(self, x, positions, slots, rope_cos_sin, kv_cache, kv_scale, index_cache, index_scale,
                   mla_q=None, index_q=None, index_w=None):
        """The launch's argument block (outputs allocated where not given) and the
        outputs (mla_q, index_q, index_w)."""
        cfg, rows, dev = self.cfg, self.rows, self.device
        _need(x, "x", torch.bfloat16, (rows, cfg.hidden))
        _need(positions, "positions", torch.int64, (rows,))
        _need(slots, "slots", torch.int64, (rows,))
        _need(rope_cos_sin, "rope_cos_sin", torch.float32, (cfg.max_position + 1, cfg.rope))
        _need(kv_cache, "kv_cache", torch.uint8)
        if mla_q is None:
            mla_q = torch.empty(rows, cfg.heads, cfg.kv_lora + cfg.rope, dtype=torch.bfloat16, device=dev)
        ih = cfg.index_heads
        if ih and index_q is None:
            index_q = torch.empty(rows, ih, 128, dtype=torch.bfloat16, device=dev)
        if ih and index_w is None:
            index_w = torch.empty(rows, ih, dtype=torch.bfloat16, device=dev)
        a = _lib.FrontArgs(self.shape, self.weights, _p(x), _p(positions), _p(slots), _p(rope_cos_sin),
                           _p(kv_cache), _p(kv_scale), _p(index_cache), _p(index_scale), _p(mla_q), _p(index_q),
                           _p(index_w), _p(self.workspace), self.workspace.numel())
        return a, (mla_q, index_q, index_w)

    def __call__(self, x, positions, slots, rope_cos_sin, kv_cache, kv_scale, index_cache, index_scale,
                 mla_q=None, index_q=None, index_w=None):
        a, outs = self._make_args(x, positions, slots, rope_cos_sin, kv_cache, kv_scale, index_cache,
                                  index_scale, mla_q, index_q, index_w)
        launch = _lib.lib().mk2_front_launch_staged if self.staged else _lib.lib().mk2_front_launch
        _lib.check(launch(ctypes.byref(a), _lib.stream_handle(self.device)))
        return outs


class TailOp:
    """The tail after the last layer: the final RMSNorm of the rows and this GPU's rows
    of the LM head, read in place from SGLang's bf16 [vocab_rows, hidden]."""

    def __init__(self, cfg: C.TailConfig, g_norm, w_head, rows: int, device=None):
        cfg.validate(rows)
        self.cfg, self.rows = cfg, rows
        self.device = torch.device(device or w_head.device)
        _need(g_norm, "g_norm", torch.bfloat16, (cfg.hidden,))
        _need(w_head, "w_head", torch.bfloat16, (cfg.vocab_rows, cfg.hidden))
        self.g_norm, self.w_head = g_norm, w_head

    def __call__(self, x, logits=None, normed=None):
        """x bf16 [rows, hidden] -> (logits f32 [rows, vocab_rows], normed bf16 [rows, hidden])."""
        cfg, rows = self.cfg, self.rows
        _need(x, "x", torch.bfloat16, (rows, cfg.hidden))
        if logits is None:
            logits = torch.empty(rows, cfg.vocab_rows, dtype=torch.float32, device=self.device)
        if normed is None:
            normed = torch.empty(rows, cfg.hidden, dtype=torch.bfloat16, device=self.device)
        _need(logits, "logits", torch.float32, (rows, cfg.vocab_rows))
        _need(normed, "normed", torch.bfloat16, (rows, cfg.hidden))
        args = _lib.TailArgs(rows, cfg.hidden, cfg.vocab_rows, cfg.eps, _p(x), _p(self.g_norm), _p(self.w_head),
                             _p(logits), _p(normed))
        _lib.check(_lib.lib().mk2_tail_launch(ctypes.byref(args), _lib.stream_handle(self.device)))
        return logits, normed


class StepRows:
    """A step's row tables for width W (the reference's Glm53Step plus ctx_len), filled
    from SGLang's rows by one launch (mk2_step_rows_launch) and read back as a seed
    (mk2_write_seed_launch)."""

    def __init__(self, width: int, topk: int = 2048, device=None):
        if not 1 <= width <= C.MAX_ROWS:
            raise ValueError(f"width must be in [1, {C.MAX_ROWS}], got {width}")
        self.width, self.k = width, topk
        self.device = torch.device(device or "cuda")
        i32, i64 = dict(dtype=torch.int32, device=self.device), dict(dtype=torch.int64, device=self.device)
        self.slots = torch.empty(width, **i64)
        self.positions = torch.empty(width, **i64)
        self.indptr = torch.empty(width + 1, **i32)
        self.req_ids = torch.empty(width, **i32)
        self.topk = torch.empty(width * topk + 1, **i32)
        self.ids = torch.empty(width, **i32)
        self.ctx_len = torch.empty(width, **i32)

    def __call__(self, out_cache_loc, positions, rows: int, max_position: int, *, ids_in=None, seed=None,
                 seed_by_position: bool = False):
        """Fill the tables for SGLang's first `rows` rows (int64 slots and positions, 1-D
        views of any stride; ids_in int32 or int64; seed int32 [rows, topk])."""
        if not 0 <= rows <= self.width:
            raise ValueError(f"rows must be in [0, {self.width}], got {rows}")
        for t, name in ((out_cache_loc, "out_cache_loc"), (positions, "positions")):
            if t.dtype != torch.int64 or t.dim() != 1 or t.shape[0] < rows or not t.is_cuda:
                raise ValueError(f"{name} must be a 1-D int64 device tensor of >= {rows} entries")
        if ids_in is not None and (ids_in.dtype not in (torch.int32, torch.int64) or ids_in.dim() != 1):
            raise ValueError("ids_in must be a 1-D int32 or int64 tensor")
        if seed is not None and (seed.dtype != torch.int32 or seed.dim() != 2 or seed.shape[1] != self.k
                                 or seed.stride(1) != 1 or seed.shape[0] < rows):
            raise ValueError(f"seed must be an int32 [rows, {self.k}] tensor with unit inner stride")
        a = _lib.StepArgs(
            self.width, rows, self.k, int(seed_by_position), max_position,
            _p(out_cache_loc), out_cache_loc.stride(0), _p(positions), positions.stride(0),
            _p(ids_in), ids_in.stride(0) if ids_in is not None else 0,
            ids_in.element_size() if ids_in is not None else 8,
            _p(seed), seed.stride(0) if seed is not None else 0,
            _p(self.slots), _p(self.positions), _p(self.indptr), _p(self.req_ids),
            _p(self.topk), _p(self.ids) if ids_in is not None else None, _p(self.ctx_len),
        )
        _lib.check(_lib.lib().mk2_step_rows_launch(ctypes.byref(a), _lib.stream_handle(self.device)))
        return self

    def write_seed(self, seed, rows: int, rows_of):
        """seed row s := the keys of step row rows_of[s], then -1 (int32 [>= rows, topk])."""
        if seed.dtype != torch.int32 or seed.dim() != 2 or seed.shape[1] != self.k or seed.stride(1) != 1:
            raise ValueError(f"seed must be an int32 [rows, {self.k}] tensor with unit inner stride")
        _need(rows_of, "rows_of", torch.int32)
        _lib.check(_lib.lib().mk2_write_seed_launch(_p(self.topk), _p(self.indptr), _p(seed), seed.stride(0),
                                                    _p(rows_of), rows, self.k, _lib.stream_handle(self.device)))
        return seed


class SparseMlaOp:
    """Sparse MLA over selected latent-KV rows, W_UV, then W_o (+ residual)."""

    def __init__(self, cfg: C.MlaConfig, w, rows: int, table_stride: int, device=None):
        cfg.validate(rows)
        self.cfg, self.rows, self.w = cfg, rows, w
        self.device = torch.device(device or w.w_o_p.device)
        _need(w.w_uv, "w_uv", torch.bfloat16, (cfg.heads, cfg.v_dim, cfg.kv_lora))
        self.shape = _lib.MlaShape(
            rows, cfg.heads, cfg.kv_lora, cfg.rope, cfg.v_dim, cfg.hidden, cfg.topk,
            table_stride, cfg.sm_scale,
        )
        nbytes = ctypes.c_size_t()
        _lib.check(_lib.lib().mk2_mla_workspace_bytes(ctypes.byref(self.shape), ctypes.byref(nbytes)))
        # zero-filled: the persistent launch's counters start at zero, and each launch
        # leaves them so
        self.workspace = torch.zeros(nbytes.value, dtype=torch.uint8, device=self.device)

    def status(self) -> int:
        """The launches' sticky status word (_block_status)."""
        return _block_status(self.workspace)

    def __call__(self, q, kv, kv_scale, page_table, req_ids, sel, h=None, out=None, o_latent=None):
        cfg, rows = self.cfg, self.rows
        _need(q, "q", torch.bfloat16, (rows, cfg.heads, cfg.qk_dim))
        _need(kv, "kv", torch.uint8)
        if kv_scale is not None:  # None: SGLang's unscaled E4M3 MLA cache
            _need(kv_scale, "kv_scale", torch.float32)
        _need(page_table, "page_table", torch.int32)
        _need(req_ids, "req_ids", torch.int32, (rows,))
        _need(sel, "sel", torch.int32, (rows, cfg.topk))
        if h is not None:
            _need(h, "h", torch.bfloat16, (rows, cfg.hidden))
        if out is None:
            out = torch.empty(rows, cfg.hidden, dtype=torch.bfloat16, device=self.device)
        _need(out, "out", torch.bfloat16, (rows, cfg.hidden))
        args = _lib.MlaArgs(
            self.shape, _p(q), _p(kv), _p(kv_scale), _p(page_table), _p(req_ids), _p(sel),
            _p(self.w.w_uv), _p(self.w.w_o_p), _p(h), _p(out), _p(self.workspace),
            self.workspace.numel(), _p(o_latent),
        )
        _lib.check(_lib.lib().mk2_sparse_mla_launch(ctypes.byref(args), _lib.stream_handle(self.device)))
        return out


class LayerOp:
    """The chained K2 layer: indexer -> top-k -> sparse MLA -> o_proj + residual ->
    RMSNorm -> MoE + residual (the reference's Glm53LayerOp.launch without the TP
    reduces, glm53/gfx950/runner.py:374-470)."""

    def __init__(self, cfg: C.K2Config, layer, rows: int, device=None, *, staged: bool = False,
                 wait_us: int = 0, static_scratch: bool = False):
        """static_scratch: launch through mk2_layer_launch_static, whose scratch is the
        library's own device array (no workspace is allocated here, and a launch
        allocates nothing); launches of such ops that overlap on one GPU race."""
        cfg.validate(rows)
        self.cfg, self.rows, self.L = cfg, rows, layer
        self.mode = _lib.MK2_LAYER_STAGED if staged else _lib.MK2_LAYER_PERSISTENT
        if not 0 <= wait_us <= _lib.MK2_MAX_WAIT_US:
            raise ValueError(f"wait_us must be in [0, {_lib.MK2_MAX_WAIT_US}], got {wait_us}")
        self.wait_us = wait_us  # a dependency wait's deadline (0: one second)
        self.device = torch.device(device or layer.h.device)
        self.idx = IndexerOp(cfg.indexer, rows, layer.idx.page_table.shape[1], self.device)
        self.mla = SparseMlaOp(cfg.mla, layer.mla, rows, layer.mla.page_table.shape[1], self.device)
        self.moe = MoEOp(cfg.moe, layer.moe, rows, norm=True, residual=True, eps=cfg.eps,
                         device=self.device)
        self._args = None
        self.static_scratch = static_scratch
        nbytes = ctypes.c_size_t()
        _lib.check(_lib.lib().mk2_layer_workspace_bytes(ctypes.byref(self._make_args()),
                                                        ctypes.byref(nbytes)))
        self.workspace_bytes = nbytes.value
        if static_scratch:
            self.workspace = None
        else:
            # zeroed once: the persistent launch's counters start at zero and every
            # launch (completed or stopped) leaves them at zero
            self.workspace = torch.zeros(nbytes.value, dtype=torch.uint8, device=self.device)
        # the launches' sticky status word: a persistent launch whose dependency wait
        # gave up ORs 1 into it (the reference's guard makes a stop visible to the host,
        # common/guard.py:100-241); check() reads it
        self.status = torch.zeros(1, dtype=torch.int32, device=self.device)

    def _make_args(self, out=None, attn_out=None, scores=None, topk=None, logits=None,
                   topk_ids=None, topk_weights=None, workspace=None, status=None, timeline=None,
                   o_latent=None):
        L = self.L
        ia = _lib.IndexerArgs(
            self.idx.shape, _p(L.idx.q), _p(L.idx.w), _p(L.idx.cache), _p(L.idx.cache_scale), _p(L.idx.page_table),
            _p(L.idx.req_ids), _p(L.idx.ctx_len), _p(scores), _p(topk), None, 0,
        )
        ma = _lib.MlaArgs(
            self.mla.shape, _p(L.mla.q), _p(L.mla.kv), _p(L.mla.kv_scale), _p(L.mla.page_table),
            _p(L.mla.req_ids), None, _p(L.mla.w_uv), _p(L.mla.w_o_p), _p(L.h), None, None, 0, _p(o_latent),
        )
        ea = _lib.MoeArgs(
            self.moe.shape, self.moe.weights, None, None, None, 0,
            _p(logits), _p(topk_ids), _p(topk_weights),
        )
        ws = workspace
        return _lib.LayerArgs(ia, ma, ea, _p(attn_out), _p(out), _p(ws),
                              0 if ws is None else ws.numel(), self.mode, self.wait_us, _p(status),
                              _p(timeline))

    def __call__(self, out=None, *, attn_out=None, scores=None, topk=None, logits=None,
                 topk_ids=None, topk_weights=None, status=None, timeline=None, o_latent=None):
        """Enqueues one layer launch on the current stream; returns out.  `status`
        (int32 [1], device) replaces the op's own sticky status word for this launch;
        the other keywords are optional outputs for checking (o_latent: f32 [rows, 16,
        512], the merged attention before W_UV)."""
        H = self.cfg.mla.hidden
        if out is None:
            out = torch.empty(self.rows, H, dtype=torch.bfloat16, device=self.device)
        _need(out, "out", torch.bfloat16, (self.rows, H))
        if status is not None:
            _need(status, "status", torch.int32, (1,))
        if o_latent is not None:
            _need(o_latent, "o_latent", torch.float32, (self.rows, self.cfg.mla.heads, self.cfg.mla.kv_lora))
        args = self._make_args(out, attn_out, scores, topk, logits, topk_ids, topk_weights,
                               self.workspace, self.status if status is None else status, timeline,
                               o_latent)
        launch = _lib.lib().mk2_layer_launch_static if self.static_scratch else _lib.lib().mk2_layer_launch
        _lib.check(launch(ctypes.byref(args), _lib.stream_handle(self.device)))
        return out

    def moe_activations(self) -> dict:
        """What the last launch left of the MoE block's activations in this op's
        workspace (moe_activation_views; mk2_layer_workspace_layout places the block)."""
        if self.workspace is None:
            raise ValueError("a static-scratch op has no workspace of its own to read")
        off = ctypes.c_int64()
        _lib.check(_lib.lib().mk2_layer_workspace_layout(ctypes.byref(self._make_args(workspace=self.workspace)),
                                                         ctypes.byref(off)))
        return moe_activation_views(self.moe.shape, self.workspace, off.value)

    def check(self) -> None:
        """Raises RuntimeError if a launch of this op stopped early since the last check
        (its outputs are not valid); clears the word.  Synchronizes with the device."""
        if int(self.status.item()) != 0:
            self.status.zero_()
            raise RuntimeError("K2 layer: a persistent launch stopped early (a dependency wait gave up); "
                               "its outputs are not valid")


class LayerStepOp:
    """The front and the K2 layer in ONE persistent launch (mk2_layer_step_launch): the
    front's stages, then the layer's.  The front writes the layer's inputs: the layer
    `layer_op.L`'s index queries, head weights, MLA queries and caches, from its
    residual rows L.h; the same bits as front_op's launch followed by layer_op's."""

    def __init__(self, front_op: FrontOp, layer_op: LayerOp):
        if front_op.rows != layer_op.rows:
            raise ValueError("front and layer rows differ")
        self.front, self.layer = front_op, layer_op

    def __call__(self, positions, slots, rope_cos_sin, out=None, *, status=None, **layer_outputs):
        L, lo = self.layer.L, self.layer
        fa, _ = self.front._make_args(L.h, positions, slots, rope_cos_sin, L.mla.kv, L.mla.kv_scale, L.idx.cache,
                                      L.idx.cache_scale, L.mla.q, L.idx.q, L.idx.w)
        H = lo.cfg.mla.hidden
        if out is None:
            out = torch.empty(lo.rows, H, dtype=torch.bfloat16, device=lo.device)
        _need(out, "out", torch.bfloat16, (lo.rows, H))
        la = lo._make_args(out, workspace=lo.workspace, status=lo.status if status is None else status,
                           **layer_outputs)
        _lib.check(_lib.lib().mk2_layer_step_launch(ctypes.byref(fa), ctypes.byref(la), _lib.stream_handle(lo.device)))
        return out
