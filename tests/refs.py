"""Oracle evaluations of synthetic cases (tests, smoke and the CPU baseline only).

Takes the canonical quantized tensors a ``sgl_amd_mono.k2.synth`` namespace holds,
dequantizes them with the oracle's own decoders and runs ``oracle.reference``.
"""

from __future__ import annotations

import torch

from oracle import codecs as oc
from oracle import reference as R


def cpu(t):
    return None if t is None else t.detach().to("cpu")


def norm_rounding_slack(x, gamma, eps, rel=1e-6):
    """Per element of the RMSNorm output bf16(x * rstd * gamma): its bf16 ulp where the
    exact (f64) value lies within `rel` (relative) of a bf16 rounding midpoint, else 0.
    Two f32 evaluations of the norm (mean(x^2) summed in different orders, each within
    a few f32 ulps of exact) may round such an element to neighbouring bf16 values."""
    xd = cpu(x).double()
    v = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps) * cpu(gamma).double()
    a = v.abs().clamp_min(1e-300)
    ulp = torch.pow(2.0, torch.floor(torch.log2(a)) - 7)
    near = ((a / ulp).frac() - 0.5).abs() * ulp <= rel * a
    return torch.where(near, ulp, torch.zeros_like(ulp))


def logit_error(logits, rlogits, w_router, slack=None):
    """The largest |kernel - oracle| router logit over its row's largest |logit|, after
    taking off what the normalized rows' rounding slack (norm_rounding_slack) can move
    a logit by: sum_k slack[k] * |W_router[e, k]|."""
    d = (cpu(logits).double() - rlogits.double()).abs()
    if slack is not None:
        d = (d - slack @ cpu(w_router).double().abs().T).clamp_min(0)
    return (d / rlogits.double().abs().amax(-1, keepdim=True)).max().item()


class MoEOracle:
    """The MoE block of a synth namespace on the CPU (experts dequantized lazily)."""

    def __init__(self, w):
        from sgl_amd_mono.k2 import config as C

        self.cfg = w.cfg
        self.C = C
        self.w_router = cpu(w.w_router).float()
        self.bias = cpu(w.bias)
        self.gamma = cpu(w.gamma)
        self.w13q, self.w13s, self.w2q, self.w2s = map(cpu, (w.w13q, w.w13s, w.w2q, w.w2s))
        self.shared = None
        if self.cfg.n_shared:
            self.shared = (
                oc.fp8_block_dequant(cpu(w.ws13q), cpu(w.ws13s)),
                oc.fp8_block_dequant(cpu(w.ws2q), cpu(w.ws2s)),
            )
        self._cache = {}

    def expert_weights(self, e):
        if e not in self._cache:
            if self.cfg.expert_fmt in self.C.FP4_WEIGHT_FMTS:
                w13 = oc.mxfp4_dequant(self.w13q[e], self.w13s[e])
                w2 = oc.mxfp4_dequant(self.w2q[e], self.w2s[e])
            else:
                w13 = oc.fp8_block_dequant(self.w13q[e], self.w13s[e])
                w2 = oc.fp8_block_dequant(self.w2q[e], self.w2s[e])
            self._cache[e] = (w13, w2)
        return self._cache[e]

    def dequant_all(self):
        for e in range(self.cfg.n_experts):
            self.expert_weights(e)

    def __call__(self, x, *, norm=False, residual=False, eps=1e-6, parts=False):
        """(out, ids, weights, logits) of the block; with parts=True also y, the f64
        route-weighted expert sum before the residual and the bf16 rounding."""
        cfg = self.cfg
        x = cpu(x).float()
        xn = R.rmsnorm(x, self.gamma, eps) if norm else x
        if cfg.router == self.C.ROUTER_SIGMOID_BIAS:
            route = lambda lg: R.route_sigmoid_bias(lg, self.bias, cfg.top_k, cfg.route_scale)  # noqa: E731
        else:
            route = lambda lg: R.route_softmax(lg, cfg.top_k)  # noqa: E731
        fn = {self.C.FMT_FP8: R.expert_fp8, self.C.FMT_MXFP4: R.expert_mxfp4, self.C.FMT_W8A8: R.expert_w8a8,
              self.C.FMT_A16W4: R.expert_fp8, self.C.FMT_A4W4: R.expert_a4w4}[cfg.expert_fmt]

        def expert(e, xr):
            w13, w2 = self.expert_weights(e)
            return fn(xr, w13, w2)

        shared = None
        if self.shared is not None:
            shared = lambda xr: R.expert_fp8(xr, *self.shared)  # noqa: E731
        res = R.moe_block(
            xn, lambda v: v @ self.w_router.T, route, expert, shared,
            residual=x if residual else None,
        )
        if not parts:
            return res
        _, ids, w, _ = res
        return (*res, R.moe_mix(xn, ids, w, expert, shared))


def index_keys_f32(cache, cache_scale, page_table, req, n, dim=128):
    """Dequantized keys of positions 0..n-1 of request `req` (oracle decoders).  With a
    cache_scale, from SGLang's FP4 index plane (score_fp4.py:9-12): token t of a page has
    its 16 code bytes of chunk c at c * 1024 + t * 16 and that chunk's E8M0 at c * 64 +
    (t % 16) * 4 + t // 16 of the page's scale row.  Without, from the FP8 DSA index
    pages [P, 64, 132] (oc.index_page_decode)."""
    cache, page_table = cpu(cache), cpu(page_table)
    pages = page_table[req, : (n + 63) // 64].long()
    if cache_scale is None:
        return oc.index_page_decode(cache[pages]).reshape(-1, dim)[:n]
    cache_scale = cpu(cache_scale)
    t = torch.arange(64)
    codes = torch.empty(len(pages), 64, 64, dtype=torch.uint8)
    scales = torch.empty(len(pages), 64, 4, dtype=torch.uint8)
    for c in range(4):
        codes[:, :, 16 * c : 16 * c + 16] = cache[pages][:, c * 1024 : (c + 1) * 1024].reshape(-1, 64, 16)
        scales[:, :, c] = cache_scale[pages][:, c * 64 + (t % 16) * 4 + t // 16]
    keys = oc.mxfp4_dequant(codes, scales).reshape(-1, dim)
    return keys[:n]


def indexer_oracle_scores(ns, r):
    """f64 scores of row r of a synth indexer namespace."""
    n = int(ns.ctx_len[r])
    keys = index_keys_f32(ns.cache, ns.cache_scale, ns.page_table, int(ns.req_ids[r]), n)
    return R.index_scores(index_queries(ns.cfg, ns.q[r]), cpu(ns.w[r]).float(), keys)


def index_queries(cfg, q):
    """A row's index queries as the scorer multiplies them: the bf16 values, or with
    FP4 queries (KEYS_FP4_Q4) their MXFP4 quantization, dequantized."""
    from sgl_amd_mono.k2 import config as C

    q = cpu(q).float()
    if cfg.keys == C.KEYS_FP4_Q4:
        q = oc.mxfp4_dequant(*oc.fp4_query_quant(q))
    return q


def mla_oracle(ns, sel=None, h="auto", parts=False):
    """(o_lat f32 [rows, 16, 512], out f32-of-bf16 [rows, hidden]) of a synth MLA case;
    with parts=True also y = o W_o^T in f64 [rows, hidden] (the attention term, before
    the residual and the bf16 rounding)."""
    cfg = ns.cfg
    sel = cpu(ns.sel if sel is None else sel).long()
    kv, pt = cpu(ns.kv), cpu(ns.page_table)
    if kv.dim() == 2:  # SGLang's flat [slots][576]: pages of 64 slots
        kv = kv.view(-1, 64, kv.shape[-1])
    ksc = torch.ones(kv.shape[:2]) if ns.kv_scale is None else cpu(ns.kv_scale)
    q, w_uv, w_o = cpu(ns.q).float(), cpu(ns.w_uv).float(), cpu(ns.w_o).float()
    hres = cpu(ns.h) if h == "auto" else (cpu(h) if h is not None else None)
    olats, outs, ys = [], [], []
    for r in range(ns.rows):
        pos = sel[r][sel[r] >= 0]
        req = int(ns.req_ids[r])
        pages = pt[req, pos // 64].long()
        rows_kv = oc.fp8_row_dequant(kv[pages, pos % 64], ksc[pages, pos % 64])
        ol = R.sparse_mla(q[r], rows_kv, cfg.sm_scale, cfg.kv_lora)
        o = R.mla_output(ol, w_uv)
        outs.append(R.o_proj(o[None], w_o, None if hres is None else hres[r : r + 1])[0])
        olats.append(ol)
        ys.append(o.double() @ w_o.double().T)
    if parts:
        return torch.stack(olats), torch.stack(outs), torch.stack(ys)
    return torch.stack(olats), torch.stack(outs)


def bf16_rounding_floor(v, ref):
    """The rel-L2 that rounding v to bf16 alone gives against a term of norm ||ref||:
    rms(ulp(v)) / sqrt(12) / rms(ref).  A check of (v - known) against ref can only
    resolve errors above this."""
    a = cpu(v).double().abs().clamp_min(1e-30)
    ulp = torch.pow(2.0, torch.floor(torch.log2(a)) - 7)
    return float(ulp.pow(2).mean().sqrt() / 12**0.5 / ref.double().pow(2).mean().sqrt().clamp_min(1e-30))


def check_layer(L, out, attn, scores, topk, logits, ids, wts, *, o_latent=None, rel_l2=1e-2, score_bound=1e-4):
    """Piecewise parity of a chained K2 layer run (kernel outputs on the CPU), each
    stage against the oracle on the kernel's own inputs to that stage:
      indexer -- scores vs f64, the list == radix_lists of the kernel's own scores;
      attention -- on the kernel's selection: o_latent (the merged attention before
        W_UV, if given) and the attention term attn - h against the oracle's o W_o^T
        in f64, each rel-L2 <= rel_l2 (the attention term is checked when the bf16
        rounding of h + o W_o^T leaves it resolvable, bf16_rounding_floor <= 0.3 *
        rel_l2: it then adds at most 5 % to the measured error; that needs a residual
        small against the term, and the parity tests draw such residuals);
      MoE -- on the kernel's attention output: router logits, ids, and the MoE term
        out - attn against the oracle's f64 route-weighted expert sum, rel-L2 <=
        rel_l2 (when resolvable in the same sense);
    plus the whole outputs attn and out within rel_l2.  Returns the measured errors."""
    cfg = L.cfg
    k = cfg.indexer.topk
    worst = 0.0
    for r in range(L.rows):
        n = int(L.idx.ctx_len[r])
        if n == 0:  # a pad row: no keys, an empty list
            assert bool((topk[r] == -1).all()), ("pad row list", r)
            continue
        got = scores[r, :n]
        ref = indexer_oracle_scores(L.idx, r)
        err = ((got.double() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
        worst = max(worst, err)
        assert err <= score_bound, ("index score", r, err)
        assert torch.equal(topk[r, : min(n, k)].long(), R.radix_lists(got, k)), ("top-k list", r)
    stats = {"score_err": worst}
    ref_lat, ref_attn, ref_y = mla_oracle(L.mla, sel=topk, h=L.h, parts=True)
    if o_latent is not None:
        stats["o_latent_rel_l2"] = R.rel_l2(o_latent.float(), ref_lat)
        assert stats["o_latent_rel_l2"] <= rel_l2, ("o_latent", stats["o_latent_rel_l2"])
    stats["attn_rel_l2"] = R.rel_l2(attn.float(), ref_attn)
    assert stats["attn_rel_l2"] <= rel_l2, ("attention", stats["attn_rel_l2"])
    h = cpu(L.h).double()
    stats["attn_term_floor"] = bf16_rounding_floor(attn, ref_y)
    stats["attn_term_rel_l2"] = R.rel_l2(attn.double() - h, ref_y)
    resolvable = 0.3 * rel_l2
    stats["attn_term_checked"] = stats["attn_term_floor"] <= resolvable
    if stats["attn_term_checked"]:
        assert stats["attn_term_rel_l2"] <= rel_l2, ("attention term attn - h", stats)
    orc = MoEOracle(L.moe)
    ref_out, rids, rw, rlogits, ref_ymoe = orc(attn, norm=True, residual=True, eps=cfg.eps, parts=True)
    slack = norm_rounding_slack(attn.float(), orc.gamma, cfg.eps)
    stats["logit_err"] = logit_error(logits, rlogits, orc.w_router, slack)
    assert stats["logit_err"] <= 1e-4, ("router logits", stats["logit_err"])
    s = torch.sigmoid(rlogits) + orc.bias
    srt = torch.sort(s, dim=-1, descending=True).values
    clear = (srt[:, cfg.moe.top_k - 1] - srt[:, cfg.moe.top_k]) > 1e-4 * s.abs().amax(-1)
    assert torch.equal(ids.long()[clear], rids[clear]), "expert ids"
    stats["clear_rows"] = int(clear.sum())
    stats["moe_term_floor"] = bf16_rounding_floor(out, ref_ymoe)
    stats["moe_term_rel_l2"] = R.rel_l2(out.double() - attn.double(), ref_ymoe)
    stats["moe_term_checked"] = stats["moe_term_floor"] <= resolvable
    if stats["moe_term_checked"]:
        assert stats["moe_term_rel_l2"] <= rel_l2, ("MoE term out - attn", stats)
    stats["out_rel_l2"] = R.rel_l2(out.float(), ref_out)
    assert stats["out_rel_l2"] <= rel_l2, ("layer out", stats["out_rel_l2"])
    return stats


class CpuLayer:
    """The oracle's forward of one chained layer with every input already on the CPU
    and every expert dequantized (the CPU baseline of bench.py)."""

    def __init__(self, L):
        from types import SimpleNamespace

        self.cfg, self.rows = L.cfg, L.rows
        self.idx = SimpleNamespace(**{k: cpu(v) if torch.is_tensor(v) else v for k, v in vars(L.idx).items()})
        self.mla = SimpleNamespace(**{k: cpu(v) if torch.is_tensor(v) else v for k, v in vars(L.mla).items()})
        self.h = cpu(L.h)
        self.moe = MoEOracle(L.moe)
        self.keys = [index_keys_f32(self.idx.cache, self.idx.cache_scale, self.idx.page_table, int(self.idx.req_ids[r]),
                                    int(self.idx.ctx_len[r])) for r in range(self.rows)]
        self.moe.dequant_all()

    def forward(self):
        cfg = self.cfg
        sel = torch.full((self.rows, cfg.indexer.topk), -1, dtype=torch.int64)
        for r in range(self.rows):
            s = R.index_scores(index_queries(cfg.indexer, self.idx.q[r]), self.idx.w[r].float(), self.keys[r]).float()
            lst = R.radix_lists(s, cfg.indexer.topk)
            sel[r, : lst.numel()] = lst
        _, attn = mla_oracle(self.mla, sel=sel, h=self.h)
        out, *_ = self.moe(attn, norm=True, residual=True, eps=cfg.eps)
        return out
