"""The K2 layer's arithmetic on the CPU (test infrastructure only).

Each function restates one piece of the reference's decode layer and cites where.
Rounding points that are part of the dataflow (bf16 hand-offs between stages,
activation quantization) are stated here explicitly, because the HIP path rounds
at the same points; everything between them is computed in f32 (f64 for scores).

Pinned by tests/test_oracle_reference.py:
  index_scores      -- explicit loops on tiny inputs; f64 closed form
  exact_topk        -- brute force, torch.sort (stable) and torch.topk set equality
  sparse_mla        -- dense softmax attention on the gathered rows (brute force),
                       key-order invariance
  rmsnorm           -- torch.nn.functional.rms_norm
  route_softmax     -- softmax over all experts, top-k, renormalize (closed form)
  route_sigmoid_bias-- sigmoid, top-k by sigmoid + bias, normalized * scale
  swiglu            -- torch.nn.functional.silu
  moe_block         -- a single expert with hand-built weights; linearity in the
                       route weights
and by tests/test_oracle_pins.py (closed forms on hand-picked exact inputs, each with
a planted mistake that must fail):
  expert_mxfp4      -- E2M1 x E8M0 weights, MXFP8 x and mid on E4M3 rounding ties
  expert_fp8        -- mid rounded to bf16 on ties
  mla_output        -- permutation W_UV, o_lat and sums on bf16 ties
  o_proj            -- permutation W_o, residual sums on bf16 ties
  moe_mix           -- route-weighted sum of hand-built experts
  expert_a4w4, expert_w8a8 -- hand-worked single experts with their activation rules
  tail              -- +-2^e rows (exact rstd at eps 0), unit-vector LM-head rows
  step_rows, write_seed -- the reference's own cases (tests/golden/step_rows_cases.json)
  rope_pairs, fwht128, layernorm, front -- a known rotation and its inverse, the
                       Hadamard matrix against scipy's and H H^T = n I, torch's
                       layer_norm, and a front worked by hand with planted mistakes
The chained layer is the composition of these, checked stage by stage on the GPU
(tests/refs.check_layer).
"""

from __future__ import annotations

import torch

from . import codecs


# ------------------------------------------------------------------- indexer scores
def index_scores(q: torch.Tensor, w: torch.Tensor, keys: torch.Tensor) -> torch.Tensor:
    """score[c] = sum_h relu(q[h] . k[c]) * w[h], in f64.

    q [H, D] (bf16 values), w [H], keys [N, D] (dequantized FP4 keys).  Restates
    deepseek_v4/gfx950/kernels/stages/indexer.py:461-602 (relu(MFMA) * w, head sum)
    and the f64 check of test/kernels/glm53/check_topk.py:107-113.
    """
    s = torch.relu(keys.double() @ q.double().T) @ w.double()
    return s + 0.0  # -0.0 -> +0.0: a sum that starts from +0 never ends at -0


def radix_lists(scores_f32: torch.Tensor, k: int) -> torch.Tensor:
    """The exact top-k of f32 scores, as the 12-bit radix select lists it.

    Keys are the radix keys of the f32 bits; the selected set is the first k of a
    stable descending sort (ties: lowest index first, check_topk.py:116-123).  The
    list order is check_topk.radix_lists at a 12-bit prefix (check_topk.py:72-85):
    keys whose top 12 bits exceed the k-th key's, in position order; then keys with
    the same 12-bit prefix that exceed the k-th key, in position order; then keys
    equal to the k-th key, in position order, as many as fill k.  When the row has
    k or fewer entries every entry is kept, in position order
    (deepseek_v4/gfx950/kernels/stages/indexer.py:466-469).
    """
    n = scores_f32.numel()
    if n <= k:
        return torch.arange(n, dtype=torch.int64)
    keys = codecs.radix_keys(scores_f32.float())
    kth = torch.sort(keys, descending=True, stable=True).values[k - 1]
    hi, khi = keys >> 20, kth >> 20
    above = (hi > khi).nonzero().flatten()
    under = ((hi == khi) & (keys > kth)).nonzero().flatten()
    ties = (keys == kth).nonzero().flatten()[: k - len(above) - len(under)]
    return torch.cat([above, under, ties])


def exact_topk_set(scores_f32: torch.Tensor, k: int) -> torch.Tensor:
    """The selected positions as a sorted set: the first k of the stable descending
    sort of radix keys (glm53/check.py:111-114, check_topk.py:116-123)."""
    n = scores_f32.numel()
    if n <= k:
        return torch.arange(n, dtype=torch.int64)
    keys = codecs.radix_keys(scores_f32.float())
    idx = torch.sort(keys, descending=True, stable=True).indices[:k]
    return torch.sort(idx).values


# ----------------------------------------------------------------------- sparse MLA
def sparse_mla(q: torch.Tensor, kv: torch.Tensor, sm_scale: float, kv_lora: int) -> torch.Tensor:
    """Softmax attention of one request over its selected latent-KV rows.

    q [Hq, kv_lora + rope] (bf16 values, W_UK already absorbed), kv [n, kv_lora + rope]
    dequantized rows; scores = (q . kv) * sm_scale; the values are the first kv_lora
    dims of the same rows.  Returns the f32 latent output [Hq, kv_lora] before W_UV.
    Restates the split softmax + merge of glm53/gfx950/kernel.py:5147-5237,5282-5340
    (a split softmax merged exactly equals one softmax over all keys).
    """
    s = (q.double() @ kv.double().T) * sm_scale
    p = torch.softmax(s, dim=-1)
    return (p @ kv[:, :kv_lora].double()).float()


def mla_output(o_lat: torch.Tensor, w_uv: torch.Tensor) -> torch.Tensor:
    """o[h, v] = sum_c W_UV[h, v, c] * bf16(o_lat[h, c]), rounded to bf16; flattened to
    [Hq * v_dim] (glm53/gfx950/kernel.py:5239-5389: the merged o_lat is handed to
    W_UV as bf16, W_UV's output to W_o as bf16)."""
    ol = codecs.bf16_round(o_lat)
    o = torch.einsum("hvc,hc->hv", w_uv.float(), ol)
    return codecs.bf16_round(o).flatten()


def o_proj(o: torch.Tensor, w_o: torch.Tensor, h: torch.Tensor | None) -> torch.Tensor:
    """a = bf16(h + o . W_o^T) (glm53/gfx950/kernel.py:5391-5469, the 1-GPU reduce path
    :2069-2074); without a residual, bf16(o . W_o^T)."""
    y = o.float() @ w_o.float().T
    if h is not None:
        y = h.float() + y
    return codecs.bf16_round(y)


# ---------------------------------------------------------------- RMSNorm and router
def rmsnorm(a: torch.Tensor, gamma: torch.Tensor, eps: float) -> torch.Tensor:
    """x = bf16(a * rsqrt(mean(a^2) + eps) * gamma) over the last dim, in f32
    (glm53/check.py:391-393; glm53/gfx950/kernel.py:5471-5562)."""
    a = a.float()
    rstd = torch.rsqrt(a.pow(2).mean(-1, keepdim=True) + eps)
    return codecs.bf16_round(a * rstd * gamma.float())


def tail(x: torch.Tensor, g_norm: torch.Tensor, w_head: torch.Tensor, eps: float):
    """The tail after the last layer: (logits f32 [rows, V], normed bf16 values as f32
    [rows, H]).  normed = bf16(rmsnorm(x) * g), logits = bf16(normed . w_head[v]) in f64,
    rounded to bf16 as the reference's tail gathers them (glm53/gfx950/kernel.py:
    2220-2350; its check's torch tail, test/kernels/glm53/check_layer.py:744-757)."""
    normed = rmsnorm(x, g_norm, eps)
    logits = codecs.bf16_round((normed.double() @ w_head.double().t()).float())
    return logits, normed


# ------------------------------------------------------------------ the layer front
def rope_pairs(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Interleaved RoPE: pairs (2i, 2i + 1) rotated by angle i (glm53/gfx950/kernel.py:
    3107-3131,3245-3251,3358-3372); cos and sin [..., n / 2]."""
    y = x.clone()
    x0, x1 = x[..., 0::2], x[..., 1::2]
    y[..., 0::2] = x0 * cos - x1 * sin
    y[..., 1::2] = x0 * sin + x1 * cos
    return y


def hadamard(n: int) -> torch.Tensor:
    """The Sylvester-order Hadamard matrix of order n (a power of two), f64."""
    h = torch.ones(1, 1, dtype=torch.float64)
    while h.shape[0] < n:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    return h


def fwht128(x: torch.Tensor) -> torch.Tensor:
    """The orthonormal 128-point Hadamard transform, Sylvester order (glm53/gfx950/
    kernel.py:778-788), of the last dim, in f64 (returned f32)."""
    return (x.double() @ hadamard(128) * 128 ** -0.5).float()


def layernorm(x: torch.Tensor, g: torch.Tensor, b: torch.Tensor, eps: float) -> torch.Tensor:
    """(x - mean) * rsqrt(var + eps) * g + b over the last dim, biased var, f32
    (the index key's norm, glm53/gfx950/kernel.py:3116-3130)."""
    x = x.float()
    mean = x.mean(-1, keepdim=True)
    var = (x - mean).pow(2).mean(-1, keepdim=True)
    return (x - mean) * torch.rsqrt(var + eps) * g.float() + b.float()


def front(x, w, positions, cos_sin, *, eps: float, index_eps: float, nope: int, heads: int,
          index_heads: int, kv_lora: int = 512, rope: int = 64) -> dict:
    """The layer's front on rows x (bf16 values) with dequantized f32 weights `w` (a
    namespace: g_in, w_qkv_a, g_q_a, g_kv_a, w_q_b, w_uk, w_iq, w_ik, g_ik, b_ik, w_iw),
    restating the reference's K1 (glm53/gfx950/kernel.py:2585-3575) and SGLang's
    DeepSeek-V3.2 / GLM-5 attention front it follows.  Returns mla_q [rows, heads, 576],
    index_q [rows, ih, 128], index_w [rows, ih] (bf16 values), the latent cache rows'
    values before E4M3 [rows, 576] and the index keys before their quant [rows, 128]."""
    rows = x.shape[0]
    QL = w.w_q_b.shape[1]
    xn = rmsnorm(x.float(), w.g_in, eps).double()
    a = (xn @ w.w_qkv_a.double().t()).float()
    q_a, kv_a, k_pe = a[:, :QL], a[:, QL:QL + kv_lora], a[:, QL + kv_lora:]
    q_an = rmsnorm(q_a, w.g_q_a, eps)
    half = rope // 2
    cs = cos_sin[positions.long()].float()
    cos, sin = cs[:, :half], cs[:, half:]
    kv_row = torch.cat([rmsnorm(kv_a, w.g_kv_a, eps), codecs.bf16_round(rope_pairs(k_pe, cos, sin))], dim=1)
    q_b = (q_an.double() @ w.w_q_b.double().t()).float().view(rows, heads, nope + rope)
    q_nope = codecs.bf16_round(q_b[..., :nope])
    q_pe = codecs.bf16_round(rope_pairs(q_b[..., nope:], cos[:, None], sin[:, None]))
    q_lat = torch.einsum("hcn,rhn->rhc", w.w_uk.double(), q_nope.double())
    mla_q = torch.cat([codecs.bf16_round(q_lat.float()), q_pe], dim=-1)
    out = {"mla_q": mla_q, "kv_row": kv_row, "q_an": q_an}
    if index_heads:
        ik = (xn @ w.w_ik.double().t()).float()
        k = layernorm(ik, w.g_ik, w.b_ik, index_eps)
        k = torch.cat([rope_pairs(k[:, :64], cos[:, :32], sin[:, :32]), k[:, 64:]], dim=1)
        out["index_key"] = fwht128(k)
        out["index_w"] = codecs.bf16_round((xn @ w.w_iw.double().t()).float())
        iq = codecs.bf16_round((q_an.double() @ w.w_iq.double().t()).float()).view(rows, index_heads, 128)
        iq = torch.cat([rope_pairs(iq[..., :64], cos[:, None, :32], sin[:, None, :32]), iq[..., 64:]], dim=-1)
        out["index_q"] = codecs.bf16_round(fwht128(iq))
    return out


# -------------------------------------------------------------------- step tables
def step_rows(loc, pos, S: int, W: int, K: int, max_position: int, ids_in=None, seed=None,
              seed_by_position: bool = False) -> dict:
    """A step's row tables from SGLang's rows, one row at a time (glm53/tables.py:26-131,
    the Triton kernel _step_rows): row s < S takes slot loc[s] (0: a pad row, -1),
    position min(pos[s], max_position), request s, id ids_in[s], and keys indptr[s] ..<
    indptr[s + 1] -- min(position + 1, K) for a row with a slot, or with a seed the
    row's entries >= 0 in order (by position: its first min(position + 1, K) entries as
    they are); rows S ..< W: slot -1, position 0, request 0, id -1, no keys.  ctx_len:
    position + 1 for a row with a slot, else 0."""
    out = {"slots": [-1] * W, "positions": [0] * W, "req_ids": [0] * W, "ids": [-1] * W,
           "ctx_len": [0] * W, "indptr": [0] * (W + 1), "topk": []}
    for s in range(W):
        count = 0
        if s < S:
            slot, p = int(loc[s]), min(int(pos[s]), max_position)
            live = slot != 0
            out["positions"][s], out["req_ids"][s] = p, s
            if ids_in is not None:
                out["ids"][s] = int(ids_in[s])
            if live:
                out["slots"][s], out["ctx_len"][s] = slot, p + 1
                if seed is not None and not seed_by_position:
                    kept = [int(v) for v in seed[s][:K] if int(v) >= 0]
                    out["topk"] += kept
                    count = len(kept)
                else:
                    count = min(p + 1, K)
                    if seed is not None:
                        out["topk"] += [int(v) for v in seed[s][:count]]
        out["indptr"][s + 1] = out["indptr"][s] + count
    return out


def write_seed(topk, indptr, rows_of, K: int) -> list:
    """Seed row s := the keys of step row rows_of[s], then -1 up to K
    (glm53/tables.py:134-167)."""
    rows = []
    for src in rows_of:
        a, b = int(indptr[src]), int(indptr[src + 1])
        keys = [int(v) for v in topk[a:b]][:K]
        rows.append(keys + [-1] * (K - len(keys)))
    return rows


def _topk_by_key(keys: torch.Tensor, k: int) -> torch.Tensor:
    """Per row, the indices of the k largest keys, equal keys by the lower index, in
    rank order (glm53/gfx950/kernel.py:1967-1999)."""
    return torch.sort(keys, dim=-1, descending=True, stable=True).indices[..., :k]


def route_softmax(logits: torch.Tensor, k: int):
    """Top-k of the f32 logits (all bits; ties -> lower expert id), weights = softmax over
    the k picked logits (qwen38_a95b_mxfp4/gfx950/layer.py:806-849, which is softmax
    over all experts, top-k, renormalized).  Returns (ids [M, k] int64, weights f32)."""
    ids = _topk_by_key(codecs.radix_keys(logits.float()), k)
    picked = torch.gather(logits.float(), -1, ids).double()
    w = torch.softmax(picked, dim=-1).float()
    return ids, w


def route_sigmoid_bias(logits: torch.Tensor, bias: torch.Tensor, k: int, scale: float):
    """s = sigmoid(logit); top-k by the f32 bits of s + bias (ties -> lower id);
    weight = s / sum of the k picked s * scale (glm53/gfx950/kernel.py:1937-1965,
    5635-5639).  Returns (ids [M, k] int64, weights f32)."""
    s = torch.sigmoid(logits.float())
    ids = _topk_by_key(codecs.radix_keys(s + bias.float()), k)
    picked = torch.gather(s, -1, ids).double()
    w = (picked / picked.sum(-1, keepdim=True) * scale).float()
    return ids, w


# -------------------------------------------------------------------------- experts
def swiglu(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """mid = silu(g) * u = g / (1 + exp(-g)) * u, f32 (glm53/gfx950/kernel.py:5719-5724)."""
    g = g.float()
    return g / (1.0 + torch.exp(-g)) * u.float()


def expert_fp8(x: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor) -> torch.Tensor:
    """One expert on bf16 rows: g|u = x . W13^T (W13 = [gate; up] dequantized), mid =
    bf16(silu(g) * u), y = mid . W2^T (f32).  glm53's block-scaled FP8 on bf16
    activations (W8A16, glm53/gfx950/kernel.py:28-34 docstring, 1008-1120); with MXFP4
    weights dequantized, the A16W4 mode (glm53/gfx950/config.py:91)."""
    inter = w13.shape[0] // 2
    gu = x.float() @ w13.T
    mid = codecs.bf16_round(swiglu(gu[..., :inter], gu[..., inter:]))
    return mid @ w2.T


def expert_mxfp4(x: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor) -> torch.Tensor:
    """One MXFP4-weight expert on MXFP8 rows: x and mid are quantized to MXFP8 per 32
    before each product (glm53 "native_fp4" A8W4: glm53/gfx950/kernel.py:1284-1307,
    1752-1766, 7032-7060)."""
    inter = w13.shape[0] // 2
    xq = codecs.mxfp8_dequant(*codecs.mxfp8_quant(x.float()))
    gu = xq @ w13.T
    mid = swiglu(gu[..., :inter], gu[..., inter:])
    mq = codecs.mxfp8_dequant(*codecs.mxfp8_quant(mid))
    return mq @ w2.T


def expert_a4w4(x: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor) -> torch.Tensor:
    """One MXFP4-weight expert on MXFP4 rows: x and mid are quantized to MXFP4 per 32
    (AITER's round-up E8M0) before each product (kernel.py:1768-1777; the reference's
    MXFP4 x MXFP4 mid, kernel.py:6958-6966)."""
    inter = w13.shape[0] // 2
    xq = codecs.mxfp4_dequant(*codecs.mxfp4_act_quant(x.float()))
    gu = xq @ w13.T
    mid = swiglu(gu[..., :inter], gu[..., inter:])
    mq = codecs.mxfp4_dequant(*codecs.mxfp4_act_quant(mid))
    return mq @ w2.T


def expert_w8a8(x: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor) -> torch.Tensor:
    """One FP8-weight expert on FP8 rows: x and mid are quantized to E4M3 with an f32
    scale per 128 before each product (MoeMode.W8A8, glm53/gfx950/config.py:89;
    kernel.py:1740-1750,6967-6985)."""
    inter = w13.shape[0] // 2
    xq = codecs.fp8_block_act_dequant(*codecs.fp8_block_act_quant(x.float()))
    gu = xq @ w13.T
    mid = swiglu(gu[..., :inter], gu[..., inter:])
    mq = codecs.fp8_block_act_dequant(*codecs.fp8_block_act_quant(mid))
    return mq @ w2.T


def moe_mix(x, ids, w, experts, shared):
    """y = sum_k w_k * expert_{id_k}(x) + shared(x), in f64, per row: the MoE block's
    sum before its residual add and bf16 rounding (glm53/gfx950/kernel.py:6676-7136:
    down + route weighting, the shared expert at slot 0 with weight 1)."""
    m = x.shape[0]
    y = torch.zeros(m, x.shape[1], dtype=torch.float64)
    for r in range(m):
        for j in range(ids.shape[1]):
            y[r] += w[r, j].double() * experts(int(ids[r, j]), x[r : r + 1])[0].double()
    if shared is not None:
        y += shared(x).double()
    return y


def moe_block(x, logits_fn, route_fn, experts, shared, residual=None):
    """y = moe_mix(...); out = bf16(residual + y) or bf16(y).

    x [M, H] bf16 values (already normalized); logits_fn(x) -> f32 [M, E]; route_fn ->
    (ids, weights); experts(e, rows_x) -> f32 [rows, H]; shared(x) -> f32 or None.
    glm53/gfx950/kernel.py:5662-7152 (up/gate, mid, down + route weighting, residual
    :7140-7151).  Returns (out f32 of bf16 values, ids, weights, logits).
    """
    logits = logits_fn(x)
    ids, w = route_fn(logits)
    y = moe_mix(x, ids, w, experts, shared)
    if residual is not None:
        y = residual.double() + y
    return codecs.bf16_round(y.float()), ids, w, logits


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    """||a - b|| / ||b||."""
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))

