// MoE block launch (every expert mode): the rows' partial sums of squares (with
// RMSNorm), router GEMV (+ RMSNorm + activation quant), route (top-k + distinct
// experts), up/gate + SwiGLU, down + combine -- as one persistent launch
// (k2_persistent.hip) for mk2_moe_launch, and as one kernel a stage for the layer's
// staged mode.
#include "indexer_stages.h"
#include "mk2_host.h"
#include "mla_stages.h"
#include "moe_stages.h"

namespace mk2 {

constexpr int MOE_NT = 512;

__global__ __launch_bounds__(128) void k_moe_sumsq(MoeDev p) { moe_sumsq<128>(p, blockIdx.y, blockIdx.x); }

template <int NCG, int FMT>
__global__ __launch_bounds__(ROUTER_NT) void k_moe_router(MoeDev p) {
  __shared__ RouterLds lds;
  moe_router<ROUTER_NT, NCG, FMT>(p, blockIdx.x, blockIdx.y, lds, 0u);
}

template <bool CMP>
__global__ __launch_bounds__(512) void k_moe_route(MoeDev p) {
  __shared__ RouteLds lds;
  moe_route<512, CMP>(p, lds, TagPoll{0u, 0, nullptr});
}

template <int NCG, int FMT>
__global__ __launch_bounds__(MOE_NT) void k_moe_upgate(MoeDev p) {
  __shared__ float red[(MOE_NT / 64) * 8 * 64 * 4];  // NW * 2 * CT * NCG * 256, CT * NCG <= 4
  __shared__ float midf[32 * 65];
  moe_upgate<MOE_NT, NCG, FMT>(p, blockIdx.x, red, midf, TagPoll{0u, 0, nullptr});
}

template <int NCG, int FMT>
__global__ __launch_bounds__(MOE_NT) void k_moe_down(MoeDev p) {
  __shared__ float red[(MOE_NT / 64) * 2 * 16 * 32];  // NW * DT * NCG * 256 (DT * NCG <= 2),
                                                     // or NW * DT * 16 * 32 (compacted rows)
  __shared__ int act_ids[512];
  __shared__ float xres[16 * 2 * 32];
  moe_down<MOE_NT, NCG, FMT>(p, blockIdx.x, red, act_ids, xres);
}

// ----------------------------------------------------------------- host side
int moe_check_shape(const mk2_moe_shape* s) {
  MK2_REQUIRE(s != nullptr, "moe: shape is NULL");
  MK2_REQUIRE(s->rows >= 1 && s->rows <= 32, "moe: rows must be in [1, 32], got %d", s->rows);
  MK2_REQUIRE(s->hidden >= 512 && s->hidden % 512 == 0, "moe: hidden must be a positive multiple of 512, got %d", s->hidden);
  MK2_REQUIRE(s->n_experts >= 64 && s->n_experts <= 256 && s->n_experts % 64 == 0,
              "moe: n_experts must be 64, 128, 192 or 256, got %d", s->n_experts);
  MK2_REQUIRE(s->top_k >= 1 && s->top_k <= 8, "moe: top_k must be in [1, 8], got %d", s->top_k);
  MK2_REQUIRE(s->router == MK2_ROUTER_SOFTMAX || s->router == MK2_ROUTER_SIGMOID_BIAS, "moe: unknown router %d", s->router);
  MK2_REQUIRE(s->expert_fmt >= MK2_FMT_FP8 && s->expert_fmt <= MK2_FMT_A4W4, "moe: unknown expert mode %d", s->expert_fmt);
  const int imax = w_fp4(s->expert_fmt) ? 4096 : 1024;
  MK2_REQUIRE(s->inter >= 128 && s->inter % 128 == 0 && s->inter <= imax,
              "moe: inter must be a multiple of 128 in [128, %d] for this mode, got %d", imax, s->inter);
  MK2_REQUIRE(s->n_shared == 0 || s->n_shared == 1, "moe: n_shared must be 0 or 1");
  if (s->n_shared)
    MK2_REQUIRE(s->shared_inter >= 128 && s->shared_inter % 128 == 0 && s->shared_inter <= 4096,
                "moe: shared_inter must be a multiple of 128 in [128, 4096], got %d", s->shared_inter);
  MK2_REQUIRE(s->norm == 0 || s->norm == 1, "moe: norm must be 0 or 1");
  MK2_REQUIRE(s->residual == 0 || s->residual == 1, "moe: residual must be 0 or 1");
  MK2_REQUIRE(s->weight_layout == MK2_WLAYOUT_TILES || s->weight_layout == MK2_WLAYOUT_AITER16,
              "moe: unknown weight_layout %d", s->weight_layout);
  if (s->weight_layout == MK2_WLAYOUT_AITER16)
    MK2_REQUIRE(!w_fp4(s->expert_fmt) || s->inter % 256 == 0,
                "moe: AITER's E8M0 layout needs inter a multiple of 256, got %d", s->inter);
  return MK2_OK;
}

// router slices of 1024 columns (512 where hidden is an odd multiple of 512)
static int router_chunks(int hidden) { return hidden / (hidden % ROUTER_CKMAX == 0 ? ROUTER_CKMAX : 512); }

// carve the MoE scratch; with base == nullptr only sizes are computed
size_t moe_carve(const mk2_moe_shape* s, void* base, MoeDev* d) {
  Carver c(base);
  const int M = s->rows, H = s->hidden, E = s->n_experts, I = s->inter;
  const int KC = router_chunks(H);
  const int Dmax = E < M * s->top_k ? E : M * s->top_k;
  MoeDev t{};
  t.KC = KC;
  t.Dmax = Dmax;
  const int fmt = s->expert_fmt;
  // up/gate chunks: 128 intermediate rows for W8A8 (its mid is quantized per 128), 64
  // for E2M1 weights up to 16 rows, else 32
  t.UC = fmt == MK2_FMT_W8A8 ? 128 : (w_fp4(fmt) && M <= 16 && I % 64 == 0) ? 64 : 32;
  // down tasks: 24 hidden rows when hidden is a multiple of 48 (6144: one task a CU of
  // MI355X), for the scaled-MFMA E2M1 modes (above 16 rows on compacted rows); else 32
  // for them up to 16 rows; 16 otherwise
  const bool mx_down = fmt == MK2_FMT_MXFP4 || fmt == MK2_FMT_A4W4;
  t.DT = !mx_down ? 1 : H % 48 == 0 ? 3 : (M <= 16 && H % 32 == 0) ? 2 : 1;
  t.ssp = c.take<float>((size_t)(H / 16) * M);
  t.xn = c.take<bf16_t>((size_t)M * H);
  t.xq = c.take<uint8_t>((size_t)M * H);
  t.xs = c.take<uint8_t>((size_t)M * H / 32);
  t.xsf = c.take<float>((size_t)M * H / 128);
  t.logit_part = c.take<uint64_t>((size_t)KC * M * E);
  t.logits = c.take<float>((size_t)M * E);
  t.topk_ids = c.take<int>((size_t)M * s->top_k);
  t.topk_w = c.take<float>((size_t)M * s->top_k);
  t.act = c.take<uint64_t>((size_t)1 + Dmax);
  t.rw = c.take<float>((size_t)Dmax * 32);
  t.act_rows = c.take<uint64_t>((size_t)Dmax);
  t.rowc = c.take<int>((size_t)Dmax * 32);
  t.picks = c.take<uint64_t>((size_t)M * s->top_k * 2);
  if (fmt == MK2_FMT_MXFP4 || fmt == MK2_FMT_A4W4 || fmt == MK2_FMT_W8A8) {
    t.mid_q = c.take<uint8_t>((size_t)Dmax * M * I);
    if (fmt == MK2_FMT_W8A8) t.mid_sf = c.take<float>((size_t)Dmax * M * I / 128);
    else t.mid_s = c.take<uint8_t>((size_t)Dmax * M * I / 32);
  } else {
    t.mid_b = c.take<bf16_t>((size_t)Dmax * M * I);
  }
  t.mid_sh = c.take<bf16_t>((size_t)M * (s->n_shared ? s->shared_inter : 0) + 1);
  if (d) {
    d->KC = t.KC; d->Dmax = t.Dmax; d->UC = t.UC; d->DT = t.DT; d->ssp = t.ssp; d->xn = t.xn; d->xq = t.xq; d->xs = t.xs;
    d->xsf = t.xsf; d->mid_sf = t.mid_sf;
    d->logit_part = t.logit_part; d->logits = t.logits; d->topk_ids = t.topk_ids;
    d->topk_w = t.topk_w; d->act = t.act; d->rw = t.rw; d->mid_q = t.mid_q;
    d->act_rows = t.act_rows; d->rowc = t.rowc; d->picks = t.picks;
    d->mid_s = t.mid_s; d->mid_b = t.mid_b; d->mid_sh = t.mid_sh;
  }
  return c.bytes();
}

int moe_fill(const mk2_moe_args* a, MoeDev* d) {
  const mk2_moe_shape* s = &a->shape;
  int rc = moe_check_shape(s);
  if (rc) return rc;
  const mk2_moe_weights* w = &a->w;
  MK2_REQUIRE(w->w_router && w->w13 && w->s13 && w->w2 && w->s2, "moe: a routed or router weight pointer is NULL");
  MK2_REQUIRE(s->router != MK2_ROUTER_SIGMOID_BIAS || w->router_bias, "moe: the sigmoid_bias router needs router_bias");
  MK2_REQUIRE(!s->n_shared || (w->ws13 && w->ss13 && w->ws2 && w->ss2), "moe: a shared-expert pointer is NULL");
  MK2_REQUIRE(!s->norm || w->gamma, "moe: norm=1 needs gamma");
  *d = MoeDev{};
  d->M = s->rows; d->H = s->hidden; d->E = s->n_experts; d->topk = s->top_k; d->I = s->inter;
  d->router = s->router; d->fmt = s->expert_fmt; d->n_shared = s->n_shared;
  d->SI = s->n_shared ? s->shared_inter : 0; d->norm = s->norm; d->residual = s->residual;
  d->route_scale = s->route_scale; d->eps = s->eps; d->wl = s->weight_layout;
  d->gamma = (const bf16_t*)w->gamma; d->w_router = (const uint8_t*)w->w_router;
  d->bias = w->router_bias; d->w13 = (const uint8_t*)w->w13; d->s13 = (const uint8_t*)w->s13;
  d->w2 = (const uint8_t*)w->w2; d->s2 = (const uint8_t*)w->s2;
  d->ws13 = (const uint8_t*)w->ws13; d->ss13 = w->ss13; d->ws2 = (const uint8_t*)w->ws2; d->ss2 = w->ss2;
  d->x = (const bf16_t*)a->x; d->out = (bf16_t*)a->out;
  return MK2_OK;
}

int k2_block_enqueue(int blk, const IdxDev* idx, const MlaDev* mla, const MoeDev* moe, int* sync, int rows,
                     hipStream_t st);
constexpr size_t BLOCK_SYNC_BYTES = (size_t)SYNC_INTS * 4;  // the persistent launch's sync block

// the layer's staged mode: one kernel a stage, in stream order
int moe_enqueue(const MoeDev& d, hipStream_t st) {
  const int ncg = d.M > 16 ? 2 : 1;
  if (d.norm) k_moe_sumsq<<<dim3(d.H / 512, d.M), 128, 0, st>>>(d);  // H: a multiple of 512
  const int up_tasks = d.Dmax * (d.I / d.UC) + d.n_shared * (d.SI / 32);
  with_moe_fmt(d.fmt, [&](auto F) {
    constexpr int FMT = decltype(F)::value;
    if (ncg == 1) k_moe_router<1, FMT><<<dim3(d.E / 16, d.KC), ROUTER_NT, 0, st>>>(d);
    else k_moe_router<2, FMT><<<dim3(d.E / 16, d.KC), ROUTER_NT, 0, st>>>(d);
    if (compact_rows(d)) k_moe_route<true><<<1, 512, 0, st>>>(d);
    else k_moe_route<false><<<1, 512, 0, st>>>(d);
    if (ncg == 1) k_moe_upgate<1, FMT><<<up_tasks, MOE_NT, 0, st>>>(d);
    else k_moe_upgate<2, FMT><<<up_tasks, MOE_NT, 0, st>>>(d);
    if (ncg == 1) k_moe_down<1, FMT><<<down_tasks(d), MOE_NT, 0, st>>>(d);
    else k_moe_down<2, FMT><<<down_tasks(d), MOE_NT, 0, st>>>(d);
    return 0;
  });
  return check_launch("moe");
}

}  // namespace mk2

using namespace mk2;

extern "C" int mk2_moe_workspace_bytes(const mk2_moe_shape* shape, size_t* bytes) {
  clear_error();
  int rc = moe_check_shape(shape);
  if (rc) return rc;
  MK2_REQUIRE(bytes != nullptr, "moe: bytes is NULL");
  *bytes = BLOCK_SYNC_BYTES + moe_carve(shape, nullptr, nullptr);
  return MK2_OK;
}

extern "C" int mk2_moe_workspace_layout(const mk2_moe_shape* shape, mk2_moe_ws_layout* out) {
  clear_error();
  int rc = moe_check_shape(shape);
  if (rc) return rc;
  MK2_REQUIRE(out != nullptr, "moe: layout is NULL");
  // carve at a stand-in base, after the sync block, and report offsets from the
  // workspace's start (nothing is dereferenced)
  char* const base = (char*)(uintptr_t)4096;
  MoeDev d{};
  d.fmt = shape->expert_fmt;
  moe_carve(shape, base + BLOCK_SYNC_BYTES, &d);
  auto off = [&](const void* p) -> int64_t { return p ? (int64_t)((const char*)p - base) : -1; };
  const int fmt = shape->expert_fmt;
  const bool q = fmt == MK2_FMT_MXFP4 || fmt == MK2_FMT_W8A8 || fmt == MK2_FMT_A4W4;
  out->xn = off(d.xn);
  out->xq = q ? off(d.xq) : -1;
  out->xs = fmt == MK2_FMT_MXFP4 || fmt == MK2_FMT_A4W4 ? off(d.xs) : -1;
  out->xsf = fmt == MK2_FMT_W8A8 ? off(d.xsf) : -1;
  out->act = off(d.act);
  out->mid_q = off(d.mid_q);
  out->mid_s = off(d.mid_s);
  out->mid_sf = off(d.mid_sf);
  out->mid_b = off(d.mid_b);
  out->mid_sh = shape->n_shared ? off(d.mid_sh) : -1;
  out->dmax = d.Dmax;
  d.M = shape->rows;
  out->compact = compact_rows(d) ? 1 : 0;
  return MK2_OK;
}

extern "C" int mk2_moe_launch(const mk2_moe_args* a, mk2_stream_t stream) {
  clear_error();
  MK2_REQUIRE(a != nullptr, "moe: args is NULL");
  MoeDev d;
  int rc = moe_fill(a, &d);
  if (rc) return rc;
  MK2_REQUIRE(a->x && a->out && a->workspace, "moe: x, out and workspace must be set");
  MK2_REQUIRE(a->x != a->out, "moe: out must not alias x");
  const size_t need = BLOCK_SYNC_BYTES + moe_carve(&a->shape, nullptr, nullptr);
  if (a->workspace_bytes < need)
    return set_error(MK2_ENOSPACE, "moe: workspace has %zu bytes, needs %zu", a->workspace_bytes, need);
  moe_carve(&a->shape, (char*)a->workspace + BLOCK_SYNC_BYTES, &d);
  if (a->logits) d.logits = a->logits;
  if (a->topk_ids) d.topk_ids = a->topk_ids;
  if (a->topk_weights) d.topk_w = a->topk_weights;
  return k2_block_enqueue(2 /* moe */, nullptr, nullptr, &d, (int*)a->workspace, d.M, (hipStream_t)stream);
}
