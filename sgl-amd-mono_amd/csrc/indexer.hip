// Indexer launch (FP4 or FP8 index keys, up to 64 heads x 128): key scores with the row
// histograms, the candidate slices, then the exact top-k of every row -- as one
// persistent launch (k2_persistent.hip) for mk2_indexer_topk_launch, and as one kernel a
// stage for the layer's staged mode.
#include "indexer_stages.h"
#include "mla_stages.h"
#include "mk2_host.h"
#include "moe_stages.h"

namespace mk2 {

constexpr int IDX_NT = 512;
static_assert(IDX_KEYS_FP4 == MK2_KEYS_FP4 && IDX_KEYS_FP8 == MK2_KEYS_FP8 && IDX_KEYS_FP4Q == MK2_KEYS_FP4_Q4,
              "key formats");

__global__ __launch_bounds__(256) void k_idx_clear(IdxDev p) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < p.rows * IDX_BINS; i += gridDim.x * 256) p.hist[i] = 0;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < p.rows * IDX_CBINS; i += gridDim.x * 256) p.chist[i] = 0;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < p.rows * p.nchk; i += gridDim.x * 256) p.ccount[i] = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.ticket = 0;
}

__global__ __launch_bounds__(IDX_NT) void k_idx_score(IdxDev p) {
  __shared__ IdxScoreLds L;
  idx_score<IDX_NT>(p, blockIdx.y, blockIdx.x, L);
}

// slices take their tasks in the order the workgroups start (a ticket), so that the
// earlier chunks a slice waits for have always started
__global__ __launch_bounds__(IDX_NT) void k_idx_slice(IdxDev p) {
  __shared__ TopkLds S;
  if (threadIdx.x == 0) S.res[3] = atomicAdd(p.ticket, 1);
  __syncthreads();
  const int t = S.res[3];
  __syncthreads();
  idx_slice<IDX_NT>(p, t / p.nchk, t % p.nchk, S, DEFAULT_WAIT_TICKS, nullptr, 0u);
}

__global__ __launch_bounds__(TOPK_NT) void k_idx_select(IdxDev p) {
  __shared__ TopkLds S;
  idx_select<TOPK_NT>(p, blockIdx.x, S, 0u);
  __syncthreads();
  idx_topk_reset<TOPK_NT>(p, blockIdx.x);  // the workspace left as a persistent launch leaves it
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.ticket = 0;
}

int idx_check_shape(const mk2_indexer_shape* s) {
  MK2_REQUIRE(s != nullptr, "indexer: shape is NULL");
  MK2_REQUIRE(s->rows >= 1 && s->rows <= 32, "indexer: rows must be in [1, 32], got %d", s->rows);
  MK2_REQUIRE(s->heads >= 16 && s->heads <= 64 && s->heads % 16 == 0,
              "indexer: heads must be 16, 32, 48 or 64, got %d", s->heads);
  MK2_REQUIRE(s->dim == 128, "indexer: dim must be 128, got %d", s->dim);
  MK2_REQUIRE(s->topk >= 64 && s->topk <= 4096 && s->topk % 64 == 0,
              "indexer: topk must be a multiple of 64 in [64, 4096], got %d", s->topk);
  MK2_REQUIRE(s->max_ctx >= 64 && s->max_ctx <= TOPK_MAXN && s->max_ctx % 64 == 0,
              "indexer: max_ctx must be a multiple of 64 in [64, %d], got %d", TOPK_MAXN, s->max_ctx);
  MK2_REQUIRE(s->table_stride >= s->max_ctx / 64, "indexer: table_stride %d < max_ctx / 64", s->table_stride);
  MK2_REQUIRE(s->key_fmt == MK2_KEYS_FP4 || s->key_fmt == MK2_KEYS_FP8 || s->key_fmt == MK2_KEYS_FP4_Q4,
              "indexer: key_fmt must be MK2_KEYS_FP4, MK2_KEYS_FP8 or MK2_KEYS_FP4_Q4, got %d", s->key_fmt);
  return MK2_OK;
}

// workspace: scores, top-k lists (used when the caller gives none), row histograms (fine, coarse),
// chunk counts, bin-b1 candidates, the slices' ticket
size_t idx_carve(const mk2_indexer_shape* s, void* base, IdxDev* d) {
  Carver c(base);
  const int nchk = (s->max_ctx + IDX_CHUNK - 1) / IDX_CHUNK;
  float* sc = c.take<float>((size_t)s->rows * s->max_ctx);
  int* tk = c.take<int>((size_t)s->rows * s->topk);
  int* hist = c.take<int>((size_t)s->rows * IDX_BINS);
  int* chist = c.take<int>((size_t)s->rows * IDX_CBINS);
  int* cnt = c.take<int>((size_t)s->rows * nchk);
  uint2* cand = c.take<uint2>((size_t)s->rows * s->max_ctx);
  int* ticket = c.take<int>(1);
  if (d) {
    if (!d->scores) d->scores = sc;
    if (!d->out) d->out = tk;
    d->hist = hist;
    d->chist = chist;
    d->ccount = cnt;
    d->cand = cand;
    d->ticket = ticket;
  }
  return c.bytes();
}

int idx_fill(const mk2_indexer_args* a, IdxDev* d) {
  int rc = idx_check_shape(&a->shape);
  if (rc) return rc;
  MK2_REQUIRE(a->q && a->w && a->cache && a->page_table && a->req_ids && a->ctx_len,
              "indexer: q, w, cache, page_table, req_ids and ctx_len must be set");
  if (a->shape.key_fmt != MK2_KEYS_FP8)
    MK2_REQUIRE(a->cache_scale != nullptr, "indexer: the FP4 index plane needs cache_scale");
  else
    MK2_REQUIRE(a->cache_scale == nullptr, "indexer: the FP8 index cache holds its scales; cache_scale must be NULL");
  *d = IdxDev{};
  d->rows = a->shape.rows; d->heads = a->shape.heads; d->topk = a->shape.topk;
  d->max_ctx = a->shape.max_ctx; d->stride = a->shape.table_stride;
  d->q = (const bf16_t*)a->q; d->w = (const bf16_t*)a->w; d->cache = a->cache;
  d->cscale = a->cache_scale; d->kfmt = a->shape.key_fmt;
  d->pt = a->page_table; d->req = a->req_ids; d->ctx = a->ctx_len;
  d->scores = a->scores; d->out = a->topk; d->keep_list = 1;
  d->scores_out = a->scores != nullptr;
  d->nchk = (d->max_ctx + IDX_CHUNK - 1) / IDX_CHUNK;
  return MK2_OK;
}

int k2_block_enqueue(int blk, const IdxDev* idx, const MlaDev* mla, const MoeDev* moe, int* sync, int rows,
                     hipStream_t st);
constexpr size_t BLOCK_SYNC_BYTES = (size_t)SYNC_INTS * 4;  // the persistent launch's sync block

// the layer's staged mode: one kernel a stage, in stream order
void idx_enqueue(const IdxDev& d, hipStream_t st) {
  k_idx_clear<<<d.rows * 4, 256, 0, st>>>(d);
  k_idx_score<<<dim3(d.nchk, d.rows), IDX_NT, 0, st>>>(d);
  k_idx_slice<<<dim3(d.nchk, d.rows), IDX_NT, 0, st>>>(d);
  k_idx_select<<<d.rows, TOPK_NT, 0, st>>>(d);
}

}  // namespace mk2

using namespace mk2;

extern "C" int mk2_indexer_workspace_bytes(const mk2_indexer_shape* shape, size_t* bytes) {
  clear_error();
  int rc = idx_check_shape(shape);
  if (rc) return rc;
  MK2_REQUIRE(bytes != nullptr, "indexer: bytes is NULL");
  *bytes = BLOCK_SYNC_BYTES + idx_carve(shape, nullptr, nullptr);
  return MK2_OK;
}

extern "C" int mk2_indexer_topk_launch(const mk2_indexer_args* a, mk2_stream_t stream) {
  clear_error();
  MK2_REQUIRE(a != nullptr, "indexer: args is NULL");
  IdxDev d;
  int rc = idx_fill(a, &d);
  if (rc) return rc;
  const size_t need = BLOCK_SYNC_BYTES + idx_carve(&a->shape, nullptr, nullptr);
  MK2_REQUIRE(a->workspace != nullptr, "indexer: workspace is NULL");
  if (a->workspace_bytes < need)
    return set_error(MK2_ENOSPACE, "indexer: workspace has %zu bytes, needs %zu", a->workspace_bytes, need);
  idx_carve(&a->shape, (char*)a->workspace + BLOCK_SYNC_BYTES, &d);
  return k2_block_enqueue(0 /* indexer */, &d, nullptr, nullptr, (int*)a->workspace, d.rows, (hipStream_t)stream);
}
