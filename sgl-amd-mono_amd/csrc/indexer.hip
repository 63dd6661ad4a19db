// Standalone indexer launch (FP4 index keys, 64 heads x 128): key scores, then the exact
// top-k of every row.
#include "indexer_stages.h"
#include "mk2_host.h"

namespace mk2 {

constexpr int IDX_NT = 512;

__global__ __launch_bounds__(IDX_NT) void k_idx_score(IdxDev p) {
  __shared__ int pages[IDX_CHUNK / 64];
  idx_score<IDX_NT>(p, blockIdx.y, blockIdx.x, pages);
}

__global__ __launch_bounds__(TOPK_NT) void k_idx_topk(IdxDev p) {
  __shared__ TopkLds S;
  idx_topk<TOPK_NT>(p, blockIdx.x, S);
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
  return MK2_OK;
}

size_t idx_carve(const mk2_indexer_shape* s, void* base, float** scores, int** topk) {
  Carver c(base);
  float* sc = c.take<float>((size_t)s->rows * s->max_ctx);
  int* tk = c.take<int>((size_t)s->rows * s->topk);
  if (scores) *scores = sc;
  if (topk) *topk = tk;
  return c.bytes();
}

int idx_fill(const mk2_indexer_args* a, IdxDev* d) {
  int rc = idx_check_shape(&a->shape);
  if (rc) return rc;
  MK2_REQUIRE(a->q && a->w && a->cache && a->page_table && a->req_ids && a->ctx_len,
              "indexer: q, w, cache, page_table, req_ids and ctx_len must be set");
  *d = IdxDev{};
  d->rows = a->shape.rows; d->heads = a->shape.heads; d->topk = a->shape.topk;
  d->max_ctx = a->shape.max_ctx; d->stride = a->shape.table_stride;
  d->q = (const bf16_t*)a->q; d->w = (const bf16_t*)a->w; d->cache = a->cache;
  d->pt = a->page_table; d->req = a->req_ids; d->ctx = a->ctx_len;
  d->scores = a->scores; d->out = a->topk;
  return MK2_OK;
}

void idx_enqueue(const IdxDev& d, hipStream_t st) {
  const int chunks = (d.max_ctx + IDX_CHUNK - 1) / IDX_CHUNK;
  k_idx_score<<<dim3(chunks, d.rows), IDX_NT, 0, st>>>(d);
  k_idx_topk<<<d.rows, TOPK_NT, 0, st>>>(d);
}

}  // namespace mk2

using namespace mk2;

extern "C" int mk2_indexer_workspace_bytes(const mk2_indexer_shape* shape, size_t* bytes) {
  clear_error();
  int rc = idx_check_shape(shape);
  if (rc) return rc;
  MK2_REQUIRE(bytes != nullptr, "indexer: bytes is NULL");
  *bytes = idx_carve(shape, nullptr, nullptr, nullptr);
  return MK2_OK;
}

extern "C" int mk2_indexer_topk_launch(const mk2_indexer_args* a, mk2_stream_t stream) {
  clear_error();
  MK2_REQUIRE(a != nullptr, "indexer: args is NULL");
  IdxDev d;
  int rc = idx_fill(a, &d);
  if (rc) return rc;
  if (!d.scores || !d.out) {
    const size_t need = idx_carve(&a->shape, nullptr, nullptr, nullptr);
    MK2_REQUIRE(a->workspace != nullptr, "indexer: scores/topk not given and no workspace");
    if (a->workspace_bytes < need)
      return set_error(MK2_ENOSPACE, "indexer: workspace has %zu bytes, needs %zu", a->workspace_bytes, need);
    float* sc;
    int* tk;
    idx_carve(&a->shape, a->workspace, &sc, &tk);
    if (!d.scores) d.scores = sc;
    if (!d.out) d.out = tk;
  }
  idx_enqueue(d, (hipStream_t)stream);
  return check_launch("indexer");
}
