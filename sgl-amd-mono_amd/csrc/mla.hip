// Sparse-MLA launch (16 heads, 512 + 64 latent dims): split attention, merge + W_UV,
// W_o + residual -- as one persistent launch (k2_persistent.hip) for
// mk2_sparse_mla_launch, and as one kernel a stage for the layer's staged mode.
#include "indexer_stages.h"
#include "mk2_host.h"
#include "mla_stages.h"
#include "moe_stages.h"

namespace mk2 {

__global__ __launch_bounds__(MLA_NT) void k_mla_split(MlaDev p) {
  __shared__ MlaSplitLds L;
  mla_split<MLA_NT>(p, blockIdx.y, blockIdx.x, L, TagPoll{0u, 0, nullptr});
}
// merge + W_UV and W_o run 512 threads, as in the persistent layer kernel: the same
// waves split the same sums, so both paths give the same bits
constexpr int MLA_NT2 = 512;
__global__ __launch_bounds__(MLA_NT2) void k_mla_merge_uv(MlaDev p) {
  __shared__ MlaMergeLds L;
  mla_merge_uv<MLA_NT2>(p, blockIdx.y, 1, blockIdx.x >> 1, blockIdx.x & 1, L);
}
template <int NCG>
__global__ __launch_bounds__(MLA_NT2) void k_mla_oproj(MlaDev p) {
  __shared__ float red[(MLA_NT2 / 64) * NCG * 64 * 4];
  mla_oproj<MLA_NT2, NCG>(p, blockIdx.x, -1, red);
}

int mla_check_shape(const mk2_mla_shape* s) {
  MK2_REQUIRE(s != nullptr, "mla: shape is NULL");
  MK2_REQUIRE(s->rows >= 1 && s->rows <= 32, "mla: rows must be in [1, 32], got %d", s->rows);
  MK2_REQUIRE(s->heads == 16 && s->kv_lora == 512 && s->rope == 64,
              "mla: the kernels serve 16 heads of 512 + 64 latent dims");
  MK2_REQUIRE(s->v_dim >= 16 && s->v_dim % 16 == 0 && (s->heads * s->v_dim) % 128 == 0 && s->v_dim <= 512,
              "mla: v_dim must be a multiple of 16 (heads * v_dim a multiple of 128), got %d", s->v_dim);
  MK2_REQUIRE(s->hidden >= 16 && s->hidden % 16 == 0, "mla: hidden must be a multiple of 16, got %d", s->hidden);
  MK2_REQUIRE(s->topk >= 64 && s->topk % 64 == 0 && s->topk <= 65536, "mla: topk must be a multiple of 64, got %d", s->topk);
  MK2_REQUIRE(s->table_stride >= 1, "mla: table_stride must be positive");
  MK2_REQUIRE(s->sm_scale > 0.f, "mla: sm_scale must be positive");
  return MK2_OK;
}

size_t mla_carve(const mk2_mla_shape* s, void* base, MlaDev* d) {
  Carver c(base);
  const int ns = s->topk / MLA_SPLIT;
  bf16_t* po = c.take<bf16_t>((size_t)s->rows * ns * MLA_HEADS * MLA_LAT);
  float* pml = c.take<float>((size_t)s->rows * ns * MLA_HEADS * 2);
  bf16_t* o = c.take<bf16_t>((size_t)s->rows * MLA_HEADS * s->v_dim);
  if (d) { d->part_o = po; d->part_ml = pml; d->o = o; d->nsplit = ns; }
  return c.bytes();
}

int mla_fill(const mk2_mla_args* a, MlaDev* d) {
  const mk2_mla_shape* s = &a->shape;
  int rc = mla_check_shape(s);
  if (rc) return rc;
  MK2_REQUIRE(a->q && a->kv && a->page_table && a->req_ids && a->w_uv && a->w_o,
              "mla: q, kv, page_table, req_ids, w_uv and w_o must be set");
  *d = MlaDev{};
  d->rows = s->rows; d->v_dim = s->v_dim; d->hidden = s->hidden; d->topk = s->topk;
  d->stride = s->table_stride; d->sm_scale = s->sm_scale;
  d->q = (const bf16_t*)a->q; d->kv = a->kv; d->kv_scale = a->kv_scale; d->pt = a->page_table;
  d->req = a->req_ids; d->sel = a->sel; d->w_uv = (const bf16_t*)a->w_uv;
  d->w_o = (const uint8_t*)a->w_o; d->h = (const bf16_t*)a->h; d->out = (bf16_t*)a->out;
  d->o_lat_f32 = a->o_latent;
  return MK2_OK;
}

int k2_block_enqueue(int blk, const IdxDev* idx, const MlaDev* mla, const MoeDev* moe, int* sync, int rows,
                     hipStream_t st);
constexpr size_t BLOCK_SYNC_BYTES = (size_t)SYNC_INTS * 4;  // the persistent launch's sync block

// the layer's staged mode: one kernel a stage, in stream order
void mla_enqueue(const MlaDev& d, hipStream_t st) {
  k_mla_split<<<dim3(d.nsplit, d.rows), MLA_NT, 0, st>>>(d);
  k_mla_merge_uv<<<dim3(2 * MLA_HEADS, d.rows), MLA_NT2, 0, st>>>(d);
  if (d.rows > 16) k_mla_oproj<2><<<d.hidden / 16, MLA_NT2, 0, st>>>(d);
  else k_mla_oproj<1><<<d.hidden / 16, MLA_NT2, 0, st>>>(d);
}

}  // namespace mk2

using namespace mk2;

extern "C" int mk2_mla_workspace_bytes(const mk2_mla_shape* shape, size_t* bytes) {
  clear_error();
  int rc = mla_check_shape(shape);
  if (rc) return rc;
  MK2_REQUIRE(bytes != nullptr, "mla: bytes is NULL");
  *bytes = BLOCK_SYNC_BYTES + mla_carve(shape, nullptr, nullptr);
  return MK2_OK;
}

extern "C" int mk2_sparse_mla_launch(const mk2_mla_args* a, mk2_stream_t stream) {
  clear_error();
  MK2_REQUIRE(a != nullptr, "mla: args is NULL");
  MlaDev d;
  int rc = mla_fill(a, &d);
  if (rc) return rc;
  MK2_REQUIRE(a->sel && a->out && a->workspace, "mla: sel, out and workspace must be set");
  MK2_REQUIRE(a->out != a->h, "mla: out must not alias h");
  const size_t need = BLOCK_SYNC_BYTES + mla_carve(&a->shape, nullptr, nullptr);
  if (a->workspace_bytes < need)
    return set_error(MK2_ENOSPACE, "mla: workspace has %zu bytes, needs %zu", a->workspace_bytes, need);
  mla_carve(&a->shape, (char*)a->workspace + BLOCK_SYNC_BYTES, &d);
  return k2_block_enqueue(1 /* mla */, nullptr, &d, nullptr, (int*)a->workspace, d.rows, (hipStream_t)stream);
}
