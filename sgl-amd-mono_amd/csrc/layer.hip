// The chained K2 layer: indexer scores -> exact top-k -> sparse MLA -> W_UV -> W_o +
// residual -> RMSNorm -> router -> top-k routing -> up/gate -> down + residual, as
// one persistent launch (k2_persistent.hip) or as one kernel a stage.
#include <mutex>

#include "front_stages.h"
#include "indexer_stages.h"
#include "mla_stages.h"
#include "mk2_host.h"
#include "moe_stages.h"

namespace mk2 {

int idx_fill(const mk2_indexer_args* a, IdxDev* d);
size_t idx_carve(const mk2_indexer_shape* s, void* base, IdxDev* d);
void idx_enqueue(const IdxDev& d, hipStream_t st);
int mla_fill(const mk2_mla_args* a, MlaDev* d);
size_t mla_carve(const mk2_mla_shape* s, void* base, MlaDev* d);
void mla_enqueue(const MlaDev& d, hipStream_t st);
int moe_fill(const mk2_moe_args* a, MoeDev* d);
size_t moe_carve(const mk2_moe_shape* s, void* base, MoeDev* d);
int moe_enqueue(const MoeDev& d, hipStream_t st);
int k2_persistent_enqueue(const IdxDev& idx, const MlaDev& mla, const MoeDev& moe, int* sync,
                          int* status, uint64_t* timeline, int rows, uint32_t wait_ticks, hipStream_t st,
                          const FrontPDev* front = nullptr, int front_key = 0);
int front_pdev(const mk2_front_args* a, FrontPDev* d, int* key);

constexpr int LAYER_SYNC_BYTES = SYNC_INTS * 4;  // the persistent launch's counters and its epoch

struct LayerPlan {
  IdxDev idx;
  MlaDev mla;
  MoeDev moe;
  int* sync;
  size_t moe_off;  // the MoE block's workspace, bytes from the layer workspace's start
};

// validate the three blocks against each other and carve one workspace for all
int layer_plan(const mk2_layer_args* a, void* ws, LayerPlan* L, size_t* bytes) {
  MK2_REQUIRE(a != nullptr, "layer: args is NULL");
  const mk2_indexer_shape& is = a->indexer.shape;
  const mk2_mla_shape& ms = a->mla.shape;
  const mk2_moe_shape& es = a->moe.shape;
  MK2_REQUIRE(is.rows == ms.rows && ms.rows == es.rows, "layer: rows differ between blocks (%d, %d, %d)",
              is.rows, ms.rows, es.rows);
  MK2_REQUIRE(is.topk == ms.topk, "layer: indexer topk %d != attention topk %d", is.topk, ms.topk);
  MK2_REQUIRE(ms.hidden == es.hidden, "layer: attention hidden %d != MoE hidden %d", ms.hidden, es.hidden);
  MK2_REQUIRE(es.norm == 1 && es.residual == 1, "layer: the MoE block runs with norm=1 and residual=1");
  int rc = idx_fill(&a->indexer, &L->idx);
  if (rc) return rc;
  rc = mla_fill(&a->mla, &L->mla);
  if (rc) return rc;
  MK2_REQUIRE(a->mla.h != nullptr, "layer: the attention residual h must be set");
  // the MoE input is the attention output; give moe_fill a stand-in to validate
  mk2_moe_args ma = a->moe;
  ma.x = (const void*)1;
  ma.out = (void*)2;
  rc = moe_fill(&ma, &L->moe);
  if (rc) return rc;
  MK2_REQUIRE(a->mode == MK2_LAYER_PERSISTENT || a->mode == MK2_LAYER_STAGED, "layer: unknown mode %d", a->mode);
  MK2_REQUIRE(a->wait_us >= 0 && a->wait_us <= MK2_MAX_WAIT_US, "layer: wait_us must be in [0, %d], got %d",
              MK2_MAX_WAIT_US, a->wait_us);
  Carver c(ws);
  int* sync = c.take<int>(LAYER_SYNC_BYTES / 4);
  const size_t b_idx = idx_carve(&is, nullptr, nullptr);
  const size_t b_mla = mla_carve(&ms, nullptr, nullptr);
  const size_t b_moe = moe_carve(&es, nullptr, nullptr);
  char* p_idx = c.take<char>(b_idx);
  char* p_mla = c.take<char>(b_mla);
  char* p_moe = c.take<char>(b_moe);
  L->moe_off = c.used - b_moe;
  bf16_t* attn = c.take<bf16_t>((size_t)ms.rows * ms.hidden);
  uint64_t* tlist = c.take<uint64_t>((size_t)is.rows * is.topk);  // the list as tagged words
  *bytes = c.bytes();
  if (!ws) return MK2_OK;
  L->sync = sync;
  idx_carve(&is, p_idx, &L->idx);
  mla_carve(&ms, p_mla, &L->mla);
  moe_carve(&es, p_moe, &L->moe);
  if (a->moe.logits) L->moe.logits = a->moe.logits;
  if (a->moe.topk_ids) L->moe.topk_ids = a->moe.topk_ids;
  if (a->moe.topk_weights) L->moe.topk_w = a->moe.topk_weights;
  L->mla.sel = L->idx.out;
  // every split reads the tagged list: the int list only for a caller that asked for it
  L->idx.keep_list = a->indexer.topk != nullptr;
  L->idx.tlist = tlist;
  L->mla.tsel = tlist;
  bf16_t* a_out = a->attn_out ? (bf16_t*)a->attn_out : attn;
  L->mla.out = a_out;
  L->moe.x = a_out;
  L->mla.ssp = L->moe.norm ? L->moe.ssp : nullptr;  // W_o leaves the RMSNorm's partial sums
  L->moe.out = (bf16_t*)a->out;
  return MK2_OK;
}

// ------------------------------------------------------ allocation-free entry point
// The layer's scratch as a file-scope device array, for callers that cannot allocate
// (code under HIP graph capture, serving loops and harnesses that forbid hipMalloc).
// Every GPU the library runs on holds its own copy until the process ends.  In host
// code `scratch` names a host-side stand-in, never a device address: the device
// address comes from hipGetSymbolAddress, taken once per device with that device
// current, and only that address is used (kernel arguments, the fill kernel).
static __device__ __align__(256) uint8_t scratch[MK2_LAYER_STATIC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[MAX_DEVICES];

static int static_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return set_error(MK2_ELAUNCH, "layer (static scratch): no current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return set_error(MK2_ELAUNCH, "layer (static scratch): hipGetSymbolAddress failed on device %d: %s", dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MK2_OK;
}

// zero what a launch needs zero on entry: the persistent launch's counters (not its
// epoch: the tags of the next launch must differ from those of every earlier launch
// on the array, whatever shape they had), the indexer's histograms, chunk counts and
// ticket, and every region of tagged words (the top-k list, the router's partial
// logits, the routing's picks, expert list and row masks).  The array is shared by
// calls of every shape, so a tagged region may lie on bytes that another layout left
// as plain data whose upper half happens to equal this launch's tag; cleared, a word
// matches only once its producer wrote it.  A fill kernel, so that a captured graph
// holds no memset node.
struct ZeroSpan {
  int* p;
  int n;
};
constexpr int ZERO_SPANS = 10;
struct ZeroSpans {
  ZeroSpan s[ZERO_SPANS];
};
__global__ __launch_bounds__(256) void k_layer_zero(ZeroSpans a) {
  for (int s = 0; s < ZERO_SPANS; ++s)
    for (int i = blockIdx.x * 256 + threadIdx.x; i < a.s[s].n; i += gridDim.x * 256) a.s[s].p[i] = 0;
}

}  // namespace mk2

using namespace mk2;

extern "C" int mk2_layer_launch_static(const mk2_layer_args* a, mk2_stream_t stream) {
  clear_error();
  LayerPlan L;
  size_t need = 0;
  int rc = layer_plan(a, nullptr, &L, &need);
  if (rc) return rc;
  MK2_REQUIRE(a->out != nullptr, "layer (static scratch): out must be set");
  MK2_REQUIRE(a->out != a->mla.h, "layer (static scratch): out must not alias the residual h");
  if (need > MK2_LAYER_STATIC_SCRATCH_BYTES)
    return set_error(MK2_ENOSPACE, "layer (static scratch): this shape needs %zu bytes of scratch, more than the "
                     "%zu bytes of the static array; use mk2_layer_launch with a workspace", need,
                     (size_t)MK2_LAYER_STATIC_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = static_scratch(&ws);
  if (rc) return rc;
  rc = layer_plan(a, ws, &L, &need);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  const IdxDev& x = L.idx;
  const MoeDev& m = L.moe;
  auto words = [](uint64_t* p, size_t n) { return ZeroSpan{(int*)p, (int)(2 * n)}; };
  const ZeroSpans z{{ZeroSpan{L.sync, SYNC_EPOCH}, ZeroSpan{x.hist, x.rows * IDX_BINS},
                     ZeroSpan{x.chist, x.rows * IDX_CBINS}, ZeroSpan{x.ccount, x.rows * x.nchk},
                     ZeroSpan{x.ticket, 1}, words(x.tlist, (size_t)x.rows * x.topk),
                     words(m.logit_part, (size_t)m.KC * m.M * m.E), words(m.act, (size_t)1 + m.Dmax),
                     words(m.act_rows, (size_t)m.Dmax), words(m.picks, (size_t)m.M * m.topk * 2)}};
  k_layer_zero<<<64, 256, 0, st>>>(z);
  rc = check_launch("layer (static scratch): clear");
  if (rc) return rc;
  if (a->mode == MK2_LAYER_PERSISTENT)
    return k2_persistent_enqueue(L.idx, L.mla, L.moe, L.sync, a->status, (uint64_t*)a->timeline,
                                 a->mla.shape.rows, wait_ticks_of(a->wait_us), st);
  idx_enqueue(L.idx, st);
  mla_enqueue(L.mla, st);
  return moe_enqueue(L.moe, st);
}

extern "C" int mk2_layer_workspace_bytes(const mk2_layer_args* a, size_t* bytes) {
  clear_error();
  MK2_REQUIRE(bytes != nullptr, "layer: bytes is NULL");
  LayerPlan L;
  return layer_plan(a, nullptr, &L, bytes);
}

extern "C" int mk2_layer_workspace_layout(const mk2_layer_args* a, int64_t* moe_offset) {
  clear_error();
  MK2_REQUIRE(moe_offset != nullptr, "layer: moe_offset is NULL");
  LayerPlan L;
  size_t bytes = 0;
  const int rc = layer_plan(a, nullptr, &L, &bytes);
  if (rc) return rc;
  // mk2_moe_workspace_layout's offsets count the standalone block's leading sync block
  *moe_offset = (int64_t)L.moe_off - (int64_t)SYNC_INTS * 4;
  return MK2_OK;
}

extern "C" int mk2_layer_launch(const mk2_layer_args* a, mk2_stream_t stream) {
  clear_error();
  LayerPlan L;
  size_t need = 0;
  int rc = layer_plan(a, nullptr, &L, &need);
  if (rc) return rc;
  MK2_REQUIRE(a->out && a->workspace, "layer: out and workspace must be set");
  MK2_REQUIRE(a->out != a->mla.h, "layer: out must not alias the residual h");
  if (a->workspace_bytes < need)
    return set_error(MK2_ENOSPACE, "layer: workspace has %zu bytes, needs %zu", a->workspace_bytes, need);
  rc = layer_plan(a, a->workspace, &L, &need);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (a->mode == MK2_LAYER_PERSISTENT)
    return k2_persistent_enqueue(L.idx, L.mla, L.moe, L.sync, a->status, (uint64_t*)a->timeline,
                                 a->mla.shape.rows,
                                 wait_ticks_of(a->wait_us), st);
  idx_enqueue(L.idx, st);
  mla_enqueue(L.mla, st);
  return moe_enqueue(L.moe, st);
}

extern "C" int mk2_layer_step_launch(const mk2_front_args* f, const mk2_layer_args* a, mk2_stream_t stream) {
  clear_error();
  MK2_REQUIRE(f != nullptr && a != nullptr, "layer step: front and layer args must be set");
  FrontPDev fd;
  int key = FRONT_FUSED_NONE;
  int rc = front_pdev(f, &fd, &key);
  if (rc) return rc;
  MK2_REQUIRE(key != FRONT_FUSED_NONE,
              "layer step: the front-and-layer launch has no instance for this front shape and weight format");
  LayerPlan L;
  size_t need = 0;
  rc = layer_plan(a, nullptr, &L, &need);
  if (rc) return rc;
  MK2_REQUIRE(a->mode == MK2_LAYER_PERSISTENT, "layer step: the layer runs persistent");
  MK2_REQUIRE(a->out && a->workspace, "layer: out and workspace must be set");
  MK2_REQUIRE(a->out != a->mla.h, "layer: out must not alias the residual h");
  if (a->workspace_bytes < need)
    return set_error(MK2_ENOSPACE, "layer: workspace has %zu bytes, needs %zu", a->workspace_bytes, need);
  // the front's outputs are the layer's inputs, its caches the layer's caches
  MK2_REQUIRE(f->shape.rows == a->mla.shape.rows, "layer step: front rows %d != layer rows %d", f->shape.rows,
              a->mla.shape.rows);
  MK2_REQUIRE(f->x == a->mla.h, "layer step: the front's residual rows x must be the layer's residual h");
  MK2_REQUIRE(f->mla_q == a->mla.q && f->kv_cache == a->mla.kv && f->kv_scale == a->mla.kv_scale,
              "layer step: the front's mla_q, kv_cache and kv_scale must be the layer's q, kv and kv_scale");
  MK2_REQUIRE(f->index_q == a->indexer.q && f->index_w == a->indexer.w && f->index_cache == a->indexer.cache &&
                  f->index_scale == a->indexer.cache_scale,
              "layer step: the front's index_q, index_w, index_cache and index_scale must be the indexer's q, w, "
              "cache and cache_scale");
  rc = layer_plan(a, a->workspace, &L, &need);
  if (rc) return rc;
  fd.wait_ticks = wait_ticks_of(a->wait_us);  // the front's waits share the layer's deadline
  return k2_persistent_enqueue(L.idx, L.mla, L.moe, L.sync, a->status, (uint64_t*)a->timeline, a->mla.shape.rows,
                               wait_ticks_of(a->wait_us), (hipStream_t)stream, &fd, key);
}
