// The step tables: a step's per-row tables, built from SGLang's rows in one small
// launch before the layer stack (reference: glm53/tables.py:26-131 step_rows, and
// write_seed, :134-167), so that a captured step needs no host work.
//
// Row s < S (SGLang's rows) takes its MLA slot from out_cache_loc (0, SGLang's padding
// slot, marks a pad row: slot -1), its position clamped to max_position, request row
// s, and keys indptr[s] ..< indptr[s + 1]: min(position + 1, K) for a row with a slot;
// with a seed (a draft step that reuses a top-k: int32 [S][K] positions, -1 unused),
// the seed row's valid entries, compacted in order into topk.  Rows S ..< W are pad
// rows.  ctx_len, the layer's per-row key count for its indexer, is position + 1 for a
// row with a slot and 0 for a pad row.
//
// One workgroup a row: each counts the valid seed entries of every row before its
// own (wave ballots into LDS) for its start in topk, then compacts its own row with a
// block-wide prefix sum.  Workgroup 0 also writes indptr.
#include "mk2_device.h"
#include "mk2_host.h"

namespace mk2 {

constexpr int STEP_NT = 1024;
constexpr int STEP_MAXW = 32;

struct StepDev {
  int W, S, K, by_position, ids_bytes;
  long long max_position;
  const long long* loc;
  long long loc_stride;
  const long long* pos;
  long long pos_stride;
  const void* ids_in;
  long long ids_stride;
  const int* seed;
  long long seed_stride;
  long long* slots;
  long long* positions;
  int* indptr;
  int* req_ids;
  int* topk;
  int* ids;
  int* ctx_len;
};

__global__ __launch_bounds__(STEP_NT) void k_step_rows(StepDev p) {
  __shared__ int cnt[STEP_MAXW];
  __shared__ int wsum[STEP_NT / 64];
  const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool compact = p.seed && !p.by_position;
  if (tid < STEP_MAXW) cnt[tid] = 0;
  __syncthreads();
  // the rows' liveness and positions (uniform loads: every thread reads the same words)
  auto live_of = [&](int r) { return r < p.S && p.loc[(long long)r * p.loc_stride] != 0; };
  auto pos_of = [&](int r) {
    const long long q = r < p.S ? p.pos[(long long)r * p.pos_stride] : 0;
    return q < p.max_position ? q : p.max_position;
  };
  // the rows' key counts this workgroup needs: with a compacted seed the valid entries
  // of rows < s (all rows on workgroup 0, which writes indptr)
  const int upto = s == 0 ? p.W : s;
  if (compact) {
    for (int r = 0; r < upto; ++r) {
      if (!live_of(r)) continue;
      const int* row = p.seed + (long long)r * p.seed_stride;
      int c = 0;  // lane 0: the wave's valid entries
      for (int j = tid; j < p.K; j += STEP_NT) c += __popcll(__ballot(row[j] >= 0));
      if (lane == 0 && c) atomicAdd(&cnt[r], c);
    }
  } else if (tid < p.W) {  // every row (by position, a row copies its own count)
    const long long q = pos_of(tid) + 1;
    cnt[tid] = live_of(tid) ? (int)(q < p.K ? q : p.K) : 0;
  }
  __syncthreads();
  int start = 0;
  for (int r = 0; r < s; ++r) start += cnt[r];
  if (s == 0 && tid <= p.W) {
    int e = 0;
    for (int r = 0; r < tid; ++r) e += cnt[r];
    p.indptr[tid] = e;
  }
  const bool live = live_of(s), in_step = s < p.S;
  const long long q = pos_of(s);
  if (tid == 0) {
    p.slots[s] = live ? p.loc[(long long)s * p.loc_stride] : -1;
    p.positions[s] = in_step ? q : 0;
    p.req_ids[s] = in_step ? s : 0;
    if (p.ctx_len) p.ctx_len[s] = live ? (int)(q + 1) : 0;
    if (p.ids) {
      long long tok = -1;
      if (in_step)
        tok = p.ids_bytes == 8 ? ((const long long*)p.ids_in)[(long long)s * p.ids_stride]
                               : ((const int*)p.ids_in)[(long long)s * p.ids_stride];
      p.ids[s] = (int)tok;
    }
  }
  if (!p.seed || !live) return;
  const int* row = p.seed + (long long)s * p.seed_stride;
  if (p.by_position) {
    const int n = cnt[s];
    for (int j = tid; j < n; j += STEP_NT) p.topk[start + j] = row[j];
    return;
  }
  // compaction in entry order: thread t holds entries j = t * E .. t * E + E - 1
  constexpr int EMAX = 4;  // K <= STEP_NT * EMAX
  const int E = (p.K + STEP_NT - 1) / STEP_NT;
  int v[EMAX], mine = 0;
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    const int j = tid * E + e;
    v[e] = (e < E && j < p.K) ? row[j] : -1;
    mine += v[e] >= 0;
  }
  // exclusive prefix of `mine` over the block: a wave scan, then the waves' totals
  int incl = mine;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < wave; ++w) before += wsum[w];
  int dst = start + before + incl - mine;
#pragma unroll
  for (int e = 0; e < EMAX; ++e)
    if (v[e] >= 0) p.topk[dst++] = v[e];
}

// seed row s := the keys of step row rows_of[s] (topk[indptr[src] ..< indptr[src + 1]]),
// then -1 up to K
__global__ __launch_bounds__(256) void k_write_seed(const int* topk, const int* indptr, int* seed,
                                                    long long seed_stride, const int* rows_of, int K) {
  const int s = blockIdx.x;
  const int src = rows_of[s];
  const int a = indptr[src], n = indptr[src + 1] - a;
  for (int j = threadIdx.x; j < K; j += 256) seed[(long long)s * seed_stride + j] = j < n ? topk[a + j] : -1;
}

}  // namespace mk2

using namespace mk2;

extern "C" int mk2_step_rows_launch(const mk2_step_args* a, mk2_stream_t stream) {
  clear_error();
  MK2_REQUIRE(a != nullptr, "step: args is NULL");
  MK2_REQUIRE(a->width >= 1 && a->width <= STEP_MAXW, "step: width must be in [1, %d], got %d", STEP_MAXW,
              a->width);
  MK2_REQUIRE(a->rows >= 0 && a->rows <= a->width, "step: rows must be in [0, width], got %d", a->rows);
  MK2_REQUIRE(a->topk >= 1 && a->topk <= 4 * STEP_NT, "step: topk must be in [1, %d], got %d", 4 * STEP_NT,
              a->topk);
  MK2_REQUIRE(a->max_position >= 0, "step: max_position must be >= 0");
  MK2_REQUIRE(a->slots && a->positions_out && a->indptr && a->req_ids,
              "step: slots, positions_out, indptr and req_ids must be set");
  MK2_REQUIRE(a->rows == 0 || (a->out_cache_loc && a->positions), "step: out_cache_loc and positions must be set");
  MK2_REQUIRE(!a->seed || a->topk_out, "step: a seed needs topk_out");
  MK2_REQUIRE(!a->ids || a->ids_in, "step: ids needs ids_in");
  MK2_REQUIRE(!a->ids_in || a->ids_in_bytes == 4 || a->ids_in_bytes == 8, "step: ids_in_bytes must be 4 or 8");
  StepDev d;
  d.W = a->width; d.S = a->rows; d.K = a->topk; d.by_position = a->seed_by_position;
  d.ids_bytes = a->ids_in_bytes; d.max_position = a->max_position;
  d.loc = (const long long*)a->out_cache_loc; d.loc_stride = a->loc_stride;
  d.pos = (const long long*)a->positions; d.pos_stride = a->pos_stride;
  d.ids_in = a->ids_in; d.ids_stride = a->ids_stride;
  d.seed = a->seed; d.seed_stride = a->seed_stride;
  d.slots = (long long*)a->slots; d.positions = (long long*)a->positions_out;
  d.indptr = a->indptr; d.req_ids = a->req_ids; d.topk = a->topk_out; d.ids = a->ids; d.ctx_len = a->ctx_len;
  k_step_rows<<<a->width, STEP_NT, 0, (hipStream_t)stream>>>(d);
  return check_launch("step rows");
}

extern "C" int mk2_write_seed_launch(const int32_t* topk, const int32_t* indptr, int32_t* seed,
                                     int64_t seed_stride, const int32_t* rows_of, int rows, int k,
                                     mk2_stream_t stream) {
  clear_error();
  MK2_REQUIRE(topk && indptr && seed && rows_of, "write_seed: topk, indptr, seed and rows_of must be set");
  MK2_REQUIRE(rows >= 0 && k >= 1 && seed_stride >= k, "write_seed: rows >= 0, k >= 1 and seed_stride >= k");
  if (rows == 0) return MK2_OK;
  k_write_seed<<<rows, 256, 0, (hipStream_t)stream>>>(topk, indptr, seed, seed_stride, rows_of, k);
  return check_launch("write seed");
}
