// The K2 layer as ONE persistent launch: one 512-thread workgroup per CU walks the
// stage list -- index scores, exact top-k, sparse-MLA splits, merge, W_UV, W_o +
// residual, RMSNorm + activation quant, router, top-k routing, up/gate + SwiGLU,
// down + residual -- taking task t of a stage when t = workgroup (mod grid).
//
// There is no grid barrier.  A task that needs the results of earlier tasks waits
// on a per-stage completion counter in the workspace (only for the producers it
// reads: e.g. row r's top-k waits for row r's 32 score chunks).  A producer
// publishes with a workgroup barrier, an agent-scope release fence and an atomic
// increment; a consumer polls the counter, then takes an agent-scope acquire fence.
// Dependencies point only to earlier stages and every workgroup is resident (one
// per CU, grid = CU count), so every wait ends; each wait is also bounded (spin
// limit) and on expiry sets a sticky error word that releases every other wait, so
// the launch always drains.  The last workgroup to finish resets the counters.
#include "indexer_stages.h"
#include "mk2_host.h"
#include "mla_stages.h"
#include "moe_stages.h"

namespace mk2 {

constexpr int K2_NT = 512;

// sync block (int words at the start of the layer workspace)
enum : int {
  SY_SCORE = 0,   // [32] score chunks done, per row
  SY_TOPK = 32,   // [32] top-k done, per row
  SY_SPLIT = 64,  // [32] attention splits done, per row
  SY_MERGE = 96,  // [16] merged rows, per head
  SY_UV = 112,
  SY_OPROJ,
  SY_PREP,
  SY_ROUTER,
  SY_ROUTE,
  SY_UP,
  SY_DONE,        // workgroups finished (the last one resets)
  SY_ERR,         // sticky: a wait ran out of its spin limit
  SY_WORDS = 128
};

struct K2Dev {
  IdxDev idx;
  MlaDev mla;
  MoeDev moe;
  int* sync;
  int* status;    // optional: the launch's error word
  int rows;
  int spin_limit;
};

union K2Lds {
  int pages[IDX_CHUNK / 64];
  TopkLds topk;
  MlaSplitLds split;
  float merge[2 * 1024 + 8];
  struct {
    float red[(K2_NT / 64) * 4 * 2 * 64 * 4];
    float midf[32 * 33];
  } up;
  struct {
    float red[(K2_NT / 64) * 2 * 64 * 4];
    int act[256];
  } down;
  struct {
    float logits[32 * 256];
    int slot[256 + 4 * (K2_NT / 64) + 24 * (K2_NT / 64)];
  } route;
  float red[(K2_NT / 64) * 2 * 64 * 4];
};

MK2_DEV void k2_signal(int* c) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    atomicAdd(c, 1);
  }
}

MK2_DEV void k2_wait(const K2Dev& p, int slot, int target) {
  if (threadIdx.x == 0) {
    const int* c = p.sync + slot;
    int* err = p.sync + SY_ERR;
    int n = 0;
    while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
      if (++n > p.spin_limit) {
        atomicOr(err, 1);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
}

template <int NCG>
__global__ __launch_bounds__(K2_NT, 1) void k_k2_layer(K2Dev p) {
  __shared__ K2Lds S;
  const int G = gridDim.x, b = blockIdx.x;
  const int R = p.rows;
  // ---- index scores
  const int nchk = (p.idx.max_ctx + IDX_CHUNK - 1) / IDX_CHUNK;
  for (int t = b; t < R * nchk; t += G) {
    idx_score<K2_NT>(p.idx, t / nchk, t % nchk, S.pages);
    k2_signal(p.sync + SY_SCORE + t / nchk);
  }
  // ---- exact top-k of each row
  for (int t = b; t < R; t += G) {
    k2_wait(p, SY_SCORE + t, nchk);
    idx_topk<K2_NT>(p.idx, t, S.topk);
    k2_signal(p.sync + SY_TOPK + t);
  }
  // ---- sparse-MLA splits
  const int ns = p.mla.nsplit;
  for (int t = b; t < R * ns; t += G) {
    const int r = t / ns;
    k2_wait(p, SY_TOPK + r, 1);
    mla_split<K2_NT>(p.mla, r, t % ns, S.split);
    k2_signal(p.sync + SY_SPLIT + r);
  }
  // ---- merge of the splits, per (row, head)
  for (int t = b; t < R * MLA_HEADS; t += G) {
    const int r = t / MLA_HEADS, h = t % MLA_HEADS;
    k2_wait(p, SY_SPLIT + r, ns);
    mla_merge<K2_NT>(p.mla, r, h, S.merge);
    k2_signal(p.sync + SY_MERGE + h);
  }
  // ---- W_UV, per (head, 16 v rows)
  const int vtn = p.mla.v_dim / 16;
  for (int t = b; t < MLA_HEADS * vtn; t += G) {
    const int h = t / vtn;
    k2_wait(p, SY_MERGE + h, R);
    mla_uv<K2_NT, NCG>(p.mla, h, t % vtn, S.red);
    k2_signal(p.sync + SY_UV);
  }
  // ---- W_o + residual, per 16 hidden rows
  const int ht = p.mla.hidden / 16;
  for (int t = b; t < ht; t += G) {
    k2_wait(p, SY_UV, MLA_HEADS * vtn);
    mla_oproj<K2_NT, NCG>(p.mla, t, S.red);
    k2_signal(p.sync + SY_OPROJ);
  }
  // ---- RMSNorm + activation quant, per row
  for (int t = b; t < R; t += G) {
    k2_wait(p, SY_OPROJ, ht);
    moe_prep<K2_NT>(p.moe, t, S.red);
    k2_signal(p.sync + SY_PREP);
  }
  // ---- router GEMV, per (16 experts, k-chunk)
  const int et = p.moe.E / 16, nrt = et * p.moe.KC;
  for (int t = b; t < nrt; t += G) {
    k2_wait(p, SY_PREP, R);
    moe_router<K2_NT, NCG>(p.moe, t % et, t / et, S.red);
    k2_signal(p.sync + SY_ROUTER);
  }
  // ---- top-k routing (one task)
  for (int t = b; t < 1; t += G) {
    k2_wait(p, SY_ROUTER, nrt);
    moe_route<K2_NT>(p.moe, S.route.logits, S.route.slot);
    k2_signal(p.sync + SY_ROUTE);
  }
  // ---- up/gate + SwiGLU: routed slots (after routing), then the shared expert
  const int up_r = p.moe.Dmax * (p.moe.I / 32);
  const int up_total = up_r + p.moe.n_shared * (p.moe.SI / 32);
  for (int t = b; t < up_total; t += G) {
    if (t < up_r) k2_wait(p, SY_ROUTE, 1);
    else k2_wait(p, SY_PREP, R);
    moe_upgate<K2_NT, NCG>(p.moe, t, S.up.red, S.up.midf);
    k2_signal(p.sync + SY_UP);
  }
  // ---- down + route weighting + residual, per 16 hidden rows
  for (int t = b; t < p.moe.H / 16; t += G) {
    k2_wait(p, SY_UP, up_total);
    moe_down<K2_NT, NCG>(p.moe, t, S.down.red, S.down.act);
  }
  // ---- the last workgroup out resets the counters for the next launch
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    if (atomicAdd(p.sync + SY_DONE, 1) == G - 1) {
      const int err = atomicAdd(p.sync + SY_ERR, 0);
      for (int i = 0; i < SY_DONE; ++i) atomicExch(p.sync + i, 0);
      if (p.status) *p.status = err;
      atomicExch(p.sync + SY_ERR, 0);
      atomicExch(p.sync + SY_DONE, 0);
      __threadfence();
    }
  }
}

static int g_cus = 0;

int k2_persistent_enqueue(const IdxDev& idx, const MlaDev& mla, const MoeDev& moe, int* sync,
                          int* status, int rows, int spin_limit, hipStream_t st) {
  if (g_cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&g_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || g_cus <= 0)
      return set_error(MK2_ELAUNCH, "layer: cannot query the CU count");
  }
  K2Dev p{idx, mla, moe, sync, status, rows, spin_limit};
  const bool two = rows > 16;
  int per_cu = 0;
  hipError_t e = two ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_k2_layer<2>, K2_NT, 0)
                     : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_k2_layer<1>, K2_NT, 0);
  if (e != hipSuccess || per_cu < 1)
    return set_error(MK2_ELAUNCH, "layer: the persistent kernel does not fit one workgroup per CU");
  if (two) k_k2_layer<2><<<g_cus, K2_NT, 0, st>>>(p);
  else k_k2_layer<1><<<g_cus, K2_NT, 0, st>>>(p);
  return check_launch("layer (persistent)");
}

}  // namespace mk2
