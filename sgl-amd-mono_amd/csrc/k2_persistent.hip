// The K2 layer as ONE persistent launch: one 512-thread workgroup per CU walks the
// stage list -- index scores (+ key histograms), top-k slices, top-k select,
// sparse-MLA splits, merge + W_UV, W_o + residual (+ the RMSNorm's partial sums),
// router (+ RMSNorm + activation quant of its slice), top-k routing, up/gate +
// SwiGLU, down + residual -- taking task t of a
// stage on workgroup (base + t) mod grid, where each stage's base continues from
// where the previous stage's tasks ended, so that work rotates over the workgroups.
//
// There is no grid barrier.  A task that needs the results of earlier tasks waits
// on a per-stage completion counter in the workspace (only for the producers it
// reads: e.g. row r's slices wait for row r's score chunks).  Everything handed
// from one workgroup to another is written and read with device-coherent (sc1)
// accesses, so a hand-off needs no cache maintenance: a producer drains its stores,
// passes a workgroup barrier and increments the counter (relaxed, agent scope); a
// consumer polls the counter, passes a barrier and reads.  Dependencies point only
// to earlier stages and every workgroup is resident (one per CU, grid = CU count),
// so every wait ends; each wait is also bounded (a deadline) and on expiry sets a
// sticky error word that releases every other wait, so the launch always drains.
// The last workgroup to finish resets the counters.
#include "front_stages.h"
#include "indexer_stages.h"
#include "mk2_host.h"
#include "mla_stages.h"
#include "moe_stages.h"

namespace mk2 {

constexpr int K2_NT = 512;

// The sync block at the start of the layer workspace: one counter a 128-byte line
// (counters that share a line serialize each other's atomics).  A counter with many
// producers is split into K2_LANES sub-counters on lines of their own, producer t
// adding to sub-counter t mod K2_LANES; a waiter sums them.
constexpr int SY_LINE = 32;  // ints a line
constexpr int K2_LANES = 16;
enum : int {
  SY_SCORE = 0,    // [32] score chunks done, per row
  SY_SLICE = 32,   // [32] top-k slices counted out (their counts and bin keys out), per row
  SY_UPT = 64,     // the up/gate task tickets handed out (above 16 rows)
  SY_UPW = 80,     // [K2_LANES] workgroups through the up/gate tasks (above 16 rows)
  SY_SPLIT = 96,   // [32] attention splits done, per row
  SY_ROUTE = 128,  // the routing's table and list are out (the down)
  SY_DONE = 130,   // workgroups finished (the last one resets)
  SY_ERR,          // sticky: a wait passed its deadline
  SY_UV = 144,     // [K2_LANES] sub-counters each: merged + W_UV (row group, head, half) tasks
  SY_OPROJ = SY_UV + K2_LANES,
  SY_ROUTER = SY_OPROJ + K2_LANES,
  SY_UP = SY_ROUTER + K2_LANES,
  SY_LINES = SY_UP + K2_LANES  // 208 lines = 26 KiB
};
static_assert(SY_LINES * SY_LINE <= SYNC_EPOCH, "the counters stay clear of the epoch word");

struct K2Dev {
  IdxDev idx;
  MlaDev mla;
  MoeDev moe;
  int* sync;
  int* status;    // optional: the launch's error word
  uint64_t* timeline;  // optional: [grid][K2_STAMPS] s_memrealtime stamps (100 MHz)
  int rows;
  uint32_t wait_ticks;  // a dependency wait's deadline (WaitClock ticks)
};

// timeline: per stage s, stamps 3s (enter), 3s+1 (first input ready), 3s+2 (leave);
// then the routing's marks: logits polled, top-k done, list out
constexpr int K2_STAGES = 10, K2_STAMPS = 3 * K2_STAGES + 3;

// The stamps collect in LDS (thread 0 takes them all) and go out once the walk is done:
// a store to memory per stamp would make thread 0's wave wait for its outstanding loads
// and stores at every stamp and move the times it measures.
__shared__ uint64_t k2_lds_stamps[K2_STAMPS];
MK2_DEV void k2_stamp(const K2Dev& p, int i) {
  if (p.timeline && threadIdx.x == 0) k2_lds_stamps[i] = __builtin_amdgcn_s_memrealtime();
}

union K2Lds {
  IdxScoreLds score;
  TopkLds topk;
  MlaSplitLds split;
  MlaMergeLds merge;
  struct {
    float red[(K2_NT / 64) * 8 * 64 * 4];  // NW * 2 * CT * NCG * 256, CT * NCG <= 4
    float midf[32 * 65];
  } up;
  struct {
    float red[(K2_NT / 64) * 2 * 16 * 32];  // NW * DT * NCG * 256, or NW * DT * 16 * 32
    int act[512];  // the slots' experts, then (compacted rows) their row counts
    float xres[16 * 2 * 32];
  } down;
  RouterLds router;
  RouteLds route;
  float red[(K2_NT / 64) * 2 * 64 * 4];
  FrontLds front;
};
static_assert(sizeof(FrontLds) <= sizeof(TopkLds), "the front's LDS fits the layer's union as it is");

MK2_DEV int* k2_ctr(const K2Dev& p, int line) { return p.sync + line * SY_LINE; }

// publish n finished tasks on counter `line` (sub-counter t mod lanes): every thread's
// stores drained, then one increment
MK2_DEV void k2_signal(const K2Dev& p, int line, int t = 0, int lanes = 1, int n = 1) {
  drain_memory();
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(k2_ctr(p, line + t % lanes), n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// publish one of n producers' tasks on a single counter and tell whether it completed
// the set: that workgroup runs the stage that needs all n (no further hand-off)
MK2_DEV bool k2_signal_last1(const K2Dev& p, int line, int n, int* flag) {
  drain_memory();
  __syncthreads();
  if (threadIdx.x == 0)
    *flag = __hip_atomic_fetch_add(k2_ctr(p, line), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n - 1;
  __syncthreads();
  return *flag != 0;
}

// wait until counter `line` (summed over `lanes` sub-counters) reaches `target`.  Wave
// 0 polls, one coherent load a lane a poll; the error word every 32 polls.  `seen`
// (LDS, by line) caches the counts this workgroup has observed (counters only grow
// within a launch), so a wait that an earlier one already satisfied costs nothing.  The
// early return is uniform: seen is written only just after this function's barrier,
// and every task ends with a barrier before the next wait reads it.
MK2_DEV bool k2_wait(const K2Dev& p, int* seen, int line, int target, int stamp = -1, int lanes = 1) {
  if (seen[line] >= target) return true;
  int v = 0;
  bool bad = false;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int* err = k2_ctr(p, SY_ERR);
    const int* ctr = k2_ctr(p, line + min(lane, lanes - 1));
    // two polls in flight: the next is issued before the last one's count is read
    auto poll = [&]() { return __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto count = [&](int c) {  // the sub-counters' sum (lanes < lanes <= 16: one DPP row)
      return __builtin_amdgcn_readfirstlane(row16_sum_i32(lane < lanes ? c : 0));
    };
    int n = 0, c0 = poll();
    WaitClock wc;
    while (true) {
      const int c1 = poll();
      v = count(c0);
      if (v >= target) break;
      c0 = poll();
      v = count(c1);
      if (v >= target) break;
      n += 2;
      if ((n & 31) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
        bad = true;
        break;
      }
      if (wc.expired(p.wait_ticks)) {
        if (lane == 0) atomicOr(k2_ctr(p, SY_ERR), 1);
        bad = true;
        break;
      }
    }
    if (lane == 0 && stamp >= 0 && p.timeline) k2_lds_stamps[stamp] = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) seen[SY_LINES] = bad;  // the workgroup's fail-stop flag
  }
  __syncthreads();
  const bool ok = seen[SY_LINES] == 0;
  __syncthreads();  // the flag is read before the next wait can write it
  if (threadIdx.x == 0 && ok) seen[line] = v;
  return ok;
}

// The up/gate tasks (up_total of them: the shared expert's chunks, then the routed
// slots' chunks in slot order) of this workgroup, the first at `first` (none when it
// is >= up_total).  Up to 16 rows (NCG 1) the rotation gives a workgroup every G-th
// task (a workgroup holds one or two; the layer's walk runs that loop in place).
// Above 16 rows a workgroup runs several and a task's time varies with its slot's
// rows, so after the first G the tasks go by ticket:
// a workgroup takes its next one from the SY_UPT counter as it starts the current one
// (the round trip overlaps the task) and stops at its first routed slot past the
// routing's count -- the tickets go out in task order, so every task before that one
// went to a workgroup that runs it.  Then every workgroup counts out on SY_UPW, which
// the down waits for.  `next`: an LDS int.  False: the walk is failing.
template <int NCG, int FMT>
MK2_DEV bool k2_upgate_walk(const K2Dev& p, K2Lds& S, int* seen, int* next, int first, int nrt, const TagPoll& tp,
                            int stamp) {
  constexpr bool ticket = NCG == 2;
  const int G = gridDim.x;
  const int up_r = p.moe.Dmax * (p.moe.I / p.moe.UC);
  const int up_sh = p.moe.n_shared * (p.moe.SI / 32);
  const int up_total = up_r + up_sh;
  for (int t = first, k = 0; t < up_total; ++k) {
    // the ticket from a wave whose next wait is on its own weight loads, not a poll
    int nxt = 0;
    if (ticket && threadIdx.x == K2_NT - 64)
      nxt = G + __hip_atomic_fetch_add(k2_ctr(p, SY_UPT), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!k2_wait(p, seen, SY_ROUTER, nrt, k == 0 ? stamp : -1, K2_LANES)) return false;
    const int rc = moe_upgate<K2_NT, NCG, FMT>(p.moe, t < up_sh ? up_r + t : t - up_sh, S.up.red, S.up.midf, tp);
    if (rc < 0) return false;
    if (!ticket) {
      k2_signal(p, SY_UP, t, K2_LANES);
      t += G;
      continue;
    }
    if (rc == 0) break;
    if (threadIdx.x == K2_NT - 64) *next = nxt;
    __syncthreads();
    t = *next;
    __syncthreads();  // read before the next task's write
  }
  if (ticket) k2_signal(p, SY_UPW, blockIdx.x, K2_LANES);
  return true;
}
// the down's wait for the up/gate tasks (k2_upgate_walk)
template <int NCG>
MK2_DEV bool k2_upgate_done(const K2Dev& p, int* seen, int stamp) {
  if constexpr (NCG == 2) return k2_wait(p, seen, SY_UPW, gridDim.x, stamp, K2_LANES);
  const int up_total = p.moe.Dmax * (p.moe.I / p.moe.UC) + p.moe.n_shared * (p.moe.SI / 32);
  return k2_wait(p, seen, SY_UP, up_total, stamp, K2_LANES);
}

// score chunks a workgroup keeps in LDS for its slices (more tasks a workgroup: the
// rest go through the scores in the workspace)
constexpr int K2_KEEP = 4;

// What the launch runs ahead of the layer's stages: nothing, or the layer's front
// (the persistent front's walk, its per-head tasks counting out, then a wait for all
// of them: the scores read the index queries and keys, the splits the MLA queries
// and latent rows, that it writes).  reset: the last workgroup out also resets its
// counters.
struct K2NoFront {
  MK2_DEV bool run(FrontLds&, int*) const { return true; }
  MK2_DEV void reset() const {}
};
template <int KUA, int KUC, int WF, int NS>
struct K2Front {
  FrontPDev f;
  MK2_DEV bool run(FrontLds& S, int* seen) const {
    if (!front_walk<KUA, KUC, WF, NS, true>(f, S, seen)) return false;
    return fp_wait(f, seen, 4, FP_HEADS, FP_LANES, f.nheads);
  }
  MK2_DEV void reset() const { front_reset(f); }
};

template <int NCG, int FMT, class Front = K2NoFront>
__global__ __launch_bounds__(K2_NT, 1) void k_k2_layer(K2Dev p, Front front) {
  __shared__ K2Lds S;
  __shared__ float kept[K2_KEEP][IDX_CHUNK];  // this workgroup's score tasks' scores, by t / G
  __shared__ int seen[SY_LINES + 1];  // counts seen by line; [SY_LINES]: a wait failed
  __shared__ int last_flag;
  __shared__ int up_next;  // the up/gate walk's next ticket
  __shared__ uint32_t s_tag;
  const int G = gridDim.x, b = blockIdx.x;
  const int R = p.rows;
  for (int i = threadIdx.x; i <= SY_LINES; i += K2_NT) seen[i] = 0;
  if (p.timeline && threadIdx.x < K2_STAMPS) k2_lds_stamps[threadIdx.x] = 0;
  // this launch's tag: one past the epoch the previous launch on this workspace left
  // (never 0; a zero-filled workspace starts at 1).  The epoch's load is issued here and
  // its value taken only after the scores, which use no tag: its round trip overlaps
  // the scores' own loads instead of holding the launch's start
  uint32_t epoch = 0;
  if (threadIdx.x == 0) epoch = (uint32_t)ld_dev_i32(p.sync + SYNC_EPOCH);
  auto tag_of = [](uint32_t e) { return e + 1u ? e + 1u : 1u; };
  __syncthreads();
  TagPoll tp{0u, p.wait_ticks, k2_ctr(p, SY_ERR)};
  // the stages in order; a wait that fails (its deadline, or another workgroup's
  // failure seen while polling) returns from the walk: the workgroup skips every task
  // left and goes straight to the counter reset (fail-stop)
  auto walk = [&]() {
    int base = 0;  // this stage's first workgroup
    // the tasks of a stage of n tasks on this workgroup; `t < G` marks the first
#define K2_TASKS(t, n) for (int t = (b - base % G + G) % G; t < (n); t += G)
#define K2_NEXT(n) base = (base + (n)) % G
    int st = 0;  // timeline stage
    // ---- index scores + row key histograms
    k2_stamp(p, 3 * st);
    const int nchk = p.idx.nchk;
    auto keep_of = [&](int t) { return t / G < K2_KEEP ? kept[t / G] : nullptr; };
    K2_TASKS(t, R * nchk) {
      idx_score<K2_NT>(p.idx, t / nchk, t % nchk, S.score, keep_of(t));
      k2_signal(p, SY_SCORE + t / nchk);
    }
    k2_stamp(p, 3 * st++ + 2);
    if (threadIdx.x == 0) s_tag = tag_of(epoch);
    __syncthreads();
    tp.tag = s_tag;
    // ---- top-k slices: each chunk lists its keys above the row's threshold bin and
    // keeps its keys in the bin
    k2_stamp(p, 3 * st);
    // slices on the workgroups of their score chunks (base unchanged).  A slice counts
    // out once its chunk's counts and bin keys are out.  With one slice a workgroup
    // (up to 8 rows) the last to count out of a row lists its own keys above the bin,
    // then finishes the row's list from the keys in the threshold bin, while the others
    // still list theirs.  With several a workgroup the selects are tasks of their own
    // after the slices: a workgroup that won one row would start its next slice late,
    // be the last of that row too, and run every round's select in turn.  A select's
    // workgroup clears the row's histograms later, where it waits for the routing
    // anyway (sel_rows: the rows it selected, a bit each)
    const bool sel_tasks = R * nchk > G;
    uint32_t sel_rows = 0;
    K2_TASKS(t, R * nchk) {
      const int r = t / nchk;
      if (!k2_wait(p, seen, SY_SCORE + r, nchk, t < G ? 3 * st + 1 : -1)) return;
      bool last = false;
      const bool known = idx_slice<K2_NT>(p.idx, r, t % nchk, S.topk, p.wait_ticks, k2_ctr(p, SY_ERR), tp.tag,
                                          [&] {
                                            if (sel_tasks)
                                              k2_signal(p, SY_SLICE + r);
                                            else
                                              last = k2_signal_last1(p, SY_SLICE + r, nchk, &last_flag);
                                          },
                                          keep_of(t));
      if (last) {
        k2_stamp(p, 3 * (st + 1));
        k2_stamp(p, 3 * (st + 1) + 1);
        // this workgroup's own slice of row r may have left the threshold in LDS
        idx_select<K2_NT>(p.idx, r, S.topk, tp.tag, known);
        k2_stamp(p, 3 * (st + 1) + 2);
        sel_rows |= 1u << r;
      }
    }
    k2_stamp(p, 3 * st + 2);
    K2_NEXT(R * nchk);
    if (sel_tasks) {
      K2_TASKS(r, R) {
        k2_stamp(p, 3 * (st + 1));
        if (!k2_wait(p, seen, SY_SLICE + r, nchk, 3 * (st + 1) + 1)) return;
        idx_select<K2_NT>(p.idx, r, S.topk, tp.tag, false);
        k2_stamp(p, 3 * (st + 1) + 2);
        sel_rows |= 1u << r;
      }
      K2_NEXT(R);
    }
    st += 2;  // the select stamps are taken above
    // ---- sparse-MLA splits
    k2_stamp(p, 3 * st);
    const int ns = p.mla.nsplit;
    K2_TASKS(t, R * ns) {
      const int r = t / ns;
      // the split polls its 64 entries of the tagged list: it starts as soon as they are
      // out (most come from the slices, ahead of the row's select)
      const int stamp = t < G ? 3 * st + 1 : -1;
      if (!mla_split<K2_NT>(p.mla, r, t % ns, S.split, tp, [&](int) { if (stamp >= 0) k2_stamp(p, stamp); }))
        return;
      k2_signal(p, SY_SPLIT + r);
    }
    K2_NEXT(R * ns);
    k2_stamp(p, 3 * st++ + 2);
    // ---- merge of the splits + W_UV, per (group of mrg rows, head, half of the head's
    // outputs): about one task a workgroup
    k2_stamp(p, 3 * st);
    const int mrg = mla_merge_rows(R, G), nmt = 2 * MLA_HEADS * ((R + mrg - 1) / mrg);
    K2_TASKS(t, nmt) {
      const int r0 = t / (2 * MLA_HEADS) * mrg, nr = min(mrg, R - r0), h = (t >> 1) % MLA_HEADS;
      mla_merge_uv<K2_NT>(p.mla, r0, nr, h, t & 1, S.merge, [&] {
        for (int i = 0; i < nr; ++i)
          if (!k2_wait(p, seen, SY_SPLIT + r0 + i, ns, t < G && i == nr - 1 ? 3 * st + 1 : -1)) return false;
        return true;
      });
      if (seen[SY_LINES]) return;
      k2_signal(p, SY_UV, t, K2_LANES);
    }
    K2_NEXT(nmt);
    k2_stamp(p, 3 * st++ + 2);
    // ---- W_o + residual, per 16 hidden rows: tasks t and t + G together (their weights
    // all in flight before the wait)
    k2_stamp(p, 3 * st);
    const int ht = p.mla.hidden / 16;
    for (int t = (b - base % G + G) % G; t < ht; t += 2 * G) {
      const int t1 = t + G < ht ? t + G : -1;
      mla_oproj<K2_NT, NCG, 2>(p.mla, t, t1, S.up.red,
                               [&] { return k2_wait(p, seen, SY_UV, nmt, t < G ? 3 * st + 1 : -1, K2_LANES); });
      if (seen[SY_LINES]) return;
      k2_signal(p, SY_OPROJ, t, K2_LANES, t1 >= 0 ? 2 : 1);
    }
    K2_NEXT(ht);
    k2_stamp(p, 3 * st++ + 2);
    // ---- router GEMV (+ RMSNorm of its slice), per (16 experts, hidden slice): the
    // partial logits go out as tagged words (the routing polls them); the counter
    // publishes the normalized rows the tasks of the first expert tile store
    k2_stamp(p, 3 * st);
    const int et = p.moe.E / 16, nrt = et * p.moe.KC;
    K2_TASKS(t, nrt) {
      moe_router<K2_NT, NCG, FMT>(p.moe, t % et, t / et, S.router, tp.tag,
                             [&] { return k2_wait(p, seen, SY_OPROJ, ht, t < G ? 3 * st + 1 : -1, K2_LANES); });
      if (seen[SY_LINES]) return;
      k2_signal(p, SY_ROUTER, t, K2_LANES);
    }
    K2_NEXT(nrt);
    k2_stamp(p, 3 * st++ + 2);
    // ---- routing, on one workgroup up to 8 rows: one without a router task (it polls
    // while they run) and with the fewest up/gate tasks.  It polls the router tasks' logits and
    // puts out the tagged expert list, then the route-weight table, published by
    // SY_ROUTE for the down
    const int up_r = p.moe.Dmax * (p.moe.I / p.moe.UC);
    const int up_sh = p.moe.n_shared * (p.moe.SI / 32);
    const int up_total = up_r + up_sh;
    // the up/gate tasks start at workgroup `base`; from base + up_total % G on, the
    // workgroups hold one fewer; the router tasks ended on the nrt workgroups before base
    // above 8 rows the rows' top-k runs on nq workgroups of 8 rows each, the first of
    // which (the lead) polls the others' picks and puts out the list and the tables
    const int nq = p.moe.M > 8 ? (p.moe.M + 7) / 8 : 1;
    int route_at = up_total % G;
    if (nrt < G && route_at > G - nrt - nq) route_at = max(0, G - nrt - nq);
    const int q = (b - base - route_at + 2 * G) % G;
    if (q < nq) {
      constexpr bool CMP = kCompact<NCG, FMT>;
      if (q == 0) k2_stamp(p, 3 * st);
      auto mark = [&](int i) { if (q == 0) k2_stamp(p, 3 * K2_STAGES + i); };
      bool ok;
      if (nq == 1)
        ok = moe_route<K2_NT, CMP>(p.moe, S.route, tp, mark);
      else if (q == 0)
        ok = moe_route<K2_NT, CMP, ROUTE_LEAD>(p.moe, S.route, tp, mark, 0, 8);
      else
        ok = moe_route<K2_NT, CMP, ROUTE_PICK>(p.moe, S.route, tp, mark, 8 * q, min(p.moe.M, 8 * q + 8));
      if (!ok) return;
      if (q == 0) {
        k2_stamp(p, 3 * st + 1);
        k2_signal(p, SY_ROUTE);
        k2_stamp(p, 3 * st + 2);
      }
    }
    ++st;
    // ---- up/gate + SwiGLU: the shared expert's chunks first (they need only the
    // normalized rows, so they run while routing is still pending), then the routed
    // slots, each polling its slot of the tagged expert list
    k2_stamp(p, 3 * st);
    // the selects' rows' histograms back to zero, here where a workgroup waits for the
    // routing anyway (every slice and select read them long ago; a stopped launch
    // leaves this to the last workgroup out)
    for (uint32_t m = sel_rows; m; m &= m - 1) idx_clear_hist<K2_NT>(p.idx, __ffs((int)m) - 1);
    if constexpr (NCG == 1) {
      K2_TASKS(t, up_total) {
        const bool sh = t < up_sh;
        if (!k2_wait(p, seen, SY_ROUTER, nrt, t < G ? 3 * st + 1 : -1, K2_LANES)) return;
        if (moe_upgate<K2_NT, NCG, FMT>(p.moe, sh ? up_r + t : t - up_sh, S.up.red, S.up.midf, tp) < 0) return;
        k2_signal(p, SY_UP, t, K2_LANES);
      }
    } else if (!k2_upgate_walk<NCG, FMT>(p, S, seen, &up_next, (b - base % G + G) % G, nrt, tp, 3 * st + 1)) {
      return;
    }
    K2_NEXT(up_total);
    k2_stamp(p, 3 * st++ + 2);
    // ---- down + route weighting + residual, per 16 hidden rows
    k2_stamp(p, 3 * st);
    K2_TASKS(t, down_tasks(p.moe)) {
      if (!k2_wait(p, seen, SY_ROUTE, 1)) return;  // the routing and its table: known long before the mid rows
      moe_down<K2_NT, NCG, FMT>(p.moe, t, S.down.red, S.down.act, S.down.xres,
                                [&] { return k2_upgate_done<NCG>(p, seen, t < G ? 3 * st + 1 : -1); });
      if (seen[SY_LINES]) return;
    }
    k2_stamp(p, 3 * st + 2);

  };
  // the front first, when the launch runs it: a failed front stops the layer's walk and
  // fails every layer wait at once
  __shared__ int fseen[FP_SEEN];
  bool front_ok = true;
  if constexpr (!std::is_same<Front, K2NoFront>::value) {
    if (threadIdx.x < FP_SEEN) fseen[threadIdx.x] = 0;
    __syncthreads();
    front_ok = front.run(S.front, fseen);
    __syncthreads();  // the front's LDS is the stages' from here on
    if (!front_ok && threadIdx.x == 0) atomicOr(k2_ctr(p, SY_ERR), 1);
  }
  if (front_ok) walk();
#undef K2_TASKS
#undef K2_NEXT
  __syncthreads();  // thread 0's stamps are in LDS
  if (p.timeline && threadIdx.x < K2_STAMPS)
    p.timeline[(size_t)blockIdx.x * K2_STAMPS + threadIdx.x] = k2_lds_stamps[threadIdx.x];
  // ---- the last workgroup out resets the counters for the next launch
  drain_memory();  // this workgroup's stores and atomics have landed before it counts out
  __syncthreads();
  if (threadIdx.x == 0)
    last_flag = __hip_atomic_fetch_add(k2_ctr(p, SY_DONE), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1;
  __syncthreads();
  if (last_flag) {
    __syncthreads();
    if (threadIdx.x == 0) last_flag = __hip_atomic_load(k2_ctr(p, SY_ERR), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (last_flag) {
      // a stopped launch skipped some rows' top-k resets: every workgroup has left, so
      // clear all rows' top-k state here and the next launch starts clean
      idx_reset_rows<K2_NT>(p.idx, R);
      if (threadIdx.x == 0 && p.status) atomicOr(p.status, 1);
      drain_memory();
      __syncthreads();
    } else {  // the chunk counts (the selects cleared the histograms)
      for (int i = threadIdx.x; i < R * p.idx.nchk; i += K2_NT) st_dev_i32(p.idx.ccount + i, 0);
    }
    for (int l = threadIdx.x; l < SY_LINES; l += K2_NT)
      __hip_atomic_store(k2_ctr(p, l), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    front.reset();
    // the epoch moves on: the next launch's tags differ from every tag of this one
    if (threadIdx.x == 0) st_dev_i32(p.sync + SYNC_EPOCH, (int)tag_of(epoch));
  }
}

// the current device's CU count (the persistent grid), queried once per device
constexpr int K2_MAX_DEVICES = 64;
static int g_cus[K2_MAX_DEVICES];
static int current_cus(int* cus) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= K2_MAX_DEVICES)
    return set_error(MK2_ELAUNCH, "persistent launch: no current HIP device");
  if (g_cus[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return set_error(MK2_ELAUNCH, "persistent launch: cannot query the CU count of device %d", dev);
    g_cus[dev] = n;
  }
  *cus = g_cus[dev];
  return MK2_OK;
}

// front: the layer's front to run ahead of the stages in the same launch, or null;
// front_key: its instantiation (FRONT_FUSED_*)
int k2_persistent_enqueue(const IdxDev& idx, const MlaDev& mla, const MoeDev& moe, int* sync,
                          int* status, uint64_t* timeline, int rows, uint32_t wait_ticks, hipStream_t st,
                          const FrontPDev* front, int front_key) {
  int ncu = 0;
  if (const int rc = current_cus(&ncu)) return rc;
  K2Dev p{idx, mla, moe, sync, status, timeline, rows, wait_ticks};
  const bool two = rows > 16;
  // one instantiation a column-group count and expert mode (and, with the front ahead,
  // front shape)
  return with_moe_fmt(moe.fmt, [&](auto F) {
    constexpr int FMT = decltype(F)::value;
    auto launch = [&](auto fr) -> int {
      using Fr = decltype(fr);
      int per_cu = 0;
      hipError_t e = two ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_k2_layer<2, FMT, Fr>, K2_NT, 0)
                         : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_k2_layer<1, FMT, Fr>, K2_NT, 0);
      if (e != hipSuccess || per_cu < 1)
        return set_error(MK2_ELAUNCH, "layer: the persistent kernel does not fit one workgroup per CU");
      if (two) k_k2_layer<2, FMT, Fr><<<ncu, K2_NT, 0, st>>>(p, fr);
      else k_k2_layer<1, FMT, Fr><<<ncu, K2_NT, 0, st>>>(p, fr);
      return check_launch("layer (persistent)");
    };
    if (!front) return launch(K2NoFront{});
    if constexpr (FMT == MK2_FMT_MXFP4) {
      if (front_key == FRONT_FUSED_C7_FP8) return launch(K2Front<6, 4, MK2_WFMT_FP8_BLOCK, 6>{*front});
      if (front_key == FRONT_FUSED_C7_AITER16) return launch(K2Front<6, 4, MK2_WFMT_FP8_AITER16, 6>{*front});
    }
    return set_error(MK2_EINVAL, "layer step: no front-and-layer launch for this expert mode and front shape");
  });
}

// ------------------------------------------------------------------------------------
// The layer's three blocks as persistent launches of their own (the entry points of
// configs[0..3]): the same stage functions, counters, hand-offs and fail-stop as the
// layer's launch, walking only the block's stages.  The block's sync block leads its
// workspace (zero-filled before the first launch; every launch leaves it so); a launch
// whose wait gave up ORs 1 into the status word at BLOCK_STATUS_INT of it.
constexpr int BLOCK_STATUS_INT = SY_LINES * SY_LINE;
static_assert(BLOCK_STATUS_INT * 4 == MK2_BLOCK_STATUS_OFFSET, "the header's status offset");
static_assert(BLOCK_STATUS_INT < SYNC_EPOCH, "the status word stays clear of the epoch word");
enum { K2_BLOCK_INDEXER = 0, K2_BLOCK_MLA = 1, K2_BLOCK_MOE = 2 };

template <int BLK, int NCG, int FMT>
__global__ __launch_bounds__(K2_NT, 1) void k_k2_block(K2Dev p) {
  __shared__ K2Lds S;
  __shared__ float kept[BLK == K2_BLOCK_INDEXER ? K2_KEEP : 1][IDX_CHUNK];
  __shared__ int seen[SY_LINES + 1];
  __shared__ int last_flag;
  __shared__ int up_next;  // the up/gate walk's next ticket
  __shared__ uint32_t s_tag;
  const int G = gridDim.x, b = blockIdx.x;
  const int R = p.rows;
  for (int i = threadIdx.x; i <= SY_LINES; i += K2_NT) seen[i] = 0;
  if (threadIdx.x == 0) {
    const uint32_t e = (uint32_t)ld_dev_i32(p.sync + SYNC_EPOCH) + 1u;
    s_tag = e ? e : 1u;
  }
  __syncthreads();
  const TagPoll tp{s_tag, p.wait_ticks, k2_ctr(p, SY_ERR)};
  uint32_t sel_rows = 0;  // the rows whose select this workgroup ran
  auto walk = [&]() {
    int base = 0;
#define K2_TASKS(t, n) for (int t = (b - base % G + G) % G; t < (n); t += G)
#define K2_NEXT(n) base = (base + (n)) % G
    if constexpr (BLK == K2_BLOCK_INDEXER) {
      // scores, slices (the last of a row to count out runs its select with one slice a
      // workgroup; with several, the selects are tasks of their own): as the layer's
      const int nchk = p.idx.nchk;
      auto keep_of = [&](int t) { return t / G < K2_KEEP ? kept[t / G] : nullptr; };
      K2_TASKS(t, R * nchk) {
        idx_score<K2_NT>(p.idx, t / nchk, t % nchk, S.score, keep_of(t));
        k2_signal(p, SY_SCORE + t / nchk);
      }
      const bool sel_tasks = R * nchk > G;
      K2_TASKS(t, R * nchk) {
        const int r = t / nchk;
        if (!k2_wait(p, seen, SY_SCORE + r, nchk)) return;
        bool last = false;
        const bool known = idx_slice<K2_NT>(p.idx, r, t % nchk, S.topk, p.wait_ticks, k2_ctr(p, SY_ERR), tp.tag,
                                            [&] {
                                              if (sel_tasks)
                                                k2_signal(p, SY_SLICE + r);
                                              else
                                                last = k2_signal_last1(p, SY_SLICE + r, nchk, &last_flag);
                                            },
                                            keep_of(t));
        if (last) {
          idx_select<K2_NT>(p.idx, r, S.topk, tp.tag, known);
          sel_rows |= 1u << r;
        }
      }
      K2_NEXT(R * nchk);
      if (sel_tasks) {
        K2_TASKS(r, R) {
          if (!k2_wait(p, seen, SY_SLICE + r, nchk)) return;
          idx_select<K2_NT>(p.idx, r, S.topk, tp.tag, false);
          sel_rows |= 1u << r;
        }
      }
      // every slice and select read the histograms: the selects' rows back to zero
      for (uint32_t m = sel_rows; m; m &= m - 1) idx_clear_hist<K2_NT>(p.idx, __ffs((int)m) - 1);
    } else if constexpr (BLK == K2_BLOCK_MLA) {
      // splits (the given positions), merge + W_UV, W_o + residual: as the layer's
      const int ns = p.mla.nsplit;
      K2_TASKS(t, R * ns) {
        if (!mla_split<K2_NT>(p.mla, t / ns, t % ns, S.split, tp)) return;
        k2_signal(p, SY_SPLIT + t / ns);
      }
      K2_NEXT(R * ns);
      const int mrg = mla_merge_rows(R, G), nmt = 2 * MLA_HEADS * ((R + mrg - 1) / mrg);
      K2_TASKS(t, nmt) {
        const int r0 = t / (2 * MLA_HEADS) * mrg, nr = min(mrg, R - r0), h = (t >> 1) % MLA_HEADS;
        mla_merge_uv<K2_NT>(p.mla, r0, nr, h, t & 1, S.merge, [&] {
          for (int i = 0; i < nr; ++i)
            if (!k2_wait(p, seen, SY_SPLIT + r0 + i, ns)) return false;
          return true;
        });
        if (seen[SY_LINES]) return;
        k2_signal(p, SY_UV, t, K2_LANES);
      }
      K2_NEXT(nmt);
      const int ht = p.mla.hidden / 16;
      for (int t = (b - base % G + G) % G; t < ht; t += 2 * G) {
        const int t1 = t + G < ht ? t + G : -1;
        mla_oproj<K2_NT, NCG, 2>(p.mla, t, t1, S.up.red,
                                 [&] { return k2_wait(p, seen, SY_UV, nmt, -1, K2_LANES); });
        if (seen[SY_LINES]) return;
      }
    } else {
      // the rows' sums of squares (with the RMSNorm), router, routing, up/gate, down:
      // as the layer's, the sums from tasks of their own (the layer's come from W_o)
      // (512 columns a task on the first 128 threads: the staged kernel's shape, so both
      // give the same bits for any hidden size a multiple of 512)
      const int per = p.moe.H / 512, nss = p.moe.norm ? p.rows * per : 0;
      K2_TASKS(t, nss) {
        if (threadIdx.x < 128) moe_sumsq<128>(p.moe, t / per, t % per);
        k2_signal(p, SY_OPROJ, t, K2_LANES);
      }
      K2_NEXT(nss);
      const int et = p.moe.E / 16, nrt = et * p.moe.KC;
      K2_TASKS(t, nrt) {
        moe_router<K2_NT, NCG, FMT>(p.moe, t % et, t / et, S.router, tp.tag,
                                    [&] { return k2_wait(p, seen, SY_OPROJ, nss, -1, K2_LANES); });
        if (seen[SY_LINES]) return;
        k2_signal(p, SY_ROUTER, t, K2_LANES);
      }
      K2_NEXT(nrt);
      const int up_r = p.moe.Dmax * (p.moe.I / p.moe.UC);
      const int up_sh = p.moe.n_shared * (p.moe.SI / 32);
      const int up_total = up_r + up_sh;
      const int nq = p.moe.M > 8 ? (p.moe.M + 7) / 8 : 1;
      int route_at = up_total % G;
      if (nrt < G && route_at > G - nrt - nq) route_at = max(0, G - nrt - nq);
      const int q = (b - base - route_at + 2 * G) % G;
      if (q < nq) {
        constexpr bool CMP = kCompact<NCG, FMT>;
        bool ok;
        if (nq == 1)
          ok = moe_route<K2_NT, CMP>(p.moe, S.route, tp);
        else if (q == 0)
          ok = moe_route<K2_NT, CMP, ROUTE_LEAD>(p.moe, S.route, tp, NoMark(), 0, 8);
        else
          ok = moe_route<K2_NT, CMP, ROUTE_PICK>(p.moe, S.route, tp, NoMark(), 8 * q, min(p.moe.M, 8 * q + 8));
        if (!ok) return;
        if (q == 0) k2_signal(p, SY_ROUTE);
      }
      if (!k2_upgate_walk<NCG, FMT>(p, S, seen, &up_next, (b - base % G + G) % G, nrt, tp, -1)) return;
      K2_NEXT(up_total);
      K2_TASKS(t, down_tasks(p.moe)) {
        if (!k2_wait(p, seen, SY_ROUTE, 1)) return;
        moe_down<K2_NT, NCG, FMT>(p.moe, t, S.down.red, S.down.act, S.down.xres,
                                  [&] { return k2_upgate_done<NCG>(p, seen, -1); });
        if (seen[SY_LINES]) return;
      }
    }
#undef K2_TASKS
#undef K2_NEXT
  };
  walk();
  // the last workgroup out resets the counters (and on a stop the top-k state it left)
  drain_memory();
  __syncthreads();
  if (threadIdx.x == 0)
    last_flag = __hip_atomic_fetch_add(k2_ctr(p, SY_DONE), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1;
  __syncthreads();
  if (last_flag) {
    __syncthreads();
    if (threadIdx.x == 0) last_flag = __hip_atomic_load(k2_ctr(p, SY_ERR), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (last_flag) {
      if constexpr (BLK == K2_BLOCK_INDEXER) idx_reset_rows<K2_NT>(p.idx, R);
      if (threadIdx.x == 0) atomicOr(p.sync + BLOCK_STATUS_INT, 1);
      drain_memory();
      __syncthreads();
    } else if constexpr (BLK == K2_BLOCK_INDEXER) {
      for (int i = threadIdx.x; i < R * p.idx.nchk; i += K2_NT) st_dev_i32(p.idx.ccount + i, 0);
    }
    for (int l = threadIdx.x; l < SY_LINES; l += K2_NT)
      __hip_atomic_store(k2_ctr(p, l), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (threadIdx.x == 0) st_dev_i32(p.sync + SYNC_EPOCH, (int)s_tag);
  }
}

// One block's persistent launch on `sync` (its workspace's leading sync block).  Returns
// MK2_ELAUNCH when the kernel would not keep one workgroup on every CU.
int k2_block_enqueue(int blk, const IdxDev* idx, const MlaDev* mla, const MoeDev* moe, int* sync, int rows,
                     hipStream_t st) {
  int ncu = 0;
  if (const int rc = current_cus(&ncu)) return rc;
  K2Dev p{};
  if (idx) p.idx = *idx;
  if (mla) p.mla = *mla;
  if (moe) p.moe = *moe;
  p.sync = sync;
  p.rows = rows;
  p.wait_ticks = DEFAULT_WAIT_TICKS;
  const bool two = rows > 16;
  auto launch = [&](auto kern) -> int {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, K2_NT, 0) != hipSuccess || per_cu < 1)
      return set_error(MK2_ELAUNCH, "block: the persistent kernel does not fit one workgroup per CU");
    kern<<<ncu, K2_NT, 0, st>>>(p);
    return check_launch("block (persistent)");
  };
  if (blk == K2_BLOCK_INDEXER) return launch(k_k2_block<K2_BLOCK_INDEXER, 1, MK2_FMT_MXFP4>);
  if (blk == K2_BLOCK_MLA)
    return two ? launch(k_k2_block<K2_BLOCK_MLA, 2, MK2_FMT_MXFP4>) : launch(k_k2_block<K2_BLOCK_MLA, 1, MK2_FMT_MXFP4>);
  return with_moe_fmt(moe->fmt, [&](auto F) {
    constexpr int FMT = decltype(F)::value;
    return two ? launch(k_k2_block<K2_BLOCK_MOE, 2, FMT>) : launch(k_k2_block<K2_BLOCK_MOE, 1, FMT>);
  });
}

}  // namespace mk2
