// Indexer stages of the K2 layer: FP4 index-key scores on the matrix cores and the
// exact radix top-k with a lowest-position tie-break.
//
// score[r][c] = sum_h relu(q[r][h] . k[c]) * w[r][h] over the FP4 keys (E2M1 codes,
// E8M0 per 32 dims) of request req[r], positions c < ctx[r].  One task scores a
// chunk of positions; a wave takes 16 keys at a time as the MFMA B operand (16
// columns) against all heads as A (16 heads a tile), widening E2M1 x 2^e exactly to
// bf16.  The head sum runs in the lanes: a lane holds 4 heads of each head group
// for one key, then two cross-row shuffles finish it.
//
// top-k: one workgroup of 1024 threads a row, 64 consecutive positions a thread in
// registers.  LDS histogram passes over at most 12 bits at a time of (key - row min)
// find the k-th key T exactly; the list is written in the radix select's order --
// keys whose top 12 bits exceed T's, then keys sharing T's top 12 bits that exceed
// T, then keys equal to T (lowest positions first) -- each group in position order.
#pragma once
#include "mk2_device.h"

namespace mk2 {

constexpr int IDX_PAGE = 64;
constexpr int IDX_PAGE_BYTES = 64 * 64 + 64 * 4;  // codes, then E8M0
constexpr int IDX_CHUNK = 2048;                    // positions a score task
constexpr int TOPK_NT = 1024;                      // top-k workgroup of the standalone launch

struct IdxDev {
  int rows, heads, topk, max_ctx, stride;
  const bf16_t* q;      // [rows][heads][128]
  const bf16_t* w;      // [rows][heads]
  const uint8_t* cache; // pages
  const int* pt;        // [requests][stride]
  const int* req;       // [rows]
  const int* ctx;       // [rows]
  float* scores;        // [rows][max_ctx]
  int* out;             // [rows][topk]
};

// ------------------------------------------------------------- stage: scores
// One task: IDX_CHUNK positions of row r; each wave owns 16 groups of 16 keys and
// issues all of their loads before the first MFMA.
// lds: IDX_CHUNK / 64 ints (the chunk's physical pages)
template <int NT>
MK2_DEV void idx_score(const IdxDev& p, int r, int chunk, int* lds_pages) {
  constexpr int NW = NT / 64;
  constexpr int GPW = IDX_CHUNK / 16 / NW;  // 16-key groups a wave
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
  const int n = p.ctx[r];
  const int k_begin = chunk * IDX_CHUNK;
  if (k_begin >= n) return;
  const int k_end = min(n, k_begin + IDX_CHUNK);
  const int ngroups = (k_end - k_begin + 15) >> 4;
  // the chunk's page ids first, through LDS: every key load below then issues
  // without waiting on another vector-memory load
  if (threadIdx.x < IDX_CHUNK / 64) {
    const int pg = (k_begin >> 6) + threadIdx.x;
    lds_pages[threadIdx.x] = pg * 64 < k_end ? p.pt[(size_t)p.req[r] * p.stride + pg] : 0;
  }
  __syncthreads();
  const int gw0 = wave * GPW;  // this wave's first group
  uint4 code[GPW];
  uint32_t sw[GPW];
#pragma unroll
  for (int j = 0; j < GPW; ++j) {
    const int key0 = k_begin + (gw0 + j) * 16;
    if (gw0 + j < ngroups) {
      const uint8_t* pg = p.cache + (size_t)lds_pages[(key0 - k_begin) >> 6] * IDX_PAGE_BYTES;
      const int tok = (key0 & 63) + c16;
      code[j] = *(const uint4*)(pg + tok * 64 + 16 * g);
      sw[j] = *(const uint32_t*)(pg + 4096 + tok * 4);
    } else {
      code[j] = make_uint4(0, 0, 0, 0);
      sw[j] = 0x7F7F7F7Fu;
    }
  }
  const int nhg = p.heads >> 4;
  // A operands: q of head 16*hg + c16, dims 32g + 8s .. +7; head weights of rows 4g+i
  bf16x8 qa[4][4];
  float wt[4][4];
#pragma unroll
  for (int hg = 0; hg < 4; ++hg) {
    if (hg < nhg) {
      const bf16_t* qr = p.q + ((size_t)r * p.heads + hg * 16 + c16) * 128 + 32 * g;
#pragma unroll
      for (int s = 0; s < 4; ++s) qa[hg][s] = __builtin_bit_cast(bf16x8, *(const uint4*)(qr + 8 * s));
      const uint2 wv = *(const uint2*)(p.w + (size_t)r * p.heads + hg * 16 + 4 * g);
      wt[hg][0] = __uint_as_float(wv.x << 16);
      wt[hg][1] = __uint_as_float(wv.x & 0xFFFF0000u);
      wt[hg][2] = __uint_as_float(wv.y << 16);
      wt[hg][3] = __uint_as_float(wv.y & 0xFFFF0000u);
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) qa[hg][s] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
#pragma unroll
      for (int i = 0; i < 4; ++i) wt[hg][i] = 0.f;
    }
  }
  float* srow = p.scores + (size_t)r * p.max_ctx;
#pragma unroll
  for (int j = 0; j < GPW; ++j) {
    if (gw0 + j >= ngroups) break;
    const float sc = e8m0_to_f32(sw[j] >> (8 * g));
    bf16x8 kb[4];
    kb[0] = e2m1x8_to_bf16(code[j].x, sc);
    kb[1] = e2m1x8_to_bf16(code[j].y, sc);
    kb[2] = e2m1x8_to_bf16(code[j].z, sc);
    kb[3] = e2m1x8_to_bf16(code[j].w, sc);
    float s = 0.f;
#pragma unroll
    for (int hg = 0; hg < 4; ++hg) {
      if (hg >= nhg) break;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) acc = mfma_bf16(qa[hg][q], kb[q], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) s += fmaxf(acc[i], 0.f) * wt[hg][i];
    }
    s += __shfl_xor(s, 16, 64);
    s += __shfl_xor(s, 32, 64);
    const int key = k_begin + (gw0 + j) * 16 + c16;
    if (g == 0 && key < k_end) srow[key] = s;
  }
  __syncthreads();
}

// ------------------------------------------------------------- stage: top-k
struct Scan3 {
  int a, b, c;
};

// exclusive scan of (a, b, c) over the workgroup in thread order; totals returned
template <int NT>
MK2_DEV Scan3 block_scan3(Scan3 v, Scan3* tot, int* lds /* 3 * NT/64 */) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  Scan3 inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int xa = __shfl_up(inc.a, o, 64), xb = __shfl_up(inc.b, o, 64), xc = __shfl_up(inc.c, o, 64);
    if (lane >= o) { inc.a += xa; inc.b += xb; inc.c += xc; }
  }
  __syncthreads();
  if (lane == 63) { lds[wave] = inc.a; lds[NW + wave] = inc.b; lds[2 * NW + wave] = inc.c; }
  __syncthreads();
  Scan3 before = {0, 0, 0}, all = {0, 0, 0};
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int a = lds[w], b = lds[NW + w], c = lds[2 * NW + w];
    if (w < wave) { before.a += a; before.b += b; before.c += c; }
    all.a += a; all.b += b; all.c += c;
  }
  *tot = all;
  return Scan3{before.a + inc.a - v.a, before.b + inc.b - v.b, before.c + inc.c - v.c};
}

template <int NT>
MK2_DEV int block_sum_int(int v, int* lds) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) t += lds[w];
  return t;
}

// The bin (of nbins, highest first) where the count from the top reaches `need`;
// returns the bin and, through *above, the count of the bins above it.  Each thread
// owns nbins / NT consecutive bins.
template <int NT>
MK2_DEV int find_bin(const int* hist, int nbins, int need, int* above_out, int* lds) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63;
  const int per = nbins / NT;  // nbins >= NT: NT-aligned runs; else threads < nbins own 1
  const int mine_n = per ? per : (tid < nbins ? 1 : 0);
  const int first = per ? tid * per : tid;
  int local = 0;
  for (int i = 0; i < mine_n; ++i) local += hist[first + i];
  // inclusive scan over reversed thread order (u = NT-1-tid): counts of higher bins
  const int u = NT - 1 - tid, uw = u >> 6, ul = u & 63;
  int* sh = lds;           // [NT] staging in u order
  __syncthreads();
  sh[u] = local;
  __syncthreads();
  int v = sh[tid];         // thread tid now scans position tid of the reversed order
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int x = __shfl_up(inc, o, 64);
    if (lane >= o) inc += x;
  }
  int* wt = lds + NT;
  __syncthreads();
  if (lane == 63) wt[tid >> 6] = inc;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < (tid >> 6); ++w) before += wt[w];
  const int excl_rev = before + inc - v;  // count in reversed positions < tid
  __syncthreads();
  sh[tid] = excl_rev;
  __syncthreads();
  int above = sh[u];  // count of bins above this thread's bins
  int* res = lds + NT + NW;
  __syncthreads();
  for (int i = mine_n - 1; i >= 0; --i) {
    const int h = hist[first + i];
    if (above < need && above + h >= need) {
      res[0] = first + i;
      res[1] = above;
    }
    above += h;
  }
  __syncthreads();
  *above_out = res[1];
  const int b = res[0];
  __syncthreads();
  (void)uw; (void)ul;
  return b;
}

// Exact top-k over values held in registers, PER a thread, in position order over
// (thread, i).  d[i] = key - kbase for the values taking part (d >= 1), 0 for the
// rest; more than k values take part.  Radix select over at most 12 bits of d at a
// time finds the k-th d; the list is written in the radix select's order: keys whose
// top 12 bits exceed the k-th key's, then keys sharing those 12 bits that exceed it,
// then keys equal to it (lowest positions first) -- each group in position order.
template <int NT, int PER, typename Pos>
MK2_DEV void select_emit(uint32_t (&d)[PER], Pos pos, uint32_t kbase, uint32_t dmax, int k,
                         int* hist, int* scratch, int* orow) {
  const int tid = threadIdx.x;
  int hib = dmax ? 32 - __clz(dmax) : 32;
  uint32_t prefix = 0;
  int need = k;
  while (hib > 0) {
    const int lob = hib > 12 ? hib - 12 : 0;
    const int nb = 1 << (hib - lob);
    __syncthreads();
    for (int i = tid; i < nb; i += NT) hist[i] = 0;
    __syncthreads();
    {
      int run_bin = -1, run_n = 0;
      const uint32_t mask = (uint32_t)(nb - 1);
      const uint32_t hmask = hib >= 32 ? 0u : ~((1u << hib) - 1u);  // bits above this digit
      const uint32_t hpfx = hib >= 32 ? 0u : (prefix << hib);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const uint32_t v = d[i];
        if ((v & hmask) == hpfx) {
          const int b = (int)((v >> lob) & mask);
          if (b != run_bin) {
            if (run_n) atomicAdd(&hist[run_bin], run_n);
            run_bin = b;
            run_n = 0;
          }
          ++run_n;
        }
      }
      if (run_n) atomicAdd(&hist[run_bin], run_n);
    }
    __syncthreads();
    int above;
    const int b = find_bin<NT>(hist, nb, need, &above, scratch);
    need -= above;
    prefix = (prefix << (hib - lob)) | (uint32_t)b;
    hib = lob;
  }
  const uint32_t T = prefix;     // the k-th d (>= 1)
  const int above = k - need;    // values > T
  const int ties_needed = need;  // values == T taken, lowest positions first
  // the 12-bit groups are defined on the true keys d + kbase; d = 0 is in no group
  Scan3 c = {0, 0, 0};
  const uint32_t tb = (T + kbase) >> 20;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint32_t v = d[i];
    const uint32_t hi = (v + kbase) >> 20;
    c.a += v != 0u && hi > tb;
    c.b += v != 0u && hi == tb && v > T;
    c.c += v == T;
  }
  Scan3 tot;
  Scan3 off = block_scan3<NT>(c, &tot, scratch);
  int o1 = off.a, o2 = tot.a + off.b, r3 = off.c;
  // an opaque copy: the group tests below are recomputed, not kept from the count
  // loop (keeping 3 x PER lane masks alive across the scan overflows the SGPRs)
#pragma unroll
  for (int i = 0; i < PER; ++i) asm volatile("" : "+v"(d[i]));
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint32_t v = d[i];
    const bool g1 = v != 0u && ((v + kbase) >> 20) > tb;
    const bool g2 = !g1 && v > T;
    const bool g3 = v == T;
    const int dst = g1 ? o1 : (g2 ? o2 : ((g3 && r3 < ties_needed) ? above + r3 : -1));
    o1 += g1;
    o2 += g2;
    r3 += g3;
    if (dst >= 0) orow[dst] = pos(i);
  }
}

constexpr int TOPK_CAP = 8192;   // candidates kept for the exact select
constexpr int TOPK_MAXN = 65536; // positions a row (a thread holds TOPK_MAXN / NT)

struct TopkLds {
  int hist[4096];
  int scratch[1024 + 1024 / 64 + 8];
  uint32_t ckey[TOPK_CAP];
  uint16_t cpos[TOPK_CAP];
};

// The select over a whole row (when the sampled bound does not hold): the keys are
// read again from the scores, in a function of its own so that the fast path does
// not carry its registers.
template <int NT>
__device__ __attribute__((noinline)) void topk_whole_row(const IdxDev& p, int r, uint32_t kmin,
                                                         uint32_t kmax, TopkLds& S) {
  constexpr int PER = TOPK_MAXN / NT;
  const int n = p.ctx[r];
  const int base = threadIdx.x * PER;
  const int nvalid = max(0, min(PER, n - base));
  const float* srow = p.scores + (size_t)r * p.max_ctx;
  uint32_t d[PER];
#pragma unroll
  for (int q = 0; q < PER / 4; ++q) {
    uint4 v = nvalid > 0 ? *(const uint4*)(srow + base + 4 * q) : make_uint4(0, 0, 0, 0);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      d[4 * q + j] = 4 * q + j < nvalid ? radix_key(__uint_as_float(w[j])) - kmin + 1u : 0u;
  }
  select_emit<NT, PER>(d, [&](int i) { return base + i; }, kmin - 1u, kmax - kmin + 1u, p.topk,
                       S.hist, S.scratch, p.out + (size_t)r * p.topk);
}

// One row; NT threads, 65536 / NT consecutive positions a thread in registers.  A sample
// (every 64th position) gives a lower bound L for the k-th key (about twice k's share
// of the sample above it, located to 24 bits with two histograms); the keys >= L
// (checked: at least k, at most TOPK_CAP) are compacted in position order into LDS
// and the exact select runs over them.  Otherwise the select runs over the whole row.
template <int NT>
MK2_DEV void idx_topk(const IdxDev& p, int r, TopkLds& S) {
  constexpr int NW = NT / 64;
  constexpr int TOPK_PER = TOPK_MAXN / NT;  // positions a thread
  constexpr int TOPK_CPT = TOPK_CAP / NT;   // candidates a thread
  constexpr int SPT = TOPK_PER / 64;        // samples a thread (one per 64 positions)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = p.ctx[r];
  const int k = p.topk;
  int* orow = p.out + (size_t)r * k;
  if (n <= k) {
    for (int i = tid; i < k; i += NT) orow[i] = i < n ? i : -1;
    return;
  }
  const int base = tid * TOPK_PER;
  const int nvalid = max(0, min(TOPK_PER, n - base));
  uint32_t key[TOPK_PER];
  const float* srow = p.scores + (size_t)r * p.max_ctx;
  if (nvalid > 0) {
#pragma unroll
    for (int q = 0; q < TOPK_PER / 4; ++q) {
      uint4 v = *(const uint4*)(srow + base + 4 * q);
      key[4 * q] = radix_key(__uint_as_float(v.x));
      key[4 * q + 1] = radix_key(__uint_as_float(v.y));
      key[4 * q + 2] = radix_key(__uint_as_float(v.z));
      key[4 * q + 3] = radix_key(__uint_as_float(v.w));
    }
  } else {
#pragma unroll
    for (int i = 0; i < TOPK_PER; ++i) key[i] = 0u;
  }
  // row min / max
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
  for (int i = 0; i < TOPK_PER; ++i) {
    if (i < nvalid) {
      kmin = min(kmin, key[i]);
      kmax = max(kmax, key[i]);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, o, 64));
    kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o, 64));
  }
  __syncthreads();
  if (lane == 0) { S.scratch[wave] = (int)kmin; S.scratch[NW + wave] = (int)kmax; }
  for (int i = tid; i < 4096; i += NT) S.hist[i] = 0;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    kmin = min(kmin, (uint32_t)S.scratch[w]);
    kmax = max(kmax, (uint32_t)S.scratch[NW + w]);
  }
  uint32_t L = kmin;
  bool ok = true;
  if (n > TOPK_CAP) {
    const int nsamp = (n + 63) / 64;  // positions 64j that exist
    const int target = min(nsamp, (int)(2ll * k * nsamp / n) + 16);
#pragma unroll
    for (int j = 0; j < SPT; ++j)
      if (64 * j < nvalid) atomicAdd(&S.hist[key[64 * j] >> 20], 1);
    __syncthreads();
    int a1, a2;
    const int b1 = find_bin<NT>(S.hist, 4096, target, &a1, S.scratch);
    for (int i = tid; i < 4096; i += NT) S.hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SPT; ++j)
      if (64 * j < nvalid && (int)(key[64 * j] >> 20) == b1) atomicAdd(&S.hist[(key[64 * j] >> 8) & 0xFFFu], 1);
    __syncthreads();
    const int b2 = find_bin<NT>(S.hist, 4096, target - a1, &a2, S.scratch);
    L = max(kmin, ((uint32_t)b1 << 20) | ((uint32_t)b2 << 8));
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < TOPK_PER; ++i) cnt += (i < nvalid && key[i] >= L) ? 1 : 0;
    cnt = block_sum_int<NT>(cnt, S.scratch);
    ok = cnt >= k && cnt <= TOPK_CAP;
  }
  if (!ok) {
    topk_whole_row<NT>(p, r, kmin, kmax, S);
    return;
  }
  // compact the keys >= L (position order) into LDS
  int mine = 0;
#pragma unroll
  for (int i = 0; i < TOPK_PER; ++i) mine += (i < nvalid && key[i] >= L) ? 1 : 0;
  Scan3 tot;
  int at = block_scan3<NT>(Scan3{mine, 0, 0}, &tot, S.scratch).a;
#pragma unroll
  for (int i = 0; i < TOPK_PER; ++i) {
    if (i < nvalid && key[i] >= L) {
      S.ckey[at] = key[i];
      S.cpos[at] = (uint16_t)(base + i);
      ++at;
    }
  }
  const int cnt = tot.a;
  __syncthreads();
  uint32_t d[TOPK_CPT];
#pragma unroll
  for (int i = 0; i < TOPK_CPT; ++i) {
    const int idx = tid * TOPK_CPT + i;
    d[i] = idx < cnt ? S.ckey[idx] - L + 1u : 0u;
  }
  select_emit<NT, TOPK_CPT>(d, [&](int i) { return (int)S.cpos[tid * TOPK_CPT + i]; }, L - 1u,
                            kmax - L + 1u, k, S.hist, S.scratch, orow);
}

}  // namespace mk2
