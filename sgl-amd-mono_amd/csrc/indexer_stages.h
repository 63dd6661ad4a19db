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
// registers.  Three LDS histogram passes (12, 12, 8 bits of the radix key) find the
// k-th key T exactly; the list is written in the radix select's order -- keys whose
// top 12 bits exceed T's, then keys sharing T's top 12 bits that exceed T, then keys
// equal to T (lowest positions first) -- each group in position order.
#pragma once
#include "mk2_device.h"

namespace mk2 {

constexpr int IDX_PAGE = 64;
constexpr int IDX_PAGE_BYTES = 64 * 64 + 64 * 4;  // codes, then E8M0
constexpr int IDX_CHUNK = 2048;                    // positions a score task
constexpr int TOPK_NT = 1024;
constexpr int TOPK_PER = 64;                       // positions a thread

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
template <int NT>
MK2_DEV void idx_score(const IdxDev& p, int r, int chunk) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
  const int n = p.ctx[r];
  const int k_begin = chunk * IDX_CHUNK;
  if (k_begin >= n) return;
  const int k_end = min(n, k_begin + IDX_CHUNK);
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
#pragma unroll
      for (int i = 0; i < 4; ++i) wt[hg][i] = bf16_to_f32(p.w[(size_t)r * p.heads + hg * 16 + 4 * g + i]);
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) qa[hg][s] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
#pragma unroll
      for (int i = 0; i < 4; ++i) wt[hg][i] = 0.f;
    }
  }
  const int* ptr = p.pt + (size_t)p.req[r] * p.stride;
  float* srow = p.scores + (size_t)r * p.max_ctx;
  constexpr int U = 4;  // 16-key groups in flight a wave
  const int ngroups = (k_end - k_begin + 15) >> 4;
  for (int g0 = wave * U; g0 < ngroups; g0 += NW * U) {
    uint4 code[U];
    uint32_t sw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int key0 = k_begin + (g0 + u) * 16;
      if (g0 + u < ngroups) {
        const int page = ptr[key0 >> 6];
        const uint8_t* pg = p.cache + (size_t)page * IDX_PAGE_BYTES;
        const int tok = (key0 & 63) + c16;
        code[u] = *(const uint4*)(pg + tok * 64 + 16 * g);
        sw[u] = *(const uint32_t*)(pg + 4096 + tok * 4);
      } else {
        code[u] = make_uint4(0, 0, 0, 0);
        sw[u] = 0x7F7F7F7Fu;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (g0 + u >= ngroups) break;
      const float sc = e8m0_to_f32(sw[u] >> (8 * g));
      bf16x8 kb[4];
      kb[0] = e2m1x8_to_bf16(code[u].x, sc);
      kb[1] = e2m1x8_to_bf16(code[u].y, sc);
      kb[2] = e2m1x8_to_bf16(code[u].z, sc);
      kb[3] = e2m1x8_to_bf16(code[u].w, sc);
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
      const int key = k_begin + (g0 + u) * 16 + c16;
      if (g == 0 && key < k_end) srow[key] = s;
    }
  }
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

// The bin (of nbins, highest first) where the count from the top reaches `need`;
// returns the bin and, through *above, the count of the bins above it.  Each thread
// owns nbins / NT consecutive bins.
template <int NT>
MK2_DEV int find_bin(const int* hist, int nbins, int need, int* above_out, int* lds) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63;
  const int per = nbins / NT;  // 4 (4096 bins) or 0 (256 bins: threads < 256 own 1)
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

// One row; NT == TOPK_NT.  lds: hist[4096] + scratch[NT + NT/64 + 8]
template <int NT>
MK2_DEV void idx_topk(const IdxDev& p, int r, int* hist, int* scratch) {
  const int tid = threadIdx.x;
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
  // ---- pass 1: top 12 bits
  for (int i = tid; i < 4096; i += NT) hist[i] = 0;
  __syncthreads();
  {
    int run_bin = -1, run_n = 0;
#pragma unroll
    for (int i = 0; i < TOPK_PER; ++i) {
      if (i < nvalid) {
        const int b = (int)(key[i] >> 20);
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
  int a1;
  const int b1 = find_bin<NT>(hist, 4096, k, &a1, scratch);
  // ---- pass 2: next 12 bits among keys with prefix b1
  for (int i = tid; i < 4096; i += NT) hist[i] = 0;
  __syncthreads();
  {
    int run_bin = -1, run_n = 0;
#pragma unroll
    for (int i = 0; i < TOPK_PER; ++i) {
      if (i < nvalid && (int)(key[i] >> 20) == b1) {
        const int b = (int)((key[i] >> 8) & 0xFFFu);
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
  int a2;
  const int b2 = find_bin<NT>(hist, 4096, k - a1, &a2, scratch);
  const uint32_t pre24 = ((uint32_t)b1 << 12) | (uint32_t)b2;
  // ---- pass 3: last 8 bits among keys with prefix (b1, b2)
  for (int i = tid; i < 256; i += NT) hist[i] = 0;
  __syncthreads();
  {
    int run_bin = -1, run_n = 0;
#pragma unroll
    for (int i = 0; i < TOPK_PER; ++i) {
      if (i < nvalid && (key[i] >> 8) == pre24) {
        const int b = (int)(key[i] & 0xFFu);
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
  int a3;
  const int b3 = find_bin<NT>(hist, 256, k - a1 - a2, &a3, scratch);
  const uint32_t T = (pre24 << 8) | (uint32_t)b3;
  const int above = a1 + a2 + a3;  // keys > T
  const int ties_needed = k - above;
  // ---- the list
  Scan3 c = {0, 0, 0};
  const uint32_t tb = T >> 20;
#pragma unroll
  for (int i = 0; i < TOPK_PER; ++i) {
    if (i < nvalid) {
      const uint32_t kk = key[i];
      c.a += (kk >> 20) > tb;
      c.b += ((kk >> 20) == tb) && kk > T;
      c.c += kk == T;
    }
  }
  Scan3 tot;
  Scan3 off = block_scan3<NT>(c, &tot, scratch);
  int o1 = off.a, o2 = a1 + off.b, r3 = off.c;
#pragma unroll
  for (int i = 0; i < TOPK_PER; ++i) {
    if (i < nvalid) {
      const uint32_t kk = key[i];
      const int pos = base + i;
      if ((kk >> 20) > tb) {
        orow[o1++] = pos;
      } else if (kk > T) {
        orow[o2++] = pos;
      } else if (kk == T) {
        if (r3 < ties_needed) orow[above + r3] = pos;
        ++r3;
      }
    }
  }
}

}  // namespace mk2
