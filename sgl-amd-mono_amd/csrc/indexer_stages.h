// Indexer stages of the K2 layer: index-key scores on the matrix cores and the
// exact radix top-k with a lowest-position tie-break.
//
// score[r][c] = sum_h relu(q[r][h] . k[c]) * w[r][h] over the keys of request req[r],
// positions c < ctx[r], from either of SGLang's index caches: the FP4 plane (E2M1
// codes, E8M0 per 32 dims, widened exactly to bf16 with their scale) or the FP8 pages
// (E4M3 values widened exactly to bf16; the key's f32 scale multiplies its lane's head
// sum, as the reference scores them, glm53/gfx950/kernel.py:3830-3845).  One task
// scores a chunk of positions; a wave takes 16 keys at a time as the MFMA B operand
// (16 columns) against all heads as A (16 heads a tile).  The head sum runs in the
// lanes: a lane holds 4 heads of each head group for one key; every four groups,
// three row-swapping permutes combine the four lane groups' sums of all four at once.
// With FP4 queries (IDX_KEYS_FP4Q, the verify-width variant after the reference's
// FP4 x FP4 scorer, deepseek_v41/gfx950/indexer/score_fp4.py:254-296) a task quantizes
// its row's queries to MXFP4 in LDS (quantize_fp4_indexer_row's rule,
// deepseek_v41/gfx950/attention/index_query.py:283-293) and a head group's 16 x 16 x
// 128 product is one scaled MFMA on the plane's codes and scales as they load.
//
// top-k, three stages over the order-preserving u32 keys of the scores:
//   score (row, chunk)  also counts its keys into the row's two-level histogram: 4096
//                       bins of the top 12 bits and 256 of the top 8 (device atomics,
//                       nonzero bins only);
//   slice (row, chunk)  finds from the finished histogram (one wave: 256 coarse bins,
//                       then 16 fine ones) the bin b1 that holds the k-th key and
//                       compacts its chunk's keys with top bits >= b1, in position
//                       order, as (key, position) candidates;
//   select (row)        gathers the row's candidates in position order (fewer than
//                       k, plus the keys of bin b1) and selects the k-th key exactly
//                       with two radix passes over the low 20 bits of bin b1's keys;
//                       the list is written in the radix select's order -- keys whose
//                       top 12 bits exceed the k-th key's, then keys sharing those bits
//                       that exceed it, then keys equal to it (lowest positions first)
//                       -- each group in position order.  It leaves the histogram
//                       zeroed for the next launch.
// A row with more than TOPK_CAP candidates (keys crowding into the threshold bin)
// runs the same select streamed over its candidates in global memory.
#pragma once
#include "mk2_device.h"

namespace mk2 {

constexpr int IDX_PAGE = 64;
// SGLang's FP4 index plane: a 64-key page is [4 chunks of 32 dims][64 keys][16 B] of
// E2M1 codes, and apart from it [4 chunks][64] E8M0 scales, key k's at (k % 16) * 4 + k / 16
constexpr int IDX_PAGE_CODES = 64 * 64;
constexpr int IDX_PAGE_SCALES = 64 * 4;
// index cache formats (MK2_KEYS_*); an FP8 page: 64 x 128 E4M3 values in 16 x 16
// tiles, then the 64 tokens' f32 scales
// IDX_KEYS_FP4Q: the FP4 plane against the queries quantized to MXFP4 (a contract of
// its own: the scores are those of the quantized queries)
constexpr int IDX_KEYS_FP4 = 0, IDX_KEYS_FP8 = 1, IDX_KEYS_FP4Q = 2;
constexpr int IDX_FP8_PAGE = 64 * 132;
constexpr int IDX_FP8_VALUES = 64 * 128;
constexpr int IDX_CHUNK = 2048;                    // positions a score task
constexpr int TOPK_NT = 1024;                      // top-k workgroup of the standalone launch

constexpr int IDX_BINS = 4096;                     // top 12 bits of a key
constexpr int IDX_CBINS = 256;                     // top 8 bits of a key

struct IdxDev {
  int rows, heads, topk, max_ctx, stride, nchk;
  const bf16_t* q;      // [rows][heads][128]
  const bf16_t* w;      // [rows][heads]
  int kfmt;             // IDX_KEYS_*
  const uint8_t* cache; // FP4, FP4Q: E2M1 plane [pages][4][64][16 B]; FP8: pages [64][132]
  const uint8_t* cscale;// FP4, FP4Q: E8M0 plane [pages][4][64]; FP8: unused
  const int* pt;        // [requests][stride]
  const int* req;       // [rows]
  const int* ctx;       // [rows]
  float* scores;        // [rows][max_ctx]
  int scores_out;       // the caller takes the scores (else the persistent layer, whose
                        // slices read them in LDS, leaves `scores` unwritten)
  int* out;             // [rows][topk]
  int keep_list;        // write `out` (with a tagged list its only readers are the
                        // caller's: the layer asked for no top-k output skips it)
  uint64_t* tlist;      // [rows][topk] the same list as tagged words (the persistent
                        // layer's splits poll it), or null
  // workspace
  int* hist;            // [rows][IDX_BINS] key counts by top 12 bits (zero between launches)
  int* chist;           // [rows][IDX_CBINS] key counts by top 8 bits (zero between launches)
  int* ccount;          // [rows][nchk] chunk counts: CC_FLAG | above | in-bin << 15 (zero between launches)
  uint2* cand;          // [rows][max_ctx] (key, position) of bin b1; chunk c from c * IDX_CHUNK
  int* ticket;          // standalone slices: the next task (zero between launches)
};

constexpr int IDX_QROW = 136;  // LDS row stride (bf16) of the staged queries

// Row r's top-k list as it is written: the int32 list and, where the layer hands it to
// its splits, the same entries as tagged words.
struct ListOut {
  int* row;        // [k] or null
  uint64_t* trow;  // [k] or null
  uint32_t tag;
  MK2_DEV void put(int i, int pos) const {
    if (row) st_dev_i32(row + i, pos);
    if (trow) st_pair(trow + i, (uint32_t)pos, tag);
  }
};
MK2_DEV ListOut list_out(const IdxDev& p, int r, uint32_t tag) {
  return ListOut{p.keep_list || !p.tlist ? p.out + (size_t)r * p.topk : nullptr,
                 p.tlist ? p.tlist + (size_t)r * p.topk : nullptr, tag};
}

struct IdxScoreLds {
  int pages[IDX_CHUNK / 64];
  int hist[IDX_BINS];
  bf16_t q[64 * IDX_QROW];  // the row's queries, [head][128] (padded rows); FP4Q: their
                            // E2M1 codes [head][64 B], then E8M0 [head][4]
  bf16_t w[64];             // its head weights
  float sc[IDX_CHUNK];      // the chunk's scores, stored once the loop is done
};

// ------------------------------------------------------------- stage: scores
// One task: IDX_CHUNK positions of row r.  The row's queries and head weights go to
// LDS first (coalesced, once a workgroup) with the chunk's page ids; then each wave
// keeps a window of its 16 groups of 16 keys in flight, takes its A operands from
// LDS, and computes group by group as the keys arrive.  The loads are unconditional
// (groups past the row's end read page id 0, and their results are dropped) and the
// scores wait in LDS until the loop is done: a store or a branch between the loads
// would make every group wait for all memory traffic.  `keep` (LDS, IDX_CHUNK floats,
// or null: L.sc) holds them for the chunk's slice on the same workgroup; with `keep`
// they go to `scores` only when the caller takes them.
template <int NT, int KF>
MK2_DEV void idx_score_keys(const IdxDev& p, int r, int chunk, IdxScoreLds& L, float* keep) {
  constexpr bool F8 = KF == IDX_KEYS_FP8;
  constexpr bool Q4 = KF == IDX_KEYS_FP4Q;
  constexpr int NW = NT / 64;
  constexpr int GPW = IDX_CHUNK / 16 / NW;  // 16-key groups a wave
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
  const int k_begin = chunk * IDX_CHUNK;
  // prologue: the row's length and request, its queries and head weights all in
  // flight together; then the chunk's page ids (through LDS, so that every key load
  // below issues without waiting on another vector-memory load)
  constexpr int QPT = (64 * 16 + NT - 1) / NT;  // 16-byte query pieces a thread
  const int n = p.ctx[r];
  const int req = p.req[r];
  uint4 qv[QPT];
  const uint4* gq = (const uint4*)(p.q + (size_t)r * p.heads * 128);
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int i = threadIdx.x + u * NT;
    qv[u] = i < p.heads * 16 ? gq[i] : make_uint4(0, 0, 0, 0);
  }
  const bf16_t wv = threadIdx.x < p.heads ? p.w[(size_t)r * p.heads + threadIdx.x] : (bf16_t)0;
  if (k_begin >= n) return;
  const int k_end = min(n, k_begin + IDX_CHUNK);
  int* lds_pages = L.pages;
  if (threadIdx.x < IDX_CHUNK / 64) {
    const int pg = (k_begin >> 6) + threadIdx.x;
    lds_pages[threadIdx.x] = pg * 64 < k_end ? p.pt[(size_t)req * p.stride + pg] : 0;
  }
  static_assert(QPT * NT >= 64 * 16, "the pieces cover 64 heads");
  if constexpr (Q4) {
    // MXFP4 queries: piece i is dims 8 (i % 16) .. + 7 of head i / 16 (zero past the
    // row's heads); a 32-dim group's four pieces sit in one DPP quad of lanes
    uint8_t* qc = (uint8_t*)L.q;
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
      const int i = threadIdx.x + u * NT;
      const uint32_t wd[4] = {qv[u].x, qv[u].y, qv[u].z, qv[u].w};
      float f[8];
      float m = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        f[2 * k] = __uint_as_float(wd[k] << 16);
        f[2 * k + 1] = __uint_as_float(wd[k] & 0xFFFF0000u);
        m = fmaxf(m, fmaxf(fabsf(f[2 * k]), fabsf(f[2 * k + 1])));
      }
      m = fmaxf(m, dpp_f32<DPP_XOR1>(m));
      m = fmaxf(m, dpp_f32<DPP_XOR2>(m));
      const uint32_t code = fp4_query_code(m);
      if (i < 64 * 16) {
        *(uint32_t*)(qc + (i >> 4) * 64 + (i & 15) * 4) = f32x8_to_e2m1x8(f, code);
        if ((i & 3) == 0) qc[64 * 64 + (i >> 4) * 4 + ((i & 15) >> 2)] = (uint8_t)code;
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
      const int i = threadIdx.x + u * NT;
      if (i < p.heads * 16) *(uint4*)(L.q + (i >> 4) * IDX_QROW + (i & 15) * 8) = qv[u];
    }
  }
  if (threadIdx.x < p.heads) L.w[threadIdx.x] = wv;
  for (int b = threadIdx.x; b < IDX_BINS; b += NT) L.hist[b] = 0;
  __syncthreads();
  const int gw0 = wave * GPW;  // this wave's first group
  static_assert(GPW % 4 == 0, "a wave's groups fill whole pages");
  // the wave's pages (4 groups each) as uniform base addresses: a key load is that base
  // plus a per-lane offset plus an immediate, no vector address arithmetic
  constexpr int PPW = GPW / 4;
  const uint8_t* pbase[PPW];
  const uint8_t* sbase[PPW];
#pragma unroll
  for (int q = 0; q < PPW; ++q) {
    const size_t pg = __builtin_amdgcn_readfirstlane(lds_pages[gw0 / 4 + q]);
    if constexpr (F8) {
      pbase[q] = p.cache + pg * IDX_FP8_PAGE;
      sbase[q] = pbase[q] + IDX_FP8_VALUES;
    } else {
      pbase[q] = p.cache + pg * IDX_PAGE_CODES;
      sbase[q] = p.cscale + pg * IDX_PAGE_SCALES;
    }
  }
  // lane (c16, g) of group j holds dims 32g .. 32g + 31 of key 16 (j & 3) + c16.  FP4:
  // chunk g's 16 code bytes, and one scale dword a page holds the lane's four keys'
  // E8M0 bytes (j & 3 = 0..3).  FP8: tiles 2g and 2g + 1 of the key's 16-token block,
  // 16 bytes each, 256 B apart, and the key's f32 scale.
  const uint32_t off_code = F8 ? g * 512 + c16 * 16 : g * 1024 + c16 * 16;
  const uint32_t off_scale = F8 ? c16 * 4 : g * 64 + c16 * 4;
  uint4 code[GPW];
  uint4 code_hi[F8 ? GPW : 1];
  float ksc[F8 ? GPW : 1];
  uint32_t sw[PPW];
  // a rolling window of KWIN key groups in flight: group j + KWIN - 1 is issued as
  // group j is widened (a full window of 16 a wave, 160 KiB a CU at once, delays every
  // CU's first groups behind the whole chip's requests)
  constexpr int KWIN = 4;
  auto issue = [&](int j) {
    if constexpr (F8) {
      const uint8_t* b = pbase[j >> 2] + off_code + (j & 3) * 2048;
      code[j] = ld_stream16(b);
      code_hi[j] = ld_stream16(b + 256);
      ksc[j] = *(const float*)(sbase[j >> 2] + off_scale + (j & 3) * 64);
    } else {
      code[j] = ld_stream16(pbase[j >> 2] + off_code + (j & 3) * 256);
      if ((j & 3) == 0) sw[j >> 2] = *(const uint32_t*)(sbase[j >> 2] + off_scale);
    }
  };
#pragma unroll
  for (int j = 0; j < KWIN; ++j) issue(j);
  const int nhg = p.heads >> 4;
  // A operands: q of head 16*hg + c16, dims 32g + 8s .. +7 (FP4Q: dims 32g .. 32g + 31
  // as codes, and their E8M0); head weights of rows 4g+i
  bf16x8 qa[4][4];
  i32x8 qa4[4];
  int qs4[4];
  float wt[4][4];
  if constexpr (Q4) {
    const uint8_t* qc = (const uint8_t*)L.q;
#pragma unroll
    for (int hg = 0; hg < 4; ++hg) {
      const uint4 c = *(const uint4*)(qc + (hg * 16 + c16) * 64 + 16 * g);
      qa4[hg] = i32x8{(int)c.x, (int)c.y, (int)c.z, (int)c.w, 0, 0, 0, 0};
      qs4[hg] = qc[64 * 64 + (hg * 16 + c16) * 4 + g];
    }
  }
#pragma unroll
  for (int hg = 0; hg < 4; ++hg) {
    if (hg < nhg) {
      const bf16_t* qr = L.q + (hg * 16 + c16) * IDX_QROW + 32 * g;
      if constexpr (!Q4) {
#pragma unroll
        for (int s = 0; s < 4; ++s) qa[hg][s] = __builtin_bit_cast(bf16x8, *(const uint4*)(qr + 8 * s));
      }
      const uint2 wv = *(const uint2*)(L.w + hg * 16 + 4 * g);
      wt[hg][0] = __uint_as_float(wv.x << 16);
      wt[hg][1] = __uint_as_float(wv.x & 0xFFFF0000u);
      wt[hg][2] = __uint_as_float(wv.y << 16);
      wt[hg][3] = __uint_as_float(wv.y & 0xFFFF0000u);
    } else {
      if constexpr (!Q4) {
#pragma unroll
        for (int s = 0; s < 4; ++s) qa[hg][s] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) wt[hg][i] = 0.f;
    }
  }
  float* srow = p.scores + (size_t)r * p.max_ctx;
  float* sc = keep ? keep : L.sc;
  // software pipeline: group j + 1's keys widened and its MFMAs issued before group
  // j's head sums, so that the matrix cores and the vector ALUs overlap
  auto keys = [&](int j, bf16x8* kb) {
    if (j >= 1 && j + KWIN - 1 < GPW) issue(j + KWIN - 1);
    if constexpr (F8) {
      kb[0] = e4m3x8_to_bf16(code[j].x, code[j].y);
      kb[1] = e4m3x8_to_bf16(code[j].z, code[j].w);
      kb[2] = e4m3x8_to_bf16(code_hi[j].x, code_hi[j].y);
      kb[3] = e4m3x8_to_bf16(code_hi[j].z, code_hi[j].w);
    } else {
      const float sc = e8m0_to_f32(sw[j >> 2] >> (8 * (j & 3)));
      kb[0] = e2m1x8_to_bf16(code[j].x, sc);
      kb[1] = e2m1x8_to_bf16(code[j].y, sc);
      kb[2] = e2m1x8_to_bf16(code[j].z, sc);
      kb[3] = e2m1x8_to_bf16(code[j].w, sc);
    }
  };
  // all four head groups, absent ones with zero queries and weights: four
  // independent MFMA chains
  auto chain = [&](const bf16x8* kb, f32x4* acc) {
#pragma unroll
    for (int hg = 0; hg < 4; ++hg) acc[hg] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int hg = 0; hg < 4; ++hg) acc[hg] = mfma_bf16(qa[hg][q], kb[q], acc[hg]);
  };
  // group j's MFMAs, its keys widened first (FP4Q: the codes as they are, with the
  // key's E8M0 from byte j % 4 of the page's scale dword)
  auto group = [&](int j, f32x4* acc) {
    if constexpr (Q4) {
      if (j >= 1 && j + KWIN - 1 < GPW) issue(j + KWIN - 1);
      const i32x8 kb4 = {(int)code[j].x, (int)code[j].y, (int)code[j].z, (int)code[j].w, 0, 0, 0, 0};
      const int ks = (int)(sw[j >> 2] >> (8 * (j & 3)));
#pragma unroll
      for (int hg = 0; hg < 4; ++hg) acc[hg] = mfma_same<4>(qa4[hg], kb4, f32x4{0.f, 0.f, 0.f, 0.f}, qs4[hg], ks);
    } else {
      bf16x8 kb[4];
      keys(j, kb);
      chain(kb, acc);
    }
  };
  // a lane's 16 heads of group j; every fourth group the four lane groups' sums are
  // combined for four groups at once, (g0 + g1) + (g2 + g3) as a single group's would
  // be, leaving group j - 3 + g's scores in lane group g: one store and one count a lane
  float part[4];
  auto finish = [&](int j, const f32x4* acc) {
    float s = 0.f;
#pragma unroll
    for (int hg = 0; hg < 4; ++hg)
#pragma unroll
      for (int i = 0; i < 4; ++i) s += relu_bits(acc[hg][i]) * wt[hg][i];
    if constexpr (F8) s *= ksc[j];  // the lane's key's scale (column c16 of group j)
    part[j & 3] = s;
    if ((j & 3) == 3) {
      // rows 0, 2 of the first swap hold groups 0 / 2 (row pairs 01, 23), rows 1, 3
      // groups 1 / 3; the 32-lane swap then pairs the halves
      const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(part[0]), __float_as_uint(part[1]), false, false);
      const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(part[2]), __float_as_uint(part[3]), false, false);
      const float pa = __uint_as_float(a[0]) + __uint_as_float(a[1]);
      const float pb = __uint_as_float(b[0]) + __uint_as_float(b[1]);
      const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(pa), __float_as_uint(pb), false, false);
      const float t = __uint_as_float(c[0]) + __uint_as_float(c[1]);
      const int loc = (gw0 + j - 3) * 16 + lane;
      if (k_begin + loc < k_end) {
        sc[loc] = t;
        atomicAdd(&L.hist[radix_key(t) >> 20], 1);
      }
    }
  };
  static_assert(GPW % 2 == 0, "groups go in pairs");
  f32x4 acc0[4], acc1[4];
  group(0, acc0);
#pragma unroll
  for (int j = 0; j < GPW; j += 2) {
    group(j + 1, acc1);
    finish(j, acc0);
    if (j + 2 < GPW) group(j + 2, acc0);
    finish(j + 1, acc1);
  }
  __syncthreads();
  for (int i = 4 * threadIdx.x; (!keep || p.scores_out) && i < k_end - k_begin; i += 4 * NT) {
    if (k_begin + i + 4 <= k_end) {
      st_dev_16(srow + k_begin + i, make_uint4(__float_as_uint(sc[i]), __float_as_uint(sc[i + 1]),
                                               __float_as_uint(sc[i + 2]), __float_as_uint(sc[i + 3])));
    } else {
      for (int u = 0; u < 4 && k_begin + i + u < k_end; ++u) st_dev_f32(srow + k_begin + i + u, sc[i + u]);
    }
  }
  // the chunk's counts into the row's histograms (device atomics, nonzero bins): two
  // adjacent fine bins a 64-bit add (no carry crosses: a row holds < 2^17 keys), half
  // the atomic lanes
  unsigned long long* gh2 = (unsigned long long*)(p.hist + (size_t)r * IDX_BINS);
  for (int b2 = threadIdx.x; b2 < IDX_BINS / 2; b2 += NT) {
    const uint2 v = *(const uint2*)(L.hist + 2 * b2);
    if (v.x | v.y)
      __hip_atomic_fetch_add(gh2 + b2, (unsigned long long)v.x | ((unsigned long long)v.y << 32), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
  int* ch = p.chist + (size_t)r * IDX_CBINS;
  for (int c = threadIdx.x; c < IDX_CBINS; c += NT) {
    int v = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) v += L.hist[16 * c + i];
    if (v) atomicAdd(ch + c, v);
  }
  __syncthreads();
}

// the scores of either index cache format (a uniform branch, once a task)
template <int NT>
MK2_DEV void idx_score(const IdxDev& p, int r, int chunk, IdxScoreLds& L, float* keep = nullptr) {
  if (p.kfmt == IDX_KEYS_FP8)
    idx_score_keys<NT, IDX_KEYS_FP8>(p, r, chunk, L, keep);
  else if (p.kfmt == IDX_KEYS_FP4Q)
    idx_score_keys<NT, IDX_KEYS_FP4Q>(p, r, chunk, L, keep);
  else
    idx_score_keys<NT, IDX_KEYS_FP4>(p, r, chunk, L, keep);
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
  const Scan3 inc = {wave_incl_scan(v.a), wave_incl_scan(v.b), wave_incl_scan(v.c)};
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

// One wave: the bin of hist[nbins] (LDS, nbins a multiple of 64, at most 4096) where
// the count from the top reaches `need`, and through *above the count of the bins
// above it.  Lane l owns the bins nbins - per*(l+1) .. nbins - per*l - 1; the lane L
// whose run holds the bin found, its run is spread over lanes 0 .. per - 1 (one bin a
// lane, from the top) and scanned again.
MK2_DEV int wave_find_bin(const int* hist, int nbins, int need, int* above) {
  const int lane = threadIdx.x & 63, per = nbins >> 6;
  const int hi = nbins - per * lane - 1;  // this lane's highest bin
  int sum = 0;
  // the lanes' runs start `per` words apart: rotate the order so they use distinct banks
  for (int i = 0; i < per; ++i) sum += hist[hi - ((i + lane) & (per - 1))];
  const int inc = wave_incl_scan(sum), excl = inc - sum;
  const uint64_t hit = __ballot(excl < need && inc >= need);
  const int L = hit ? __ffsll((long long)hit) - 1 : 63;
  const int hiL = nbins - per * L - 1, aL = __builtin_amdgcn_readlane(excl, L);
  const int h = lane < per ? hist[hiL - lane] : 0;
  const int a = aL + wave_incl_scan(h);  // the count down to bin hiL - lane
  const uint64_t hit2 = __ballot(lane < per && a >= need);
  const int i = hit2 ? __ffsll((long long)hit2) - 1 : per - 1;
  *above = hit2 ? __builtin_amdgcn_readlane(a - h, i) : aL;
  return hiL - i;
}

// One wave: the 12-bit bin b1 of row r's k-th key from the two-level histogram in
// global memory (256 coarse bins, then the 16 fine bins of the coarse one), and the
// count of keys above it.
MK2_DEV int wave_threshold(const IdxDev& p, int r, int k, int* above) {
  const int lane = threadIdx.x & 63;
  const int* ch = p.chist + (size_t)r * IDX_CBINS;
  const int* fh = p.hist + (size_t)r * IDX_BINS;
  int c[4], sum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c[i] = ld_dev_i32(ch + IDX_CBINS - 1 - 4 * lane - i);
    sum += c[i];
  }
  int inc = wave_incl_scan(sum), excl = inc - sum;
  uint64_t hit = __ballot(excl < k && inc >= k);
  int L = hit ? __ffsll((long long)hit) - 1 : 63;
  int cb = 0, ca = 0;
  if (lane == L) {
    int a = excl;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (a < k && a + c[i] >= k) {
        cb = IDX_CBINS - 1 - 4 * lane - i;
        ca = a;
      }
      a += c[i];
    }
  }
  cb = __builtin_amdgcn_readlane(cb, L);
  ca = __builtin_amdgcn_readlane(ca, L);
  const int f = lane < 16 ? ld_dev_i32(fh + 16 * cb + 15 - lane) : 0;
  inc = ca + wave_incl_scan(f);
  excl = inc - f;
  hit = __ballot(lane < 16 && excl < k && inc >= k);
  L = hit ? __ffsll((long long)hit) - 1 : 15;
  *above = __builtin_amdgcn_readlane(excl, L);
  return 16 * cb + 15 - L;
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
  const int inc = wave_incl_scan(v);
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

constexpr int TOPK_CAP = 16384;  // candidates the select keeps in LDS
constexpr int TOPK_MAXN = 65536; // positions a row

struct TopkLds {
  int hist[IDX_BINS];
  int scratch[1024 + 1024 / 64 + 8];
  int offs[TOPK_MAXN / IDX_CHUNK + 8];
  int res[4];
  uint32_t ckey[TOPK_CAP];
  uint16_t cpos[TOPK_CAP];
  int gcount[2][TOPK_CAP / 64];  // per (round, wave): counts above / equal to the k-th key, then offsets
};

// Row r's histograms back to zero (every reader is done): the fine bins of each
// nonzero coarse bin, then the coarse bins.
template <int NT>
MK2_DEV void idx_clear_hist(const IdxDev& p, int r) {
  int* ch = p.chist + (size_t)r * IDX_CBINS;
  int* fh = p.hist + (size_t)r * IDX_BINS;
  for (int c = threadIdx.x; c < IDX_CBINS; c += NT) {
    if (ld_dev_i32(ch + c)) {
#pragma unroll
      for (int i = 0; i < 16; ++i) st_dev_i32(fh + 16 * c + i, 0);
      st_dev_i32(ch + c, 0);
    }
  }
}

// ---------------------------------------------------------------- stage: slice
// Task (row r, chunk), with b1 the 12-bit bin of the row's k-th key: the chunk's keys
// above bin b1 all make the list, and go to it directly, in position order, after
// the row's earlier chunks' (the list's first part); the keys in bin b1 go to
// cand[r][chunk * IDX_CHUNK ..], in position order, for the row's select to finish
// the list.  The chunk's two counts are published in ccount[r][chunk] first, then its
// bin-b1 keys are stored and `published()` runs (every thread, every path: the
// persistent layer counts the chunk out there, so that the row's select can start
// while the slices still list their keys above the bin); then the task waits for the
// earlier chunks' counts (tasks only wait on chunks of lower index, which publish
// before they wait, so with every task started every wait ends; a wait past its
// deadline of `wait_ticks` (WaitClock), or the sticky error word `err` set, gives up
// and sets it).  `kept`: the
// chunk's scores in LDS (its score task's `keep`), or null: read from `scores`.
// Returns whether S.res[0..1] now hold b1 and the count above it.
constexpr int CC_FLAG = 1 << 30;
struct NoPub {
  MK2_DEV void operator()() const {}
};
template <int NT, class Pub = NoPub>
MK2_DEV bool idx_slice(const IdxDev& p, int r, int chunk, TopkLds& S, uint32_t wait_ticks, int* err, uint32_t tag,
                       Pub published = Pub(), const float* kept = nullptr) {
  constexpr int PER = IDX_CHUNK / NT;  // consecutive positions a thread
  static_assert(PER % 4 == 0, "a thread reads whole 16-byte groups of scores");
  const int tid = threadIdx.x;
  const int n = p.ctx[r], k = p.topk;
  const int k_begin = chunk * IDX_CHUNK;
  int* cnt_out = p.ccount + (size_t)r * p.nchk + chunk;
  if (n <= k || k_begin >= n) {
    if (tid == 0) st_dev_i32(cnt_out, CC_FLAG);
    published();
    return false;
  }
  // the chunk's scores first: their loads overlap the threshold search
  const float* srow = p.scores + (size_t)r * p.max_ctx;
  const int base = k_begin + tid * PER;
  uint4 raw[PER / 4];
#pragma unroll
  for (int q = 0; q < PER / 4; ++q)
    raw[q] = base + 4 * q >= n ? make_uint4(0, 0, 0, 0)
             : kept            ? *(const uint4*)(kept + tid * PER + 4 * q)
                               : ldp_16(srow + base + 4 * q);
  if (tid < 64) {
    int above;
    const int b1 = wave_threshold(p, r, k, &above);
    if (tid == 0) { S.res[0] = b1; S.res[1] = above; }
  }
  __syncthreads();
  const uint32_t b1 = (uint32_t)S.res[0];
  uint32_t key[PER];
#pragma unroll
  for (int q = 0; q < PER / 4; ++q) {
    key[4 * q] = radix_key(__uint_as_float(raw[q].x));
    key[4 * q + 1] = radix_key(__uint_as_float(raw[q].y));
    key[4 * q + 2] = radix_key(__uint_as_float(raw[q].z));
    key[4 * q + 3] = radix_key(__uint_as_float(raw[q].w));
  }
  int m1 = 0, mb = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const bool valid = base + i < n;
    m1 += (valid && (key[i] >> 20) > b1) ? 1 : 0;
    mb += (valid && (key[i] >> 20) == b1) ? 1 : 0;
  }
  Scan3 tot;
  const Scan3 off = block_scan3<NT>(Scan3{m1, mb, 0}, &tot, S.scratch);
  if (tid == 0) st_dev_i32(cnt_out, CC_FLAG | tot.a | (tot.b << 15));
  uint2* dst = p.cand + (size_t)r * p.max_ctx + k_begin;
  int at = off.b;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (base + i < n && (key[i] >> 20) == b1) {
      st_dev_8(dst + at, make_uint2(key[i], (uint32_t)(base + i)));
      ++at;
    }
  }
  published();
  // the keys above bin b1 in the row's earlier chunks (nchk <= 64: a lane a chunk)
  if (tid < 64) {
    const int lane = tid;
    int v = CC_FLAG;
    if (chunk > 0) {
      const int* cc = p.ccount + (size_t)r * p.nchk;
      WaitClock wc;
      for (int polls = 1;; ++polls) {
        v = lane < chunk ? ld_dev_i32(cc + lane) : CC_FLAG;
        if (__ballot((v & CC_FLAG) == 0) == 0) break;
        if (wc.expired(wait_ticks) || ((polls & 31) == 0 && err && ld_dev_i32(err))) {
          if (lane == 0 && err) atomicOr(err, 1);
          break;
        }
      }
    }
    int pre = lane < chunk ? (v & 0x7FFF) : 0;  // a count not yet published reads 0
    pre = __builtin_amdgcn_readlane(wave_incl_scan(pre), 63);
    if (tid == 0) S.res[2] = pre;
  }
  __syncthreads();
  const ListOut lo = list_out(p, r, tag);
  at = S.res[2] + off.a;  // < the count above bin b1 < k (checked all the same)
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (base + i < n && (key[i] >> 20) > b1) {
      if (at < k) lo.put(at, base + i);
      ++at;
    }
  }
  return true;
}

// The list's bin-b1 part when more than TOPK_CAP keys share bin b1 (a row whose keys
// crowd into one bin): the k-th key's radix select and the list entries base ..
// base + k - 1, streamed over the candidates in global memory, NT at a time in
// position order.
template <int NT>
MK2_DEV void topk_stream(const IdxDev& p, int r, uint32_t kbase, int m, int k, int base, TopkLds& S,
                         const ListOut& lo) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nchk = p.nchk;
  const uint2* cr = p.cand + (size_t)r * p.max_ctx;
  auto cand_d = [&](int j) -> uint32_t {  // candidate j (position order) - kbase
    int lo = 0, hi = nchk;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (S.offs[mid] <= j) lo = mid;
      else hi = mid;
    }
    return ldp_u32(cr + (size_t)lo * IDX_CHUNK + (j - S.offs[lo])) - kbase;
  };
  auto cand_pos = [&](int j) -> int {
    int lo = 0, hi = nchk;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (S.offs[mid] <= j) lo = mid;
      else hi = mid;
    }
    return (int)ldp_8(cr + (size_t)lo * IDX_CHUNK + (j - S.offs[lo])).y;
  };
  uint32_t dmax = 0;
  for (int j = tid; j < m; j += NT) dmax = max(dmax, cand_d(j));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) dmax = max(dmax, (uint32_t)__shfl_xor((int)dmax, o, 64));
  __syncthreads();
  if (lane == 0) S.scratch[wave] = (int)dmax;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NW; ++w) dmax = max(dmax, (uint32_t)S.scratch[w]);
  // radix select of the k-th d, 12 bits at a time
  int hib = dmax ? 32 - __clz(dmax) : 32;
  uint32_t prefix = 0;
  int need = k;
  while (hib > 0) {
    const int lob = hib > 12 ? hib - 12 : 0;
    const int nb = 1 << (hib - lob);
    __syncthreads();
    for (int i = tid; i < nb; i += NT) S.hist[i] = 0;
    __syncthreads();
    const uint32_t mask = (uint32_t)(nb - 1);
    const uint32_t hmask = hib >= 32 ? 0u : ~((1u << hib) - 1u);
    const uint32_t hpfx = hib >= 32 ? 0u : (prefix << hib);
    for (int j = tid; j < m; j += NT) {
      const uint32_t v = cand_d(j);
      if ((v & hmask) == hpfx) atomicAdd(&S.hist[(v >> lob) & mask], 1);
    }
    __syncthreads();
    int above;
    const int b = find_bin<NT>(S.hist, nb, need, &above, S.scratch);
    need -= above;
    prefix = (prefix << (hib - lob)) | (uint32_t)b;
    hib = lob;
  }
  const uint32_t T = prefix;
  const int above_T = k - need, ties_needed = need;
  const uint32_t tb = (T + kbase) >> 20;
  // the list, NT candidates a round in position order
  int o1 = 0, o2 = 0, r3 = 0;  // running group counts before this round
  int n1 = 0;                  // keys of group 1 in all: counted first
  for (int j = tid; j < m; j += NT) {
    const uint32_t v = cand_d(j);
    n1 += ((v + kbase) >> 20) > tb;
  }
  n1 = block_sum_int<NT>(n1, S.scratch);
  for (int j0 = 0; j0 < m; j0 += NT) {
    const int j = j0 + tid;
    const uint32_t v = j < m ? cand_d(j) : 0u;
    const bool g1 = j < m && ((v + kbase) >> 20) > tb;
    const bool g2 = j < m && !g1 && v > T;
    const bool g3 = j < m && v == T;
    Scan3 tot;
    const Scan3 off = block_scan3<NT>(Scan3{g1, g2, g3}, &tot, S.scratch);
    int dst = -1;
    if (g1) dst = o1 + off.a;
    else if (g2) dst = n1 + o2 + off.b;
    else if (g3 && r3 + off.c < ties_needed) dst = above_T + r3 + off.c;
    if (dst >= 0 && dst < k) lo.put(base + dst, cand_pos(j));
    o1 += tot.a;
    o2 += tot.b;
    r3 += tot.c;
  }
}

// The list entries base .. k - 1 from the m <= TOPK_CAP keys of bin b1 in LDS
// (position order): the need = k - base largest by their low 20 bits, ties by
// position.  Two 10-bit radix digits, each located by one wave over its own histogram
// (S.hist[1024 * pass ..], cleared by the caller; the first digit's filled by the
// caller as it gathers the keys); then the keys above the k-th key in position
// order, then the keys equal to it, as many as fill.  Round
// i gives thread t the candidate j = i * NT + t, so lanes read consecutive words; a
// candidate's rank in its group is its wave's offset for the round (one scan over all
// (round, wave) counts) plus the ballot count of the lanes below it.
template <int NT, int CPT>
MK2_DEV void bin_select(TopkLds& S, int m, int base, int k, const ListOut& lo) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
  const int nr = (m + NT - 1) / NT;  // rounds that hold candidates (<= CPT)
  int need = k - base;
  uint32_t prefix = 0;  // the digits found so far
#pragma unroll 1
  for (int pass = 0; pass < 2; ++pass) {
    int* h = S.hist + 1024 * pass;
    if (pass == 1) {  // the first digit's histogram was built as the candidates were gathered
      for (int j = tid; j < m; j += NT) {
        const uint32_t v = S.ckey[j] & 0xFFFFFu;
        if ((v >> 10) == prefix) atomicAdd(&h[v & 1023u], 1);
      }
      __syncthreads();
    }
    if (tid < 64) {
      int ab;
      const int b = wave_find_bin(h, 1024, need, &ab);
      if (tid == 0) { S.res[0] = b; S.res[1] = ab; }
    }
    __syncthreads();
    // every thread reads S.res before it reaches the next pass's barrier, after which
    // wave 0 rewrites it
    prefix = (prefix << 10) | (uint32_t)S.res[0];
    need -= S.res[1];
  }
  const uint32_t T = prefix;              // low 20 bits of the k-th key
  const int ties = need, n_gt = k - base - need;
  // group counts per (round, wave): 0 = above T, 1 = equal to T
#pragma unroll 4
  for (int i = 0; i < nr; ++i) {
    const int j = i * NT + tid;
    const bool valid = j < m;
    const uint32_t low = valid ? S.ckey[j] & 0xFFFFFu : 0u;
    const int n2 = __popcll(__ballot(valid && low > T));
    const int n3 = __popcll(__ballot(valid && low == T));
    if (lane == 0) {
      S.gcount[0][i * NW + wave] = n2;
      S.gcount[1][i * NW + wave] = n3;
    }
  }
  __syncthreads();
  // exclusive scans of the two count sequences, in (round, wave) order
  if (wave < 2) {
    constexpr int PER = (CPT * NW + 63) / 64;
    const int E = nr * NW;
    int* gc = S.gcount[wave];
    int v[PER], sum = 0;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      v[e] = lane * PER + e < E ? gc[lane * PER + e] : 0;
      sum += v[e];
    }
    int run = wave_incl_scan(sum) - sum;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      if (lane * PER + e < E) gc[lane * PER + e] = run;
      run += v[e];
    }
  }
  __syncthreads();
#pragma unroll 4
  for (int i = 0; i < nr; ++i) {
    const int j = i * NT + tid;
    const bool valid = j < m;
    const uint32_t low = valid ? S.ckey[j] & 0xFFFFFu : 0u;
    const bool g2 = valid && low > T, g3 = valid && low == T;
    const uint64_t b2m = __ballot(g2), b3m = __ballot(g3);
    const int e = i * NW + wave;
    int dst = -1;
    if (g2) dst = base + S.gcount[0][e] + __popcll(b2m & below);
    else if (g3) {
      const int r3 = S.gcount[1][e] + __popcll(b3m & below);
      if (r3 < ties) dst = base + n_gt + r3;
    }
    if (dst >= 0 && dst < k) lo.put(dst, (int)S.cpos[j]);
  }
}

// The same list part from the 2048-bin histogram of the candidates' bits 19 .. 9 (built
// as they were gathered), when the bin b of the need-th largest holds at most 64 of them
// (else false, and nothing is written): every candidate of a higher bin lies above the
// k-th key; one wave ranks bin b's few by (low bits desc, candidate order) and finds the
// k-th key T and the count above it; then one block scan of (above T, equal to T) over
// the candidates in their order (position order) places every entry, the reference's
// order: the keys above the k-th, then the ties, lowest positions first.
template <int NT>
MK2_DEV bool bin_select_fast(TopkLds& S, int m, int base, int k, const ListOut& lo) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int need = k - base;  // >= 1: the k-th key lies in bin b1
  if (tid < 64) {
    int ab;
    const int bb = wave_find_bin(S.hist, 2048, need, &ab);
    if (tid == 0) {
      S.res[0] = bb;
      S.res[1] = ab;
      S.res[2] = 0;
    }
  }
  __syncthreads();
  const uint32_t bb = (uint32_t)S.res[0];
  const int above = S.res[1];
  const int inb = S.hist[bb];
  if (inb > 64) return false;  // uniform: every thread read the same words
  // bin b's candidates (their indices, in any order)
  for (int j = tid; j < m; j += NT)
    if (((S.ckey[j] & 0xFFFFFu) >> 9) == bb) S.scratch[atomicAdd(&S.res[2], 1)] = j;
  __syncthreads();
  if (tid < 64) {
    const int j = lane < inb ? S.scratch[lane] : 0;
    const uint32_t key = lane < inb ? (S.ckey[j] & 0x1FFu) : 0u;
    int rank = 0;  // bin b's candidates before this one in (key desc, candidate asc)
    for (int o = 0; o < inb; ++o) {
      const uint32_t ko = (uint32_t)__builtin_amdgcn_readlane((int)key, o);
      const int jo = __builtin_amdgcn_readlane(j, o);
      rank += (ko > key || (ko == key && jo < j)) ? 1 : 0;
    }
    const int need2 = need - above;  // 1 .. inb
    const uint64_t hit = __ballot(lane < inb && rank == need2 - 1);
    const uint32_t t9 = (uint32_t)__builtin_amdgcn_readlane((int)key, __ffsll((long long)hit) - 1);
    const int gt = __popcll(__ballot(lane < inb && key > t9));
    if (tid == 0) {
      S.res[0] = (int)((bb << 9) | t9);
      S.res[1] = above + gt;
    }
  }
  __syncthreads();
  const uint32_t T = (uint32_t)S.res[0];  // low 20 bits of the k-th key
  const int n_gt = S.res[1], ties = need - n_gt;
  // thread t takes candidates t c .. t c + c - 1: a count pass, the scan, an emit pass
  const int c = (m + NT - 1) / NT, j0 = tid * c;
  int na = 0, ne = 0;
  for (int i = 0; i < c; ++i) {
    const int j = j0 + i;
    if (j < m) {
      const uint32_t low = S.ckey[j] & 0xFFFFFu;
      na += low > T ? 1 : 0;
      ne += low == T ? 1 : 0;
    }
  }
  Scan3 tot;
  const Scan3 off = block_scan3<NT>(Scan3{na, ne, 0}, &tot, (int*)S.gcount);
  int ra = off.a, re = off.b;
  for (int i = 0; i < c; ++i) {
    const int j = j0 + i;
    if (j >= m) break;
    const uint32_t low = S.ckey[j] & 0xFFFFFu;
    int dst = -1;
    if (low > T) {
      dst = base + ra++;
    } else if (low == T) {
      if (re < ties) dst = base + n_gt + re;
      ++re;
    }
    if (dst >= 0 && dst < k) lo.put(dst, (int)S.cpos[j]);
  }
  return true;
}

// --------------------------------------------------------------- stage: select
// Task (row r), once every slice of the row is done: the list's bin-b1 part.  The
// keys above bin b1 (above1 of them) are already listed by the slices; of the keys in
// bin b1 the need = k - above1 largest follow, as list entries above1 .. k - 1.
// `known`: S.res[0..1] already hold b1 and above1 (the workgroup ran one of the
// row's slices just before).
template <int NT>
MK2_DEV void idx_select(const IdxDev& p, int r, TopkLds& S, uint32_t tag, bool known = false) {
  constexpr int CPT = TOPK_CAP / NT;                  // candidates a thread
  constexpr int TPC = NT / (TOPK_MAXN / IDX_CHUNK);   // gather threads a chunk
  constexpr int SPEC = 8;                             // candidates a thread loads with the counts
  const int tid = threadIdx.x;
  const int n = p.ctx[r];
  const int k = p.topk;
  const ListOut lo = list_out(p, r, tag);
  if (n <= k) {
    for (int i = tid; i < k; i += NT) lo.put(i, i < n ? i : -1);
    return;
  }
  const int nchk = p.nchk;
  if (!known && tid < 64) {
    int above;
    const int b1 = wave_threshold(p, r, k, &above);
    if (tid == 0) { S.res[0] = b1; S.res[1] = above; }
  }
  for (int i = tid; i < 2048; i += NT) S.hist[i] = 0;  // the bits-19..9 histogram
  // one round trip: each chunk's count of bin-b1 keys and its first SPEC * TPC of them
  const int c = tid / TPC, sub = tid % TPC;
  const uint2* src = p.cand + (size_t)r * p.max_ctx + (size_t)c * IDX_CHUNK;
  int cnt = 0;
  uint2 v[SPEC];
  if (c < nchk) {
    const int lim = min(IDX_CHUNK, p.max_ctx - c * IDX_CHUNK);  // the chunk's area (>= 64)
    // device-coherent: the slices polled this line (ld_dev) while later chunks' counts
    // were still unpublished, so a plain load could hit a copy taken before them
    cnt = min((ld_dev_i32(p.ccount + (size_t)r * nchk + c) >> 15) & 0x7FFF, lim);
#pragma unroll
    for (int u = 0; u < SPEC; ++u) v[u] = ldp_8(src + min(sub + u * TPC, lim - 1));
  }
  Scan3 tot;  // a chunk's count enters at its last thread: every thread of the chunk gets its offset
  const int off = block_scan3<NT>(Scan3{sub == TPC - 1 ? cnt : 0, 0, 0}, &tot, S.scratch).a;
  if (sub == 0 && c < nchk) S.offs[c] = off;
  if (tid == 0) S.offs[nchk] = tot.a;
  __syncthreads();
  const uint32_t b1 = (uint32_t)S.res[0];
  const int above1 = S.res[1];
  const int m = tot.a;
  if (m > TOPK_CAP) {
    // keys relative to the bottom of bin b1: d >= 1 for every candidate
    topk_stream<NT>(p, r, (b1 << 20) - 1u, m, k - above1, above1, S, lo);
    return;
  }
  if (c < nchk) {
#pragma unroll
    for (int u = 0; u < SPEC; ++u) {
      const int i = sub + u * TPC;
      if (i < cnt) {
        S.ckey[off + i] = v[u].x;
        S.cpos[off + i] = (uint16_t)v[u].y;
        atomicAdd(&S.hist[(v[u].x >> 9) & 2047u], 1);  // bits 19 .. 9 of the key
      }
    }
    for (int i0 = SPEC * TPC; i0 < cnt; i0 += SPEC * TPC) {  // a crowded chunk's rest
#pragma unroll
      for (int u = 0; u < SPEC; ++u) {
        const int i = i0 + sub + u * TPC;
        v[u] = i < cnt ? ldp_8(src + i) : make_uint2(0, 0);
      }
#pragma unroll
      for (int u = 0; u < SPEC; ++u) {
        const int i = i0 + sub + u * TPC;
        if (i < cnt) {
          S.ckey[off + i] = v[u].x;
          S.cpos[off + i] = (uint16_t)v[u].y;
          atomicAdd(&S.hist[(v[u].x >> 9) & 2047u], 1);
        }
      }
    }
  }
  __syncthreads();
  if (bin_select_fast<NT>(S, m, above1, k, lo)) return;
  // a crowded bin (keys that tie, or lie close together): the two-digit radix select,
  // its first digit's histogram (bits 19 .. 10) built again over the candidates
  for (int i = tid; i < 2 * 1024; i += NT) S.hist[i] = 0;
  __syncthreads();
  for (int j = tid; j < m; j += NT) atomicAdd(&S.hist[(S.ckey[j] >> 10) & 1023u], 1);
  __syncthreads();
  bin_select<NT, CPT>(S, m, above1, k, lo);
}

// Row r's top-k state back to zero for the next launch (every reader is done): the
// histograms and the chunk counts.
template <int NT>
MK2_DEV void idx_topk_reset(const IdxDev& p, int r) {
  idx_clear_hist<NT>(p, r);
  for (int c = threadIdx.x; c < p.nchk; c += NT) st_dev_i32(p.ccount + (size_t)r * p.nchk + c, 0);
}

// Every row's top-k state to zero, whatever a stopped launch left in it (one
// workgroup, once no other is running): all fine and coarse bins and chunk counts.
template <int NT>
MK2_DEV void idx_reset_rows(const IdxDev& p, int rows) {
  const uint4 z = make_uint4(0, 0, 0, 0);
  for (int i = threadIdx.x; i < rows * IDX_BINS / 4; i += NT) st_dev_16(p.hist + 4 * i, z);
  for (int i = threadIdx.x; i < rows * IDX_CBINS / 4; i += NT) st_dev_16(p.chist + 4 * i, z);
  for (int i = threadIdx.x; i < rows * p.nchk; i += NT) st_dev_i32(p.ccount + i, 0);
}

}  // namespace mk2
