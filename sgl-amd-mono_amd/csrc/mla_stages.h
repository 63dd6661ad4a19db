// Sparse-MLA stages of the K2 layer: split attention over gathered FP8 latent-KV
// rows, the merge of the splits, W_UV, and W_o with the residual.
//
// split task (row r, split s): 64 selected positions -> page table -> 576-byte E4M3
// rows, gathered with 16-byte loads into LDS twice: row-major (the QK operand) and,
// for the first 512 dims, transposed to [dim][key] (the PV operand, 8 keys a lane
// read).  S = q . k on bf16 MFMA (E4M3 widens exactly), x (scale_k * sm_scale); a
// split-local softmax per head; P' = p * scale_k rounded to bf16; O = P' V on bf16
// MFMA.  The split writes O (unnormalized), its max m and sum l.
// merge task (up to 4 rows, head h, half): exact combination of each row's splits ->
// o_lat (bf16), then o[r][h] = W_UV[h] o_lat on bf16 MFMA, the rows as its columns.
// oproj task (16 hidden rows): a = bf16(h + W_o o) on bf16 MFMA.
#pragma once
#include "mk2_device.h"

namespace mk2 {

constexpr int MLA_D = 576;        // latent 512 + rope 64
constexpr int MLA_LAT = 512;
constexpr int MLA_HEADS = 16;
constexpr int MLA_SPLIT = 64;     // keys a split task
constexpr int MLA_KROW = 584;     // LDS row stride of the gathered rows (bytes)
constexpr int MLA_VROW = 72;      // LDS row stride of the transposed latent (bytes)
// In the transposed latent, dim d's 4-key word w sits at word w ^ mla_vswz(d): the
// gather writes one word of 16 consecutive dims a lane, and without the swizzle all
// lanes of a store would hit one bank (16 rows of 18 words is 0 mod 32).  The swizzle
// is even, so the two words of an aligned 8-key read stay an aligned pair.
MK2_DEV int mla_vswz(int d) { return 2 * ((d >> 4) & 7); }
constexpr int MLA_NT = 256;

struct MlaDev {
  int rows, v_dim, hidden, topk, stride, nsplit;
  float sm_scale;
  const bf16_t* q;       // [rows][16][576]
  const uint8_t* kv;     // [pages][64][576]
  const float* kv_scale; // [pages][64]; null: unscaled E4M3 (scale 1)
  const int* pt;
  const int* req;
  const int* sel;        // [rows][topk]
  const uint64_t* tsel;  // the same list as tagged words (the persistent layer polls
                         // its split's entries), or null: sel
  const bf16_t* w_uv;    // [16][v_dim][512]
  const uint8_t* w_o;    // tiles of [hidden][16*v_dim]
  const bf16_t* h;       // [rows][hidden] or null
  bf16_t* out;           // [rows][hidden]
  // workspace
  bf16_t* part_o;        // [rows][nsplit][16][512] the splits' P.V, rounded to bf16
  float* part_ml;        // [rows][nsplit][16][2]
  float* o_lat_f32;      // optional [rows][16][512]
  bf16_t* o;             // [rows][16 * v_dim]
  float* ssp;            // optional [rows][hidden/16]: sums of squares of out over 16 columns
};

struct MlaSplitLds {
  uint8_t k[MLA_SPLIT * MLA_KROW];       // gathered rows, row-major
  uint8_t vt[MLA_LAT * MLA_VROW];        // latent dims transposed: [dim][key]
  bf16_t p[MLA_HEADS * (MLA_SPLIT + 8)]; // P' [head][key]
  int row[MLA_SPLIT + 1];                // cache row of each key (-1: unused); [64]: a poll gave up
  float sc[MLA_SPLIT];                   // per-key scale * sm_scale
  float kscale[MLA_SPLIT];
  float red[4][MLA_HEADS];
};

// ---------------------------------------------------------------- stage: split
// NT = 256 or 512: waves 0-3 run QK and the softmax (16 keys each), every wave
// gathers and takes a share of the PV dim tiles.
template <int NT, typename Mark = NoMark>
MK2_DEV bool mla_split(const MlaDev& p, int r, int s, MlaSplitLds& L, const TagPoll& tp, Mark mark = Mark()) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, c16 = lane & 15;
  const bool qk_wave = wave < 4;
  const int* selr = p.sel + (size_t)r * p.topk + s * MLA_SPLIT;
  const int* ptr = p.pt + (size_t)p.req[r] * p.stride;
  // q operands for this wave's QK: head c16, dims 8g + 32ks .. +7.  Wave 0 loads its
  // own behind the gather: ahead of its list poll and page-table read they would hold
  // both up (a wave's loads complete in order)
  bf16x8 qa[18];
  const bf16_t* qr = p.q + ((size_t)r * MLA_HEADS + c16) * MLA_D + 8 * g;
  auto load_q = [&] {
#pragma unroll
    for (int ks = 0; ks < 18; ++ks) qa[ks] = __builtin_bit_cast(bf16x8, *(const uint4*)(qr + 32 * ks));
  };
  if (qk_wave && wave != 0) load_q();
  // resolve the 64 positions to cache rows (one dependent round); the rows' scales
  // are loaded with the rows below.  A tagged list is polled here, one entry a lane of
  // wave 0: the split starts as soon as its own 64 entries are out.
  if (tid < MLA_SPLIT) {
    int pos;
    bool bad = false;
    if (p.tsel) {
      const uint64_t* src = p.tsel + (size_t)r * p.topk + s * MLA_SPLIT + tid;
      uint64_t w = ld_pair(src);
      WaitClock wc;
      for (int polls = 1;; polls += 2) {  // two polls in flight
        const uint64_t w1 = ld_pair(src);
        if (poll_done(pair_ready(w, tp), polls, wc, tp, &bad)) break;
        w = ld_pair(src);
        if (poll_done(pair_ready(w1, tp), polls + 1, wc, tp, &bad)) {
          w = w1;
          break;
        }
      }
      pos = (int)pair_value(w);
    } else {
      pos = ldp_i32(selr + tid);
    }
    if (tid == 0) L.row[MLA_SPLIT] = bad;  // wave-uniform
    int row = -1;
    if (pos >= 0 && pos < p.stride * 64) row = ptr[pos >> 6] * 64 + (pos & 63);
    L.row[tid] = row;
  }
  if (tid == 0) mark(0);
  __syncthreads();
  if (L.row[MLA_SPLIT]) return false;
  float ksc = 0.f;
  if (tid < MLA_SPLIT) {
    const int row = L.row[tid];
    ksc = row < 0 ? 0.f : (p.kv_scale ? p.kv_scale[row] : 1.f);
  }
  // gather: job = (4-key group kg, 16-byte dim chunk dc), 16 x 36 jobs; every load of
  // a thread is issued before the first LDS store
  constexpr int JOBS = 16 * 36, JPT = (JOBS + NT - 1) / NT;
  uint4 v[JPT][4];
#pragma unroll
  for (int it = 0; it < JPT; ++it) {
    const int job = tid + it * NT;
    const int kg = job / 36, dc = job % 36;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = job < JOBS ? L.row[kg * 4 + j] : -1;
      v[it][j] = row >= 0 ? ld_stream16(p.kv + (size_t)row * MLA_D + dc * 16) : make_uint4(0, 0, 0, 0);
    }
  }
  if (wave == 0) load_q();
  if (tid < MLA_SPLIT) {
    L.kscale[tid] = ksc;
    L.sc[tid] = ksc * p.sm_scale;
  }
#pragma unroll
  for (int it = 0; it < JPT; ++it) {
    const int job = tid + it * NT;
    if (job >= JOBS) break;
    const int kg = job / 36, dc = job % 36;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint8_t* dst = L.k + (kg * 4 + j) * MLA_KROW + dc * 16;
      *(uint2*)dst = make_uint2(v[it][j].x, v[it][j].y);
      *(uint2*)(dst + 8) = make_uint2(v[it][j].z, v[it][j].w);
    }
    if (dc < 32) {
      // transpose 4 keys x 16 dims of bytes -> 16 words of 4 keys
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t w0 = ((const uint32_t*)&v[it][0])[q], w1 = ((const uint32_t*)&v[it][1])[q];
        const uint32_t w2 = ((const uint32_t*)&v[it][2])[q], w3 = ((const uint32_t*)&v[it][3])[q];
        const uint32_t lo01 = __builtin_amdgcn_perm(w1, w0, 0x05010400u);  // b0 of w0,w1 | b1 of w0,w1
        const uint32_t hi01 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);  // b2.. | b3..
        const uint32_t lo23 = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
        const uint32_t hi23 = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
        const int d = dc * 16 + q * 4;
        const int w = (kg ^ mla_vswz(d)) * 4;  // the four dims share d >> 4
        *(uint32_t*)(L.vt + (d + 0) * MLA_VROW + w) = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
        *(uint32_t*)(L.vt + (d + 1) * MLA_VROW + w) = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
        *(uint32_t*)(L.vt + (d + 2) * MLA_VROW + w) = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
        *(uint32_t*)(L.vt + (d + 3) * MLA_VROW + w) = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
      }
    }
  }
  __syncthreads();
  // QK: wave w < 4 takes keys 16w .. 16w+15 as the MFMA columns
  const int key = (wave & 3) * 16 + c16;
  const bool valid = L.row[key] >= 0;
  float sv[4], m[4];
  if (qk_wave) {
    // every LDS read first, then two interleaved accumulator chains
    const uint8_t* krow = L.k + key * MLA_KROW + 8 * g;
    uint2 kw[18];
#pragma unroll
    for (int ks = 0; ks < 18; ++ks) kw[ks] = *(const uint2*)(krow + 32 * ks);
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 18; ks += 2) {
      acc0 = mfma_bf16(qa[ks], e4m3x8_to_bf16(kw[ks].x, kw[ks].y), acc0);
      acc1 = mfma_bf16(qa[ks + 1], e4m3x8_to_bf16(kw[ks + 1].x, kw[ks + 1].y), acc1);
    }
    const f32x4 acc = acc0 + acc1;
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = valid ? acc[i] * L.sc[key] : -INFINITY;
    // split-local softmax per head (heads 4g + i)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float mx = row16_max(sv[i]);
      if (c16 == 0) L.red[wave][4 * g + i] = mx;
    }
  }
  __syncthreads();
  float ls[4];
  if (qk_wave) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int hd = 4 * g + i;
      m[i] = fmaxf(fmaxf(L.red[0][hd], L.red[1][hd]), fmaxf(L.red[2][hd], L.red[3][hd]));
      const float pe = (valid && m[i] != -INFINITY) ? expf(sv[i] - m[i]) : 0.f;
      ls[i] = row16_sum(pe);
      L.p[hd * (MLA_SPLIT + 8) + key] = f32_to_bf16(pe * L.kscale[key]);
    }
  }
  __syncthreads();
  if (qk_wave && c16 == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) L.red[wave][4 * g + i] = ls[i];
  }
  __syncthreads();
  float* mlo = p.part_ml + (((size_t)r * p.nsplit + s) * MLA_HEADS) * 2;
  if (wave == 0 && c16 == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int hd = 4 * g + i;
      st_dev_f32(mlo + hd * 2, m[i]);
      st_dev_f32(mlo + hd * 2 + 1, L.red[0][hd] + L.red[1][hd] + L.red[2][hd] + L.red[3][hd]);
    }
  }
  // PV: wave w takes dim tiles TPW*w .. +TPW-1 (16 dims each), 2 key steps of 32
  constexpr int TPW = 32 / NW;
  bf16x8 pa[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    pa[ks] = __builtin_bit_cast(bf16x8, *(const uint4*)(L.p + c16 * (MLA_SPLIT + 8) + 32 * ks + 8 * g));
  bf16_t* orow = p.part_o + ((size_t)r * p.nsplit + s) * MLA_HEADS * MLA_LAT;
  static_assert(TPW % 2 == 0, "dim tiles go in pairs");
#pragma unroll
  for (int t = 0; t < TPW; t += 2) {
    const int d0 = (wave * TPW + t) * 16;
    f32x4 o[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      o[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int w = (8 * ks + 2 * g) ^ mla_vswz(d0 + 16 * tt);  // d0 + c16 shares d0 >> 4
        const uint2 vw = *(const uint2*)(L.vt + (d0 + 16 * tt + c16) * MLA_VROW + 4 * w);
        o[tt] = mfma_bf16(pa[ks], e4m3x8_to_bf16(vw.x, vw.y), o[tt]);
      }
    }
    // the pair's 32 columns as bf16 pairs, lane c16 taking columns 2 c16, 2 c16 + 1 of
    // them (from lanes 2 c16 and 2 c16 + 1 of the first tile, or of the second), so
    // that a row's 16 lanes store one whole 64-byte piece (half the bytes the merge
    // tasks read, each (row, head) twice)
    const int src = ((lane & 48) | ((2 * c16) & 15)) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int a0 = __builtin_amdgcn_ds_bpermute(src, __float_as_int(o[0][i]));
      const int a1 = __builtin_amdgcn_ds_bpermute(src + 4, __float_as_int(o[0][i]));
      const int b0 = __builtin_amdgcn_ds_bpermute(src, __float_as_int(o[1][i]));
      const int b1 = __builtin_amdgcn_ds_bpermute(src + 4, __float_as_int(o[1][i]));
      const bool first = c16 < 8;
      st_dev_u32(orow + (4 * g + i) * MLA_LAT + d0 + 2 * c16,
                 pack_bf16x2(__int_as_float(first ? a0 : b0), __int_as_float(first ? a1 : b1)));
    }
  }
  __syncthreads();
  return true;
}

// ---------------------------------------------------------------- stage: merge + W_UV
// Task (rows r0 .. r0 + nr - 1, head h, half hf), nr <= MLA_MRG: for each row the exact
// combination of its splits for head h -> o_lat (rounded to bf16, in LDS), then half
// hf of o[r][h] = W_UV[h] o_lat on bf16 MFMA: the half's 16-row W_UV tiles go to waves
// 1, 2, ... over all 512 latent dims, with row r0 + i's o_lat as MFMA column i (the
// W_UV bytes a task moves serve all its rows).  Every row's sums and every MFMA column
// are computed alike whatever the task's rows, and the two halves of (r, h) compute
// the same o_lat bits, so the output does not depend on either split.  A wave's first
// tile is static and loaded before `wait` (the splits' dependency); wave 0, which
// polls the dependency, loads none.
constexpr int MLA_MRG = 4;            // rows a merge task at most
constexpr int MLA_OLROW = MLA_LAT + 8; // LDS row stride (bf16) of o_lat: rows in distinct banks
struct MlaMergeLds {
  float w[MLA_MRG][2 * 1024 + 8];  // per row, per split: exp(m_s - M), then l_s (nsplit <= 1024)
  float hi[MLA_MRG][MLA_LAT];      // the second half of the splits' weighted sums
  float inv[MLA_MRG];              // 1 / sum_s l_s exp(m_s - M)
  bf16_t ol[MLA_MRG][MLA_OLROW];
};

// rows a merge task of a persistent launch takes: about one task a workgroup
MK2_DEV int mla_merge_rows(int rows, int G) { return min(MLA_MRG, max(1, rows * 2 * MLA_HEADS / G)); }

template <int NT, typename Wait = NoWait>
MK2_DEV void mla_merge_uv(const MlaDev& p, int r0, int nr, int h, int hf, MlaMergeLds& L, Wait wait = Wait()) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, c16 = lane & 15;
  const int ns = p.nsplit, nvt = p.v_dim / 16;
  const int vlo = hf ? (nvt + 1) / 2 : 0, vhi = hf ? nvt : (nvt + 1) / 2;  // this half's tiles
  const int vt0 = vlo + wave - 1;  // wave w >= 1 takes tiles vt0, vt0 + NW - 1, ...
  auto load_a = [&](int vt, bf16x8* a) {  // W_UV[h] rows vt*16 + c16, dims 128 kb + 32 g + 8 q
    const bf16_t* wrow = p.w_uv + ((size_t)h * p.v_dim + vt * 16 + c16) * MLA_LAT + 32 * g;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int q = 0; q < 4; ++q) a[kb * 4 + q] = __builtin_bit_cast(bf16x8, ld_stream16(wrow + kb * 128 + 8 * q));
  };
  bf16x8 a[16];
  if (wave >= 1 && vt0 < vhi) load_a(vt0, a);
  if (!wait()) return;
  // the splits' bf16 partials: thread t takes dims 2 (t % 256) and + 1 of every row (one
  // 32-bit load a split) over half of the splits (the first or the second), 16 loads a
  // row in flight; the second half's sums go through LDS and are added to the first's.
  // The first 16 of every row go out right behind the splits' (m, l), so that all
  // arrive in one round trip.
  static_assert(NT == 2 * (MLA_LAT / 2), "two threads a dim pair");
  const int dp = tid % (MLA_LAT / 2), sh = tid / (MLA_LAT / 2);
  const int nh = (ns + 1) / 2, sa = sh * nh, sb = min(ns, sa + nh);
  constexpr int U = 16;
  uint32_t v[MLA_MRG][U];
  auto load_po = [&](int i, int s0) {
    const uint32_t* po = (const uint32_t*)(p.part_o + ((size_t)(r0 + i) * ns * MLA_HEADS + h) * MLA_LAT) + dp;
#pragma unroll
    for (int u = 0; u < U; ++u) v[i][u] = s0 + u < sb ? ldp_u32(po + (size_t)(s0 + u) * (MLA_HEADS * MLA_LAT / 2)) : 0u;
  };
  // (m, l) of split s of row i at flat index f = i * ns + s
  auto ml_at = [&](int f) {
    const int i = f / ns, s = f - i * ns;
    return ldp_8(p.part_ml + (((size_t)(r0 + i) * ns + s) * MLA_HEADS + h) * 2);
  };
  const int nml = nr * ns;
  const uint2 ml0 = tid < nml ? ml_at(tid) : make_uint2(0, 0);
#pragma unroll
  for (int i = 0; i < MLA_MRG; ++i)
    if (i < nr) load_po(i, sa);
  if (tid < nml) {
    const int i = tid / ns, s = tid - i * ns;
    L.w[i][s] = __uint_as_float(ml0.x);
    L.w[i][ns + s] = __uint_as_float(ml0.y);
  }
  for (int f = tid + NT; f < nml; f += NT) {  // more than NT splits in the task
    const uint2 m1 = ml_at(f);
    const int i = f / ns, s = f - i * ns;
    L.w[i][s] = __uint_as_float(m1.x);
    L.w[i][ns + s] = __uint_as_float(m1.y);
  }
  __syncthreads();
  // row i on wave i: M = max_s m_s, the split weights exp(m_s - M), and 1 / sum_s l_s w_s
  if (wave < nr) {
    float* wg = L.w[wave];
    float M = -INFINITY;
    for (int s = lane; s < ns; s += 64) M = fmaxf(M, wg[s]);
    M = wave_max(M);
    float ls = 0.f;
    for (int s = lane; s < ns; s += 64) {
      const float e = wg[s] == -INFINITY ? 0.f : expf(wg[s] - M);
      wg[s] = e;
      ls += wg[ns + s] * e;
    }
    ls = wave_sum(ls);
    if (lane == 0) L.inv[wave] = ls > 0.f ? 1.0f / ls : 0.f;
  }
  __syncthreads();
  float o[MLA_MRG][2];
#pragma unroll
  for (int i = 0; i < MLA_MRG; ++i) {
    o[i][0] = o[i][1] = 0.f;
    if (i >= nr) continue;
    for (int s0 = sa; s0 < sb; s0 += U) {
      if (s0 != sa) load_po(i, s0);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float w = s0 + u < sb ? L.w[i][s0 + u] : 0.f;
        o[i][0] += __uint_as_float(v[i][u] << 16) * w;
        o[i][1] += __uint_as_float(v[i][u] & 0xFFFF0000u) * w;
      }
    }
    if (sh == 1) {
      L.hi[i][2 * dp] = o[i][0];
      L.hi[i][2 * dp + 1] = o[i][1];
    }
  }
  __syncthreads();
  if (sh == 0) {
#pragma unroll
    for (int i = 0; i < MLA_MRG; ++i) {
      if (i >= nr) break;
      const float inv = L.inv[i];
      const float f0 = (o[i][0] + L.hi[i][2 * dp]) * inv, f1 = (o[i][1] + L.hi[i][2 * dp + 1]) * inv;
      *(uint32_t*)(L.ol[i] + 2 * dp) = pack_bf16x2(f0, f1);
      if (p.o_lat_f32 && hf == 0) {
        const size_t at = ((size_t)(r0 + i) * MLA_HEADS + h) * MLA_LAT + 2 * dp;
        p.o_lat_f32[at] = f0;
        p.o_lat_f32[at + 1] = f1;
      }
    }
  }
  __syncthreads();
  // column c16: row r0 + c16 (columns past nr repeat the last row and are not stored)
  const bf16_t* olc = L.ol[min(c16, nr - 1)];
  for (int vt = vt0; wave >= 1 && vt < vhi; vt += NW - 1) {
    if (vt != vt0) load_a(vt, a);
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int q = 0; q < 4; ++q) c = mfma_bf16(a[kb * 4 + q], *(const bf16x8*)(olc + kb * 128 + 32 * g + 8 * q), c);
    if (c16 < nr) {  // column c16: v rows 4 g + i of row r0 + c16
      bf16_t* dst = p.o + (size_t)(r0 + c16) * (MLA_HEADS * p.v_dim) + h * p.v_dim + vt * 16 + 4 * g;
      st_dev_8(dst, make_uint2(pack_bf16x2(c[0], c[1]), pack_bf16x2(c[2], c[3])));
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------- stage: W_o
// Tasks (16 hidden rows nt0) and, with NTL = 2, (16 hidden rows nt1; -1: none): both
// tiles' first PF k-blocks a wave are loaded before `wait` (the attention rows'
// dependency), the rest after; the attention rows are loaded once for both.  Without
// a second tile the first is computed twice and stored once.  With `ssp` set, the
// epilogue also leaves each output row's sum of squares over the tile's 16 columns
// (the next RMSNorm's partial sums).
template <int NT, int NCG, int NTL = 1, typename Wait = NoWait>
MK2_DEV void mla_oproj(const MlaDev& p, int nt0, int nt1, float* red, Wait wait = Wait()) {
  constexpr int NW = NT / 64, PF = 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
  const int K = MLA_HEADS * p.v_dim, KB = K / 128;
  const uint8_t* tiles[NTL];
#pragma unroll
  for (int j = 0; j < NTL; ++j) tiles[j] = p.w_o + (size_t)(j == 0 || nt1 < 0 ? nt0 : nt1) * KB * 64 * 64;
  bf16x8 apf[NTL][PF][4];
#pragma unroll
  for (int j = 0; j < NTL; ++j)
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      const int kb = wave + u * NW;
      const uint4* t = (const uint4*)(tiles[j] + ((size_t)min(kb, KB - 1) * 64 + lane) * 64);
#pragma unroll
      for (int q = 0; q < 4; ++q) apf[j][u][q] = __builtin_bit_cast(bf16x8, ld_stream16(t + q));
    }
  // the residual rows (the layer's input, static) for the epilogue: entry idx = tid +
  // i * NT of the ntl * 16 * rows outputs
  const int ntl = NTL > 1 && nt1 >= 0 ? 2 : 1;
  constexpr int EPI = (NTL * 16 * 32 + NT - 1) / NT;
  float hres[EPI];
#pragma unroll
  for (int i = 0; i < EPI; ++i) {
    const int idx = threadIdx.x + i * NT;
    hres[i] = 0.f;
    if (p.h && idx < ntl * 16 * p.rows) {
      const int j = idx / (16 * p.rows), jdx = idx - j * 16 * p.rows;
      hres[i] = bf16_to_f32(p.h[(size_t)(jdx >> 4) * p.hidden + (j == 0 ? nt0 : nt1) * 16 + (jdx & 15)]);
    }
  }
  if (!wait()) return;
  f32x4 acc[NTL][NCG];
#pragma unroll
  for (int j = 0; j < NTL; ++j)
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) acc[j][cg] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto step = [&](int kb, bf16x8 (*a)[4]) {
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) {
      const int row = cg * 16 + c16;
      bf16x8 b[4];
      if (row < p.rows) {
        const bf16_t* src = p.o + (size_t)row * K + kb * 128 + 32 * g;
#pragma unroll
        for (int q = 0; q < 4; ++q) b[q] = __builtin_bit_cast(bf16x8, ldp_16(src + 8 * q));
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) b[q] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
      }
#pragma unroll
      for (int j = 0; j < NTL; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[j][cg] = mfma_bf16(a[j][q], b[q], acc[j][cg]);
    }
  };
#pragma unroll
  for (int u = 0; u < PF; ++u)
    if (wave + u * NW < KB) {
      bf16x8 a[NTL][4];
#pragma unroll
      for (int j = 0; j < NTL; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) a[j][q] = apf[j][u][q];
      step(wave + u * NW, a);
    }
  for (int kb = wave + PF * NW; kb < KB; kb += NW) {
    bf16x8 a[NTL][4];
#pragma unroll
    for (int j = 0; j < NTL; ++j) {
      const uint4* t = (const uint4*)(tiles[j] + ((size_t)kb * 64 + lane) * 64);
#pragma unroll
      for (int q = 0; q < 4; ++q) a[j][q] = __builtin_bit_cast(bf16x8, ld_stream16(t + q));
    }
    step(kb, a);
  }
#pragma unroll
  for (int j = 0; j < NTL; ++j)
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) *(f32x4*)(red + (((j * NW + wave) * NCG + cg) * 64 + lane) * 4) = acc[j][cg];
  __syncthreads();
#pragma unroll
  for (int it = 0; it < EPI; ++it) {
    const int idx = threadIdx.x + it * NT;
    if (idx >= ntl * 16 * p.rows) break;
    const int j = idx / (16 * p.rows), jdx = idx - j * 16 * p.rows;
    const int n16 = jdx & 15, row = jdx >> 4, cg = row >> 4, s16 = row & 15;
    const int l = (n16 >> 2) * 16 + s16, i = n16 & 3;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += red[(((j * NW + w) * NCG + cg) * 64 + l) * 4 + i];
    const size_t o = (size_t)row * p.hidden + (j == 0 ? nt0 : nt1) * 16 + n16;
    if (p.h) v += hres[it];
    const bf16_t ob = f32_to_bf16(v);
    st_dev_u16(p.out + o, ob);
    if (p.ssp) {  // the 16 columns of (tile, row) are one DPP row: 16 * rows and NT are multiples of 16
      const float vb = bf16_to_f32(ob);
      const float ss = row16_sum(vb * vb);
      if (n16 == 0) st_dev_f32(p.ssp + (size_t)row * (p.hidden / 16) + (j == 0 ? nt0 : nt1), ss);
    }
  }
  __syncthreads();
}

}  // namespace mk2
