// The layer front's device code (the reference's K1; the arithmetic is described in
// front.hip): the GEMV engine, the per-row and per-head stages, and the persistent
// front's counters and walk.  front.hip launches them on their own; the persistent
// layer can run the walk ahead of its stages in the same launch.
#pragma once
#include "mk2.h"
#include "mk2_device.h"

namespace mk2 {

constexpr int GV_NT = 512;
constexpr int GV_WAVES = GV_NT / 64;
constexpr int GV_CHUNK = 8;  // tiles whose partials wait in LDS for one barrier
constexpr int FR_NT = 512;

struct GemvSeg {
  const void* w;   // [rows][K] bf16 or E4M3, row-major
  const float* s;  // E4M3: f32 [ceil(rows / 128)][K / 128] block scales
  float* out;      // f32 partial planes: K part p, row m at out + p * pstride + m * ld
  int rows;        // multiple of 16
  int ld;
  long long pstride;
};

struct GemvDev {
  int M;   // rows this pass, 1..16
  int K;
  int ks;  // K parts: workgroup b takes part b % ks (the grid is a multiple of ks)
  float eps;
  const bf16_t* x;  // [M][K]: raw rows (with g) or the GEMV input as it is (g null)
  const bf16_t* g;  // RMSNorm weight [K], or null
  GemvSeg seg[2];
  int tiles0;  // 16-row tiles of segment 0
  int ntiles;
};

struct GemvLds {
  float ssum[16];
  uint4 gam[8192 / 8];
  float red[GV_CHUNK][GV_WAVES][256];
};

// One engine workgroup's work: workgroup b of nblocks (a multiple of p.ks).  KU: 64-k
// units a wave (K / ks = 8 * 64 * KU); WF: the weights' MK2_WFMT_* (bf16, E4M3
// row-major, or E4M3 in AITER's (16, 16) layout).  `wait` (the input rows'
// dependency, in the persistent front) runs once the first tile's weights are in
// flight; false from it returns false at once.  The f32 partial planes are stored
// device-coherently (the next stage may run on another XCD within the same launch).
template <int KU, int WF, typename Wait = NoWait>
MK2_DEV bool gemv_run(const GemvDev& p, int b, int nblocks, GemvLds& S, Wait wait = Wait()) {
  constexpr bool F8 = WF != MK2_WFMT_BF16, SHUF = WF == MK2_WFMT_FP8_AITER16;
  constexpr int L = F8 ? KU : 2 * KU;      // 16-byte weight loads a lane a tile
  constexpr int WIN = L <= 24 ? L : L / 2;  // loads in flight a lane
  static_assert(L % WIN == 0, "a window divides the loads of a tile");
  static_assert(!F8 || KU % 2 == 0, "FP8 slices are whole 128-k blocks");
  float* ssum = S.ssum;
  uint4* gam = S.gam;
  auto& red = S.red;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, c16 = lane & 15, g = lane >> 4;
  const int K = p.K, M = p.M;
  const int part = b % p.ks, G = nblocks / p.ks, q = b / p.ks;
  const int t0 = (int)((long long)q * p.ntiles / G), t1 = (int)((long long)(q + 1) * p.ntiles / G);
  // k map: unit u of the wave's slice holds k = kw + 64 u + 0 .. 15 for lane group g;
  // MFMA step 2u takes its first 8, step 2u + 1 the next 8 (A and B alike)
  const int kw = part * (K / p.ks) + wave * KU * 64 + 16 * g;
  const bool live = c16 < M;
  // the tile sequence: tile t of segment sid at row (t - base) * 16; this lane's row
  auto seg_of = [&](int t) { return t < p.tiles0 ? 0 : 1; };
  // In AITER's (16, 16) layout ([rows/16][K/32][2][16 rows][16 B]) the 16 bytes of
  // row c16 at k = kw + 64 u (k % 16 == 0) sit at tile * 16 K + (kw - 16 g + 64 u) * 16
  // + lane * 16: a wave's load of a unit is one contiguous 1 KiB.
  auto w_row = [&](int t) -> const uint8_t* {
    const int sid = seg_of(t);
    const int nt = t - (sid ? p.tiles0 : 0);
    if constexpr (SHUF)
      return (const uint8_t*)p.seg[sid].w + (size_t)nt * 16 * K + (size_t)(kw - 16 * g) * 16 + lane * 16;
    return (const uint8_t*)p.seg[sid].w + ((size_t)(nt * 16 + c16) * K + kw) * (F8 ? 1 : 2);
  };
  // a lane's load j of a tile: F8 unit j (16 E4M3); bf16 unit j / 2, half j % 2
  auto w_off = [&](int j) { return SHUF ? 1024 * j : F8 ? 64 * j : 128 * (j >> 1) + 16 * (j & 1); };
  const uint8_t* wrow = w_row(t0 < t1 ? t0 : 0);
  uint4 wv[WIN];
  if (t0 < t1) {
#pragma unroll
    for (int j = 0; j < WIN; ++j) wv[j] = ld_stream16(wrow + w_off(j));
  }
  if (!wait()) return false;
  // the rows: this lane's fragments of row c16 (16 k a unit)
  const bf16_t* xr = p.x + (size_t)(live ? c16 : 0) * K + kw;
  uint4 xq[2 * KU];
#pragma unroll
  for (int u = 0; u < KU; ++u) {
    xq[2 * u] = *(const uint4*)(xr + 64 * u);
    xq[2 * u + 1] = *(const uint4*)(xr + 64 * u + 8);
  }
  // the norm: each row's sum of squares over all K (the rows are L2-resident): 32
  // threads a row, 16-byte pieces, every load issued before the sums
  float rs = 1.f;
  if (p.g) {
    constexpr int PB = 12;  // pieces a thread a batch
    const int mr = threadIdx.x >> 5, tr = threadIdx.x & 31;
    const uint4* xrow = (const uint4*)(p.x + (size_t)(mr < M ? mr : 0) * K);
    float ss = 0.f;
    for (int i0 = tr; i0 < K / 8; i0 += 32 * PB) {
      uint4 v[PB];
#pragma unroll
      for (int j = 0; j < PB; ++j) v[j] = i0 + 32 * j < K / 8 ? xrow[i0 + 32 * j] : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < PB; ++j) {
        const uint32_t u4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bf16x2 h = __builtin_bit_cast(bf16x2, u4[e]);
          ss = __builtin_amdgcn_fdot2_f32_bf16(h, h, ss, false);
        }
      }
    }
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) ss += __shfl_xor(ss, m);
    if (tr == 0 && mr < M) ssum[mr] = ss;
    for (int j = threadIdx.x; j < K / 8; j += GV_NT) gam[j] = ((const uint4*)p.g)[j];
    __syncthreads();
    rs = live ? 1.0f / sqrtf(ssum[c16] / (float)K + p.eps) : 0.f;
  }
  // B operands: bf16(x * rstd * g), or x as it is; zero columns past the rows
  bf16x8 bq[2 * KU];
#pragma unroll
  for (int i = 0; i < 2 * KU; ++i) {
    uint4 ov = xq[i];
    if (p.g) {
      const uint4 gv = gam[(kw + 64 * (i >> 1) + 8 * (i & 1)) >> 3];
      const uint32_t xu[4] = {xq[i].x, xq[i].y, xq[i].z, xq[i].w}, gu[4] = {gv.x, gv.y, gv.z, gv.w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf16x2(__uint_as_float(xu[j] << 16) * rs * __uint_as_float(gu[j] << 16),
                           __uint_as_float(xu[j] & 0xFFFF0000u) * rs * __uint_as_float(gu[j] & 0xFFFF0000u));
      ov = make_uint4(o[0], o[1], o[2], o[3]);
    }
    if (!live) ov = make_uint4(0, 0, 0, 0);
    bq[i] = __builtin_bit_cast(bf16x8, ov);
  }
  // the tiles, in chunks of GV_CHUNK whose partials wait in LDS (no barrier a tile)
  for (int c0 = t0; c0 < t1; c0 += GV_CHUNK) {
#pragma unroll
    for (int i = 0; i < GV_CHUNK; ++i) {
      const int t = c0 + i;
      if (t >= t1) break;
      const bool more = t + 1 < t1;
      const uint8_t* nrow = w_row(more ? t + 1 : t);
      const int sid = seg_of(t);
      const int row0 = (t - (sid ? p.tiles0 : 0)) * 16;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (F8) {
        // the tile's block scales (one a 128-k block of the wave's slice; the tile's 16
        // rows are in one 128-row block)
        const float* sr = p.seg[sid].s + (size_t)(row0 >> 7) * (K >> 7) + ((kw - 16 * g) >> 7);
#pragma unroll
        for (int kb = 0; kb < KU / 2; ++kb) {
          f32x4 pa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int j = 2 * kb + h;
            const uint4 w = wv[j % WIN];
            pa = mfma_bf16(e4m3x8_to_bf16(w.x, w.y), bq[2 * j], pa);
            pa = mfma_bf16(e4m3x8_to_bf16(w.z, w.w), bq[2 * j + 1], pa);
            const int nj = j + WIN;
            if (nj < L)
              wv[j % WIN] = ld_stream16(wrow + w_off(nj));
            else if (more)
              wv[j % WIN] = ld_stream16(nrow + w_off(nj - L));
          }
          const float sc = sr[kb];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[e] += pa[e] * sc;
        }
      } else {
#pragma unroll
        for (int j = 0; j < L; ++j) {
          acc = mfma_bf16(__builtin_bit_cast(bf16x8, wv[j % WIN]), bq[j], acc);
          const int nj = j + WIN;
          if (nj < L)
            wv[j % WIN] = ld_stream16(wrow + w_off(nj));
          else if (more)
            wv[j % WIN] = ld_stream16(nrow + w_off(nj - L));
        }
      }
      // lane (c16, g) holds D[v = 4 g + e][m = c16]
      float* rw = red[i][wave];
#pragma unroll
      for (int e = 0; e < 4; ++e) rw[(4 * g + e) * 16 + c16] = acc[e];
      wrow = nrow;
    }
    __syncthreads();
    const int nt = min(GV_CHUNK, t1 - c0);
    for (int e = threadIdx.x; e < nt * 256; e += GV_NT) {
      const int i = e >> 8, m = (e >> 4) & 15, v = e & 15;
      const int t = c0 + i, sid = seg_of(t);
      const int row = (t - (sid ? p.tiles0 : 0)) * 16 + v;
      float s = red[i][0][v * 16 + m];
#pragma unroll
      for (int w = 1; w < GV_WAVES; ++w) s += red[i][w][v * 16 + m];
      if (m < M) st_dev_f32(p.seg[sid].out + part * p.seg[sid].pstride + (size_t)m * p.seg[sid].ld + row, s);
    }
    __syncthreads();
  }
  return true;
}


// ------------------------------------------------------------------ per-row stage
struct FrontDev {
  int M, q_lora, kv_lora, rope, nope, heads, ih, max_position, key_fmt, kv_scaled;
  float eps, index_eps;
  const long long* positions;  // [M]
  const long long* slots;      // [M], < 0: a pad row (no cache writes)
  const float* rope_cs;        // [positions][rope]: cos | sin
  // the GEMV outputs (workspace): f32 partial planes over K parts, summed in part order
  const float* qkv_a;  // [ksA][M][q_lora + kv_lora + rope]
  const float* ik;     // [ksA][M][128]
  const float* iw;     // [ksW][M][ih]
  const float* q_b;    // [ksC][M][heads * (nope + rope)]
  const float* iq;     // [ksC][M][ih * 128]
  int ksA, ksW, ksC;
  // weights
  const bf16_t* g_q_a;
  const bf16_t* g_kv_a;
  const float* g_ik;
  const float* b_ik;
  const bf16_t* w_uk;  // [heads][kv_lora][nope] (SGLang's w_kc memory)
  // outputs
  bf16_t* q_an;     // [M][q_lora] (workspace)
  uint8_t* kv;      // latent cache [slots][576]
  float* kv_scale;  // [slots], or null (unscaled)
  uint8_t* icache;  // index cache (FP8 pages, or the FP4 plane's codes)
  uint8_t* iscale;  // FP4 plane scales, or null
  bf16_t* mla_q;    // [M][heads][kv_lora + rope]
  bf16_t* index_q;  // [M][ih][128]
  bf16_t* index_w;  // [M][ih]
};

// element i of plane row `row` (length n) summed over `parts` planes in order
MK2_DEV float parts_sum(const float* base, int parts, long long pstride, size_t at) {
  float v = base[at];
  for (int k = 1; k < parts; ++k) v += base[k * pstride + at];
  return v;
}
// N elements (at[i], those with on[i]; 0 for the rest) summed over `parts` planes in
// order, as parts_sum, with each plane's N loads issued together (one round trip a
// plane rather than one an element)
template <int N>
MK2_DEV void parts_sum_n(const float* base, int parts, long long pstride, const size_t* at, const bool* on, float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = on[i] ? base[at[i]] : 0.f;
  for (int k = 1; k < parts; ++k) {
    float w[N];
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = on[i] ? base[k * pstride + at[i]] : 0.f;
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += w[i];
  }
}

MK2_DEV float block_sum512(float v, float* sh) {  // all 512 threads; sh: 8 floats
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < FR_NT / 64; ++w) t += sh[w];
  return t;
}

// the orthonormal 128-point Hadamard transform (Sylvester order) of one wave's values,
// lane l holding entries 2l and 2l + 1
MK2_DEV void fwht128(float& v0, float& v1) {
  const int lane = threadIdx.x & 63;
  float a = v0 + v1, b = v0 - v1;
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    const int m = 1 << j;
    const float pa = __shfl_xor(a, m), pb = __shfl_xor(b, m);
    const bool up = (lane & m) != 0;
    a = up ? pa - a : a + pa;
    b = up ? pb - b : b + pb;
  }
  const float r = 0.08838834764831845f;  // 128^-1/2
  v0 = a * r;
  v1 = b * r;
}

MK2_DEV const float* rope_row(const FrontDev& p, int s) {
  const long long pos = p.positions[s] < p.max_position ? p.positions[s] : p.max_position;
  return p.rope_cs + (size_t)(pos < 0 ? 0 : pos) * p.rope;
}

// the normed input rows x_n = bf16(x * rstd * g_in), one workgroup a row (row s), for
// every hidden-input GEMV (so that each of their workgroups reads only its k slice);
// stored device-coherently (the GEMVs may run on another XCD in the same launch)
MK2_DEV void front_norm_row(const bf16_t* x, const bf16_t* gw, bf16_t* xn, int K, float eps, int s, float* sh) {
  constexpr int PT = 2;  // 16-byte pieces a thread (K <= 8192)
  const uint4* xr = (const uint4*)(x + (size_t)s * K);
  uint4 v[PT];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PT; ++i) {
    const int j = threadIdx.x + i * FR_NT;
    v[i] = j < K / 8 ? xr[j] : make_uint4(0, 0, 0, 0);
    const uint32_t u4[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bf16x2 h = __builtin_bit_cast(bf16x2, u4[e]);
      ss = __builtin_amdgcn_fdot2_f32_bf16(h, h, ss, false);
    }
  }
  const float rs = 1.0f / sqrtf(block_sum512(ss, sh) / (float)K + eps);
#pragma unroll
  for (int i = 0; i < PT; ++i) {
    const int j = threadIdx.x + i * FR_NT;
    if (j >= K / 8) continue;
    const uint4 gv = ((const uint4*)gw)[j];
    const uint32_t xu[4] = {v[i].x, v[i].y, v[i].z, v[i].w}, gu[4] = {gv.x, gv.y, gv.z, gv.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack_bf16x2(__uint_as_float(xu[e] << 16) * rs * __uint_as_float(gu[e] << 16),
                         __uint_as_float(xu[e] & 0xFFFF0000u) * rs * __uint_as_float(gu[e] & 0xFFFF0000u));
    st_dev_16((uint4*)(xn + (size_t)s * K) + j, make_uint4(o[0], o[1], o[2], o[3]));
  }
}

// three workgroups a row (task b of 3 M): role 0 the normed q_a (stored
// device-coherently: the q_b GEMV may run on another XCD in the same launch); role 1
// the latent cache row; role 2 the index key and the head weights.  sh: 8 floats, kvv:
// 576 floats of LDS.
MK2_DEV void front_rows_task(const FrontDev& p, int b, float* sh, float* kvv) {
  const int role = b / p.M, s = b % p.M;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int NA = p.q_lora + p.kv_lora + p.rope;
  const long long pA = (long long)p.M * NA;
  const size_t ra = (size_t)s * NA;
  const long long slot = p.slots[s];
  const float* cs = rope_row(p, s);
  if (role == 0) {  // q_an = bf16(rmsnorm(q_a) * g)
    constexpr int QPT = 16;  // q_lora <= 8192: 16 a thread
    float v[QPT];
    size_t at[QPT];
    bool on[QPT];
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      at[i] = ra + tid + i * FR_NT;
      on[i] = tid + i * FR_NT < p.q_lora;
    }
    parts_sum_n<QPT>(p.qkv_a, p.ksA, pA, at, on, v);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < QPT; ++i) ss += v[i] * v[i];
    const float rs = 1.0f / sqrtf(block_sum512(ss, sh) / (float)p.q_lora + p.eps);
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int k = tid + i * FR_NT;
      if (k < p.q_lora) st_dev_u16(p.q_an + (size_t)s * p.q_lora + k, f32_to_bf16(v[i] * rs * bf16_to_f32(p.g_q_a[k])));
    }
    return;
  }
  if (role == 1) {  // the latent row: bf16(rmsnorm(kv_a) * g) | bf16(rope(k_pe)), then E4M3
    const int D = p.kv_lora + p.rope;
    const size_t at[3] = {ra + p.q_lora + tid, ra + p.q_lora + p.kv_lora + 2 * tid,
                          ra + p.q_lora + p.kv_lora + 2 * tid + 1};
    const bool on[3] = {tid < p.kv_lora, tid < p.rope / 2, tid < p.rope / 2};
    float r3[3];
    parts_sum_n<3>(p.qkv_a, p.ksA, pA, at, on, r3);
    const float v = r3[0], x0 = r3[1], x1 = r3[2];
    const float rs = 1.0f / sqrtf(block_sum512(v * v, sh) / (float)p.kv_lora + p.eps);
    if (tid < p.kv_lora) kvv[tid] = bf16_to_f32(f32_to_bf16(v * rs * bf16_to_f32(p.g_kv_a[tid])));
    if (tid < p.rope / 2) {
      const float c = cs[tid], sn = cs[p.rope / 2 + tid];
      kvv[p.kv_lora + 2 * tid] = bf16_to_f32(f32_to_bf16(x0 * c - x1 * sn));
      kvv[p.kv_lora + 2 * tid + 1] = bf16_to_f32(f32_to_bf16(x0 * sn + x1 * c));
    }
    __syncthreads();
    float scale = 1.f;
    if (p.kv_scaled) {
      float am = 0.f;
      for (int k = tid; k < D; k += FR_NT) am = fmaxf(am, fabsf(kvv[k]));
      am = wave_max(am);
      if (lane == 0) sh[wave] = am;
      __syncthreads();
      am = sh[0];
#pragma unroll
      for (int w = 1; w < FR_NT / 64; ++w) am = fmaxf(am, sh[w]);
      scale = am > 0.f ? am / 448.0f : 1.0f;
    }
    if (slot >= 0 && tid < D / 4) {  // four E4M3 a thread, one dword store
      const float* k4 = kvv + 4 * tid;
      const uint32_t w = p.kv_scaled ? f32x4_to_e4m3x4(k4[0] / scale, k4[1] / scale, k4[2] / scale, k4[3] / scale)
                                     : f32x4_to_e4m3x4(k4[0], k4[1], k4[2], k4[3]);
      st_dev_u32(p.kv + (size_t)slot * D + 4 * tid, w);
      if (p.kv_scaled && tid == 0) st_dev_f32(p.kv_scale + slot, scale);
    }
    return;
  }
  // role 2: the index key (wave 0): LayerNorm, RoPE on the first 64 dims, Hadamard,
  // quant; the head weights (the other threads)
  if (wave > 0) {
    const long long pW = (long long)p.M * p.ih;
    for (int h = tid - 64; h < p.ih; h += FR_NT - 64)
      st_dev_u16(p.index_w + (size_t)s * p.ih + h, f32_to_bf16(parts_sum(p.iw, p.ksW, pW, (size_t)s * p.ih + h)));
    return;
  }
  const long long pK = (long long)p.M * 128;
  const size_t at2[2] = {(size_t)s * 128 + 2 * lane, (size_t)s * 128 + 2 * lane + 1};
  const bool on2[2] = {true, true};
  float r2[2];
  parts_sum_n<2>(p.ik, p.ksA, pK, at2, on2, r2);
  float v0 = r2[0], v1 = r2[1];
  const float mean = wave_sum(v0 + v1) * (1.0f / 128);
  const float d0 = v0 - mean, d1 = v1 - mean;
  const float rstd = 1.0f / sqrtf(wave_sum(d0 * d0 + d1 * d1) * (1.0f / 128) + p.index_eps);
  v0 = d0 * rstd * p.g_ik[2 * lane] + p.b_ik[2 * lane];
  v1 = d1 * rstd * p.g_ik[2 * lane + 1] + p.b_ik[2 * lane + 1];
  if (2 * lane < 64) {
    const float c = cs[lane], sn = cs[p.rope / 2 + lane];
    const float r0 = v0 * c - v1 * sn, r1 = v0 * sn + v1 * c;
    v0 = r0;
    v1 = r1;
  }
  fwht128(v0, v1);
  if (slot < 0) return;
  const long long page = slot >> 6;
  const int t = (int)(slot & 63);
  if (p.key_fmt == MK2_KEYS_FP8) {
    // ue8m0: 2^ceil(log2(max(amax, 1e-4) / 448)), the values times its inverse
    const float am = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
    const uint32_t bits = __float_as_uint(fmaxf(am, 1.0e-4f) / 448.0f);
    const uint32_t e = ((bits >> 23) & 0xFF) + ((bits & 0x7FFFFF) != 0);
    const float inv = __uint_as_float((254u - e) << 23);
    uint8_t* pg = p.icache + (size_t)page * (64 * 132);
    const int d = 2 * lane;  // dims d, d + 1: tile d / 16, byte d % 16
    const uint32_t q = f32x4_to_e4m3x4(v0 * inv, v1 * inv, 0.f, 0.f);
    st_dev_u16(pg + (t >> 4) * 2048 + (d >> 4) * 256 + (t & 15) * 16 + (d & 15), q & 0xFFFF);
    if (lane == 0) st_dev_f32((float*)(pg + 64 * 128 + 4 * t), __uint_as_float(e << 23));
  } else {
    // MXFP4 per 32 dims (16 lanes): E8M0 = pow2_ceil(max(amax, 6 * 2^-126) / 6),
    // E2M1 codes of v * 2^-e, two a byte (the even dim in the low nibble)
    float am = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) am = fmaxf(am, __shfl_xor(am, m));
    const uint32_t bits = __float_as_uint(fmaxf(am, 6.0f * 1.1754944e-38f) * (1.0f / 6.0f));
    uint32_t e = ((bits >> 23) & 0xFF) + ((bits & 0x7FFFFF) != 0);
    e = e > 254 ? 254 : e;
    const int c = lane >> 4;  // the 32-dim chunk
    st_dev_u8(p.icache + (size_t)page * 4096 + c * 1024 + t * 16 + (lane & 15), f32x2_to_e2m1x2(v0, v1, e));
    if ((lane & 15) == 0) st_dev_u8(p.iscale + (size_t)page * 256 + c * 64 + (t & 15) * 4 + (t >> 4), e);
  }
}

// ---------------------------------------------------------------- per-head stage
// Workgroups [0, 4 heads): head h, latent rows [128 j, 128 j + 128) of every row, a
// 16-row tile a wave on MFMA (A = W_UK[h] rows c, k = nope; B = bf16(q_nope) of the
// rows); quarter 0 also rotates the head's q_pe.  The rest: the index queries, one
// (row, index head) a wave.
// Task b: W_UK tasks below 4 heads, then index-query tasks.  qn: LDS of 32 * NS * 4
// uint4 (the head's bf16 q_nope, [row][nope] in 16-byte pieces).  `wait` (the q_b
// planes' dependency, in the persistent front) runs after the task's static loads;
// false from it returns false at once.
template <int NS, typename Wait = NoWait>  // NS: nope / 32 k-steps
MK2_DEV bool front_heads_task(const FrontDev& p, int b, uint4* qn, Wait wait = Wait()) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c16 = lane & 15, g = lane >> 4;
  const int QD = p.nope + p.rope, D = p.kv_lora + p.rope, QB = p.heads * QD;
  const long long pC = (long long)p.M * QB;
  if (b < 4 * p.heads) {
    const int h = b >> 2, quarter = b & 3;
    const int c0 = quarter * 128 + wave * 16;
    const bf16_t* wr = p.w_uk + ((size_t)h * p.kv_lora + c0 + c16) * p.nope + 8 * g;
    uint4 wv[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) wv[s] = *(const uint4*)(wr + 32 * s);
    if (!wait()) return false;
    // the head's q_nope rows as bf16 in LDS: 8 consecutive k a thread (coalesced f32 reads)
    for (int e = tid; e < p.M * NS * 4; e += FR_NT) {
      const int m = e / (NS * 4), k8 = (e % (NS * 4)) * 8;
      const size_t at = (size_t)m * QB + (size_t)h * QD + k8;
      size_t a8[8];
      bool on8[8];
      float r8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a8[j] = at + j;
        on8[j] = true;
      }
      parts_sum_n<8>(p.q_b, p.ksC, pC, a8, on8, r8);
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = pack_bf16x2(r8[2 * j], r8[2 * j + 1]);
      qn[e] = make_uint4(o[0], o[1], o[2], o[3]);
    }
    __syncthreads();
    for (int m0 = 0; m0 < p.M; m0 += 16) {
      // B operands: bf16(q_nope[m0 + c16][h]) at k = 32 s + 8 g
      const int m = m0 + c16;
      const bool live = m < p.M;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const uint4 b = live ? qn[m * NS * 4 + 4 * s + g] : make_uint4(0, 0, 0, 0);
        acc = mfma_bf16(__builtin_bit_cast(bf16x8, wv[s]), __builtin_bit_cast(bf16x8, b), acc);
      }
      // lane (c16, g): latent rows c0 + 4 g + e of row m0 + c16
      if (live) {
        bf16_t* out = p.mla_q + ((size_t)m * p.heads + h) * D + c0 + 4 * g;
        st_dev_8(out, make_uint2(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])));
      }
    }
    if (quarter == 0) {  // q_pe rotated: pairs (2i, 2i + 1) of every row
      for (int e = tid; e < p.M * (p.rope / 2); e += FR_NT) {
        const int m = e / (p.rope / 2), i = e % (p.rope / 2);
        const float* cs = rope_row(p, m);
        const size_t at = (size_t)m * QB + (size_t)h * QD + p.nope + 2 * i;
        const float x0 = parts_sum(p.q_b, p.ksC, pC, at), x1 = parts_sum(p.q_b, p.ksC, pC, at + 1);
        const float c = cs[i], sn = cs[p.rope / 2 + i];
        st_dev_u32(p.mla_q + ((size_t)m * p.heads + h) * D + p.kv_lora + 2 * i,
                   pack_bf16x2(x0 * c - x1 * sn, x0 * sn + x1 * c));
      }
    }
    return true;
  }
  // index queries: wave task (row, index head)
  if (!wait()) return false;
  const int task = (b - 4 * p.heads) * (FR_NT / 64) + wave;
  if (task >= p.M * p.ih) return true;
  const int m = task / p.ih, h = task % p.ih;
  const long long pQ = (long long)p.M * p.ih * 128;
  const size_t at = ((size_t)m * p.ih + h) * 128 + 2 * lane;
  float v0 = bf16_to_f32(f32_to_bf16(parts_sum(p.iq, p.ksC, pQ, at)));
  float v1 = bf16_to_f32(f32_to_bf16(parts_sum(p.iq, p.ksC, pQ, at + 1)));
  if (2 * lane < 64) {
    const float* cs = rope_row(p, m);
    const float c = cs[lane], sn = cs[p.rope / 2 + lane];
    const float r0 = v0 * c - v1 * sn, r1 = v0 * sn + v1 * c;
    v0 = r0;
    v1 = r1;
  }
  fwht128(v0, v1);
  st_dev_u32(p.index_q + ((size_t)m * p.ih + h) * 128 + 2 * lane, pack_bf16x2(v0, v1));
  return true;
}

// ------------------------------------------------------------- the persistent front
// The five stages in ONE launch of one workgroup a CU (the staged launches' device
// code, task by task): task t of a stage runs on workgroup (base + t) mod grid, each
// stage's base continuing from the previous stage's last task, and a task that needs
// an earlier stage's results waits on that stage's completion counter, as the
// persistent layer does: producers store their hand-off data device-coherently,
// drain, pass a barrier and add to the counter (16 sub-counters on their own lines
// for the wide stages); wave 0 of a consumer polls the counter (bounded; a wait that
// runs out, or sees another's failure, stops the workgroup's walk and sets the sticky
// error word), then the workgroup reads with plain loads.  Every dependency points
// back and every workgroup is resident, so every wait ends.  The last workgroup out
// resets the counters and ORs a failure into the status word.
constexpr int FP_LINE = 32, FP_LANES = 16;
// the front shapes the front-and-layer launch instantiates (with A8W4 experts): C7's
// GEMV steps and nope 192, block-FP8 weights row-major or in AITER's layout
enum : int { FRONT_FUSED_NONE = 0, FRONT_FUSED_C7_FP8 = 1, FRONT_FUSED_C7_AITER16 = 2 };
enum : int {
  FP_NORM = 0,                 // normed rows done
  FP_A = 1,                    // [FP_LANES] hidden-input GEMV workgroups done
  FP_ROWS = FP_A + FP_LANES,   // [FP_LANES] per-row tasks done
  FP_C = FP_ROWS + FP_LANES,   // [FP_LANES] q_an-input GEMV workgroups done
  FP_DONE = FP_C + FP_LANES,   // workgroups finished
  FP_ERR,                      // sticky within a launch
  FP_STATUS,                   // nonzero once a launch failed; never cleared here
  FP_HEADS,                    // [FP_LANES] per-head tasks done (when the layer follows in the launch)
  FP_LINES = FP_HEADS + FP_LANES
};
static_assert(FP_STATUS * FP_LINE * 4 == MK2_FRONT_STATUS_OFFSET, "the status word's documented offset");

struct FrontPDev {
  FrontDev f;
  GemvDev A[2], W[2], C[2];  // passes of 16 rows
  int passes, gridA, gridW, gridC, nheads;
  const bf16_t* x;
  const bf16_t* g_in;
  bf16_t* x_n;
  int hidden;
  float eps;
  int* sync;
  uint32_t wait_ticks;  // a dependency wait's deadline (WaitClock ticks)
};

union FrontLds {
  GemvLds gemv;
  struct {
    float sh[FR_NT / 64];
    float kvv[576];
  } rows;
  uint4 qn[32 * 8 * 4];
};

MK2_DEV int* fp_ctr(const FrontPDev& p, int line) { return p.sync + line * FP_LINE; }

MK2_DEV void fp_signal(const FrontPDev& p, int line, int t, int lanes) {
  drain_memory();
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(fp_ctr(p, line + t % lanes), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// until the sub-counters of `line` sum to target; seen[k] (k < FP_SEEN - 1) caches what
// wait k saw and seen[FP_SEEN - 1] is the workgroup's failure flag (every thread
// returns the same)
constexpr int FP_SEEN = 8;
MK2_DEV bool fp_wait(const FrontPDev& p, int* seen, int k, int line, int lanes, int target) {
  if (seen[k] >= target) return true;
  int v = 0;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int* ctr = fp_ctr(p, line + min(lane, lanes - 1));
    const int* err = fp_ctr(p, FP_ERR);
    auto poll = [&]() { return __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto count = [&](int c) { return __builtin_amdgcn_readfirstlane(row16_sum_i32(lane < lanes ? c : 0)); };
    bool bad = false;
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
        if (lane == 0) atomicOr(fp_ctr(p, FP_ERR), 1);
        bad = true;
        break;
      }
    }
    if (lane == 0) seen[FP_SEEN - 1] = bad;
  }
  __syncthreads();
  const bool ok = seen[FP_SEEN - 1] == 0;
  __syncthreads();  // the flag is read before the next wait can write it
  if (threadIdx.x == 0 && ok) seen[k] = v;
  return ok;
}


// The persistent front's stages (see front.hip), task by task on this workgroup; false
// when a wait failed (the walk stopped).  seen: FP_SEEN ints of LDS, zero at the
// start.  With HEADS the per-head tasks also count out on FP_HEADS (the persistent
// layer that runs the front ahead of its own stages waits on it); their outputs and
// the cache rows are stored device-coherently either way.
template <int KUA, int KUC, int WF, int NS, bool HEADS = false>
MK2_DEV bool front_walk(const FrontPDev& p, FrontLds& S, int* seen) {
  const int G = gridDim.x, b = blockIdx.x, M = p.f.M;
  int base = 0;
#define FP_TASKS(t, n) for (int t = (b - base % G + G) % G; t < (n); t += G)
#define FP_NEXT(n) base = (base + (n)) % G
  // 0. the normed input rows
  FP_TASKS(t, M) {
    front_norm_row(p.x, p.g_in, p.x_n, p.hidden, p.eps, t, S.rows.sh);
    fp_signal(p, FP_NORM, 0, 1);
  }
  FP_NEXT(M);
  // 1. the hidden-input GEMVs, per pass of 16 rows: [W_qkv_a | W_ik], then W_iw
  const int nA = p.gridA + p.gridW;
  FP_TASKS(t, p.passes * nA) {
    const int pass = t / nA, u = t % nA;
    auto w = [&] { return fp_wait(p, seen, 0, FP_NORM, 1, M); };
    const bool ok = u < p.gridA ? gemv_run<KUA, WF>(p.A[pass], u, p.gridA, S.gemv, w)
                                : gemv_run<1, MK2_WFMT_BF16>(p.W[pass], u - p.gridA, p.gridW, S.gemv, w);
    if (!ok) return false;
    fp_signal(p, FP_A, t, FP_LANES);
  }
  FP_NEXT(p.passes * nA);
  // 2. the per-row stage
  const int nR = (p.f.ih ? 3 : 2) * M;
  FP_TASKS(t, nR) {
    if (!fp_wait(p, seen, 1, FP_A, FP_LANES, p.passes * nA)) return false;
    front_rows_task(p.f, t, S.rows.sh, S.rows.kvv);
    fp_signal(p, FP_ROWS, t, FP_LANES);
  }
  FP_NEXT(nR);
  // 3. the q_an-input GEMVs
  FP_TASKS(t, p.passes * p.gridC) {
    const int pass = t / p.gridC, u = t % p.gridC;
    if (!gemv_run<KUC, WF>(p.C[pass], u, p.gridC, S.gemv, [&] { return fp_wait(p, seen, 2, FP_ROWS, FP_LANES, nR); }))
      return false;
    fp_signal(p, FP_C, t, FP_LANES);
  }
  FP_NEXT(p.passes * p.gridC);
  // 4. the per-head stage
  FP_TASKS(t, p.nheads) {
    if (!front_heads_task<NS>(p.f, t, S.qn, [&] { return fp_wait(p, seen, 3, FP_C, FP_LANES, p.passes * p.gridC); }))
      return false;
    if constexpr (HEADS) fp_signal(p, FP_HEADS, t, FP_LANES);
    else __syncthreads();  // this workgroup's next head task rewrites qn
  }
#undef FP_TASKS
#undef FP_NEXT
  return true;
}

// the last workgroup out (every workgroup counted out on FP_DONE): a failure into the
// status word, every counter back to zero for the next launch
MK2_DEV void front_reset(const FrontPDev& p) {
  if (threadIdx.x == 0 && __hip_atomic_load(fp_ctr(p, FP_ERR), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
    atomicOr(fp_ctr(p, FP_STATUS), 1);
  for (int l = threadIdx.x; l < FP_LINES; l += FR_NT)
    if (l != FP_STATUS) __hip_atomic_store(fp_ctr(p, l), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace mk2
