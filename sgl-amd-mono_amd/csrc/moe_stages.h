// MoE block stages of the K2 layer: RMSNorm + activation quant, router GEMV,
// top-k routing, up/gate + SwiGLU (+ mid quant), down + route weighting + residual.
//
// Each stage is a device function that runs one task on one workgroup of NT
// threads; the standalone kernels map task = blockIdx, the persistent layer kernel
// walks task lists.  All expert GEMVs run on the matrix cores with the weights as
// MFMA A (16 output rows a tile) and the decode rows as the 16 (or 32) columns.
#pragma once
#include "mk2_device.h"

namespace mk2 {

struct MoeDev {
  int M, H, E, topk, I, router, fmt, n_shared, SI, norm, residual;
  int KC;    // router k-chunks
  int Dmax;  // capacity of the distinct-expert list
  float route_scale, eps;
  const bf16_t* x;
  const bf16_t* gamma;
  const uint8_t* w_router;
  const float* bias;
  const uint8_t* w13;
  const uint8_t* s13;
  const uint8_t* w2;
  const uint8_t* s2;
  const uint8_t* ws13;
  const float* ss13;
  const uint8_t* ws2;
  const float* ss2;
  bf16_t* out;
  // workspace
  bf16_t* xn;        // [M][H] normalized rows
  uint8_t* xq;       // [M][H] MXFP8 codes (MXFP4 experts)
  uint8_t* xs;       // [M][H/32] E8M0
  float* logit_part; // [KC][M][E]
  float* logits;     // [M][E]
  int* topk_ids;     // [M][topk]
  float* topk_w;     // [M][topk]
  int* act;          // [1 + E]: count D, then the distinct expert ids ascending
  float* rw;         // [Dmax][32] route weight of slot j for row r (0: not routed)
  uint8_t* mid_q;    // [Dmax][M][I] MXFP8 mid (MXFP4 experts)
  uint8_t* mid_s;    // [Dmax][M][I/32]
  bf16_t* mid_b;     // [Dmax][M][I] bf16 mid (FP8 experts)
  bf16_t* mid_sh;    // [M][SI] shared-expert mid
};

template <int NT>
MK2_DEV float block_sum(float v, float* lds) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) t += lds[w];
  return t;
}

// ---------------------------------------------------------------- stage: prep
// Row r: xn = norm ? bf16(x * rstd * gamma) : x, then (MXFP4 experts) MXFP8 codes.
template <int NT>
MK2_DEV void moe_prep(const MoeDev& p, int r, float* lds) {
  const int tid = threadIdx.x;
  const bf16_t* xr = p.x + (size_t)r * p.H;
  float rstd = 1.f;
  if (p.norm) {
    float ss = 0.f;
    for (int k = tid * 8; k < p.H; k += NT * 8) {
      uint4 v = *(const uint4*)(xr + k);
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = __uint_as_float(w[i] << 16), b = __uint_as_float(w[i] & 0xFFFF0000u);
        ss += a * a + b * b;
      }
    }
    ss = block_sum<NT>(ss, lds);
    rstd = 1.0f / sqrtf(ss / (float)p.H + p.eps);
  }
  for (int blk = tid; blk < p.H / 32; blk += NT) {
    float f[32];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint4 v = *(const uint4*)(xr + blk * 32 + q * 8);
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[q * 8 + 2 * i] = __uint_as_float(w[i] << 16);
        f[q * 8 + 2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
      }
    }
    if (p.norm) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint4 g = *(const uint4*)(p.gamma + blk * 32 + q * 8);
        uint32_t w[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float g0 = __uint_as_float(w[i] << 16), g1 = __uint_as_float(w[i] & 0xFFFF0000u);
          f[q * 8 + 2 * i] = bf16_to_f32(f32_to_bf16(f[q * 8 + 2 * i] * rstd * g0));
          f[q * 8 + 2 * i + 1] = bf16_to_f32(f32_to_bf16(f[q * 8 + 2 * i + 1] * rstd * g1));
        }
      }
    }
    uint32_t packed[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) packed[i] = pack_bf16x2_exact(f[2 * i], f[2 * i + 1]);
    uint4* dst = (uint4*)(p.xn + (size_t)r * p.H + blk * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      dst[q] = make_uint4(packed[4 * q], packed[4 * q + 1], packed[4 * q + 2], packed[4 * q + 3]);
    if (p.fmt == MK2_FMT_MXFP4) {
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(f[i]));
      uint32_t code = mxfp8_scale_code(amax);
      float inv = e8m0_inverse(code);
      uint32_t qw[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        qw[i] = f32x4_to_e4m3x4(f[4 * i] * inv, f[4 * i + 1] * inv, f[4 * i + 2] * inv,
                                f[4 * i + 3] * inv);
      uint4* qd = (uint4*)(p.xq + (size_t)r * p.H + blk * 32);
      qd[0] = make_uint4(qw[0], qw[1], qw[2], qw[3]);
      qd[1] = make_uint4(qw[4], qw[5], qw[6], qw[7]);
      p.xs[(size_t)r * (p.H / 32) + blk] = (uint8_t)code;
    }
  }
}

// B operand: 32 bf16 of row `row` at k0 (4 MFMA k-steps), zeros past the last row
MK2_DEV void load_b_bf16(const bf16_t* base, int row, int nrows, int ld, int k0, bf16x8* b) {
  if (row < nrows) {
    const uint4* s = (const uint4*)(base + (size_t)row * ld + k0);
#pragma unroll
    for (int q = 0; q < 4; ++q) b[q] = __builtin_bit_cast(bf16x8, s[q]);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) b[q] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
  }
}
// B operand of one scaled MFMA: 32 E4M3 of row `row` in the 128-k block at kb0, lane
// group g.  An 8-VGPR E4M3 operand holds k = 16g .. 16g+15 in its first four VGPRs
// and k = 64 + 16g .. +15 in the last four (the E2M1 A operand is plain: 32g .. 32g+31).
MK2_DEV i32x8 load_b_fp8(const uint8_t* base, int row, int nrows, int ld, int kb0, int g) {
  i32x8 b = {0, 0, 0, 0, 0, 0, 0, 0};
  if (row < nrows) {
    const uint8_t* s = base + (size_t)row * ld + kb0 + 16 * g;
    uint4 u0 = *(const uint4*)s, u1 = *(const uint4*)(s + 64);
    b[0] = u0.x; b[1] = u0.y; b[2] = u0.z; b[3] = u0.w;
    b[4] = u1.x; b[5] = u1.y; b[6] = u1.z; b[7] = u1.w;
  }
  return b;
}
// A operand of a bf16 tile: 64 B a lane -> four k-steps
MK2_DEV void load_a_bf16(const uint8_t* tile, int lane, bf16x8* a) {
  const uint4* s = (const uint4*)(tile + lane * 64);
#pragma unroll
  for (int q = 0; q < 4; ++q) a[q] = __builtin_bit_cast(bf16x8, s[q]);
}
// A operand of an E4M3 tile widened to bf16: 32 B a lane -> four k-steps
MK2_DEV void load_a_fp8(const uint8_t* tile, int lane, bf16x8* a) {
  const uint4* s = (const uint4*)(tile + lane * 32);
  uint4 u0 = s[0], u1 = s[1];
  a[0] = e4m3x8_to_bf16(u0.x, u0.y);
  a[1] = e4m3x8_to_bf16(u0.z, u0.w);
  a[2] = e4m3x8_to_bf16(u1.x, u1.y);
  a[3] = e4m3x8_to_bf16(u1.z, u1.w);
}
MK2_DEV i32x8 load_a_fp4(const uint8_t* tile, int lane) {
  uint4 u = *(const uint4*)(tile + lane * 16);
  i32x8 a = {(int)u.x, (int)u.y, (int)u.z, (int)u.w, 0, 0, 0, 0};
  return a;
}
MK2_DEV f32x4 mfma4_bf16(const bf16x8* a, const bf16x8* b, f32x4 c) {
#pragma unroll
  for (int q = 0; q < 4; ++q) c = mfma_bf16(a[q], b[q], c);
  return c;
}

// ------------------------------------------------------------- stage: router GEMV
// task (nt, kc): 16 experts x the kc-th slice of hidden -> logit_part[kc]
template <int NT, int NCG>
MK2_DEV void moe_router(const MoeDev& p, int nt, int kc, float* red) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4;
  const int KB = p.H / 128, kbs = KB / p.KC;
  f32x4 acc[NCG];
#pragma unroll
  for (int c = 0; c < NCG; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int i = wave; i < kbs; i += NW) {
    const int kb = kc * kbs + i;
    bf16x8 a[4];
    load_a_bf16(p.w_router + ((size_t)nt * KB + kb) * 4096, lane, a);
#pragma unroll
    for (int c = 0; c < NCG; ++c) {
      bf16x8 b[4];
      load_b_bf16(p.xn, c * 16 + (lane & 15), p.M, p.H, kb * 128 + 32 * g, b);
      acc[c] = mfma4_bf16(a, b, acc[c]);
    }
  }
#pragma unroll
  for (int c = 0; c < NCG; ++c)
    *(f32x4*)(red + ((wave * NCG + c) * 64 + lane) * 4) = acc[c];
  __syncthreads();
  for (int idx = threadIdx.x; idx < 16 * p.M; idx += NT) {
    const int e16 = idx & 15, row = idx >> 4, c = row >> 4, s16 = row & 15;
    const int l = (e16 >> 2) * 16 + s16, i = e16 & 3;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += red[((w * NCG + c) * 64 + l) * 4 + i];
    p.logit_part[((size_t)kc * p.M + row) * p.E + nt * 16 + e16] = v;
  }
  __syncthreads();
}

// ------------------------------------------------------------- stage: route
// One workgroup: logits = sum of the k-chunk partials (in order), per row the top-k
// by (key desc, expert asc), the weights, the distinct-expert list and rw.
template <int NT>
MK2_DEV void moe_route(const MoeDev& p, float* lds_logits /*[M*E]*/, int* lds_slot /*[E+NT/64]*/) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ME = p.M * p.E;
  for (int idx = tid; idx < ME; idx += NT) {
    float v = 0.f;
    for (int kc = 0; kc < p.KC; ++kc) v += p.logit_part[(size_t)kc * ME + idx];
    lds_logits[idx] = v;
    if (p.logits) p.logits[idx] = v;
  }
  for (int e = tid; e < p.E; e += NT) lds_slot[e] = 0;
  __syncthreads();
  const int per = p.E / 64;  // experts a lane holds: e = lane + 64 * i
  for (int r = wave; r < p.M; r += NW) {
    uint32_t key[4] = {0u, 0u, 0u, 0u};
    float sv[4] = {0.f, 0.f, 0.f, 0.f};
    bool taken[4] = {false, false, false, false};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i >= per) break;
      const int e = lane + 64 * i;
      const float lg = lds_logits[r * p.E + e];
      if (p.router == MK2_ROUTER_SIGMOID_BIAS) {
        const float s = 1.0f / (1.0f + expf(-lg));
        sv[i] = s;
        key[i] = radix_key(s + p.bias[e]);
      } else {
        sv[i] = lg;
        key[i] = radix_key(lg);
      }
    }
    float picked_v = 0.f;  // lane j < topk: the value of pick j
    int picked_e = 0;
    for (int k = 0; k < p.topk; ++k) {
      // best of this lane: max key, then lowest expert id
      uint64_t best = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (i >= per || taken[i]) continue;
        const uint64_t c = ((uint64_t)key[i] << 32) | (uint32_t)(0xFFFFu - (lane + 64 * i));
        best = c > best ? c : best;
      }
      uint64_t m = best;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        uint32_t lo = __shfl_xor((uint32_t)m, o, 64), hi = __shfl_xor((uint32_t)(m >> 32), o, 64);
        uint64_t other = ((uint64_t)hi << 32) | lo;
        m = other > m ? other : m;
      }
      const int e = 0xFFFF - (int)(m & 0xFFFFu);
      const int ei = e >> 6;
      const float mine_v = ei == 0 ? sv[0] : (ei == 1 ? sv[1] : (ei == 2 ? sv[2] : sv[3]));
      const float val = __shfl(mine_v, e & 63, 64);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (e == lane + 64 * i) taken[i] = true;
      if (lane == k) { picked_v = val; picked_e = e; }
    }
    // weights of the picks (lanes < topk)
    float w = 0.f;
    if (p.router == MK2_ROUTER_SIGMOID_BIAS) {
      float tot = lane < p.topk ? picked_v : 0.f;
      tot = wave_sum(tot);
      w = picked_v / tot * p.route_scale;
    } else {
      const float top = __shfl(picked_v, 0, 64);
      float ex = lane < p.topk ? expf(picked_v - top) : 0.f;
      const float tot = wave_sum(ex);
      w = ex / tot;
    }
    if (lane < p.topk) {
      p.topk_ids[r * p.topk + lane] = picked_e;
      p.topk_w[r * p.topk + lane] = w;
      lds_slot[picked_e] = 1;
    }
  }
  __syncthreads();
  // distinct experts, ascending: exclusive scan of the flags
  int flag[4] = {0, 0, 0, 0}, mine = 0;
  const int per_t = (p.E + NT - 1) / NT;  // <= 4 (E <= 256, NT >= 64)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = tid * per_t + i;
    flag[i] = (i < per_t && e < p.E) ? lds_slot[e] : 0;
    mine += flag[i];
  }
  int incl = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  int* wtot = lds_slot + p.E;
  __syncthreads();
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < wave; ++w) before += wtot[w];
  int total = 0;
  for (int w = 0; w < NW; ++w) total += wtot[w];
  int pos = before + incl - mine;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = tid * per_t + i;
    if (i < per_t && e < p.E) {
      lds_slot[e] = flag[i] ? pos : -1;
      if (flag[i]) p.act[1 + pos] = e;
      pos += flag[i];
    }
  }
  if (tid == 0) p.act[0] = total;
  for (int idx = tid; idx < total * 32; idx += NT) p.rw[idx] = 0.f;
  __syncthreads();
  for (int idx = tid; idx < p.M * p.topk; idx += NT) {
    const int r = idx / p.topk;
    p.rw[lds_slot[p.topk_ids[idx]] * 32 + r] = p.topk_w[idx];
  }
}

// ------------------------------------------------------- stage: up/gate + SwiGLU
// task t < Dmax * I/32: routed slot j = t / (I/32), 32-row chunk c; past that the
// shared expert's chunks.  mid = silu(gate) * up for the chunk's 32 rows x all rows.
template <int NT, int NCG>
MK2_DEV void moe_upgate(const MoeDev& p, int t, float* red, float* midf) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4;
  const int KB = p.H / 128;
  const int chunks_r = p.I / 32;
  bool shared = false;
  int j = 0, e = 0, c = 0;
  if (t < p.Dmax * chunks_r) {
    j = t / chunks_r;
    c = t % chunks_r;
    if (j >= p.act[0]) return;
    e = p.act[1 + j];
  } else {
    shared = true;
    c = t - p.Dmax * chunks_r;
  }
  const int I = shared ? p.SI : p.I;
  const int NT16 = 2 * I / 16;  // 16-row tiles of the stacked gate|up
  int nts[4] = {2 * c, 2 * c + 1, I / 16 + 2 * c, I / 16 + 2 * c + 1};
  f32x4 acc[4][NCG];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) acc[q][cg] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (!shared && p.fmt == MK2_FMT_MXFP4) {
    const int G = (KB + 3) / 4;
    const uint8_t* wbase = p.w13 + (size_t)e * NT16 * KB * 1024;
    const uint8_t* sbase = p.s13 + (size_t)e * NT16 * G * 256;
    for (int kb = wave; kb < KB; kb += NW) {
      i32x8 a[4];
      int sa[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        a[q] = load_a_fp4(wbase + ((size_t)nts[q] * KB + kb) * 1024, lane);
        sa[q] = (int)(*(const uint32_t*)(sbase + (((size_t)nts[q] * G + kb / 4) * 64 + lane) * 4) >>
                      (8 * (kb & 3)));
      }
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        const int row = cg * 16 + (lane & 15);
        i32x8 b = load_b_fp8(p.xq, row, p.M, p.H, kb * 128, g);
        const int sb = row < p.M ? p.xs[(size_t)row * (p.H / 32) + kb * 4 + g] : 127;
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q][cg] = mfma_fp4_fp8<0, 0>(a[q], b, acc[q][cg], sa[q], sb);
      }
    }
  } else {
    const uint8_t* wbase = shared ? p.ws13 : p.w13 + (size_t)e * NT16 * KB * 2048;
    const float* sbase = shared ? p.ss13 : (const float*)p.s13 + (size_t)e * (2 * I / 128) * KB;
    for (int kb = wave; kb < KB; kb += NW) {
      bf16x8 a[4][4];
      float sc[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        load_a_fp8(wbase + ((size_t)nts[q] * KB + kb) * 2048, lane, a[q]);
        sc[q] = sbase[(nts[q] * 16 / 128) * KB + kb];
      }
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        bf16x8 b[4];
        load_b_bf16(p.xn, cg * 16 + (lane & 15), p.M, p.H, kb * 128 + 32 * g, b);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          f32x4 tmp = mfma4_bf16(a[q], b, f32x4{0.f, 0.f, 0.f, 0.f});
          acc[q][cg] += tmp * sc[q];
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg)
      *(f32x4*)(red + (((wave * 4 + q) * NCG + cg) * 64 + lane) * 4) = acc[q][cg];
  __syncthreads();
  for (int idx = threadIdx.x; idx < 32 * 16 * NCG; idx += NT) {
    const int n = idx & 31, s = idx >> 5;
    const int t2 = n >> 4, n16 = n & 15, cg = s >> 4, s16 = s & 15;
    const int l = (n16 >> 2) * 16 + s16, i = n16 & 3;
    float gs = 0.f, us = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      gs += red[(((w * 4 + t2) * NCG + cg) * 64 + l) * 4 + i];
      us += red[(((w * 4 + 2 + t2) * NCG + cg) * 64 + l) * 4 + i];
    }
    midf[s * 33 + n] = silu_mul(gs, us);
  }
  __syncthreads();
  if (!shared && p.fmt == MK2_FMT_MXFP4) {
    for (int s = threadIdx.x; s < p.M; s += NT) {
      float amax = 0.f;
      for (int n = 0; n < 32; ++n) amax = fmaxf(amax, fabsf(midf[s * 33 + n]));
      const uint32_t code = mxfp8_scale_code(amax);
      const float inv = e8m0_inverse(code);
      uint32_t qw[8];
      for (int i = 0; i < 8; ++i)
        qw[i] = f32x4_to_e4m3x4(midf[s * 33 + 4 * i] * inv, midf[s * 33 + 4 * i + 1] * inv,
                                midf[s * 33 + 4 * i + 2] * inv, midf[s * 33 + 4 * i + 3] * inv);
      uint4* dst = (uint4*)(p.mid_q + ((size_t)j * p.M + s) * p.I + c * 32);
      dst[0] = make_uint4(qw[0], qw[1], qw[2], qw[3]);
      dst[1] = make_uint4(qw[4], qw[5], qw[6], qw[7]);
      p.mid_s[((size_t)j * p.M + s) * (p.I / 32) + c] = (uint8_t)code;
    }
  } else {
    bf16_t* dst = shared ? p.mid_sh : p.mid_b + (size_t)j * p.M * p.I;
    for (int idx = threadIdx.x; idx < 32 * p.M; idx += NT) {
      const int n = idx & 31, s = idx >> 5;
      dst[(size_t)s * I + c * 32 + n] = f32_to_bf16(midf[s * 33 + n]);
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------- stage: down + combine
// task nt: 16 hidden rows; every slot (shared, then the D routed experts) adds
// rw * W_down[e] . mid into the rows' accumulators; out = bf16(y [+ x]).
template <int NT, int NCG>
MK2_DEV void moe_down(const MoeDev& p, int nt, float* red) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4;
  const int D = p.act[0];
  const int slots = p.n_shared + D;
  const int HT = p.H / 16;
  f32x4 acc[NCG];
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) acc[cg] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int sl = wave; sl < slots; sl += NW) {
    if (sl < p.n_shared) {
      const int KB2 = p.SI / 128;
      for (int kb = 0; kb < KB2; ++kb) {
        bf16x8 a[4];
        load_a_fp8(p.ws2 + ((size_t)nt * KB2 + kb) * 2048, lane, a);
        const float sc = p.ss2[(nt * 16 / 128) * KB2 + kb];
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) {
          bf16x8 b[4];
          load_b_bf16(p.mid_sh, cg * 16 + (lane & 15), p.M, p.SI, kb * 128 + 32 * g, b);
          acc[cg] += mfma4_bf16(a, b, f32x4{0.f, 0.f, 0.f, 0.f}) * sc;
        }
      }
      continue;
    }
    const int j = sl - p.n_shared;
    const int e = p.act[1 + j];
    const int KB2 = p.I / 128;
    if (p.fmt == MK2_FMT_MXFP4) {
      const int G2 = (KB2 + 3) / 4;
      const uint8_t* wbase = p.w2 + ((size_t)e * HT + nt) * KB2 * 1024;
      const uint8_t* sbase = p.s2 + ((size_t)e * HT + nt) * G2 * 256;
      f32x4 tmp[NCG];
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) tmp[cg] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int kb = 0; kb < KB2; ++kb) {
        i32x8 a = load_a_fp4(wbase + (size_t)kb * 1024, lane);
        const int sa = (int)(*(const uint32_t*)(sbase + ((kb / 4) * 64 + lane) * 4) >> (8 * (kb & 3)));
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) {
          const int row = cg * 16 + (lane & 15);
          i32x8 b = load_b_fp8(p.mid_q + (size_t)j * p.M * p.I, row, p.M, p.I, kb * 128, g);
          const int sb = row < p.M ? p.mid_s[((size_t)j * p.M + row) * (p.I / 32) + kb * 4 + g] : 127;
          tmp[cg] = mfma_fp4_fp8<0, 0>(a, b, tmp[cg], sa, sb);
        }
      }
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) acc[cg] += tmp[cg] * p.rw[j * 32 + cg * 16 + (lane & 15)];
    } else {
      const uint8_t* wbase = p.w2 + ((size_t)e * HT + nt) * KB2 * 2048;
      const float* sbase = (const float*)p.s2 + (size_t)e * (p.H / 128) * KB2;
      for (int kb = 0; kb < KB2; ++kb) {
        bf16x8 a[4];
        load_a_fp8(wbase + (size_t)kb * 2048, lane, a);
        const float sc = sbase[(nt * 16 / 128) * KB2 + kb];
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) {
          bf16x8 b[4];
          load_b_bf16(p.mid_b + (size_t)j * p.M * p.I, cg * 16 + (lane & 15), p.M, p.I,
                      kb * 128 + 32 * g, b);
          acc[cg] += mfma4_bf16(a, b, f32x4{0.f, 0.f, 0.f, 0.f}) *
                     (sc * p.rw[j * 32 + cg * 16 + (lane & 15)]);
        }
      }
    }
  }
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) *(f32x4*)(red + ((wave * NCG + cg) * 64 + lane) * 4) = acc[cg];
  __syncthreads();
  for (int idx = threadIdx.x; idx < 16 * p.M; idx += NT) {
    const int n16 = idx & 15, s = idx >> 4, cg = s >> 4, s16 = s & 15;
    const int l = (n16 >> 2) * 16 + s16, i = n16 & 3;
    float y = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) y += red[((w * NCG + cg) * 64 + l) * 4 + i];
    const size_t o = (size_t)s * p.H + nt * 16 + n16;
    if (p.residual) y += bf16_to_f32(p.x[o]);
    p.out[o] = f32_to_bf16(y);
  }
  __syncthreads();
}

}  // namespace mk2
