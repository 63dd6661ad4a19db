// MoE block stages of the K2 layer: RMSNorm partial sums, router GEMV (+ RMSNorm +
// activation quant of its slice), top-k routing, up/gate + SwiGLU (+ mid quant), down
// + route weighting + residual.
//
// Each stage is a device function that runs one task on one workgroup of NT
// threads; the standalone kernels map task = blockIdx, the persistent layer kernel
// walks task lists.  All expert GEMVs run on the matrix cores with the weights as
// MFMA A (16 output rows a tile) and the decode rows as the 16 (or 32) columns.
#pragma once
#include <type_traits>

#include "mk2_device.h"

namespace mk2 {

// the expert modes whose routed weights are E2M1 (the others are E4M3)
__host__ __device__ inline bool w_fp4(int fmt) {
  return fmt == MK2_FMT_MXFP4 || fmt == MK2_FMT_A16W4 || fmt == MK2_FMT_A4W4;
}

struct MoeDev {
  int M, H, E, topk, I, router, fmt, n_shared, SI, norm, residual;
  int KC;    // router k-chunks
  int Dmax;  // capacity of the distinct-expert list
  int UC;    // intermediate rows of a routed up/gate task (64: MXFP4 at <= 16 rows, else 32)
  int DT;    // 16-row hidden tiles of a down task (2: MXFP4 at <= 16 rows, else 1; 3: 24 rows,
            // a tile and a half, when hidden is a multiple of 48)
  float route_scale, eps;
  int wl;    // MK2_WLAYOUT_*: the expert weights' layout
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
  float* ssp;        // [M][H/16] the rows' sums of squares over 16 columns (RMSNorm)
  bf16_t* xn;        // [M][H] normalized rows
  uint8_t* xq;       // [M][H] E4M3 codes (A8W4, W8A8) or [M][H/2] E2M1 codes (A4W4)
  uint8_t* xs;       // [M][H/32] E8M0 (A8W4, A4W4)
  float* xsf;        // [M][H/128] f32 scales (W8A8)
  uint64_t* logit_part; // [KC][M][E] tagged f32 partial logits
  float* logits;     // [M][E]
  int* topk_ids;     // [M][topk]
  float* topk_w;     // [M][topk]
  uint64_t* act;     // [1 + Dmax] tagged: count D, then the distinct expert ids ascending
                     // (-1 past D)
  float* rw;         // [Dmax][32] route weight of slot j for row r (0: not routed); with
                     // compacted rows (compact_rows), of slot j's c-th row
  uint64_t* act_rows; // [Dmax] tagged: slot j's rows as a bit mask (compacted rows)
  uint64_t* picks;   // [M][topk][2] tagged: row r's k-th pick, expert then weight bits
                     // (the persistent layer's route pick tasks, above 8 rows)
  int* rowc;         // [Dmax][32] slot j's rows, ascending (compacted rows)
  uint8_t* mid_q;    // [Dmax][M][I] E4M3 mid (A8W4, W8A8) or [Dmax][M][I/2] E2M1 (A4W4)
  uint8_t* mid_s;    // [Dmax][M][I/32] E8M0 (A8W4, A4W4)
  float* mid_sf;     // [Dmax][M][I/128] f32 scales (W8A8)
  bf16_t* mid_b;     // [Dmax][M][I] bf16 mid (W8A16, A16W4)
  bf16_t* mid_sh;    // [M][SI] shared-expert mid
};

// Expert jobs with compacted rows: above 16 rows, the scaled-MFMA E2M1 modes (A8W4,
// A4W4) run each routed slot's up/gate on the rows that picked its expert only (the
// MFMA columns: the slot's c-th row, not row c), store the mid compacted, and the down
// adds each slot's columns into its rows through LDS (the reference's expert jobs,
// glm53/gfx950/kernel.py:6189-6305).  Every row's sums keep their order, so the bits
// equal the uncompacted path's.
__host__ __device__ inline bool compact_rows(const MoeDev& p) {
  return p.M > 16 && (p.fmt == MK2_FMT_MXFP4 || p.fmt == MK2_FMT_A4W4);
}
template <int NCG, int FMT>
constexpr bool kCompact = NCG == 2 && (FMT == MK2_FMT_MXFP4 || FMT == MK2_FMT_A4W4);
// the c-th set bit of m (c < popcount(m))
MK2_DEV int nth_bit(uint32_t m, int c) {
  for (int i = 0; i < c; ++i) m &= m - 1;
  return __ffs((int)m) - 1;
}

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

// ------------------------------------------------------- stage: sums of squares
// Row r, columns blk * 4 NT ..: ssp[r][t] = sum of x^2 over columns 16t .. 16t+15,
// reduced across one DPP row of 16 lanes.  W_o's epilogue produces the same sums of
// its output tiles with the same reduction, so either producer gives the same bits.
// NT is a multiple of 64 and H of 4 NT, so every pass runs whole 16-lane rows.
template <int NT>
MK2_DEV void moe_sumsq(const MoeDev& p, int r, int blk) {  // columns blk * 4 NT .. + 4 NT - 1
  const bf16_t* xr = p.x + (size_t)r * p.H + blk * 4 * NT;
  uint32_t x[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = ldp_u16(xr + threadIdx.x + i * NT);  // all in flight
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = blk * 4 * NT + threadIdx.x + i * NT;
    const float v = bf16_to_f32((bf16_t)x[i]);
    const float ss = row16_sum(v * v);
    if ((c & 15) == 0) st_dev_f32(p.ssp + (size_t)r * (p.H / 16) + (c >> 4), ss);
  }
}

// B operands are activations produced inside the launch: device-coherent loads.
// B operand: 32 bf16 of row `row` at k0 (4 MFMA k-steps), zeros past the last row
MK2_DEV void load_b_bf16(const bf16_t* base, int row, int nrows, int ld, int k0, bf16x8* b) {
  if (row < nrows) {
    const bf16_t* s = base + (size_t)row * ld + k0;
#pragma unroll
    for (int q = 0; q < 4; ++q) b[q] = __builtin_bit_cast(bf16x8, ldp_16(s + 8 * q));
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
    uint4 u0 = ldp_16(s), u1 = ldp_16(s + 64);
    b[0] = u0.x; b[1] = u0.y; b[2] = u0.z; b[3] = u0.w;
    b[4] = u1.x; b[5] = u1.y; b[6] = u1.z; b[7] = u1.w;
  }
  return b;
}
// B operand of an E2M1 x E2M1 product: 32 E2M1 (16 B) of row `row` at byte kb0 (a
// 128-k block is 64 B), lane group g: k = 32g .. 32g+31 in the low 4 dwords
MK2_DEV i32x8 load_b_fp4(const uint8_t* base, int row, int nrows, int ld, int kb0, int g) {
  i32x8 b = {0, 0, 0, 0, 0, 0, 0, 0};
  if (row < nrows) {
    const uint4 u = ldp_16(base + (size_t)row * ld + kb0 + 16 * g);
    b[0] = u.x; b[1] = u.y; b[2] = u.z; b[3] = u.w;
  }
  return b;
}
// B operand of an E4M3 x E4M3 product: 32 E4M3 of row `row` at k = k0 + 32g .. +31 in
// 8 dwords, the same k map as the weight tiles' A operand (a dot product is free in its
// k order as long as both operands share the map)
MK2_DEV i32x8 load_b_fp8_same(const uint8_t* base, int row, int nrows, int ld, int k0, int g) {
  i32x8 b = {0, 0, 0, 0, 0, 0, 0, 0};
  if (row < nrows) {
    const uint8_t* s = base + (size_t)row * ld + k0 + 32 * g;
    const uint4 u0 = ldp_16(s), u1 = ldp_16(s + 16);
    b[0] = u0.x; b[1] = u0.y; b[2] = u0.z; b[3] = u0.w;
    b[4] = u1.x; b[5] = u1.y; b[6] = u1.z; b[7] = u1.w;
  }
  return b;
}
// A operand of a bf16 tile: 64 B a lane -> four k-steps
MK2_DEV void load_a_bf16(const uint8_t* tile, int lane, bf16x8* a) {
  const uint4* s = (const uint4*)(tile + lane * 64);
#pragma unroll
  for (int q = 0; q < 4; ++q) a[q] = __builtin_bit_cast(bf16x8, ld_stream16(s + q));
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
// ---- the expert weights' two layouts (MK2_WLAYOUT_*).  Both keep a 16-row group's
// 16-row x 128-k block at the same place (2 KiB of E4M3, 1 KiB of E2M1, k-block-major
// inside the group).  Inside a block:
//  - E4M3: lane (g, c16) takes k 32 g .. 32 g + 31 of row c16 as two 16-byte halves
//    at fp8_half: tiles [64 lanes][32 B], AITER [4 groups][2 halves][16 rows][16 B];
//  - E2M1: [4 groups][16 rows][16 B] in both.
MK2_DEV uint32_t fp8_half(int wl, int lane, int h) {
  return wl == MK2_WLAYOUT_AITER16 ? (uint32_t)((lane >> 4) * 512 + h * 256 + (lane & 15) * 16)
                                   : (uint32_t)(lane * 32 + h * 16);
}
// the lane's two halves of the E4M3 block at `blk`
MK2_DEV void load_fp8_block(const uint8_t* blk, int wl, int lane, uint4& lo, uint4& hi) {
  lo = ld_stream16(blk + fp8_half(wl, lane, 0));
  hi = ld_stream16(blk + fp8_half(wl, lane, 1));
}
// The E8M0 scales of an expert's E2M1 [N][K] matrix: one expert's bytes; the 32-bit
// word lane `lane` reads for 16-row tile t and k-block kb; the shift that brings kb's
// code to the word's low byte.  Tiles: [N/16][ceil(K/512)][64 lanes] words of four
// k-blocks.  AITER (e8m0_shuffle over the experts' rows, N a multiple of 32, K of
// 256): [N/32][K/256][64 lanes] words, each two k-blocks of two 16-row tiles, byte
// 2 (kb & 1) + (t & 1).
MK2_DEV size_t e8m0_expert_bytes(int wl, int N, int K) {
  return wl == MK2_WLAYOUT_AITER16 ? (size_t)N * (K / 32) : (size_t)(N / 16) * ((K / 128 + 3) / 4) * 256;
}
MK2_DEV uint32_t e8m0_word(const uint8_t* s_e, int wl, int K, int t, int kb, int lane) {
  const size_t w = wl == MK2_WLAYOUT_AITER16 ? ((size_t)(t >> 1) * (K / 256) + (kb >> 1)) * 64 + lane
                                             : ((size_t)t * ((K / 128 + 3) / 4) + (kb >> 2)) * 64 + lane;
  return *(const uint32_t*)(s_e + w * 4);
}
MK2_DEV int e8m0_shift(int wl, int t, int kb) {
  return wl == MK2_WLAYOUT_AITER16 ? 8 * (2 * (kb & 1) + (t & 1)) : 8 * (kb & 3);
}

// the same 16 bytes through a buffer resource: an offset past its end reads zeros
// (no branch for a lane outside the task)
MK2_DEV i32x8 load_a_fp4_rs(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  const i32x4 u = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
  return i32x8{u.x, u.y, u.z, u.w, 0, 0, 0, 0};
}
MK2_DEV i32x8 load_a_fp4(const uint8_t* tile, int lane) {
  uint4 u = ld_stream16(tile + lane * 16);
  i32x8 a = {(int)u.x, (int)u.y, (int)u.z, (int)u.w, 0, 0, 0, 0};
  return a;
}
MK2_DEV f32x4 mfma4_bf16(const bf16x8* a, const bf16x8* b, f32x4 c) {
#pragma unroll
  for (int q = 0; q < 4; ++q) c = mfma_bf16(a[q], b[q], c);
  return c;
}

// ------------------------------------------------------------- stage: router GEMV
// Task (nt, kc): 16 experts x the kc-th slice of hidden (CK = H / KC columns: 1024, or
// 512 where H is an odd multiple of 512) -> logit_part[kc], as tagged words (the
// routing polls them).  The task normalizes its
// slice of the rows itself: rstd from the rows' partial sums of squares (summed in a
// fixed order, so that every task gets the same bits), then xn = bf16(x * rstd *
// gamma) into LDS as the MFMA B operand.  The nt == 0 task of each slice also stores
// the slice for the expert stages (bf16 rows, and MXFP8 codes + E8M0 scales for MXFP4
// experts).  The router weights and gamma are static: loaded before `wait` (the rows'
// dependency).  NT = 512.
constexpr int ROUTER_NT = 512, ROUTER_CKMAX = 1024;
struct RouterLds {
  float red[8 * 2 * 256];  // NW * NCG * 256
  float rstd[32];
  bf16_t xn[32 * (ROUTER_CKMAX + 8)];
};

template <int NT, int NCG, int FMT, typename Wait = NoWait>
MK2_DEV void moe_router(const MoeDev& p, int nt, int kc, RouterLds& L, uint32_t tag, Wait wait = Wait()) {
  static_assert(NT == ROUTER_NT, "the router task is laid out for 512 threads");
  constexpr int NW = NT / 64, RMAX = 32 * ROUTER_CKMAX / 8 / NT;  // row passes a thread at most
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4;
  const int KB = p.H / 128, kbs = KB / p.KC, CK = kbs * 128, XR = CK + 8, c0 = kc * CK;
  const int cpr = CK / 8, rstep = NT / cpr;                 // 8-column groups a row, rows a pass
  const int c8 = 8 * (tid % cpr), r0 = tid / cpr;          // this thread: columns c8.., rows r0 + rstep*i
  bf16x8 a0[4];
  load_a_bf16(p.w_router + ((size_t)nt * KB + kc * kbs + min(wave, kbs - 1)) * 4096, lane, a0);
  const uint4 gam = p.norm ? *(const uint4*)(p.gamma + c0 + c8) : make_uint4(0, 0, 0, 0);
  if (!wait()) return;
  uint4 xv[RMAX];  // rows past M are not loaded (uniform in a wave: its lanes share a row)
#pragma unroll
  for (int i = 0; i < RMAX; ++i)
    xv[i] = r0 + rstep * i < p.M ? ldp_16(p.x + (size_t)(r0 + rstep * i) * p.H + c0 + c8) : make_uint4(0, 0, 0, 0);
  if (p.norm) {
    const int nt16 = p.H / 16;
    for (int r = wave; r < p.M; r += NW) {
      float ss = 0.f;
      for (int t0 = 0; t0 < nt16; t0 += 64 * 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = ldp_f32(p.ssp + (size_t)r * nt16 + min(t0 + lane + 64 * u, nt16 - 1));
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (t0 + lane + 64 * u < nt16) ss += v[u];
      }
      ss = wave_sum(ss);
      if (lane == 0) L.rstd[r] = 1.0f / sqrtf(ss / (float)p.H + p.eps);
    }
    __syncthreads();
  }
  const uint32_t gw[4] = {gam.x, gam.y, gam.z, gam.w};
#pragma unroll
  for (int i = 0; i < RMAX; ++i) {
    const int r = r0 + rstep * i;
    if (r >= p.M) break;  // uniform in the wave: a wave's lanes share a row
    const uint32_t w[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
    float f[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[2 * j] = __uint_as_float(w[j] << 16);
      f[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
    }
    if (p.norm) {
      const float rs = L.rstd[r];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f[2 * j] = bf16_to_f32(f32_to_bf16(f[2 * j] * rs * __uint_as_float(gw[j] << 16)));
        f[2 * j + 1] = bf16_to_f32(f32_to_bf16(f[2 * j + 1] * rs * __uint_as_float(gw[j] & 0xFFFF0000u)));
      }
    }
    const uint4 packed = make_uint4(pack_bf16x2_exact(f[0], f[1]), pack_bf16x2_exact(f[2], f[3]),
                                    pack_bf16x2_exact(f[4], f[5]), pack_bf16x2_exact(f[6], f[7]));
    *(uint4*)(L.xn + r * XR + c8) = packed;
    if (nt == 0) {
      st_dev_16(p.xn + (size_t)r * p.H + c0 + c8, packed);
      if constexpr (FMT == MK2_FMT_MXFP4) {  // a 32-column block is 4 lanes (a DPP quad)
        float amax = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(f[j]));
        amax = fmaxf(amax, dpp_f32<DPP_XOR1>(amax));
        amax = fmaxf(amax, dpp_f32<DPP_XOR2>(amax));
        const uint32_t code = mxfp8_scale_code(amax);
        const float inv = e8m0_inverse(code);
        st_dev_8(p.xq + (size_t)r * p.H + c0 + c8,
                 make_uint2(f32x4_to_e4m3x4(f[0] * inv, f[1] * inv, f[2] * inv, f[3] * inv),
                            f32x4_to_e4m3x4(f[4] * inv, f[5] * inv, f[6] * inv, f[7] * inv)));
        if ((lane & 3) == 0) st_dev_u8(p.xs + (size_t)r * (p.H / 32) + (c0 + c8) / 32, code);
      } else if constexpr (FMT == MK2_FMT_A4W4) {  // MXFP4 per 32: a DPP quad
        float amax = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(f[j]));
        amax = fmaxf(amax, dpp_f32<DPP_XOR1>(amax));
        amax = fmaxf(amax, dpp_f32<DPP_XOR2>(amax));
        const uint32_t code = mxfp4_act_code(amax);
        st_dev_u32(p.xq + ((size_t)r * p.H + c0 + c8) / 2, f32x8_to_e2m1x8(f, code));
        if ((lane & 3) == 0) st_dev_u8(p.xs + (size_t)r * (p.H / 32) + (c0 + c8) / 32, code);
      } else if constexpr (FMT == MK2_FMT_W8A8) {  // E4M3 per 128 with an f32 scale: a DPP row
        float amax = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(f[j]));
        amax = row16_max(amax);
        float qs, inv;
        fp8_block_scale(amax, &qs, &inv);
        st_dev_8(p.xq + (size_t)r * p.H + c0 + c8,
                 make_uint2(f32x4_to_e4m3x4(f[0] * inv, f[1] * inv, f[2] * inv, f[3] * inv),
                            f32x4_to_e4m3x4(f[4] * inv, f[5] * inv, f[6] * inv, f[7] * inv)));
        if ((lane & 15) == 0) st_dev_f32(p.xsf + (size_t)r * (p.H / 128) + (c0 + c8) / 128, qs);
      }
    }
  }
  __syncthreads();
  f32x4 acc[NCG];
#pragma unroll
  for (int c = 0; c < NCG; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int i = wave; i < kbs; i += NW) {
    const int kb = kc * kbs + i;
    bf16x8 a[4];
    if (i == wave) {
#pragma unroll
      for (int q = 0; q < 4; ++q) a[q] = a0[q];
    } else {
      load_a_bf16(p.w_router + ((size_t)nt * KB + kb) * 4096, lane, a);
    }
#pragma unroll
    for (int c = 0; c < NCG; ++c) {
      const int row = c * 16 + (lane & 15);
      bf16x8 b[4];
      if (row < p.M) {
        const bf16_t* src = L.xn + row * XR + i * 128 + 32 * g;
#pragma unroll
        for (int q = 0; q < 4; ++q) b[q] = *(const bf16x8*)(src + 8 * q);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) b[q] = __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
      }
      acc[c] = mfma4_bf16(a, b, acc[c]);
    }
  }
#pragma unroll
  for (int c = 0; c < NCG; ++c)
    *(f32x4*)(L.red + ((wave * NCG + c) * 64 + lane) * 4) = acc[c];
  __syncthreads();
  const int nw_used = NW < kbs ? NW : kbs;
  for (int idx = threadIdx.x; idx < 16 * p.M; idx += NT) {
    const int e16 = idx & 15, row = idx >> 4, c = row >> 4, s16 = row & 15;
    const int l = (e16 >> 2) * 16 + s16, i = e16 & 3;
    float v = 0.f;
    for (int w = 0; w < nw_used; ++w) v += L.red[((w * NCG + c) * 64 + l) * 4 + i];
    st_pair(p.logit_part + ((size_t)kc * p.M + row) * p.E + nt * 16 + e16, __float_as_uint(v), tag);
  }
  __syncthreads();
}

// ------------------------------------------------------------- stage: route
// One workgroup of NT = 512; wave w takes rows w, w + NW, ...  Lane l holds experts
// 4l .. 4l+3 of the row: their logits are the slice partials, polled as tagged words
// and summed in slice order.  The row's top-k by (key desc, expert asc): each lane
// orders its 4 candidates (a stable bubble pass, so equal keys keep expert order), then
// each of topk rounds takes the largest head key of the wave (DPP max) and, among equal
// heads, the lowest lane, whose experts all lie below a higher lane's; the winning lane
// moves its head on.  Round k's pick lands in lane k, so the picks come out ranked.
// Then the distinct-expert list (ascending) from the expert flags, as tagged words
// (every slot up to Dmax, -1 past the count, so that an up/gate task polls its own
// slot and the count together), and the dense route-weight table rw [slot][row] for
// the down (published by the caller's counter).  Returns false when the launch is
// failing (a poll gave up).
// Above 8 rows the persistent layer spreads the rows' top-k over several workgroups:
// ROUTE_PICK takes rows r0 .. r1-1 (logits, top-k) and stores their picks as tagged
// words; ROUTE_LEAD takes its own rows the same way, polls every other row's picks,
// then puts out the list and the tables as ROUTE_ALL does.
struct RouteLds {
  int flag[256];     // expert: 1 if picked, then its slot (-1: none)
  int ids[32 * 8];   // [M][topk]
  float w[32 * 8];   // [M][topk]
  float rw[256 * 32];
  uint32_t mask[256];  // slot: its rows (compacted rows)
  float lg[32 * 256];  // [M][E] logits
  float bias[256];
  int tot;
  int bad;
};

template <int CTRL, int ROWS>
MK2_DEV uint32_t dpp_u32(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWS, 0xF, false);
}
MK2_DEV uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<DPP_XOR1, 0xF>(0u, v));
  v = max(v, dpp_u32<DPP_XOR2, 0xF>(0u, v));
  v = max(v, dpp_u32<DPP_HALF_MIRROR, 0xF>(0u, v));
  v = max(v, dpp_u32<DPP_MIRROR, 0xF>(0u, v));
  v = max(v, dpp_u32<DPP_BCAST15, 0xA>(0u, v));
  v = max(v, dpp_u32<DPP_BCAST31, 0xC>(0u, v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

enum { ROUTE_ALL = 0, ROUTE_PICK = 1, ROUTE_LEAD = 2 };
// CMP: the compacted-row tables as well (compact_rows(p) must agree)
template <int NT, bool CMP = false, int MODE = ROUTE_ALL, typename Mark = NoMark>
MK2_DEV bool moe_route(const MoeDev& p, RouteLds& L, const TagPoll& tp, Mark mark = Mark(), int r0 = 0, int r1 = 0) {
  if (MODE == ROUTE_ALL) r0 = 0, r1 = p.M;
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int el = min(lane, p.E / 4 - 1);  // lanes past E/4 repeat the last group, unused
  const bool sig = p.router == MK2_ROUTER_SIGMOID_BIAS;
  // the bias through LDS: no load of it stays in flight past the polls (a wait for it
  // later would also wait for every store issued since)
  for (int e = tid; e < p.E; e += NT) {
    L.flag[e] = 0;
    L.bias[e] = sig ? p.bias[e] : 0.f;
    if (CMP) L.mask[e] = 0u;
  }
  for (int i = tid; i < p.Dmax * 32; i += NT) L.rw[i] = 0.f;
  if (tid == 0) L.bad = 0;
  __syncthreads();
  // the logits: each thread takes 16-byte pieces (two experts of a row) of the [M][E]
  // plane and polls that piece in every slice's plane (coalesced device-coherent loads
  // of two tagged words) until all carry the tag, then sums the slices in slice order
  bool bad = false;
  {
    const int pieces = r1 * p.E / 2;
    const uint32_t plane = (uint32_t)(p.M * p.E) * 8u;  // bytes a slice
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.logit_part, (short)0, (int)(plane * p.KC), 0x00020000);
    for (int c0 = r0 * p.E / 2; c0 < pieces && !bad; c0 += 2 * NT) {
      float sum[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
      // up to eight slices a poll round: one round trip for hidden <= 8192
      constexpr int KU = 8;
      for (int kc0 = 0; kc0 < p.KC && !bad; kc0 += KU) {
        i32x4 t[2][KU];
        WaitClock wc;
        for (int polls = 1;; ++polls) {
          bool ready = true;
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int u = 0; u < KU; ++u) {
              const int c = min(c0 + tid + i * NT, pieces - 1), kc = min(kc0 + u, p.KC - 1);
              t[i][u] = __builtin_amdgcn_raw_buffer_load_b128(rs, kc * plane + (uint32_t)c * 16u, 0, 16 /* sc1 */);
            }
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int u = 0; u < KU; ++u)
              ready = ready && (tp.tag == 0 || ((uint32_t)t[i][u].y == tp.tag && (uint32_t)t[i][u].w == tp.tag));
          if (poll_done(ready, polls, wc, tp, &bad)) break;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int u = 0; u < KU; ++u)
            if (kc0 + u < p.KC) {
              sum[i][0] += __int_as_float(t[i][u].x);
              sum[i][1] += __int_as_float(t[i][u].z);
            }
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int c = c0 + tid + i * NT;
        if (c < pieces) {
          L.lg[2 * c] = sum[i][0];
          L.lg[2 * c + 1] = sum[i][1];
        }
      }
    }
  }
  if (bad && lane == 0) L.bad = 1;
  __syncthreads();
  if (L.bad) return false;
  mark(0);
  constexpr float LOG2E = 1.4426950408889634f;
  for (int r = r0 + wave; r < r1; r += NW) {
    const float4 v = *(const float4*)(L.lg + r * p.E + 4 * el);
    const float4 bias = *(const float4*)(L.bias + 4 * el);
    const bool live = 4 * lane < p.E;
    if (p.logits && live) *(float4*)(p.logits + (size_t)r * p.E + 4 * lane) = v;
    const float lg[4] = {v.x, v.y, v.z, v.w}, bs[4] = {bias.x, bias.y, bias.z, bias.w};
    // the score a pick is weighted by: sigmoid as the reference kernel takes it, rcp(1 +
    // exp2(-x log2 e)) with the hardware exp2 and rcp; the softmax router's is the logit
    float sv[4];
    uint32_t key[4];
    int ix[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sv[i] = sig ? __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-lg[i] * LOG2E)) : lg[i];
      key[i] = live ? radix_key(sig ? sv[i] + bs[i] : lg[i]) : 0u;  // live keys are > 0
      ix[i] = i;
    }
    // stable bubble order, keys descending
#pragma unroll
    for (int j = 1; j < 4; ++j)
#pragma unroll
      for (int k = j; k > 0; --k) {
        const bool sw = key[k] > key[k - 1];
        const uint32_t tk = key[k];
        const int ti = ix[k];
        key[k] = sw ? key[k - 1] : key[k];
        ix[k] = sw ? ix[k - 1] : ix[k];
        key[k - 1] = sw ? tk : key[k - 1];
        ix[k - 1] = sw ? ti : ix[k - 1];
      }
    // round k takes the wave's largest head key; among equal heads the lowest lane,
    // whose experts all lie below a higher lane's.  The winning lane moves its head on
    // and notes the round in which its c-th candidate went.
    int taken = 0, rk[4] = {-1, -1, -1, -1};
    for (int k = 0; k < p.topk; ++k) {
      const uint32_t top = wave_max_u32(key[0]);
      const int wl = __ffsll((unsigned long long)__ballot(key[0] == top)) - 1;
      if (lane == wl) {
        rk[0] = taken == 0 ? k : rk[0];
        rk[1] = taken == 1 ? k : rk[1];
        rk[2] = taken == 2 ? k : rk[2];
        rk[3] = taken == 3 ? k : rk[3];
        ++taken;
        key[0] = key[1];
        key[1] = key[2];
        key[2] = key[3];
        key[3] = 0u;
      }
    }
    // the picks to LDS by round, then lane k holds pick k
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (c < taken) {
        const int i = ix[c];
        L.ids[r * p.topk + rk[c]] = 4 * lane + i;
        L.w[r * p.topk + rk[c]] = i == 0 ? sv[0] : i == 1 ? sv[1] : i == 2 ? sv[2] : sv[3];
      }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    const int my_e = lane < p.topk ? L.ids[r * p.topk + lane] : 0;
    const float my_v = lane < p.topk ? L.w[r * p.topk + lane] : 0.f;
    float w;
    if (sig) {
      const float tot = wave_sum(lane < p.topk ? my_v : 0.f);
      w = my_v * (__builtin_amdgcn_rcpf(tot) * p.route_scale);
    } else {
      const float top = wave_max(lane < p.topk ? my_v : -INFINITY);
      const float ex = lane < p.topk ? __builtin_amdgcn_exp2f((my_v - top) * LOG2E) : 0.f;
      w = ex * __builtin_amdgcn_rcpf(wave_sum(ex));
    }
    if (lane < p.topk) {
      st_dev_i32(p.topk_ids + r * p.topk + lane, my_e);
      st_dev_f32(p.topk_w + r * p.topk + lane, w);
      if (MODE == ROUTE_PICK) {
        st_pair(p.picks + 2 * (r * p.topk + lane), (uint32_t)my_e, tp.tag);
        st_pair(p.picks + 2 * (r * p.topk + lane) + 1, __float_as_uint(w), tp.tag);
      }
      L.w[r * p.topk + lane] = w;
      L.flag[my_e] = 1;
    }
  }
  if (MODE == ROUTE_PICK) {
    __syncthreads();  // the caller's next stage reuses this LDS
    return true;
  }
  if (MODE == ROUTE_LEAD) {
    // every other row's picks, one tagged word a thread a round
    const int words = 2 * p.M * p.topk;
    for (int i0 = 0; i0 < words && !bad; i0 += NT) {
      const int i = min(i0 + tid, words - 1);
      const bool own = i / (2 * p.topk) >= r0 && i / (2 * p.topk) < r1;
      uint64_t w = 0;
      WaitClock wc;
      for (int polls = 1;; ++polls) {
        w = own ? 0 : ld_pair(p.picks + i);
        if (poll_done(own || pair_ready(w, tp), polls, wc, tp, &bad)) break;
      }
      if (i0 + tid < words && !own && !bad) {
        const int j = i >> 1;
        if (i & 1) {
          L.w[j] = __uint_as_float(pair_value(w));
        } else {  // an id out of range (never written by a pick task) flags nothing
          const uint32_t e = pair_value(w);
          L.ids[j] = e < (uint32_t)p.E ? (int)e : 0;
          if (e < (uint32_t)p.E) L.flag[e] = 1;
        }
      }
    }
    if (bad && lane == 0) L.bad = 1;
    __syncthreads();
    if (L.bad) return false;
  }
  __syncthreads();
  mark(1);
  // the distinct experts, ascending (one wave: four ballots over e = lane + 64 i); the
  // list's slots past the count hold -1
  if (wave == 0) {
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    int tot = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane + 64 * i;
      const int f = e < p.E ? L.flag[e] : 0;
      const uint64_t m = __ballot(f != 0);
      if (e < p.E) {
        const int pos = tot + __popcll(m & below);
        L.flag[e] = f ? pos : -1;
        if (f) st_pair(p.act + 1 + pos, (uint32_t)e, tp.tag);
      }
      tot += __popcll(m);
    }
    for (int j = tot + lane; j < p.Dmax; j += 64) st_pair(p.act + 1 + j, 0xFFFFFFFFu, tp.tag);
    if (lane == 0) {
      st_pair(p.act, (uint32_t)tot, tp.tag);
      L.tot = tot;
    }
  }
  __syncthreads();
  mark(2);
  const int total = L.tot;
  for (int idx = tid; idx < p.M * p.topk; idx += NT) {
    const int s = L.flag[L.ids[idx]], r = idx / p.topk;
    L.rw[s * 32 + r] = L.w[idx];
    if (CMP) atomicOr(&L.mask[s], 1u << r);
  }
  __syncthreads();
  if constexpr (!CMP) {
    for (int idx = 4 * tid; idx < total * 32; idx += 4 * NT)
      st_dev_16(p.rw + idx, make_uint4(__float_as_uint(L.rw[idx]), __float_as_uint(L.rw[idx + 1]),
                                       __float_as_uint(L.rw[idx + 2]), __float_as_uint(L.rw[idx + 3])));
    return true;
  }
  // compacted rows: slot j's rows (a tagged mask for its up/gate tasks, which poll it
  // with their expert id), their route weights and row ids in row order
  for (int j = tid; j < p.Dmax; j += NT) {
    const uint32_t m = j < total ? L.mask[j] : 0u;
    st_pair(p.act_rows + j, m, tp.tag);
    uint32_t mm = m;
    for (int c = 0; mm; ++c, mm &= mm - 1) {
      const int r = __ffs((int)mm) - 1;
      st_dev_f32(p.rw + j * 32 + c, L.rw[j * 32 + r]);
      st_dev_i32(p.rowc + j * 32 + c, r);
    }
  }
  return true;
}

// ------------------------------------------------------- stage: up/gate + SwiGLU
// A chunk is 16*CT intermediate rows of one expert: CT gate tiles and the CT matching
// up tiles of the stacked [gate; up] matrix, against all decode rows; mid =
// silu(gate) * up.  Each wave owns every NW-th 128-k block and issues the loads of a
// batch of its blocks (weights, scales, activations) before the first MFMA.
template <int NT, int NCG, int CT, int FMT>
MK2_DEV void upgate_chunk(const MoeDev& p, bool shared, int j, int e, int c, float* red, float* midf,
                          uint32_t rows = 0u) {
  constexpr int NW = NT / 64, NQ = 2 * CT, R = 16 * CT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4;
  const int KB = p.H / 128;
  const int I = shared ? p.SI : p.I;
  const int NT16 = 2 * I / 16;  // 16-row tiles of the stacked gate|up
  int nts[NQ];
#pragma unroll
  for (int q = 0; q < CT; ++q) {
    nts[q] = CT * c + q;
    nts[CT + q] = I / 16 + CT * c + q;
  }
  f32x4 acc[NQ][NCG];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) acc[q][cg] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (!shared && (FMT == MK2_FMT_MXFP4 || FMT == MK2_FMT_A4W4)) {
    // scaled MFMA: E2M1 weights against MXFP8 (A8W4) or MXFP4 (A4W4) activations
    constexpr bool a4 = FMT == MK2_FMT_A4W4;
    constexpr int B = CT == 4 ? (NCG == 1 ? 3 : 2) : (NCG == 1 ? 4 : 3);  // k-blocks in flight
    const uint8_t* wbase = p.w13 + (size_t)e * NT16 * KB * 1024;
    const uint8_t* sbase = p.s13 + e * e8m0_expert_bytes(p.wl, 2 * I, p.H);
    // the MFMA columns: rows 16 cg + c16, or with compacted rows the slot's (16 cg +
    // c16)-th row (p.M: none, read as zeros); a second column group only if the slot
    // has more than 16 rows
    constexpr bool CMP = kCompact<NCG, FMT>;
    const int cnt = CMP ? __popc(rows) : p.M;
    int xrow[NCG];
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) {
      const int cc = cg * 16 + (lane & 15);
      xrow[cg] = CMP ? (cc < cnt ? nth_bit(rows, cc) : p.M) : cc;
    }
    const bool two = !CMP || cnt > 16;
    for (int kb0 = wave; kb0 < KB; kb0 += NW * B) {
      i32x8 a[B][NQ], b[B][NCG];
      int sa[B][NQ], sb[B][NCG];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int kb = min(kb0 + u * NW, KB - 1);  // past the end: a valid block, unused
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          a[u][q] = load_a_fp4(wbase + ((size_t)nts[q] * KB + kb) * 1024, lane);
          sa[u][q] = (int)(e8m0_word(sbase, p.wl, p.H, nts[q], kb, lane) >> e8m0_shift(p.wl, nts[q], kb));
        }
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) {
          const int row = xrow[cg];
          b[u][cg] = a4 ? load_b_fp4(p.xq, row, p.M, p.H / 2, kb * 64, g) : load_b_fp8(p.xq, row, p.M, p.H, kb * 128, g);
          sb[u][cg] = row < p.M ? (int)ldp_u8(p.xs + (size_t)row * (p.H / 32) + kb * 4 + g) : E8M0_ONE;
        }
      }
#pragma unroll
      for (int u = 0; u < B; ++u) {
        if (kb0 + u * NW >= KB) break;
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) {
          if (cg == 1 && !two) break;  // no rows there (uniform)
#pragma unroll
          for (int q = 0; q < NQ; ++q)
            acc[q][cg] = a4 ? mfma_same<4>(a[u][q], b[u][cg], acc[q][cg], sa[u][q], sb[u][cg])
                            : mfma_fp4_fp8<0, 0>(a[u][q], b[u][cg], acc[q][cg], sa[u][q], sb[u][cg]);
        }
      }
    }
  } else if (!shared && FMT == MK2_FMT_A16W4) {
    // E2M1 weights widened exactly to bf16 (x their E8M0) right before bf16 MFMAs on the
    // bf16 rows: no scale to apply after
    constexpr int B = NCG == 1 ? 2 : 1;
    const uint8_t* wbase = p.w13 + (size_t)e * NT16 * KB * 1024;
    const uint8_t* sbase = p.s13 + e * e8m0_expert_bytes(p.wl, 2 * I, p.H);
    for (int kb0 = wave; kb0 < KB; kb0 += NW * B) {
      uint4 raw[B][NQ];
      uint32_t sw[B][NQ];
      bf16x8 bx[B][NCG][4];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int kb = min(kb0 + u * NW, KB - 1);
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          raw[u][q] = ld_stream16(wbase + (((size_t)nts[q] * KB + kb) * 64 + lane) * 16);
          sw[u][q] = (e8m0_word(sbase, p.wl, p.H, nts[q], kb, lane) >> e8m0_shift(p.wl, nts[q], kb)) & 0xFFu;
        }
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg)
          load_b_bf16(p.xn, cg * 16 + (lane & 15), p.M, p.H, kb * 128 + 32 * g, bx[u][cg]);
      }
#pragma unroll
      for (int u = 0; u < B; ++u) {
        if (kb0 + u * NW >= KB) break;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const float sc = e8m0_to_f32(sw[u][q]);
          bf16x8 aa[4];
          aa[0] = e2m1x8_to_bf16(raw[u][q].x, sc);
          aa[1] = e2m1x8_to_bf16(raw[u][q].y, sc);
          aa[2] = e2m1x8_to_bf16(raw[u][q].z, sc);
          aa[3] = e2m1x8_to_bf16(raw[u][q].w, sc);
#pragma unroll
          for (int cg = 0; cg < NCG; ++cg) acc[q][cg] = mfma4_bf16(aa, bx[u][cg], acc[q][cg]);
        }
      }
    }
  } else if constexpr (CT == 2) {
    constexpr int B = NCG == 1 ? 3 : 2;
    const uint8_t* wbase = shared ? p.ws13 : p.w13 + (size_t)e * NT16 * KB * 2048;
    const float* sbase = shared ? p.ss13 : (const float*)p.s13 + (size_t)e * (2 * I / 128) * KB;
    for (int kb0 = wave; kb0 < KB; kb0 += NW * B) {
      uint4 raw[B][NQ][2];
      bf16x8 bx[B][NCG][4];
      float sc[B][NQ];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int kb = min(kb0 + u * NW, KB - 1);
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          load_fp8_block(wbase + ((size_t)nts[q] * KB + kb) * 2048, p.wl, lane, raw[u][q][0], raw[u][q][1]);
          sc[u][q] = sbase[(nts[q] * 16 / 128) * KB + kb];
        }
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg)
          load_b_bf16(p.xn, cg * 16 + (lane & 15), p.M, p.H, kb * 128 + 32 * g, bx[u][cg]);
      }
#pragma unroll
      for (int u = 0; u < B; ++u) {
        if (kb0 + u * NW >= KB) break;
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) {
          const bf16x8* bb = bx[u][cg];
#pragma unroll
          for (int q = 0; q < NQ; ++q) {
            bf16x8 aa[4];
            aa[0] = e4m3x8_to_bf16(raw[u][q][0].x, raw[u][q][0].y);
            aa[1] = e4m3x8_to_bf16(raw[u][q][0].z, raw[u][q][0].w);
            aa[2] = e4m3x8_to_bf16(raw[u][q][1].x, raw[u][q][1].y);
            aa[3] = e4m3x8_to_bf16(raw[u][q][1].z, raw[u][q][1].w);
            acc[q][cg] += mfma4_bf16(aa, bb, f32x4{0.f, 0.f, 0.f, 0.f}) * sc[u][q];
          }
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg)
      *(f32x4*)(red + (((wave * NQ + q) * NCG + cg) * 64 + lane) * 4) = acc[q][cg];
  __syncthreads();
  // gate tile t2 and up tile CT + t2 summed over the waves, columns 4k .. 4k + 3 of
  // one row a thread: a wave's lanes take consecutive rows, so every read is a whole
  // 16-byte word and the lanes' words fall in distinct banks
  for (int idx = threadIdx.x; idx < 64 * CT * NCG; idx += NT) {
    const int s16 = idx & 15, k = (idx >> 4) & 3, t2 = (idx >> 6) % CT, cg = (idx >> 6) / CT;
    const int l = k * 16 + s16;
    f32x4 gs = {0.f, 0.f, 0.f, 0.f}, us = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      gs += *(const f32x4*)(red + (((w * NQ + t2) * NCG + cg) * 64 + l) * 4);
      us += *(const f32x4*)(red + (((w * NQ + CT + t2) * NCG + cg) * 64 + l) * 4);
    }
    const int s = cg * 16 + s16, n = t2 * 16 + 4 * k;
#pragma unroll
    for (int i = 0; i < 4; ++i) midf[s * (R + 1) + n + i] = silu_mul(gs[i], us[i]);
  }
  __syncthreads();
  if (!shared && FMT == MK2_FMT_A4W4) {
    // MXFP4 per 32 values of a row: 32 lanes a block as below, 8 codes a store
    for (int idx = threadIdx.x; idx < R * p.M; idx += NT) {
      const int n = idx % R, s = idx / R;
      const float v = midf[s * (R + 1) + n];
      const float amax = max_xor16(row16_max(fabsf(v)));
      const uint32_t code = mxfp4_act_code(amax);
      const float sc = __uint_as_float(code ? code << 23 : 0x00400000u);
      const uint32_t q = (uint32_t)__builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, v, 0.f, sc, 0) & 0xFu;
      const uint32_t w = q | (dpp_shl<1>(q) << 4) | (dpp_shl<2>(q) << 8) | (dpp_shl<3>(q) << 12) |
                         (dpp_shl<4>(q) << 16) | (dpp_shl<5>(q) << 20) | (dpp_shl<6>(q) << 24) | (dpp_shl<7>(q) << 28);
      if ((n & 7) == 0) st_dev_u32(p.mid_q + (((size_t)j * p.M + s) * p.I + c * R + n) / 2, w);
      if ((n & 31) == 0) st_dev_u8(p.mid_s + ((size_t)j * p.M + s) * (p.I / 32) + (c * R + n) / 32, code);
    }
  } else if (!shared && FMT == MK2_FMT_MXFP4) {
    // MXFP8 per 32 values of a row: 32 lanes (two DPP rows) a block, amax by DPP and a
    // row swap, 4 codes a store (DPP row shifts)
    for (int idx = threadIdx.x; idx < R * p.M; idx += NT) {
      const int n = idx % R, s = idx / R;
      const float v = midf[s * (R + 1) + n];
      const float amax = max_xor16(row16_max(fabsf(v)));
      const uint32_t code = mxfp8_scale_code(amax);
      const uint32_t q = f32_to_e4m3(v * e8m0_inverse(code));
      const uint32_t w = q | (dpp_shl<1>(q) << 8) | (dpp_shl<2>(q) << 16) | (dpp_shl<3>(q) << 24);
      if ((n & 3) == 0) st_dev_u32(p.mid_q + ((size_t)j * p.M + s) * p.I + c * R + n, w);
      if ((n & 31) == 0) st_dev_u8(p.mid_s + ((size_t)j * p.M + s) * (p.I / 32) + c * (R / 32) + (n >> 5), code);
    }
  } else {
    bf16_t* dst = shared ? p.mid_sh : p.mid_b + (size_t)j * p.M * p.I;
    for (int idx = threadIdx.x; idx < R * p.M; idx += NT) {
      const int n = idx % R, s = idx / R;
      st_dev_u16(dst + (size_t)s * I + c * R + n, f32_to_bf16(midf[s * (R + 1) + n]));
    }
  }
  __syncthreads();
}

// W8A8 routed chunk c of slot j (expert e): 128 intermediate rows, wave w taking gate
// tile 8c + w and its up tile over the whole hidden dim (no cross-wave sum), E4M3
// weights against the rows' E4M3 activations on the scaled MFMA (E8M0 = 1), each
// k-block's product times w_scale x x_scale (the x scale per decode row, one a lane).
// mid = silu(g) u is quantized to E4M3 per 128 (the chunk's rows of a decode row: its
// amax from all eight waves through LDS) with an f32 scale.  red: >= NW * 32 floats.
template <int NT, int NCG>
MK2_DEV void upgate_w8a8(const MoeDev& p, int j, int e, int c, float* red) {
  static_assert(NT / 64 == 8, "eight gate/up tile pairs, one a wave");
  constexpr int KBB = 2;  // k-blocks a batch
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
  const int KB = p.H / 128, I = p.I;
  const int NT16 = 2 * I / 16;
  const int tg = 8 * c + wave, tu = I / 16 + 8 * c + wave;
  const uint8_t* wbase = p.w13 + (size_t)e * NT16 * KB * 2048;
  const float* sg = (const float*)p.s13 + ((size_t)e * (2 * I / 128) + c) * KB;
  const float* su = (const float*)p.s13 + ((size_t)e * (2 * I / 128) + I / 128 + c) * KB;
  f32x4 ag[NCG], au[NCG];
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) ag[cg] = au[cg] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int kb0 = 0; kb0 < KB; kb0 += KBB) {
    uint4 rg[KBB][2], ru[KBB][2];
    i32x8 bq[KBB][NCG];
    float xs[KBB][NCG], wsg[KBB], wsu[KBB];
#pragma unroll
    for (int u = 0; u < KBB; ++u) {
      const int kb = min(kb0 + u, KB - 1);
      load_fp8_block(wbase + ((size_t)tg * KB + kb) * 2048, p.wl, lane, rg[u][0], rg[u][1]);
      load_fp8_block(wbase + ((size_t)tu * KB + kb) * 2048, p.wl, lane, ru[u][0], ru[u][1]);
      wsg[u] = sg[kb];
      wsu[u] = su[kb];
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        const int row = cg * 16 + c16;
        bq[u][cg] = load_b_fp8_same(p.xq, row, p.M, p.H, kb * 128, g);
        xs[u][cg] = row < p.M ? ldp_f32(p.xsf + (size_t)row * (p.H / 128) + kb) : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < KBB; ++u) {
      if (kb0 + u >= KB) break;
      const i32x8 A = {(int)rg[u][0].x, (int)rg[u][0].y, (int)rg[u][0].z, (int)rg[u][0].w,
                       (int)rg[u][1].x, (int)rg[u][1].y, (int)rg[u][1].z, (int)rg[u][1].w};
      const i32x8 U = {(int)ru[u][0].x, (int)ru[u][0].y, (int)ru[u][0].z, (int)ru[u][0].w,
                       (int)ru[u][1].x, (int)ru[u][1].y, (int)ru[u][1].z, (int)ru[u][1].w};
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        ag[cg] += mfma_same<0>(A, bq[u][cg], z, E8M0_ONE, E8M0_ONE) * (wsg[u] * xs[u][cg]);
        au[cg] += mfma_same<0>(U, bq[u][cg], z, E8M0_ONE, E8M0_ONE) * (wsu[u] * xs[u][cg]);
      }
    }
  }
  // lane (g, c16) holds intermediate rows 128c + 16w + 4g + i of decode row cg*16 + c16
  float mid[NCG][4], amax[NCG];
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mid[cg][i] = silu_mul(ag[cg][i], au[cg][i]);
      m = fmaxf(m, fabsf(mid[cg][i]));
    }
    m = max_xor16(m);  // the column's 16 rows of this wave: over the four lane groups
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    m = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    if (g == 0) red[wave * 32 + cg * 16 + c16] = m;
  }
  __syncthreads();
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    float m = 0.f;
#pragma unroll
    for (int w = 0; w < 8; ++w) m = fmaxf(m, red[w * 32 + cg * 16 + c16]);
    amax[cg] = m;
  }
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    const int row = cg * 16 + c16;
    float qs, inv;
    fp8_block_scale(amax[cg], &qs, &inv);
    if (row < p.M) {
      const uint32_t w = f32x4_to_e4m3x4(mid[cg][0] * inv, mid[cg][1] * inv, mid[cg][2] * inv, mid[cg][3] * inv);
      st_dev_u32(p.mid_q + ((size_t)j * p.M + row) * I + 128 * c + 16 * wave + 4 * g, w);
      if (wave == 0 && g == 0) st_dev_f32(p.mid_sf + ((size_t)j * p.M + row) * (I / 128) + c, qs);
    }
  }
  __syncthreads();
}

// task t < Dmax * (I / UC): routed slot j = t / (I / UC), chunk of UC rows; past that
// the shared expert's 32-row chunks.  red: NW * 2 * CT * NCG * 256 floats (CT = UC/16);
// midf: 32 * (UC + 1) floats.
// Routed slot j's expert from the routing's tagged list: one wave polls the count and
// the slot's word together (-1 past the list); -2 when the launch is failing.
// With compacted rows (CMP) lane 2 also polls the slot's row mask: *rows (else all
// rows).
template <bool CMP>
MK2_DEV int slot_expert(const MoeDev& p, int j, const TagPoll& tp, int* lds, uint32_t* rows) {
  constexpr int nl = CMP ? 3 : 2;  // lanes that poll
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    bool bad = false;
    // two polls in flight: the next is issued before the last one is looked at
    const uint64_t* src = lane == 2 ? p.act_rows + j : p.act + (lane ? 1 + j : 0);
    uint64_t w = lane < nl ? ld_pair(src) : 0;
    WaitClock wc;
    for (int polls = 1;; polls += 2) {
      const uint64_t w1 = lane < nl ? ld_pair(src) : 0;
      if (poll_done(lane >= nl || pair_ready(w, tp), polls, wc, tp, &bad)) break;
      w = lane < nl ? ld_pair(src) : 0;
      if (poll_done(lane >= nl || pair_ready(w1, tp), polls + 1, wc, tp, &bad)) {
        w = w1;
        break;
      }
    }
    const int cnt = __builtin_amdgcn_readlane((int)pair_value(w), 0);
    const int e = __builtin_amdgcn_readlane((int)pair_value(w), 1);
    const uint32_t m = (uint32_t)__builtin_amdgcn_readlane((int)pair_value(w), 2);
    if (lane == 0) {
      lds[0] = bad ? -2 : (j >= cnt || e < 0 || e >= p.E ? -1 : e);
      lds[1] = nl == 3 ? (int)m : (int)(p.M >= 32 ? 0xFFFFFFFFu : (1u << p.M) - 1u);
    }
  }
  __syncthreads();
  const int e = lds[0];
  *rows = (uint32_t)lds[1];
  __syncthreads();
  return e;
}

// Task t: 1 when it ran, 0 for a routed slot past the routing's count (nothing to do),
// -1 when its wait failed (the same value in every thread)
template <int NT, int NCG, int FMT>
MK2_DEV int moe_upgate(const MoeDev& p, int t, float* red, float* midf, const TagPoll& tp) {
  const int chunks_r = p.I / p.UC;
  if (t < p.Dmax * chunks_r) {
    const int j = t / chunks_r, c = t % chunks_r;
    uint32_t rows;
    const int e = slot_expert<kCompact<NCG, FMT>>(p, j, tp, (int*)midf, &rows);
    if (e == -2) return -1;
    if (e < 0) return 0;
    if constexpr (FMT == MK2_FMT_W8A8) upgate_w8a8<NT, NCG>(p, j, e, c, red);
    else if (NCG == 1 && p.UC == 64) upgate_chunk<NT, NCG, (NCG == 1 ? 4 : 2), FMT>(p, false, j, e, c, red, midf, rows);
    else upgate_chunk<NT, NCG, 2, FMT>(p, false, j, e, c, red, midf, rows);
  } else {
    upgate_chunk<NT, NCG, 2, FMT>(p, true, 0, 0, t - p.Dmax * chunks_r, red, midf);
  }
  return 1;
}

// ---------------------------------------------------------- stage: down + combine
// A down task's hidden rows: tile tl[d], rows rlo[d] .. rhi[d] - 1 of it (every row of
// DT tiles, or with p.DT == 3 (DT 2) 24 rows: a whole tile and half of the next, in
// either order); c0 the first (its output column), ncol how many, live[d] whether
// lane row c16 is one of tile d's
template <int DT>
struct DownRows {
  int tl[DT], rlo[DT], rhi[DT], c0, ncol;
  bool live[DT];
  MK2_DEV DownRows(const MoeDev& p, int nt, int c16) {
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      tl[d] = nt * DT + d;
      rlo[d] = 0;
      rhi[d] = 16;
    }
    if (DT == 2 && p.DT == 3) {
      const int ta = (3 * nt) >> 1;
      tl[0] = ta;
      tl[DT - 1] = ta + 1;
      rlo[0] = nt & 1 ? 8 : 0;
      rhi[DT - 1] = nt & 1 ? 16 : 8;
    }
    c0 = tl[0] * 16 + rlo[0];
    ncol = 0;
#pragma unroll
    for (int d = 0; d < DT; ++d) ncol += rhi[d] - rlo[d];
#pragma unroll
    for (int d = 0; d < DT; ++d) live[d] = c16 >= rlo[d] && c16 < rhi[d];
  }
};

// The shared expert's first k-block of this wave (weights only, static: loaded before
// the mid activations' wait)
template <int DT>
MK2_DEV void down_shared_first(const MoeDev& p, const DownRows<DT>& t, int KB2s, int wave, int lane,
                               uint4 (&shraw)[DT][2], float (&shsc)[DT]) {
  const int kb = min(wave, max(KB2s, 1) - 1);
#pragma unroll
  for (int d = 0; d < DT; ++d) {
    shraw[d][0] = shraw[d][1] = make_uint4(0, 0, 0, 0);
    shsc[d] = 0.f;
    if (KB2s) {
      if (t.live[d]) load_fp8_block(p.ws2 + ((size_t)t.tl[d] * KB2s + kb) * 2048, p.wl, lane, shraw[d][0], shraw[d][1]);
      shsc[d] = p.ss2[(t.tl[d] * 16 / 128) * KB2s + kb];
    }
  }
}

// The residual rows (the W_o output, published before the routing) for the epilogue,
// straight into LDS (no registers held): dword d of the ncol / 2 * M is row
// d / (ncol / 2), columns 2 (d % (ncol / 2)) .. + 1 of the task's
template <int DT>
MK2_DEV void down_residual_lds(const MoeDev& p, const DownRows<DT>& t, float* xres, int wave) {
  const int half = t.ncol / 2;
  const int nxd = p.residual ? half * p.M : 0;
  if (threadIdx.x < nxd)
    __builtin_amdgcn_global_load_lds((const uint32_t*)(p.x + (size_t)(threadIdx.x / half) * p.H + t.c0) + threadIdx.x % half,
                                     (uint32_t*)xres + 64 * wave, 4, 0, 0);
}

// The shared expert (FP8, bf16 mid) into acc: its k-blocks spread over the NW waves,
// the first from shraw / shsc (down_shared_first)
template <int NW, int NCG, int DT>
MK2_DEV void down_shared(const MoeDev& p, const DownRows<DT>& t, int KB2s, int wave, int lane,
                         const uint4 (&shraw)[DT][2], const float (&shsc)[DT], f32x4 (&acc)[DT][NCG]) {
  const int g = lane >> 4, c16 = lane & 15;
  for (int kb = wave; kb < KB2s; kb += NW) {
    bf16x8 b[NCG][4];
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) load_b_bf16(p.mid_sh, cg * 16 + c16, p.M, p.SI, kb * 128 + 32 * g, b[cg]);
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      uint4 r0, r1;
      float sc;
      if (kb == wave) {
        r0 = shraw[d][0];
        r1 = shraw[d][1];
        sc = shsc[d];
      } else {
        r0 = r1 = make_uint4(0, 0, 0, 0);
        if (t.live[d]) load_fp8_block(p.ws2 + ((size_t)t.tl[d] * KB2s + kb) * 2048, p.wl, lane, r0, r1);
        sc = p.ss2[(t.tl[d] * 16 / 128) * KB2s + kb];
      }
      bf16x8 a[4];
      a[0] = e4m3x8_to_bf16(r0.x, r0.y);
      a[1] = e4m3x8_to_bf16(r0.z, r0.w);
      a[2] = e4m3x8_to_bf16(r1.x, r1.y);
      a[3] = e4m3x8_to_bf16(r1.z, r1.w);
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) acc[d][cg] += mfma4_bf16(a, b[cg], f32x4{0.f, 0.f, 0.f, 0.f}) * sc;
    }
  }
}

// The task's outputs: the waves' partial sums from LDS (CMP: each wave's [DT][16
// hidden][32 rows] accumulator; else its f32x4 MFMA tiles, which acc still holds and
// this stores first), plus the residual, rounded to bf16
template <int NT, int NCG, int DT, bool CMP>
MK2_DEV void down_epilogue(const MoeDev& p, const DownRows<DT>& t, float* red, const float* xres,
                           const f32x4 (*acc)[NCG] = nullptr) {
  constexpr int NW = NT / 64;
  if constexpr (!CMP) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) *(f32x4*)(red + (((wave * DT + d) * NCG + cg) * 64 + lane) * 4) = acc[d][cg];
  }
  drain_memory();  // this wave's residual dwords have landed in LDS
  __syncthreads();
  const int n0 = t.rhi[0] - t.rlo[0];  // the first tile's columns
  for (int idx = threadIdx.x; idx < t.ncol * p.M; idx += NT) {
    const int n = idx % t.ncol, s = idx / t.ncol;  // column c0 + n of row s
    const int d = n < n0 ? 0 : DT - 1, n16 = n < n0 ? t.rlo[0] + n : t.rlo[DT - 1] + n - n0;
    const int cg = s >> 4, s16 = s & 15;
    const int l = (n16 >> 2) * 16 + s16, i = n16 & 3;
    float y = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w)
      y += CMP ? red[((w * DT + d) * 16 + n16) * 32 + s] : red[(((w * DT + d) * NCG + cg) * 64 + l) * 4 + i];
    const size_t o = (size_t)s * p.H + t.c0 + n;
    if (p.residual) y += bf16_to_f32(((const bf16_t*)xres)[idx]);
    p.out[o] = f32_to_bf16(y);
  }
  __syncthreads();
}

// A task is 16*DT hidden rows (24 with p.DT == 3); every slot (the shared expert, then the D routed
// experts) adds rw * W_down[e] . mid into the rows' accumulators; out = bf16(y [+ x]).
// Waves take every NW-th slot, B slots a unit, the next unit's weight tiles and mid
// rows (shared by the DT tiles) in flight while a unit's MFMAs run.  act_ids: LDS >=
// 512 ints; red: NW * DT * NCG * 256 floats; xres: LDS >= 8 * DT * M words (the residual
// rows, bf16).
template <int NT, int NCG, int DT, int FMT, typename Wait>
MK2_DEV void down_rows(const MoeDev& p, int nt, float* red, int* act_ids, float* xres, Wait wait) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
  // the list, published by the routing's counter; read device-coherently: up/gate
  // tasks on this XCD polled its words before all of them were out
  const int D = min((int)pair_value(ld_pair(p.act)), p.Dmax);
  for (int j = threadIdx.x; j < D; j += NT) act_ids[j] = min(max((int)pair_value(ld_pair(p.act + 1 + j)), 0), p.E - 1);
  __syncthreads();
  const int HT = p.H / 16;
  const DownRows<DT> t(p, nt, c16);
  const auto& tl = t.tl;
  const auto& live = t.live;
  const int KB2s = p.n_shared ? p.SI / 128 : 0;
  const int KB2 = p.I / 128;
  constexpr int B = 1;                                 // MXFP4 slots a unit
  constexpr int KC = 2;                                // k-blocks of a slot a pass
  // weights only (static, or known since routing): the shared expert's first k-block
  // of this wave and its first batch of routed slots, loaded before `wait` (the mid
  // activations' dependency)
  uint4 shraw[DT][2];
  float shsc[DT];
  down_shared_first<DT>(p, t, KB2s, wave, lane, shraw, shsc);
  // the scaled-MFMA unit pipeline: E2M1 weights against MXFP8 (A8W4) or MXFP4 (A4W4) mid
  constexpr bool mx = FMT == MK2_FMT_MXFP4 || FMT == MK2_FMT_A4W4;
  constexpr bool a4 = FMT == MK2_FMT_A4W4;
  down_residual_lds<DT>(p, t, xres, wave);
  // the routed slots (MXFP4): a unit is a batch of B slots (wave + NW * (B * i + u))
  // over KC k-blocks; units u + 1 and u + 2 (weights, mid rows, scales and route
  // weights) are in flight while unit u's MFMAs run
  struct Unit {
    i32x8 a[B][DT][KC];
    i32x8 bq[B][KC][NCG];
    int sa[B][DT];
    int sbq[B][KC][NCG];
    float wr[B][NCG];
  };
  const int nkc = (KB2 + KC - 1) / KC;  // units a batch
  const int nu = mx && D > wave ? (D - wave + NW * B - 1) / (NW * B) * nkc : 0;
  auto load_w = [&](int u, Unit& x) {  // weights: known since the routing
    const int j0 = wave + (u / nkc) * NW * B, kb0 = (u % nkc) * KC;
#pragma unroll
    for (int ub = 0; ub < B; ++ub) {
      const int e = act_ids[min(j0 + ub * NW, D - 1)];  // past the list: a valid slot, unused
#pragma unroll
      for (int c = 0; c < KC; ++c)
#pragma unroll
        for (int d = 0; d < DT; ++d)
          x.a[ub][d][c] = live[d] ? load_a_fp4(p.w2 + (((size_t)e * HT + tl[d]) * KB2 + min(kb0 + c, KB2 - 1)) * 1024, lane)
                                  : i32x8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int d = 0; d < DT; ++d)
        x.sa[ub][d] = live[d] ? (int)e8m0_word(p.s2 + e * e8m0_expert_bytes(p.wl, p.H, p.I), p.wl, p.I, tl[d], kb0, lane)
                              : 127;
    }
  };
  auto load_m = [&](int u, Unit& x) {  // mid rows and route weights: after the wait
    const int j0 = wave + (u / nkc) * NW * B, kb0 = (u % nkc) * KC;
#pragma unroll
    for (int ub = 0; ub < B; ++ub) {
      const int j = min(j0 + ub * NW, D - 1);
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const int kb = min(kb0 + c, KB2 - 1);
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) {
          const int row = cg * 16 + c16;
          x.bq[ub][c][cg] = a4 ? load_b_fp4(p.mid_q + (size_t)j * p.M * (p.I / 2), row, p.M, p.I / 2, kb * 64, g)
                               : load_b_fp8(p.mid_q + (size_t)j * p.M * p.I, row, p.M, p.I, kb * 128, g);
          x.sbq[ub][c][cg] = row < p.M ? (int)ldp_u8(p.mid_s + ((size_t)j * p.M + row) * (p.I / 32) + kb * 4 + g) : 127;
        }
      }
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) x.wr[ub][cg] = ldp_f32(p.rw + j * 32 + cg * 16 + c16);
    }
  };
  f32x4 acc[DT][NCG], tmp[B][DT][NCG];
#pragma unroll
  for (int d = 0; d < DT; ++d)
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) acc[d][cg] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int u, Unit& x) {
    const int j0 = wave + (u / nkc) * NW * B, kb0 = (u % nkc) * KC;
    if (kb0 == 0) {
#pragma unroll
      for (int ub = 0; ub < B; ++ub)
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
          for (int cg = 0; cg < NCG; ++cg) tmp[ub][d][cg] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int ub = 0; ub < B; ++ub) {
      if (j0 + ub * NW >= D) break;
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const int kb = kb0 + c;
        if (kb >= KB2) break;
#pragma unroll
        for (int d = 0; d < DT; ++d) {
          const int sak = x.sa[ub][d] >> e8m0_shift(p.wl, tl[d], kb);
#pragma unroll
          for (int cg = 0; cg < NCG; ++cg)
            tmp[ub][d][cg] = a4 ? mfma_same<4>(x.a[ub][d][c], x.bq[ub][c][cg], tmp[ub][d][cg], sak, x.sbq[ub][c][cg])
                                : mfma_fp4_fp8<0, 0>(x.a[ub][d][c], x.bq[ub][c][cg], tmp[ub][d][cg], sak, x.sbq[ub][c][cg]);
        }
      }
    }
    if (kb0 + KC >= KB2) {
#pragma unroll
      for (int ub = 0; ub < B; ++ub) {
        if (j0 + ub * NW >= D) break;
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg)
#pragma unroll
          for (int d = 0; d < DT; ++d) acc[d][cg] += tmp[ub][d][cg] * x.wr[ub][cg];
      }
    }
  };
  Unit x0, x1, x2;
  if (nu > 0) load_w(0, x0);
  if (nu > 1) load_w(1, x1);
  if (!wait()) return;
  if (nu > 0) load_m(0, x0);
  if (nu > 1) load_m(1, x1);
  down_shared<NW, NCG, DT>(p, t, KB2s, wave, lane, shraw, shsc, acc);
  if constexpr (mx) {
    auto step = [&](int u, Unit& cur, Unit& nxt2) {
      if (u + 2 < nu) {
        load_w(u + 2, nxt2);
        load_m(u + 2, nxt2);
      }
      if (u < nu) compute(u, cur);
    };
    for (int u = 0; u < nu; u += 3) {
      step(u, x0, x2);
      step(u + 1, x1, x0);
      step(u + 2, x2, x1);
    }
  } else if constexpr (DT == 1) {
    if constexpr (FMT == MK2_FMT_A16W4) {
      // E2M1 weights widened exactly to bf16 against the bf16 mid, 8 k-blocks a batch
      constexpr int KMAX = 8;
      for (int j = wave; j < D; j += NW) {
        const int e = act_ids[j];
        const uint8_t* wb = p.w2 + ((size_t)e * HT + tl[0]) * KB2 * 1024;
        const uint8_t* sb = p.s2 + e * e8m0_expert_bytes(p.wl, p.H, p.I);
        f32x4 t[NCG];
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) t[cg] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int kb0 = 0; kb0 < KB2; kb0 += KMAX) {
          uint4 raw[KMAX];
          uint32_t sw[KMAX];
#pragma unroll
          for (int u = 0; u < KMAX; ++u) {
            const int kb = min(kb0 + u, KB2 - 1);
            raw[u] = ld_stream16(wb + ((size_t)kb * 64 + lane) * 16);
            sw[u] = (e8m0_word(sb, p.wl, p.I, tl[0], kb, lane) >> e8m0_shift(p.wl, tl[0], kb)) & 0xFFu;
          }
#pragma unroll
          for (int u = 0; u < KMAX; ++u) {
            const int kb = kb0 + u;
            if (kb >= KB2) break;
            const float sc = e8m0_to_f32(sw[u]);
            bf16x8 a[4];
            a[0] = e2m1x8_to_bf16(raw[u].x, sc);
            a[1] = e2m1x8_to_bf16(raw[u].y, sc);
            a[2] = e2m1x8_to_bf16(raw[u].z, sc);
            a[3] = e2m1x8_to_bf16(raw[u].w, sc);
#pragma unroll
            for (int cg = 0; cg < NCG; ++cg) {
              bf16x8 b[4];
              load_b_bf16(p.mid_b + (size_t)j * p.M * p.I, cg * 16 + c16, p.M, p.I, kb * 128 + 32 * g, b);
              t[cg] = mfma4_bf16(a, b, t[cg]);
            }
          }
        }
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) acc[0][cg] += t[cg] * ldp_f32(p.rw + j * 32 + cg * 16 + c16);
      }
    } else {
      // E4M3 weights (f32 scale per 128 x 128 block): widened to bf16 against the bf16
      // mid (W8A16), or on the scaled MFMA against the E4M3 mid (W8A8, f32 scale per 128
      // a row); each k-block's product times its scales and the route weight
      constexpr int KMAX = 8;  // inter <= 1024
      constexpr bool w8a8 = FMT == MK2_FMT_W8A8;
      for (int j = wave; j < D; j += NW) {
        const int e = act_ids[j];
        const uint8_t* wb = p.w2 + ((size_t)e * HT + tl[0]) * KB2 * 2048;
        const float* sbase = (const float*)p.s2 + (size_t)e * (p.H / 128) * KB2 + (tl[0] * 16 / 128) * KB2;
        uint4 raw[KMAX][2];
#pragma unroll
        for (int kb = 0; kb < KMAX; ++kb) {
          load_fp8_block(wb + (size_t)min(kb, KB2 - 1) * 2048, p.wl, lane, raw[kb][0], raw[kb][1]);
        }
#pragma unroll
        for (int kb = 0; kb < KMAX; ++kb) {
          if (kb >= KB2) break;
          const float sc = sbase[kb];
          if constexpr (w8a8) {
            const i32x8 A = {(int)raw[kb][0].x, (int)raw[kb][0].y, (int)raw[kb][0].z, (int)raw[kb][0].w,
                             (int)raw[kb][1].x, (int)raw[kb][1].y, (int)raw[kb][1].z, (int)raw[kb][1].w};
#pragma unroll
            for (int cg = 0; cg < NCG; ++cg) {
              const int row = cg * 16 + c16;
              const i32x8 bq = load_b_fp8_same(p.mid_q + (size_t)j * p.M * p.I, row, p.M, p.I, kb * 128, g);
              const float ms = row < p.M ? ldp_f32(p.mid_sf + ((size_t)j * p.M + row) * (p.I / 128) + kb) : 0.f;
              acc[0][cg] += mfma_same<0>(A, bq, f32x4{0.f, 0.f, 0.f, 0.f}, E8M0_ONE, E8M0_ONE) *
                            (sc * ms * ldp_f32(p.rw + j * 32 + row));
            }
          } else {
            bf16x8 a[4];
            a[0] = e4m3x8_to_bf16(raw[kb][0].x, raw[kb][0].y);
            a[1] = e4m3x8_to_bf16(raw[kb][0].z, raw[kb][0].w);
            a[2] = e4m3x8_to_bf16(raw[kb][1].x, raw[kb][1].y);
            a[3] = e4m3x8_to_bf16(raw[kb][1].z, raw[kb][1].w);
#pragma unroll
            for (int cg = 0; cg < NCG; ++cg) {
              bf16x8 b[4];
              load_b_bf16(p.mid_b + (size_t)j * p.M * p.I, cg * 16 + c16, p.M, p.I, kb * 128 + 32 * g, b);
              acc[0][cg] += mfma4_bf16(a, b, f32x4{0.f, 0.f, 0.f, 0.f}) * (sc * ldp_f32(p.rw + j * 32 + cg * 16 + c16));
            }
          }
        }
      }
    }
  }
  down_epilogue<NT, NCG, DT, false>(p, t, red, xres, acc);
}

// The down with compacted rows (kCompact: the scaled-MFMA modes above 16 rows): as
// down_rows' scaled-MFMA path, each slot's columns being its rows in order, added into
// per-wave [DT][16 hidden][32 rows] accumulators in LDS.  The unit pipeline is its own
// (the compacted columns change every unit's loads and accumulation); the task rows,
// the shared expert's first k-block and the residual are down_rows' helpers.  Its
// shared-expert loop and epilogue stay written out here: as calls of down_shared and
// down_epilogue the 32-row kernel spilled more registers and ran 0.8-0.9 us slower each.
template <int NT, int NCG, int DT, int FMT, typename Wait>
MK2_DEV void down_rows_cmp(const MoeDev& p, int nt, float* red, int* act_ids, float* xres, Wait wait) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
  static_assert(kCompact<NCG, FMT>, "compacted rows: the scaled-MFMA modes above 16 rows");
  // the list, published by the routing's counter; read device-coherently: up/gate
  // tasks on this XCD polled its words before all of them were out
  const int D = min((int)pair_value(ld_pair(p.act)), p.Dmax);
  for (int j = threadIdx.x; j < D; j += NT) {
    act_ids[j] = min(max((int)pair_value(ld_pair(p.act + 1 + j)), 0), p.E - 1);
    act_ids[256 + j] = __popc((uint32_t)pair_value(ld_pair(p.act_rows + j)));  // the slot's rows
  }
  __syncthreads();
  const int HT = p.H / 16;
  const DownRows<DT> t(p, nt, c16);
  const auto& tl = t.tl;
  const auto& live = t.live;
  const int KB2s = p.n_shared ? p.SI / 128 : 0;
  const int KB2 = p.I / 128;
  constexpr int B = 1;                                 // MXFP4 slots a unit
  constexpr int KC = 2;                                // k-blocks of a slot a pass
  // weights only (static, or known since routing): the shared expert's first k-block
  // of this wave and its first batch of routed slots, loaded before `wait` (the mid
  // activations' dependency)
  uint4 shraw[DT][2];
  float shsc[DT];
  down_shared_first<DT>(p, t, KB2s, wave, lane, shraw, shsc);
  // the scaled-MFMA unit pipeline: E2M1 weights against MXFP8 (A8W4) or MXFP4 (A4W4) mid
  constexpr bool a4 = FMT == MK2_FMT_A4W4;
  down_residual_lds<DT>(p, t, xres, wave);
  // the routed slots (MXFP4): a unit is a batch of B slots (wave + NW * (B * i + u))
  // over KC k-blocks; units u + 1 and u + 2 (u + 1 alone for 24-row tasks: weights,
  // mid rows, scales and route weights) are in flight while unit u's MFMAs run
  struct Unit {
    i32x8 a[B][DT][KC];
    i32x8 bq[B][KC][NCG];
    int sa[B][DT];
    int sbq[B][KC][NCG];
    float wr[B][NCG];
    int rr[B][NCG];  // compacted rows: the column's row (-1: none)
    int cnt[B];      // compacted rows: the slot's rows
  };
  const int nkc = (KB2 + KC - 1) / KC;  // units a batch
  const int nu = D > wave ? (D - wave + NW * B - 1) / (NW * B) * nkc : 0;
  auto load_w = [&](int u, Unit& x) {  // weights: known since the routing
    const int j0 = wave + (u / nkc) * NW * B, kb0 = (u % nkc) * KC;
#pragma unroll
    for (int ub = 0; ub < B; ++ub) {
      // past the list: a valid slot, unused
      const int e = __builtin_amdgcn_readfirstlane(act_ids[min(j0 + ub * NW, D - 1)]);
      // the expert's E2M1 bytes as a buffer: a lane outside the task's rows reads
      // zeros past its end, with no branch around the load
      const uint32_t ebytes = (uint32_t)HT * KB2 * 1024;
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc((void*)(p.w2 + (size_t)e * ebytes), (short)0, (int)ebytes, 0x00020000);
#pragma unroll
      for (int c = 0; c < KC; ++c)
#pragma unroll
        for (int d = 0; d < DT; ++d)
          x.a[ub][d][c] = load_a_fp4_rs(
              rs, live[d] ? (uint32_t)(tl[d] * KB2 + min(kb0 + c, KB2 - 1)) * 1024u + lane * 16u : ebytes);
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const uint32_t w = e8m0_word(p.s2 + e * e8m0_expert_bytes(p.wl, p.H, p.I), p.wl, p.I, tl[d], kb0, lane);
        x.sa[ub][d] = live[d] ? (int)w : 127;
      }
    }
  };
  auto load_m = [&](int u, Unit& x) {  // mid rows and route weights: after the wait
    const int j0 = wave + (u / nkc) * NW * B, kb0 = (u % nkc) * KC;
#pragma unroll
    for (int ub = 0; ub < B; ++ub) {
      const int j = min(j0 + ub * NW, D - 1);
      // the mid's rows: the slot's rows compacted (row c its c-th)
      const int lim = act_ids[256 + j];
      x.cnt[ub] = lim;
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const int kb = min(kb0 + c, KB2 - 1);
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) {
          const int row = cg * 16 + c16;
          x.bq[ub][c][cg] = a4 ? load_b_fp4(p.mid_q + (size_t)j * p.M * (p.I / 2), row, lim, p.I / 2, kb * 64, g)
                               : load_b_fp8(p.mid_q + (size_t)j * p.M * p.I, row, lim, p.I, kb * 128, g);
          x.sbq[ub][c][cg] = row < lim ? (int)ldp_u8(p.mid_s + ((size_t)j * p.M + row) * (p.I / 32) + kb * 4 + g) : 127;
        }
      }
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        const int row = cg * 16 + c16;
        x.wr[ub][cg] = row < lim ? ldp_f32(p.rw + j * 32 + row) : 0.f;
        x.rr[ub][cg] = row < lim ? ldp_i32(p.rowc + j * 32 + row) : -1;
      }
    }
  };
  f32x4 acc[DT][NCG], tmp[B][DT][NCG];
#pragma unroll
  for (int d = 0; d < DT; ++d)
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) acc[d][cg] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int u, Unit& x) {
    const int j0 = wave + (u / nkc) * NW * B, kb0 = (u % nkc) * KC;
    if (kb0 == 0) {
#pragma unroll
      for (int ub = 0; ub < B; ++ub)
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
          for (int cg = 0; cg < NCG; ++cg) tmp[ub][d][cg] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int ub = 0; ub < B; ++ub) {
      if (j0 + ub * NW >= D) break;
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const int kb = kb0 + c;
        if (kb >= KB2) break;
#pragma unroll
        for (int d = 0; d < DT; ++d) {
          const int sak = x.sa[ub][d] >> e8m0_shift(p.wl, tl[d], kb);
#pragma unroll
          for (int cg = 0; cg < NCG; ++cg) {
            if (cg == 1 && x.cnt[ub] <= 16) break;  // no rows there (uniform)
            tmp[ub][d][cg] = a4 ? mfma_same<4>(x.a[ub][d][c], x.bq[ub][c][cg], tmp[ub][d][cg], sak, x.sbq[ub][c][cg])
                                : mfma_fp4_fp8<0, 0>(x.a[ub][d][c], x.bq[ub][c][cg], tmp[ub][d][cg], sak, x.sbq[ub][c][cg]);
          }
        }
      }
    }
    if (kb0 + KC >= KB2) {
#pragma unroll
      for (int ub = 0; ub < B; ++ub) {
        if (j0 + ub * NW >= D) break;
        // each column into its row of this wave's accumulators [DT][16 hidden][32 rows]
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg)
          if (x.rr[ub][cg] >= 0) {
#pragma unroll
            for (int d = 0; d < DT; ++d)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                red[((wave * DT + d) * 16 + 4 * g + i) * 32 + x.rr[ub][cg]] += tmp[ub][d][cg][i] * x.wr[ub][cg];
          }
      }
    }
  };
  // units in flight: 3, or 2 of two tiles each (24-row tasks), within the registers
  constexpr int DEPTH = DT == 2 ? 2 : 3;
  Unit x0, x1, x2;
  if (nu > 0) load_w(0, x0);
  if (DEPTH == 3 && nu > 1) load_w(1, x1);
  if (!wait()) return;
  if (nu > 0) load_m(0, x0);
  if (DEPTH == 3 && nu > 1) load_m(1, x1);
  // the shared expert (FP8, bf16 mid): its k-blocks spread over the waves
  for (int kb = wave; kb < KB2s; kb += NW) {
    bf16x8 b[NCG][4];
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) load_b_bf16(p.mid_sh, cg * 16 + c16, p.M, p.SI, kb * 128 + 32 * g, b[cg]);
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      uint4 r0, r1;
      float sc;
      if (kb == wave) {
        r0 = shraw[d][0];
        r1 = shraw[d][1];
        sc = shsc[d];
      } else {
        r0 = r1 = make_uint4(0, 0, 0, 0);
        if (live[d]) load_fp8_block(p.ws2 + ((size_t)tl[d] * KB2s + kb) * 2048, p.wl, lane, r0, r1);
        sc = p.ss2[(tl[d] * 16 / 128) * KB2s + kb];
      }
      bf16x8 a[4];
      a[0] = e4m3x8_to_bf16(r0.x, r0.y);
      a[1] = e4m3x8_to_bf16(r0.z, r0.w);
      a[2] = e4m3x8_to_bf16(r1.x, r1.y);
      a[3] = e4m3x8_to_bf16(r1.z, r1.w);
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) acc[d][cg] += mfma4_bf16(a, b[cg], f32x4{0.f, 0.f, 0.f, 0.f}) * sc;
    }
  }
  // this wave's accumulators [DT][16 hidden][32 rows] in LDS, from its shared-expert
  // sums; the routed slots add into their rows
#pragma unroll
  for (int d = 0; d < DT; ++d)
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[((wave * DT + d) * 16 + 4 * g + i) * 32 + cg * 16 + c16] = acc[d][cg][i];
  if constexpr (DEPTH == 2) {
    auto step = [&](int u, Unit& cur, Unit& nxt) {
      if (u + 1 < nu) {
        load_w(u + 1, nxt);
        load_m(u + 1, nxt);
      }
      if (u < nu) compute(u, cur);
    };
    for (int u = 0; u < nu; u += 2) {
      step(u, x0, x1);
      step(u + 1, x1, x0);
    }
  } else {
    auto step = [&](int u, Unit& cur, Unit& nxt2) {
      if (u + 2 < nu) {
        load_w(u + 2, nxt2);
        load_m(u + 2, nxt2);
      }
      if (u < nu) compute(u, cur);
    };
    for (int u = 0; u < nu; u += 3) {
      step(u, x0, x2);
      step(u + 1, x1, x0);
      step(u + 2, x2, x1);
    }
  }
  drain_memory();  // this wave's residual dwords have landed in LDS
  __syncthreads();
  const int n0 = t.rhi[0] - t.rlo[0];  // the first tile's columns
  for (int idx = threadIdx.x; idx < t.ncol * p.M; idx += NT) {
    const int n = idx % t.ncol, s = idx / t.ncol;  // column c0 + n of row s
    const int d = n < n0 ? 0 : DT - 1, n16 = n < n0 ? t.rlo[0] + n : t.rlo[DT - 1] + n - n0;
    float y = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) y += red[((w * DT + d) * 16 + n16) * 32 + s];
    const size_t o = (size_t)s * p.H + t.c0 + n;
    if (p.residual) y += bf16_to_f32(((const bf16_t*)xres)[idx]);
    p.out[o] = f32_to_bf16(y);
  }
  __syncthreads();
}

// down tasks of a launch: 16 * DT hidden rows each, or 24 with DT == 3
__host__ __device__ inline int down_tasks(const MoeDev& p) { return p.DT == 3 ? p.H / 24 : p.H / (16 * p.DT); }

// task nt of down_tasks(p).  Needs the routing (act, rw) on entry; `wait` is the
// mid activations' dependency, run once the task's static and routed weight loads
// are in flight.
template <int NT, int NCG, int FMT, typename Wait = NoWait>
MK2_DEV void moe_down(const MoeDev& p, int nt, float* red, int* act_ids, float* xres, Wait wait = Wait()) {
  if constexpr (kCompact<NCG, FMT>) {
    // 24 hidden rows a task where hidden is a multiple of 48 (one task a CU at 6144),
    // else 16
    if (p.DT == 3) down_rows_cmp<NT, NCG, 2, FMT>(p, nt, red, act_ids, xres, wait);
    else down_rows_cmp<NT, NCG, 1, FMT>(p, nt, red, act_ids, xres, wait);
  } else {
    if constexpr (FMT == MK2_FMT_MXFP4 || FMT == MK2_FMT_A4W4) {
      if (NCG == 1 && p.DT >= 2) {
        down_rows<NT, NCG, (NCG == 1 ? 2 : 1), FMT>(p, nt, red, act_ids, xres, wait);
        return;
      }
    }
    down_rows<NT, NCG, 1, FMT>(p, nt, red, act_ids, xres, wait);
  }
}

// runs f(std::integral_constant<int, FMT>) for the expert mode fmt (a kernel
// instantiation a mode, so that each carries only its own mode's code)
template <typename F>
inline int with_moe_fmt(int fmt, F&& f) {
  switch (fmt) {
    case MK2_FMT_FP8: return f(std::integral_constant<int, MK2_FMT_FP8>{});
    case MK2_FMT_MXFP4: return f(std::integral_constant<int, MK2_FMT_MXFP4>{});
    case MK2_FMT_W8A8: return f(std::integral_constant<int, MK2_FMT_W8A8>{});
    case MK2_FMT_A16W4: return f(std::integral_constant<int, MK2_FMT_A16W4>{});
    default: return f(std::integral_constant<int, MK2_FMT_A4W4>{});
  }
}

}  // namespace mk2
