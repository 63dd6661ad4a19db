// The tail launch: the final RMSNorm of the last layer's rows and this GPU's rows of
// the LM head (reference: glm53/gfx950/kernel.py:2220-2350, a `tail` build; host side
// Glm53HeadOp.launch, runner.py:473-545):
//   normed[r]    = bf16(x[r] * rsqrt(mean(x[r]^2) + eps) * g_norm)
//   logits[r][v] = f32(bf16(normed[r] . w_head[v]))
// w_head is SGLang's LM head as loaded, bf16 [vocab_rows][hidden] row-major, read in
// place; the logits are rounded to bf16 as the reference gathers them.
//
// One 512-thread workgroup a CU takes a contiguous range of vocab rows (within one of
// every other's: the launch is HBM-bound, so work is rows) and walks it in 16-row
// tiles, the last one partial: its dead lanes load a live row's addresses, which the
// same instruction already fetches, and store nothing.
// Wave w owns the k slice [w * hidden / 8, (w + 1) * hidden / 8) of every tile: the
// normed rows' B operands for that slice (the rows as the MFMA's 16 columns) are built
// once and stay in registers, and the tile's W rows stream through a window of WIN
// 16-byte loads a lane, each refilled from the same tile or the next one as its MFMA
// consumes it.  The norm costs no extra pass over the rows: the x fragments a wave
// loads for its operands give its slice's sums of squares, which the eight waves
// combine through LDS; they and the norm weight are loaded ahead of the first window,
// so the norm runs while the first W bytes are in flight.  A lane (c16, g) loads 16 B
// of row c16 at k = 32 s + 8 g of its slice: a wave instruction reads 64 contiguous
// bytes of each of 16 rows, and two consecutive k-steps fill whole 128-byte lines.  The eight waves' 16 x 16 partial
// tiles are summed in wave order through LDS (double-buffered by tile parity).
// A call of more than 16 rows runs as two passes over the LM head.
#include "mk2_device.h"
#include "mk2_host.h"

namespace mk2 {

constexpr int TAIL_NT = 512;
constexpr int TAIL_WAVES = TAIL_NT / 64;
constexpr int TAIL_ROWS = 16;  // rows a pass (the MFMA's columns)
constexpr int TAIL_CHUNK = 8;  // tiles whose partials wait in LDS for one barrier

struct TailDev {
  int rows;        // rows of this pass, 1..16
  int hidden;
  int vocab_rows;
  float eps;
  const bf16_t* x;       // [rows][hidden] of this pass
  const bf16_t* g;       // [hidden]
  const bf16_t* w;       // [vocab_rows][hidden]
  float* logits;         // [rows][vocab_rows] of this pass
  bf16_t* normed;        // [rows][hidden] of this pass, or null
};

template <int KS>
__global__ __launch_bounds__(TAIL_NT) void k_tail(TailDev p) {
  constexpr int WIN = KS <= 24 ? KS : KS / 2;  // W loads in flight a lane
  static_assert(KS % WIN == 0, "a window divides the k-steps");
  __shared__ float part[TAIL_WAVES][TAIL_ROWS];  // the waves' sums of squares by row
  __shared__ uint4 gam[8192 / 8];                // g_norm
  __shared__ float red[TAIL_CHUNK][TAIL_WAVES][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, c16 = lane & 15, g = lane >> 4;
  const int H = p.hidden, G = gridDim.x, b = blockIdx.x, M = p.rows;
  // this workgroup's rows [r0, r1): at least one (G <= vocab_rows)
  const int r0 = (int)((long long)b * p.vocab_rows / G), r1 = (int)((long long)(b + 1) * p.vocab_rows / G);
  const int kw = wave * KS * 32 + 8 * g;  // this lane's first k of its wave's slice
  // 1. this lane's x fragments (row c16, its k-steps) and the norm weight, then the
  //    first tile's W window: the rows and the weight are in hand before the first W
  //    bytes arrive
  const bool live = c16 < M;
  const bf16_t* xr = p.x + (size_t)(live ? c16 : 0) * H + kw;
  uint4 xq[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) xq[s] = *(const uint4*)(xr + 32 * s);
  uint4 gq[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int i = threadIdx.x + u * TAIL_NT;
    gq[u] = i < H / 8 ? ((const uint4*)p.g)[i] : make_uint4(0, 0, 0, 0);
  }
  // the W row of this lane in the tile from row t (the range's last row past its end)
  auto w_row = [&](int t) { return p.w + (size_t)min(t + c16, r1 - 1) * H + kw; };
  const bf16_t* wrow = w_row(r0);
  uint4 wv[WIN];
#pragma unroll
  for (int s = 0; s < WIN; ++s) wv[s] = ld_stream16(wrow + 32 * s);
  // 2. sums of squares: the lane's k-steps, the four lanes of its row, then the eight
  //    waves' slices in wave order (every lane of row c16 gets the same rstd bits)
  // (packed dot products of the bf16 pairs with themselves: nothing is unpacked here
  // for the conversion below to keep alive across the barrier)
  float ss = 0.f;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const uint32_t u[4] = {xq[s].x, xq[s].y, xq[s].z, xq[s].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x2 v = __builtin_bit_cast(bf16x2, u[j]);
      ss = __builtin_amdgcn_fdot2_f32_bf16(v, v, ss, false);
    }
  }
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  if (g == 0) part[wave][c16] = ss;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int i = threadIdx.x + u * TAIL_NT;
    if (i < H / 8) gam[i] = gq[u];
  }
  __syncthreads();
  float tot = part[0][c16];
#pragma unroll
  for (int w = 1; w < TAIL_WAVES; ++w) tot += part[w][c16];
  const float rs = live ? 1.0f / sqrtf(tot / (float)H + p.eps) : 0.f;
  // 3. B operands in place: bf16(x * rstd * g) of row c16 (zero columns past the rows)
  bf16x8 bq[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const uint4 gv = gam[(kw + 32 * s) >> 3];
    const uint32_t xu[4] = {xq[s].x, xq[s].y, xq[s].z, xq[s].w}, gu[4] = {gv.x, gv.y, gv.z, gv.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = __uint_as_float(xu[j] << 16) * rs * __uint_as_float(gu[j] << 16);
      const float hi = __uint_as_float(xu[j] & 0xFFFF0000u) * rs * __uint_as_float(gu[j] & 0xFFFF0000u);
      o[j] = live ? pack_bf16x2(lo, hi) : 0u;
    }
    const uint4 ov = make_uint4(o[0], o[1], o[2], o[3]);
    bq[s] = __builtin_bit_cast(bf16x8, ov);
    if (b == 0 && live && p.normed) *(uint4*)(p.normed + (size_t)c16 * H + kw + 32 * s) = ov;
  }
  // 4. the tiles, in chunks of up to TAIL_CHUNK: each wave runs its chain for every
  //    tile of the chunk and leaves its partial tile in LDS with no barrier between
  //    tiles (a barrier a tile would hold every wave to the slowest one while no load
  //    can issue); the chunk's partials are then summed in wave order and stored
  for (int c0 = r0; c0 < r1; c0 += 16 * TAIL_CHUNK) {
#pragma unroll
    for (int i = 0; i < TAIL_CHUNK; ++i) {
      const int t = c0 + 16 * i;
      if (t >= r1) break;
      const bool more = t + 16 < r1;
      const bf16_t* nrow = w_row(t + 16);  // this lane's row of the next tile
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        acc = mfma_bf16(__builtin_bit_cast(bf16x8, wv[s % WIN]), bq[s], acc);
        const int u = s + WIN;
        if (u < KS)
          wv[s % WIN] = ld_stream16(wrow + 32 * u);
        else if (more)
          wv[s % WIN] = ld_stream16(nrow + 32 * (u - KS));
      }
      // lane (c16, g) holds D[v = 4 g + i][m = c16]
      float* rw = red[i][wave];
#pragma unroll
      for (int j = 0; j < 4; ++j) rw[(4 * g + j) * 16 + c16] = acc[j];
      wrow = nrow;
    }
    __syncthreads();
    const int nt = min(TAIL_CHUNK, (r1 - c0 + 15) / 16);
    for (int e = threadIdx.x; e < nt * 256; e += TAIL_NT) {
      const int i = e >> 8, m = (e >> 4) & 15, v = e & 15;
      const int row = c0 + 16 * i + v;
      float s = red[i][0][v * 16 + m];
#pragma unroll
      for (int w = 1; w < TAIL_WAVES; ++w) s += red[i][w][v * 16 + m];
      if (m < M && row < r1) p.logits[(size_t)m * p.vocab_rows + row] = bf16_to_f32(f32_to_bf16(s));
    }
    __syncthreads();
  }
}

template <int KS>
static void tail_enqueue(const TailDev& d, int grid, hipStream_t st) {
  k_tail<KS><<<grid, TAIL_NT, 0, st>>>(d);
}

static int tail_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0 && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus[dev] = 0;
  return cus[dev];
}

}  // namespace mk2

using namespace mk2;

extern "C" int mk2_tail_launch(const mk2_tail_args* a, mk2_stream_t stream) {
  clear_error();
  MK2_REQUIRE(a != nullptr, "tail: args is NULL");
  MK2_REQUIRE(a->rows >= 1 && a->rows <= 32, "tail: rows must be in [1, 32], got %d", a->rows);
  MK2_REQUIRE(a->hidden >= 2048 && a->hidden <= 8192 && a->hidden % 1024 == 0,
              "tail: hidden must be a multiple of 1024 in [2048, 8192], got %d", a->hidden);
  MK2_REQUIRE(a->vocab_rows >= 1, "tail: vocab_rows must be positive, got %d", a->vocab_rows);
  MK2_REQUIRE(a->eps > 0.f, "tail: eps must be positive");
  MK2_REQUIRE(a->x && a->g_norm && a->w_head && a->logits, "tail: x, g_norm, w_head and logits must be set");
  MK2_REQUIRE(a->normed != a->x, "tail: normed must not alias x");
  const int cus = tail_cus();
  if (cus <= 0) return set_error(MK2_ELAUNCH, "tail: cannot query the CU count");
  const int grid = a->vocab_rows < cus ? a->vocab_rows : cus;
  hipStream_t st = (hipStream_t)stream;
  for (int r0 = 0; r0 < a->rows; r0 += TAIL_ROWS) {
    TailDev d;
    d.rows = a->rows - r0 < TAIL_ROWS ? a->rows - r0 : TAIL_ROWS;
    d.hidden = a->hidden;
    d.vocab_rows = a->vocab_rows;
    d.eps = a->eps;
    d.x = (const bf16_t*)a->x + (size_t)r0 * a->hidden;
    d.g = (const bf16_t*)a->g_norm;
    d.w = (const bf16_t*)a->w_head;
    d.logits = a->logits + (size_t)r0 * a->vocab_rows;
    d.normed = a->normed ? (bf16_t*)a->normed + (size_t)r0 * a->hidden : nullptr;
    switch (a->hidden / 256) {
      case 8: tail_enqueue<8>(d, grid, st); break;
      case 12: tail_enqueue<12>(d, grid, st); break;
      case 16: tail_enqueue<16>(d, grid, st); break;
      case 20: tail_enqueue<20>(d, grid, st); break;
      case 24: tail_enqueue<24>(d, grid, st); break;
      case 28: tail_enqueue<28>(d, grid, st); break;
      default: tail_enqueue<32>(d, grid, st); break;
    }
    const int rc = check_launch("tail");
    if (rc) return rc;
  }
  return MK2_OK;
}
