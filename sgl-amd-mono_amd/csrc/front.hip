// The layer's front (the reference's K1): from the residual rows h to what the K2 layer
// takes -- the absorbed MLA queries, the index queries and head weights -- and this
// step's rows of the latent-KV and index caches.  Reference: glm53/gfx950/kernel.py:
// 2585-3575 (the front stages of its fused launch); the arithmetic is SGLang's
// DeepSeek-V3.2 / GLM-5 attention front (DeepseekV2AttentionMLA with the DSA indexer),
// which the reference's check runs as its truth (glm53/check.py:200-272):
//
//   x_n  = bf16(rmsnorm(h) * g_in)
//   [q_a | kv_a | k_pe] = W_qkv_a x_n,  ik = W_ik x_n,  iw = W_iw x_n        (f32)
//   q_an = bf16(rmsnorm(q_a) * g_q_a)
//   latent cache row = e4m3(bf16(rmsnorm(kv_a) * g_kv_a)) | e4m3(bf16(rope(k_pe)))
//   index cache row  = quant(fwht(rope64(layernorm(ik) * g_ik + b_ik)))
//   q_b  = W_q_b q_an: per head q_nope | q_pe;  iq = W_iq q_an                 (f32)
//   mla_q[h]   = bf16(W_UK[h] . bf16(q_nope[h])) | bf16(rope(q_pe[h]))
//   index_q[h] = bf16(fwht(rope64(bf16(iq[h])))),  index_w = bf16(iw)
//
// rope: interleaved pairs (2i, 2i + 1) rotated by the position's angle i (cos/sin from
// SGLang's cos_sin_cache [positions][rope]: cos in the first half, sin in the second;
// kernel.py:3107-3131,3245-3251); rope64: the same on the first 64 dims; fwht: the
// orthonormal 128-point Hadamard transform in Sylvester order (kernel.py:778-788);
// the index key's quant is its cache's (the FP8 pages' ue8m0 rule, kernel.py:
// 3134-3147, or the FP4 plane's MXFP4).
//
// Launches in stream order:
//   0. k_front_norm, one workgroup a row: x_n;
//   1. k_gemv over [W_qkv_a | W_ik], then over W_iw (bf16): the hidden-input GEMVs;
//   2. k_front_rows, three workgroups a row: the q_a norm; the latent cache row (kv_a
//      norm, RoPE); the index key and the head weights;
//   3. k_gemv over [W_q_b | W_iq] from q_an;
//   4. k_front_heads: W_UK absorption on MFMA and the index queries' RoPE + Hadamard.
// The GEMV engine is HBM-bound: each workgroup takes one K part (several when the
// tiles are fewer than the CUs; their f32 partial planes are summed in part order by
// the next stage) and a contiguous range of 16-row tiles, and each wave a k slice; the
// input rows are register-resident MFMA operands;
// FP8 weights (SGLang's row-major E4M3 with 128 x 128 f32 block scales, read in place)
// widen exactly to bf16 and each 128-k block's partial sum takes its block scale.
#include "front_stages.h"
#include "mk2_host.h"

namespace mk2 {

template <int KU, int WF>
__global__ __launch_bounds__(GV_NT) void k_gemv(GemvDev p) {
  __shared__ GemvLds S;
  gemv_run<KU, WF>(p, blockIdx.x, gridDim.x, S);
}

template <int KU, int WF>
static void gemv_launch1(const GemvDev& d, int grid, hipStream_t st) {
  k_gemv<KU, WF><<<grid, GV_NT, 0, st>>>(d);
}

// the engine's k-step counts: KU = K / (512 ks)
static bool gemv_ku_ok(int ku, bool f8) {
  return (!f8 && ku == 1) || ku == 2 || ku == 4 || ku == 6 || ku == 8 || ku == 12 || ku == 14 || ku == 16;
}

// K parts for `tiles` tiles on `cus` CUs: the fewest that give every CU a tile, among
// those the engine instantiates
static int gemv_parts(int K, int tiles, int cus, bool f8) {
  int best = 1;
  for (int ks = 1; ks <= 16; ++ks) {
    if (K % (512 * ks) || !gemv_ku_ok(K / (512 * ks), f8)) continue;
    best = ks;
    if (tiles * ks >= cus) break;
  }
  return best;
}

template <int WF>
static int gemv_launch(const GemvDev& d, int cus, hipStream_t st) {
  const int per = d.ntiles < cus / d.ks ? d.ntiles : cus / d.ks;  // workgroups a K part
  const int grid = d.ks * (per > 0 ? per : 1);
  switch (d.K / (512 * d.ks)) {
    case 1:
      if constexpr (WF != MK2_WFMT_BF16) return set_error(MK2_EINVAL, "front: FP8 K parts must hold whole 128-k blocks");
      else gemv_launch1<1, WF>(d, grid, st);
      break;
    case 2: gemv_launch1<2, WF>(d, grid, st); break;
    case 4: gemv_launch1<4, WF>(d, grid, st); break;
    case 6: gemv_launch1<6, WF>(d, grid, st); break;
    case 8: gemv_launch1<8, WF>(d, grid, st); break;
    case 12: gemv_launch1<12, WF>(d, grid, st); break;
    case 14: gemv_launch1<14, WF>(d, grid, st); break;
    case 16: gemv_launch1<16, WF>(d, grid, st); break;
    default: return set_error(MK2_EINVAL, "front: no GEMV engine for K = %d in %d parts", d.K, d.ks);
  }
  return MK2_OK;
}

__global__ __launch_bounds__(FR_NT) void k_front_norm(const bf16_t* x, const bf16_t* gw, bf16_t* xn, int K, float eps) {
  __shared__ float sh[FR_NT / 64];
  front_norm_row(x, gw, xn, K, eps, blockIdx.x, sh);
}

__global__ __launch_bounds__(FR_NT) void k_front_rows(FrontDev p) {
  __shared__ float sh[FR_NT / 64];
  __shared__ float kvv[576];
  front_rows_task(p, blockIdx.x, sh, kvv);
}

template <int NS>
__global__ __launch_bounds__(FR_NT) void k_front_heads(FrontDev p) {
  __shared__ uint4 qn[32 * NS * 4];
  front_heads_task<NS>(p, blockIdx.x, qn);
}


template <int KUA, int KUC, int WF, int NS>
__global__ __launch_bounds__(FR_NT, 1) void k_front_persistent(FrontPDev p) {
  __shared__ FrontLds S;
  __shared__ int seen[FP_SEEN];
  __shared__ int last;
  const int G = gridDim.x;
  if (threadIdx.x < FP_SEEN) seen[threadIdx.x] = 0;
  __syncthreads();
  front_walk<KUA, KUC, WF, NS>(p, S, seen);
  // the last workgroup out resets the counters for the next launch
  drain_memory();
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(fp_ctr(p, FP_DONE), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1;
  __syncthreads();
  if (last) front_reset(p);
}

static int front_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0 && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus[dev] = 0;
  return cus[dev];
}

// the K parts of the three GEMV launches, planned for MI355X's 256 CUs (so that the
// workspace and the bits do not depend on the device)
constexpr int FRONT_PLAN_CUS = 256;
struct FrontPlan {
  int ksA, ksW, ksC;
};
static FrontPlan front_plan(const mk2_front_shape* s) {
  const bool f8 = s->weight_fmt != MK2_WFMT_BF16;
  const int NA = s->q_lora + s->kv_lora + s->rope, QB = s->heads * (s->nope + s->rope);
  const int tA = NA / 16 + (s->index_heads > 0 ? 128 / 16 : 0);
  const int tC = QB / 16 + s->index_heads * 128 / 16;
  FrontPlan pl;
  pl.ksA = gemv_parts(s->hidden, tA, FRONT_PLAN_CUS, f8);
  pl.ksW = s->index_heads > 0 ? gemv_parts(s->hidden, s->index_heads / 16, FRONT_PLAN_CUS, false) : 1;
  pl.ksC = gemv_parts(s->q_lora, tC, FRONT_PLAN_CUS, f8);
  return pl;
}

// workspace: the persistent launch's counters, the GEMV outputs' partial planes, the
// normed q_a rows and the normed input rows
struct FrontWs {
  int* sync;
  float *qkv_a, *ik, *iw, *q_b, *iq;
  bf16_t *q_an, *x_n;
};
static size_t front_carve(const mk2_front_shape* s, void* base, FrontWs* w) {
  Carver c(base);
  int* sync = c.take<int>(FP_LINES * FP_LINE);
  const FrontPlan pl = front_plan(s);
  const size_t M = s->rows, ih = s->index_heads > 0 ? s->index_heads : 1;
  float* qkv_a = c.take<float>(pl.ksA * M * (s->q_lora + s->kv_lora + s->rope));
  float* ik = c.take<float>(pl.ksA * M * 128);
  float* iw = c.take<float>(pl.ksW * M * ih);
  float* q_b = c.take<float>(pl.ksC * M * s->heads * (s->nope + s->rope));
  float* iq = c.take<float>(pl.ksC * M * ih * 128);
  bf16_t* q_an = c.take<bf16_t>(M * s->q_lora);
  bf16_t* x_n = c.take<bf16_t>(M * s->hidden);
  if (w) *w = FrontWs{sync, qkv_a, ik, iw, q_b, iq, q_an, x_n};
  return c.bytes();
}

static int front_check_shape(const mk2_front_shape* s) {
  MK2_REQUIRE(s != nullptr, "front: shape is NULL");
  MK2_REQUIRE(s->rows >= 1 && s->rows <= 32, "front: rows must be in [1, 32], got %d", s->rows);
  auto engine_k = [](int k) { return k == 1024 || k == 2048 || k == 3072 || k == 4096 || k == 6144 || k == 7168 || k == 8192; };
  MK2_REQUIRE(engine_k(s->hidden), "front: hidden must be 1024, 2048, 3072, 4096, 6144, 7168 or 8192, got %d",
              s->hidden);
  MK2_REQUIRE(engine_k(s->q_lora), "front: q_lora must be 1024, 2048, 3072, 4096, 6144, 7168 or 8192, got %d",
              s->q_lora);
  MK2_REQUIRE(s->kv_lora == 512 && s->rope == 64, "front: kv_lora must be 512 and rope 64");
  MK2_REQUIRE(s->nope == 128 || s->nope == 192 || s->nope == 256, "front: nope must be 128, 192 or 256, got %d",
              s->nope);
  MK2_REQUIRE(s->heads >= 1 && s->heads <= 128, "front: heads must be in [1, 128], got %d", s->heads);
  MK2_REQUIRE(s->index_heads == 0 || (s->index_heads % 16 == 0 && s->index_heads <= 64),
              "front: index_heads must be 0 or a multiple of 16 up to 64, got %d", s->index_heads);
  MK2_REQUIRE(s->weight_fmt == MK2_WFMT_BF16 || s->weight_fmt == MK2_WFMT_FP8_BLOCK ||
                  s->weight_fmt == MK2_WFMT_FP8_AITER16,
              "front: weight_fmt must be MK2_WFMT_BF16, MK2_WFMT_FP8_BLOCK or MK2_WFMT_FP8_AITER16, got %d",
              s->weight_fmt);
  MK2_REQUIRE(s->key_fmt == MK2_KEYS_FP4 || s->key_fmt == MK2_KEYS_FP8, "front: key_fmt must be MK2_KEYS_*");
  MK2_REQUIRE(s->max_position >= 0, "front: max_position must be >= 0");
  MK2_REQUIRE(s->eps > 0.f && s->index_eps > 0.f, "front: eps and index_eps must be positive");
  return MK2_OK;
}

}  // namespace mk2

using namespace mk2;

extern "C" int mk2_front_workspace_bytes(const mk2_front_shape* shape, size_t* bytes) {
  clear_error();
  int rc = front_check_shape(shape);
  if (rc) return rc;
  MK2_REQUIRE(bytes != nullptr, "front: bytes is NULL");
  *bytes = front_carve(shape, nullptr, nullptr);
  return MK2_OK;
}

namespace mk2 {

// the persistent front's instantiations: (KUA, KUC, NS) of the hidden- and q_an-input
// GEMVs' K steps and nope / 32, for each weight format; X(WF, KUA, KUC, NS)
#define MK2_FRONT_PERSISTENT_SHAPES(X, WF) X(WF, 6, 4, 6) X(WF, 6, 4, 4) X(WF, 2, 2, 4) X(WF, 2, 2, 6)

// the K steps of the three GEMVs and nope / 32 of a valid shape
struct FrontSteps {
  int kua, kuw, kuc, ns;
};
static FrontSteps front_steps(const mk2_front_shape* s) {
  const FrontPlan pl = front_plan(s);
  return FrontSteps{s->hidden / (512 * pl.ksA), s->hidden / (512 * pl.ksW), s->q_lora / (512 * pl.ksC), s->nope / 32};
}
static bool front_persistent_ok(const mk2_front_shape* s) {
  const FrontSteps k = front_steps(s);
  if (s->index_heads > 0 && k.kuw != 1) return false;
#define MK2_FP_MATCH(WF, A, C, N) || (k.kua == A && k.kuc == C && k.ns == N)
  return false MK2_FRONT_PERSISTENT_SHAPES(MK2_FP_MATCH, 0);
#undef MK2_FP_MATCH
}

template <int KUA, int KUC, int WF, int NS>
static int front_persistent_launch(const FrontPDev& d, int cus, hipStream_t st) {
  static int fits = -1;  // one workgroup a CU
  if (fits < 0) {
    int per_cu = 0;
    fits = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_front_persistent<KUA, KUC, WF, NS>, FR_NT, 0) ==
                   hipSuccess &&
           per_cu >= 1;
  }
  if (!fits) return set_error(MK2_ELAUNCH, "front: the persistent kernel does not fit one workgroup per CU");
  k_front_persistent<KUA, KUC, WF, NS><<<cus, FR_NT, 0, st>>>(d);
  return check_launch("front (persistent)");
}

static int front_persistent_dispatch(const FrontPDev& d, int wf, const FrontSteps& k, int cus, hipStream_t st) {
#define MK2_FP_CASE(WF, A, C, N) \
  if (wf == WF && k.kua == A && k.kuc == C && k.ns == N) return front_persistent_launch<A, C, WF, N>(d, cus, st);
  MK2_FRONT_PERSISTENT_SHAPES(MK2_FP_CASE, MK2_WFMT_BF16)
  MK2_FRONT_PERSISTENT_SHAPES(MK2_FP_CASE, MK2_WFMT_FP8_BLOCK)
  MK2_FRONT_PERSISTENT_SHAPES(MK2_FP_CASE, MK2_WFMT_FP8_AITER16)
#undef MK2_FP_CASE
  return set_error(MK2_EINVAL, "front: no persistent front for these K steps");
}

// the grid of one GEMV pass as its stage launch runs it
static int gemv_grid(const GemvDev& d, int cus) {
  const int per = d.ntiles < cus / d.ks ? d.ntiles : cus / d.ks;
  return d.ks * (per > 0 ? per : 1);
}

// a front launch's validated arguments, workspace and stage descriptions
struct FrontPrep {
  FrontWs ws;
  FrontPlan pl;
  int cus, passes, heads_grid;
  GemvDev gA[2], gW[2], gC[2];
  FrontDev f;
};

static int front_prepare(const mk2_front_args* a, FrontPrep* P) {
  MK2_REQUIRE(a != nullptr, "front: args is NULL");
  int rc = front_check_shape(&a->shape);
  if (rc) return rc;
  const mk2_front_shape& s = a->shape;
  const mk2_front_weights& w = a->weights;
  const bool f8 = s.weight_fmt != MK2_WFMT_BF16;
  const bool idx = s.index_heads > 0;
  MK2_REQUIRE(a->x && a->positions && a->slots && a->rope_cos_sin && a->kv_cache && a->mla_q,
              "front: x, positions, slots, rope_cos_sin, kv_cache and mla_q must be set");
  MK2_REQUIRE(w.g_in && w.w_qkv_a && w.g_q_a && w.g_kv_a && w.w_q_b && w.w_uk,
              "front: g_in, w_qkv_a, g_q_a, g_kv_a, w_q_b and w_uk must be set");
  MK2_REQUIRE(!f8 || (w.s_qkv_a && w.s_q_b), "front: FP8 weights need s_qkv_a and s_q_b");
  MK2_REQUIRE(!(s.kv_scaled) || a->kv_scale, "front: a scaled latent cache needs kv_scale");
  if (idx) {
    MK2_REQUIRE(w.w_iq && w.w_ik && w.g_ik && w.b_ik && w.w_iw && a->index_cache && a->index_q && a->index_w,
                "front: the indexer needs w_iq, w_ik, g_ik, b_ik, w_iw, index_cache, index_q and index_w");
    MK2_REQUIRE(!f8 || (w.s_iq && w.s_ik), "front: FP8 weights need s_iq and s_ik");
    MK2_REQUIRE(s.key_fmt == MK2_KEYS_FP8 || a->index_scale, "front: the FP4 index plane needs index_scale");
  }
  const size_t need = front_carve(&s, nullptr, nullptr);
  MK2_REQUIRE(a->workspace != nullptr, "front: workspace is NULL");
  if (a->workspace_bytes < need)
    return set_error(MK2_ENOSPACE, "front: workspace has %zu bytes, needs %zu", a->workspace_bytes, need);
  P->cus = front_cus();
  if (P->cus <= 0) return set_error(MK2_ELAUNCH, "front: cannot query the CU count");
  FrontWs& ws = P->ws;
  front_carve(&s, a->workspace, &ws);
  const FrontPlan pl = P->pl = front_plan(&s);
  const int M = s.rows, NA = s.q_lora + s.kv_lora + s.rope, QB = s.heads * (s.nope + s.rope), IH = s.index_heads;
  auto seg = [](const void* w, const float* sc, float* out, int rows, int ld, long long pstride) {
    return GemvSeg{w, sc, out, rows, ld, pstride};
  };
  // the GEMV passes of 16 rows: hidden-input [W_qkv_a | W_ik] and W_iw, q_an-input
  // [W_q_b | W_iq]
  const int passes = P->passes = (M + 15) / 16;
  for (int pi = 0; pi < 2; ++pi) P->gA[pi] = P->gW[pi] = P->gC[pi] = GemvDev{};
  for (int pi = 0; pi < passes; ++pi) {
    const int r0 = 16 * pi;
    GemvDev& d = P->gA[pi];
    d.M = M - r0 < 16 ? M - r0 : 16; d.K = s.hidden; d.ks = pl.ksA; d.eps = s.eps;
    d.x = ws.x_n + (size_t)r0 * s.hidden; d.g = nullptr;
    d.seg[0] = seg(w.w_qkv_a, w.s_qkv_a, ws.qkv_a + (size_t)r0 * NA, NA, NA, (long long)M * NA);
    d.tiles0 = NA / 16; d.ntiles = d.tiles0;
    if (idx) {
      d.seg[1] = seg(w.w_ik, w.s_ik, ws.ik + (size_t)r0 * 128, 128, 128, (long long)M * 128);
      d.ntiles += 128 / 16;
      GemvDev& e = P->gW[pi];  // the head weights are bf16 in every checkpoint format
      e = d;
      e.ks = pl.ksW;
      e.seg[0] = seg(w.w_iw, nullptr, ws.iw + (size_t)r0 * IH, IH, IH, (long long)M * IH);
      e.tiles0 = IH / 16; e.ntiles = e.tiles0;
    }
    GemvDev& c = P->gC[pi];
    c.M = d.M; c.K = s.q_lora; c.ks = pl.ksC; c.eps = s.eps;
    c.x = ws.q_an + (size_t)r0 * s.q_lora; c.g = nullptr;
    c.seg[0] = seg(w.w_q_b, w.s_q_b, ws.q_b + (size_t)r0 * QB, QB, QB, (long long)M * QB);
    c.tiles0 = QB / 16; c.ntiles = c.tiles0;
    if (idx) {
      c.seg[1] = seg(w.w_iq, w.s_iq, ws.iq + (size_t)r0 * IH * 128, IH * 128, IH * 128, (long long)M * IH * 128);
      c.ntiles += IH * 128 / 16;
    }
  }
  FrontDev& f = P->f;
  f = FrontDev{};
  f.M = M; f.q_lora = s.q_lora; f.kv_lora = s.kv_lora; f.rope = s.rope; f.nope = s.nope; f.heads = s.heads;
  f.ih = IH; f.max_position = s.max_position; f.key_fmt = s.key_fmt; f.kv_scaled = s.kv_scaled;
  f.eps = s.eps; f.index_eps = s.index_eps;
  f.positions = (const long long*)a->positions; f.slots = (const long long*)a->slots;
  f.rope_cs = a->rope_cos_sin;
  f.qkv_a = ws.qkv_a; f.ik = ws.ik; f.iw = ws.iw; f.q_b = ws.q_b; f.iq = ws.iq;
  f.ksA = pl.ksA; f.ksW = pl.ksW; f.ksC = pl.ksC;
  f.g_q_a = (const bf16_t*)w.g_q_a; f.g_kv_a = (const bf16_t*)w.g_kv_a; f.g_ik = w.g_ik; f.b_ik = w.b_ik;
  f.w_uk = (const bf16_t*)w.w_uk;
  f.q_an = ws.q_an; f.kv = (uint8_t*)a->kv_cache; f.kv_scale = a->kv_scale;
  f.icache = (uint8_t*)a->index_cache; f.iscale = (uint8_t*)a->index_scale;
  f.mla_q = (bf16_t*)a->mla_q; f.index_q = (bf16_t*)a->index_q; f.index_w = (bf16_t*)a->index_w;
  P->heads_grid = 4 * s.heads + (idx ? (M * IH + FR_NT / 64 - 1) / (FR_NT / 64) : 0);
  return MK2_OK;
}

// the persistent front's arguments
static FrontPDev front_pdev_of(const mk2_front_args* a, const FrontPrep& P) {
  const mk2_front_shape& s = a->shape;
  const bool idx = s.index_heads > 0;
  FrontPDev d{};
  d.f = P.f;
  for (int pi = 0; pi < 2; ++pi) { d.A[pi] = P.gA[pi]; d.W[pi] = P.gW[pi]; d.C[pi] = P.gC[pi]; }
  d.passes = P.passes;
  // one round of workgroups for a pass's hidden-input GEMVs: the W_iw workgroups
  // first, [W_qkv_a | W_ik] on the rest (a tile's bits do not depend on which
  // workgroup or how many take the tiles)
  d.gridW = idx ? gemv_grid(P.gW[0], P.cus) : 0;
  d.gridA = gemv_grid(P.gA[0], P.cus - d.gridW > P.gA[0].ks ? P.cus - d.gridW : P.cus);
  d.gridC = gemv_grid(P.gC[0], P.cus);
  d.nheads = P.heads_grid;
  d.x = (const bf16_t*)a->x; d.g_in = (const bf16_t*)a->weights.g_in; d.x_n = P.ws.x_n; d.hidden = s.hidden;
  d.eps = s.eps;
  d.sync = P.ws.sync;
  d.wait_ticks = DEFAULT_WAIT_TICKS;
  return d;
}

// the front-and-layer launch's instantiation of a (checked) front shape, FRONT_FUSED_*
static int front_fused_key(const mk2_front_shape* s) {
  const FrontSteps k = front_steps(s);
  const bool c7 = front_persistent_ok(s) && k.kua == 6 && k.kuc == 4 && k.ns == 6;
  return !c7                                     ? FRONT_FUSED_NONE
         : s->weight_fmt == MK2_WFMT_FP8_BLOCK   ? FRONT_FUSED_C7_FP8
         : s->weight_fmt == MK2_WFMT_FP8_AITER16 ? FRONT_FUSED_C7_AITER16
                                                 : FRONT_FUSED_NONE;
}

int front_pdev(const mk2_front_args* a, FrontPDev* d, int* key) {
  FrontPrep P;
  int rc = front_prepare(a, &P);
  if (rc) return rc;
  *d = front_pdev_of(a, P);
  *key = front_fused_key(&a->shape);
  return MK2_OK;
}

static int front_run(const mk2_front_args* a, hipStream_t st, bool persistent) {
  FrontPrep P;
  int rc = front_prepare(a, &P);
  if (rc) return rc;
  const mk2_front_shape& s = a->shape;
  const mk2_front_weights& w = a->weights;
  const bool f8 = s.weight_fmt != MK2_WFMT_BF16;
  const bool idx = s.index_heads > 0;
  const int cus = P.cus, M = s.rows;
  if (persistent && front_persistent_ok(&s))
    return front_persistent_dispatch(front_pdev_of(a, P), s.weight_fmt, front_steps(&s), cus, st);
  auto gemv_fmt = [&](const GemvDev& d) {
    return s.weight_fmt == MK2_WFMT_FP8_AITER16 ? gemv_launch<MK2_WFMT_FP8_AITER16>(d, cus, st)
           : f8                                 ? gemv_launch<MK2_WFMT_FP8_BLOCK>(d, cus, st)
                                                : gemv_launch<MK2_WFMT_BF16>(d, cus, st);
  };
  // 0. the normed input rows
  k_front_norm<<<M, FR_NT, 0, st>>>((const bf16_t*)a->x, (const bf16_t*)w.g_in, P.ws.x_n, s.hidden, s.eps);
  rc = check_launch("front (norm)");
  if (rc) return rc;
  // 1. the hidden-input GEMVs
  for (int pi = 0; pi < P.passes; ++pi) {
    rc = gemv_fmt(P.gA[pi]);
    if (rc) return rc;
    if (idx) {
      rc = gemv_launch<MK2_WFMT_BF16>(P.gW[pi], cus, st);
      if (rc) return rc;
    }
  }
  // 2. the per-row stage: three workgroups a row
  k_front_rows<<<(idx ? 3 : 2) * M, FR_NT, 0, st>>>(P.f);
  rc = check_launch("front (rows)");
  if (rc) return rc;
  // 3. the q_an-input GEMVs
  for (int pi = 0; pi < P.passes; ++pi) {
    rc = gemv_fmt(P.gC[pi]);
    if (rc) return rc;
  }
  // 4. the per-head stage
  switch (s.nope / 32) {
    case 4: k_front_heads<4><<<P.heads_grid, FR_NT, 0, st>>>(P.f); break;
    case 6: k_front_heads<6><<<P.heads_grid, FR_NT, 0, st>>>(P.f); break;
    default: k_front_heads<8><<<P.heads_grid, FR_NT, 0, st>>>(P.f); break;
  }
  return check_launch("front (heads)");
}

}  // namespace mk2

extern "C" int mk2_front_launch(const mk2_front_args* a, mk2_stream_t stream) {
  clear_error();
  return front_run(a, (hipStream_t)stream, true);
}

extern "C" int mk2_front_launch_staged(const mk2_front_args* a, mk2_stream_t stream) {
  clear_error();
  return front_run(a, (hipStream_t)stream, false);
}

extern "C" int mk2_front_is_persistent(const mk2_front_shape* shape) {
  clear_error();
  int rc = front_check_shape(shape);
  if (rc) return -rc;
  return front_persistent_ok(shape) ? 1 : 0;
}

extern "C" int mk2_layer_step_is_fused(const mk2_front_shape* shape, int expert_fmt) {
  clear_error();
  int rc = front_check_shape(shape);
  if (rc) return -rc;
  return front_fused_key(shape) != FRONT_FUSED_NONE && expert_fmt == MK2_FMT_MXFP4 ? 1 : 0;
}
