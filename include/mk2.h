/* mk2.h -- C ABI of the MI355X (gfx950) K2 decode-layer kernels.
 *
 * One GPU's share of the sgl-amd-mono decoder-layer monokernel: the FP4 indexer
 * scores and exact top-k, sparse-MLA decode over the selected FP8 latent-KV rows,
 * W_UV and o_proj, RMSNorm, the router top-k and the FP8 / MXFP4 routed and shared
 * experts.  The TP all-reduces of the reference are omitted (one GPU).
 *
 * Every entry point takes plain device pointers and sizes, enqueues work on the
 * given HIP stream and returns 0, or a nonzero MK2_E* code with a message readable
 * through mk2_last_error() (thread-local).  Nothing here allocates device memory or
 * synchronizes the host: scratch is a caller-owned workspace whose size the
 * *_workspace_bytes queries report, so every launch can be captured in a HIP graph.
 * Buffers are caller-owned and must stay alive until the stream work completes.
 *
 * Reference interfaces replaced (paths in sgl-project/sgl-amd-mono):
 *   mk2_layer_launch          Glm53LayerOp.launch -> glm5_monokernel(...).launch
 *                             sgl_amd_mono/glm53/gfx950/runner.py:374-470,
 *                             sgl_amd_mono/glm53/gfx950/kernel.py:7155-7245
 *   mk2_moe_launch            the router/ug/down stages of that launch
 *                             kernel.py:5471-7152
 *   mk2_indexer_topk_launch   index_score + index_slice stages, kernel.py:3577-4883,
 *                             with the FP4 keys of deepseek_v4/gfx950/kernels/stages/
 *                             indexer.py:412-803
 *   mk2_sparse_mla_launch     split + uv + o stages, kernel.py:4885-5469
 *   *_workspace_bytes         the scratch layout of glm53/gfx950/layout.py:181-318
 *   mk2_last_error            the ValueError/RuntimeError text the reference's host
 *                             raises before a launch (runner.py:312-318,388-421)
 */
#ifndef MK2_H
#define MK2_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MK2_ABI_VERSION 4

/* the longest dependency-wait deadline a persistent launch takes (its waits compare
 * 32-bit differences of the 100 MHz clock) */
#define MK2_MAX_WAIT_US 40000000

/* return codes */
#define MK2_OK 0
#define MK2_EINVAL 1   /* a shape, pointer or size argument is invalid */
#define MK2_ELAUNCH 2  /* the HIP runtime refused a launch */
#define MK2_ENOSPACE 3 /* the workspace is smaller than *_workspace_bytes reports */

/* router kinds */
#define MK2_ROUTER_SOFTMAX 0      /* top-k of logits, softmax over the k picked */
#define MK2_ROUTER_SIGMOID_BIAS 1 /* top-k of sigmoid + bias, sigmoid / sum * scale */

/* expert modes: the routed experts' weight format and what their activations (the
 * normalized rows and the SwiGLU mid) are quantized to -- the reference's MoE modes
 * (glm53/gfx950/config.py:88-93) plus MXFP4 rows (kernel.py:1768-1777).  E4M3 weights
 * carry an f32 scale per 128 x 128 block; E2M1 weights an E8M0 per 32 (tile layouts
 * below).  The shared expert is always E4M3 weights on bf16 rows. */
#define MK2_FMT_FP8 0   /* W8A16: E4M3 weights, bf16 activations */
#define MK2_FMT_MXFP4 1 /* A8W4: E2M1 weights, activations MXFP8 (E8M0 = ceil-pow2 of amax/448) */
#define MK2_FMT_W8A8 2  /* E4M3 weights, activations E4M3 with an f32 scale per 128
                           (amax/448; q = clamp(x * 448/amax)) */
#define MK2_FMT_A16W4 3 /* E2M1 weights widened exactly to bf16, bf16 activations */
#define MK2_FMT_A4W4 4  /* E2M1 weights, activations MXFP4 (E8M0 = ceil-pow2 of amax/6, at
                           most 254: AITER's round-up rule; E2M1 round to nearest even) */

typedef void* mk2_stream_t; /* a hipStream_t */

/* ---------------------------------------------------------------------- MoE
 * Weight layouts (tile packing): every weight matrix [N, K] is
 * stored as tiles [N/16][K/128][64 lanes][chunk] where lane l holds row l%16 and
 * k = 32*(l/16) .. +31 of the 128-k block; chunk = 64 B (bf16), 32 B (E4M3),
 * 16 B (E2M1).  MXFP4 E8M0 scales: [N/16][ceil(K/512)][64 lanes][4 B].
 * gate and up are stacked as one [2*inter, hidden] matrix (gate first).
 *
 * The expert weights (routed and shared) may instead be in AITER's (16, 16) layout,
 * as SGLang leaves them for AITER's MoE (shuffle_weight(w, (16, 16)), e8m0_shuffle):
 * the weight bytes [N/16][K_bytes/32][2][16 rows][16 B] -- for E2M1 this is byte for
 * byte the tile layout above; for E4M3 a lane's 32 bytes are its row's two 16-byte
 * halves 256 bytes apart -- and the E8M0 scales of [N][K/32] (rows counted across the
 * experts) in e8m0_shuffle's order: byte (row, col) at
 * ((((row/32 * K/256 + col/8) * 4 + col%4) * 16 + row%16) * 2 + col/4%2) * 2 + row/16%2.
 * The E4M3 block scales are plain in both. */
#define MK2_WLAYOUT_TILES 0   /* the tile packing above */
#define MK2_WLAYOUT_AITER16 1 /* AITER's (16, 16) shuffle (the reference's fp8_shuffled
                                 mode, glm53/gfx950/kernel.py:1015-1050; E2M1 with
                                 e8m0_shuffle, runner.py:83-89) */
typedef struct mk2_moe_shape {
  int rows;         /* M: decode rows, 1..32 */
  int hidden;       /* H, multiple of 512 */
  int n_experts;    /* E, multiple of 64, <= 256 */
  int top_k;        /* 1..8 */
  int inter;        /* routed expert intermediate size */
  int router;       /* MK2_ROUTER_* */
  int expert_fmt;   /* MK2_FMT_*: the routed experts' mode */
  int n_shared;     /* 0 or 1 shared expert, always MK2_FMT_FP8 */
  int shared_inter; /* shared expert intermediate size */
  int norm;         /* 1: RMSNorm(x) * gamma feeds the router and experts */
  int residual;     /* 1: out = x + moe, else out = moe */
  float route_scale;
  float eps;
  int weight_layout; /* MK2_WLAYOUT_*: the routed and shared experts' weights; AITER16
                        needs inter and shared_inter multiples of 32, and with E2M1
                        weights inter a multiple of 256 */
} mk2_moe_shape;

typedef struct mk2_moe_weights {
  const void* gamma;       /* bf16 [H] (norm only) */
  const void* w_router;    /* bf16 tiles of [E, H] */
  const float* router_bias;/* f32 [E] (sigmoid_bias only) */
  const void* w13;         /* routed gate|up: [E] x tiles of [2*inter, H] */
  const void* s13;         /* E4M3 weights: f32 [E][2*inter/128][H/128]; E2M1: E8M0 tiles */
  const void* w2;          /* routed down: [E] x tiles of [H, inter] */
  const void* s2;          /* E4M3 weights: f32 [E][H/128][inter/128]; E2M1: E8M0 tiles */
  const void* ws13;        /* shared gate|up E4M3 tiles of [2*shared_inter, H] */
  const float* ss13;       /* f32 [2*shared_inter/128][H/128] */
  const void* ws2;         /* shared down E4M3 tiles of [H, shared_inter] */
  const float* ss2;        /* f32 [H/128][shared_inter/128] */
} mk2_moe_weights;

typedef struct mk2_moe_args {
  mk2_moe_shape shape;
  mk2_moe_weights w;
  const void* x;           /* bf16 [M][H] input rows (the residual when residual=1) */
  void* out;               /* bf16 [M][H]; must not alias x */
  void* workspace;
  size_t workspace_bytes;
  /* optional outputs for checking; NULL skips each */
  float* logits;           /* f32 [M][E] router logits */
  int32_t* topk_ids;       /* [M][top_k], rank order */
  float* topk_weights;     /* [M][top_k] */
} mk2_moe_args;

/* The block entry points below (mk2_moe_launch, mk2_indexer_topk_launch,
 * mk2_sparse_mla_launch) each run their block as ONE persistent launch (one workgroup
 * a CU, the stages handing off through counters, as the layer's launch does).  Their
 * workspace is zero-filled before its first launch, and every launch (completed or
 * stopped) leaves it ready for the next.  The int at byte MK2_BLOCK_STATUS_OFFSET of
 * the workspace becomes nonzero once a launch's dependency wait passed its deadline
 * (one second of the device clock; that launch's outputs are undefined); only the
 * caller clears it. */
#define MK2_BLOCK_STATUS_OFFSET 26624
int mk2_moe_workspace_bytes(const mk2_moe_shape* shape, size_t* bytes);
int mk2_moe_launch(const mk2_moe_args* args, mk2_stream_t stream);
/* Where a launch leaves the MoE block's activations in its workspace: byte offsets
 * from the workspace's start, -1 where the expert mode has no such buffer.  They are
 * what the device quantizers wrote -- the normalized rows and their codes and scales
 * (the reference's activation quant, kernel.py:1740-1777,5563-5614) and the SwiGLU
 * mid's (kernel.py:6955-6985,7032-7060) -- and stay there until the next launch on
 * the workspace.  The reference's checks read the same buffers through its scratch
 * layout (glm53/gfx950/layout.py:181-318).  Slot j is the j-th distinct routed
 * expert, ascending (act); with compact = 1 (rows > 16, A8W4 or A4W4) row c of slot
 * j's mid is the c-th of the rows that picked its expert, ascending. */
typedef struct mk2_moe_ws_layout {
  int64_t xn;      /* bf16 [rows][hidden]: bf16(x * rstd * gamma) (x itself without norm) */
  int64_t xq;      /* A8W4, W8A8: E4M3 [rows][hidden]; A4W4: E2M1 [rows][hidden/2] */
  int64_t xs;      /* A8W4, A4W4: E8M0 [rows][hidden/32] */
  int64_t xsf;     /* W8A8: f32 [rows][hidden/128] */
  int64_t act;     /* u64 [1 + dmax], low 32 bits: the count D, then the experts */
  int64_t mid_q;   /* A8W4, W8A8: E4M3 [dmax][rows][inter]; A4W4: E2M1 [dmax][rows][inter/2] */
  int64_t mid_s;   /* A8W4, A4W4: E8M0 [dmax][rows][inter/32] */
  int64_t mid_sf;  /* W8A8: f32 [dmax][rows][inter/128] */
  int64_t mid_b;   /* W8A16, A16W4: bf16 [dmax][rows][inter] */
  int64_t mid_sh;  /* bf16 [rows][shared_inter]: the shared expert's mid */
  int32_t dmax;    /* capacity of the slot list */
  int32_t compact; /* 1: compacted rows (see above) */
} mk2_moe_ws_layout;
int mk2_moe_workspace_layout(const mk2_moe_shape* shape, mk2_moe_ws_layout* layout);

/* ------------------------------------------------------------ indexer + top-k
 * Index cache, one of SGLang's two formats, read in place:
 *  MK2_KEYS_FP4: the FP4 index plane (reference: deepseek_v41/gfx950/indexer/
 *    score_fp4.py:9-12,45-49).  cache: E2M1 codes [pages][4 chunks of 32 dims][64
 *    tokens][16 B], 4096 B a page; cache_scale: E8M0 [pages][4 chunks][64], token t's
 *    scale at (t % 16) * 4 + t / 16.
 *  MK2_KEYS_FP8: the DSA index cache, uint8 [pages][64][132] (reference:
 *    glm53/gfx950/runner.py:28-31,412-421).  A page is 64 x 128 E4M3 values in tiles of
 *    16 tokens x 16 dims -- token t's dim d at byte (t / 16) * 2048 + (d / 16) * 256 +
 *    (t % 16) * 16 + d % 16 (kernel.py:698-705) -- then 64 f32 scales, token t's at
 *    byte 8192 + 4 t; a key is its values times its scale.  cache_scale is NULL.
 *  MK2_KEYS_FP4_Q4: the FP4 index plane as MK2_KEYS_FP4, scored against the queries
 *    quantized to MXFP4 in the kernel (E2M1 with an E8M0 per 32 dims by the rule of
 *    quantize_fp4_indexer_row, deepseek_v41/gfx950/attention/index_query.py:283-293)
 *    on the FP4 x FP4 scaled MFMA, as the reference's verify-width scorer
 *    (deepseek_v41/gfx950/indexer/score_fp4.py:254-296).  A contract of its own: the
 *    scores are those of the quantized queries.
 * Page table int32 [requests][table_stride], logical page -> physical page.  Row r
 * scores the context positions 0 .. ctx_len[r]-1 of request req_ids[r]. */
#define MK2_KEYS_FP4 0
#define MK2_KEYS_FP8 1
#define MK2_KEYS_FP4_Q4 2

typedef struct mk2_indexer_shape {
  int rows;        /* 1..32 */
  int heads;       /* index heads, multiple of 16, <= 64 */
  int dim;         /* 128 */
  int topk;        /* multiple of 64, 64..4096 */
  int max_ctx;     /* upper bound of ctx_len, <= 65536, multiple of 64 */
  int table_stride;/* page table row stride (entries) */
  int key_fmt;     /* MK2_KEYS_*: the index cache's format (and, FP4_Q4, the queries') */
} mk2_indexer_shape;

typedef struct mk2_indexer_args {
  mk2_indexer_shape shape;
  const void* q;            /* bf16 [rows][heads][128] */
  const void* w;            /* bf16 [rows][heads] head weights */
  const uint8_t* cache;     /* FP4: E2M1 plane [pages][4][64][16]; FP8: [pages][64][132] */
  const uint8_t* cache_scale;/* FP4: E8M0 plane [pages][4][64]; FP8: NULL */
  const int32_t* page_table;/* [requests][table_stride] */
  const int32_t* req_ids;   /* [rows] */
  const int32_t* ctx_len;   /* [rows] */
  float* scores;            /* f32 [rows][max_ctx] (written for 0..ctx_len-1) or NULL */
  int32_t* topk;            /* [rows][topk] positions, -1 padded, or NULL */
  void* workspace;          /* required: key histograms and top-k candidates (and the
                               scores / lists when those are NULL) */
  size_t workspace_bytes;
} mk2_indexer_args;

int mk2_indexer_workspace_bytes(const mk2_indexer_shape* shape, size_t* bytes);
int mk2_indexer_topk_launch(const mk2_indexer_args* args, mk2_stream_t stream);

/* --------------------------------------------------------------- sparse MLA
 * Latent KV pages: [pages][64 tokens][576 B E4M3] with one f32 scale per token
 * in kv_scale [pages][64], or kv_scale NULL for SGLang's unscaled MLA cache
 * [slots][576] e4m3 (reference: glm53/spec.py:542-547), read as scale 1.  Row r attends the positions sel[r][0..topk-1] (-1 =
 * unused) of request req_ids[r]; then W_UV (bf16 [heads][v_dim][512]) and W_o
 * (bf16 tiles of [hidden, heads*v_dim]); out = bf16(h + o W_o^T) (h may be NULL). */
typedef struct mk2_mla_shape {
  int rows;        /* 1..32 */
  int heads;       /* 16 */
  int kv_lora;     /* 512 */
  int rope;        /* 64 */
  int v_dim;       /* multiple of 16 */
  int hidden;      /* multiple of 16 */
  int topk;        /* selected positions a row, multiple of 64 */
  int table_stride;
  float sm_scale;
} mk2_mla_shape;

typedef struct mk2_mla_args {
  mk2_mla_shape shape;
  const void* q;            /* bf16 [rows][heads][576] (W_UK absorbed) */
  const uint8_t* kv;        /* latent KV pages */
  const float* kv_scale;    /* [pages][64], or NULL (scale 1) */
  const int32_t* page_table;
  const int32_t* req_ids;   /* [rows] */
  const int32_t* sel;       /* [rows][topk] positions */
  const void* w_uv;         /* bf16 [heads][v_dim][512] */
  const void* w_o;          /* bf16 tiles of [hidden, heads*v_dim] */
  const void* h;            /* bf16 [rows][hidden] residual or NULL */
  void* out;                /* bf16 [rows][hidden] */
  void* workspace;
  size_t workspace_bytes;
  float* o_latent;          /* optional f32 [rows][heads][512] merged latent output */
} mk2_mla_args;

int mk2_mla_workspace_bytes(const mk2_mla_shape* shape, size_t* bytes);
int mk2_sparse_mla_launch(const mk2_mla_args* args, mk2_stream_t stream);

/* ------------------------------------------------------------ the K2 layer
 * indexer -> top-k -> sparse MLA -> o_proj + residual h -> RMSNorm(eps) -> MoE +
 * residual.  The three argument blocks are the ones above; their q/sel/out fields
 * that the chain produces itself are ignored.  out: bf16 [rows][hidden]. */
#define MK2_LAYER_PERSISTENT 0 /* one persistent launch (default) */
#define MK2_LAYER_STAGED 1     /* the same stages as one kernel each, stream-ordered */

typedef struct mk2_layer_args {
  mk2_indexer_args indexer; /* scores/topk may be NULL (then kept in the workspace) */
  mk2_mla_args mla;         /* sel, out are ignored: the chain supplies them */
  mk2_moe_args moe;         /* x is ignored (the attention output); norm=1, residual=1 */
  void* attn_out;           /* optional bf16 [rows][hidden]: the residual after attention */
  void* out;
  void* workspace;          /* zero-filled before its first launch; every launch
                               (completed or stopped) leaves it ready for the next */
  size_t workspace_bytes;
  int mode;                 /* MK2_LAYER_PERSISTENT or MK2_LAYER_STAGED */
  int wait_us;              /* persistent: a dependency wait's deadline in microseconds
                               of the device's 100 MHz clock, from the wait's first
                               unmet poll (0: one second; at most MK2_MAX_WAIT_US) */
  int32_t* status;          /* optional device word, sticky: a persistent launch whose
                               wait gave up stops early (its out is not valid) and ORs 1
                               into it; a completed launch leaves it as it is.  A stopped
                               launch still leaves the workspace ready for the next. */
  uint64_t* timeline;       /* optional [grid][33] stage stamps of the persistent launch
                               (100 MHz device clock): per stage enter, input ready, leave;
                               then the routing's logits polled, top-k done, list out */
} mk2_layer_args;

int mk2_layer_workspace_bytes(const mk2_layer_args* args, size_t* bytes);
int mk2_layer_launch(const mk2_layer_args* args, mk2_stream_t stream);
/* The MoE block's part of a layer workspace: its buffers lie at *moe_offset plus the
 * offsets mk2_moe_workspace_layout(&args->moe.shape) reports (the reference's scratch
 * layout, glm53/gfx950/layout.py:181-318). */
int mk2_layer_workspace_layout(const mk2_layer_args* args, int64_t* moe_offset);

/* The same layer launch without a caller workspace: no counterpart in the reference.
 * It is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  args->workspace and
 * workspace_bytes are ignored; the scratch is a device array of
 * MK2_LAYER_STATIC_SCRATCH_BYTES inside the library, which each GPU the library runs
 * on holds until the process ends.  A shape whose mk2_layer_workspace_bytes exceeds it
 * fails with MK2_ENOSPACE (the configs[4] layer needs about 1.9 MiB a row at context
 * 65536: 60.4 MiB at 32 rows).  Nothing is allocated: each call enqueues a small fill
 * kernel that clears the counters and histograms a launch needs zero and every region
 * of tagged hand-off words (the array keeps the last call's other contents, and calls
 * of different shapes lay their regions over each other's), then the launch.  Every
 * call on one GPU shares that GPU's array, so calls that overlap on one GPU (other
 * streams, other host threads) race; calls ordered on one stream do not. */
#define MK2_LAYER_STATIC_SCRATCH_BYTES ((size_t)64 << 20)
int mk2_layer_launch_static(const mk2_layer_args* args, mk2_stream_t stream);

/* ----------------------------------------------------------------- front
 * The layer's front, the reference's K1 (glm53/gfx950/kernel.py:2585-3575): from the
 * residual rows h to what mk2_layer_launch takes -- the absorbed MLA queries, the
 * index queries and head weights -- and this step's latent-KV and index cache rows:
 *   x_n  = bf16(rmsnorm(h) * g_in)
 *   [q_a | kv_a | k_pe] = W_qkv_a x_n,  ik = W_ik x_n,  iw = W_iw x_n        (f32)
 *   q_an = bf16(rmsnorm(q_a) * g_q_a)
 *   latent row = e4m3(bf16(rmsnorm(kv_a) * g_kv_a) | bf16(rope(k_pe))) (/ its scale)
 *   index row  = quant(fwht(rope64(layernorm(ik) * g_ik + b_ik)))
 *   mla_q[h]   = bf16(W_UK[h] . bf16(q_nope[h])) | bf16(rope(q_pe[h])), q_b = W_q_b q_an
 *   index_q[h] = bf16(fwht(rope64(bf16(W_iq q_an)[h]))),  index_w = bf16(iw)
 * rope: interleaved pairs (2i, 2i+1) by rope_cos_sin[position] (SGLang's cos_sin_cache
 * f32 [positions][rope], cos | sin); fwht: the orthonormal 128-point Hadamard
 * transform (Sylvester order); quant: the index cache's (MK2_KEYS_FP8: ue8m0 +
 * E4M3, MK2_KEYS_FP4: MXFP4).  Weights are SGLang's as loaded, read in place: bf16
 * or E4M3 row-major, or E4M3 in AITER's (16, 16) layout, with f32 128 x 128 block
 * scales [ceil(rows/128)][K/128] (W_iw is bf16 in all).  W_UK is SGLang's w_kc, bf16
 * [heads][kv_lora][nope] in memory.  A row with slot < 0 (a pad row) writes no cache
 * rows.  mk2_front_launch runs ONE persistent launch (one workgroup a CU, the stages
 * handing off through counters in the workspace) for the shapes whose GEMV steps it
 * instantiates (mk2_front_is_persistent), else the six stage launches in stream
 * order, which mk2_front_launch_staged always runs; both give the same bits.  The
 * workspace is zero-filled before its first launch and holds the launch's counters,
 * the normed rows and the f32 GEMV outputs; the int at byte MK2_FRONT_STATUS_OFFSET
 * of it becomes nonzero once a persistent launch's dependency wait passed its
 * deadline (that launch's outputs are undefined) and only the caller clears it. */
#define MK2_FRONT_STATUS_OFFSET 6528
#define MK2_WFMT_BF16 0
#define MK2_WFMT_FP8_BLOCK 1
#define MK2_WFMT_FP8_AITER16 2 /* E4M3 with the same block scales, the weight bytes in
                                  AITER's (16, 16) layout [rows/16][K/32][2][16][16 B], as
                                  SGLang leaves linears it preshuffled for AITER's GEMM
                                  (the reference's fp8_shuffled, kernel.py:1015-1050) */

typedef struct mk2_front_shape {
  int rows;          /* 1..32 */
  int hidden;        /* 1024, 2048, 3072, 4096, 6144, 7168 or 8192 */
  int q_lora;        /* as hidden */
  int kv_lora;       /* 512 */
  int rope;          /* 64 */
  int nope;          /* 128, 192 or 256 */
  int heads;         /* MLA heads of this GPU */
  int index_heads;   /* 0 (no indexer) or a multiple of 16 up to 64; index dim 128 */
  int weight_fmt;    /* MK2_WFMT_* of W_qkv_a, W_q_b, W_iq, W_ik (one format for all four) */
  int key_fmt;       /* MK2_KEYS_*: the index cache's format */
  int kv_scaled;     /* 1: latent rows with a f32 scale (amax / 448) each; 0: SGLang's unscaled */
  int max_position;  /* the last position of rope_cos_sin */
  float eps;         /* the RMSNorms' */
  float index_eps;   /* the index key LayerNorm's */
} mk2_front_shape;

typedef struct mk2_front_weights {
  const void* g_in;      /* bf16 [hidden] */
  const void* w_qkv_a;   /* [q_lora + kv_lora + rope][hidden] */
  const float* s_qkv_a;
  const void* g_q_a;     /* bf16 [q_lora] */
  const void* g_kv_a;    /* bf16 [kv_lora] */
  const void* w_q_b;     /* [heads * (nope + rope)][q_lora] */
  const float* s_q_b;
  const void* w_uk;      /* bf16 [heads][kv_lora][nope] */
  const void* w_iq;      /* [index_heads * 128][q_lora] */
  const float* s_iq;
  const void* w_ik;      /* [128][hidden] */
  const float* s_ik;
  const float* g_ik;     /* f32 [128] */
  const float* b_ik;     /* f32 [128] */
  const void* w_iw;      /* bf16 [index_heads][hidden] */
} mk2_front_weights;

typedef struct mk2_front_args {
  mk2_front_shape shape;
  mk2_front_weights weights;
  const void* x;             /* bf16 [rows][hidden]: the residual rows */
  const int64_t* positions;  /* [rows] (clamped to max_position) */
  const int64_t* slots;      /* [rows] cache slots, < 0: a pad row */
  const float* rope_cos_sin; /* f32 [max_position + 1][rope] */
  uint8_t* kv_cache;         /* [slots][kv_lora + rope] E4M3 */
  float* kv_scale;           /* [slots] (kv_scaled), or NULL */
  uint8_t* index_cache;      /* FP8: [pages][64][132]; FP4: the plane's codes [pages][4][64][16] */
  uint8_t* index_scale;      /* FP4: the plane's E8M0 [pages][4][64]; FP8: NULL */
  void* mla_q;               /* bf16 [rows][heads][kv_lora + rope] */
  void* index_q;             /* bf16 [rows][index_heads][128] */
  void* index_w;             /* bf16 [rows][index_heads] */
  void* workspace;
  size_t workspace_bytes;
} mk2_front_args;

int mk2_front_workspace_bytes(const mk2_front_shape* shape, size_t* bytes);
/* reference: the front stages of glm53/gfx950/kernel.py:2585-3575 (one launch there) */
int mk2_front_launch(const mk2_front_args* args, mk2_stream_t stream);
/* the same front as six stage launches in stream order (every valid shape) */
int mk2_front_launch_staged(const mk2_front_args* args, mk2_stream_t stream);
/* 1: mk2_front_launch runs one persistent launch for this shape; 0: the six stage
   launches; < 0: an invalid shape (minus its MK2_E* code; mk2_last_error says why) */
int mk2_front_is_persistent(const mk2_front_shape* shape);

/* The front and the layer in ONE persistent launch: the front's stages first (as
 * mk2_front_launch's persistent launch runs them), then the layer's, which wait for
 * the front's per-head tasks.  The front's outputs and caches must be the layer's
 * inputs (index_q/index_w/index_cache/index_scale = indexer q/w/cache/cache_scale,
 * mla_q/kv_cache/kv_scale = mla q/kv/kv_scale, x = mla h) and the layer persistent;
 * both workspaces as for their own launches.  Instanced for A8W4 experts
 * (MK2_FMT_MXFP4) with the C7 front shape (hidden 6144, q_lora 2048, nope 192, 64
 * index heads), block-FP8 front weights row-major or in AITER's layout; other shapes
 * get MK2_EINVAL (launch the front and the layer on their own).  The same bits as the
 * two launches.  Reference: its K2 launch runs the front's stages ahead of the
 * layer's in one launch (glm53/gfx950/kernel.py:2585-3575). */
int mk2_layer_step_launch(const mk2_front_args* front, const mk2_layer_args* layer, mk2_stream_t stream);
/* 1: mk2_layer_step_launch has an instance for this front shape with experts of
   expert_fmt (MK2_FMT_*); 0: launch the front and the layer on their own; < 0: an
   invalid front shape (minus its MK2_E* code).  The serving host's choice; the
   reference's K2 launch always carries its front (glm53/gfx950/kernel.py:2585-3575). */
int mk2_layer_step_is_fused(const mk2_front_shape* shape, int expert_fmt);

/* ------------------------------------------------------------------ tail
 * The steps after the last layer, on this GPU's rows of the LM head: the final
 * RMSNorm and the logits.  Replaces the reference's tail launch,
 * Glm53HeadOp.launch (glm53/gfx950/runner.py:473-545; kernel glm53/gfx950/kernel.py:
 * 2220-2350, run_head), without its TP gather of the logits:
 *   normed[r]    = bf16(x[r] * rsqrt(mean(x[r]^2) + eps) * g_norm)
 *   logits[r][v] = f32(bf16(normed[r] . w_head[v]))   (bf16 as the reference gathers)
 * w_head is SGLang's LM head as loaded, bf16 [vocab_rows][hidden] row-major, read in
 * place.  No workspace.  More than 16 rows stream the LM head twice. */
typedef struct mk2_tail_args {
  int rows;             /* 1..32 */
  int hidden;           /* multiple of 1024 in [2048, 8192] */
  int vocab_rows;       /* this GPU's LM-head rows, >= 1 */
  float eps;
  const void* x;        /* bf16 [rows][hidden]: the last layer's output rows */
  const void* g_norm;   /* bf16 [hidden] */
  const void* w_head;   /* bf16 [vocab_rows][hidden] */
  float* logits;        /* f32 [rows][vocab_rows] */
  void* normed;         /* bf16 [rows][hidden], or NULL; must not alias x */
} mk2_tail_args;

int mk2_tail_launch(const mk2_tail_args* args, mk2_stream_t stream);

/* ------------------------------------------------------------ step tables
 * A step's per-row tables, from SGLang's rows, in one launch before the layer stack.
 * Replaces the reference's tables.step_rows (glm53/tables.py:26-131); the outputs
 * are its Glm53Step's (runner.py:138-151) plus ctx_len, the layer's per-row key
 * counts.  Row s < rows takes its slot from out_cache_loc[s] (0 = SGLang's padding
 * slot: a pad row, slot -1), its position min(positions[s], max_position), request
 * row s, and keys indptr[s] ..< indptr[s + 1]: min(position + 1, topk) for a row with
 * a slot, 0 for a pad row, or with a seed (a draft step reusing a top-k: int32
 * [rows][topk], -1 unused) the seed row's valid entries, compacted in order into
 * topk_out (seed_by_position: its first min(position + 1, topk) entries as they
 * are).  Rows rows ..< width are pad rows (slot -1, position 0, request 0, id -1).
 * ctx_len[s] = position + 1 for a row with a slot, else 0. */
typedef struct mk2_step_args {
  int width;                 /* W: 1..32 */
  int rows;                  /* S: SGLang's rows this step, 0..W */
  int topk;                  /* K: the keys a row attends at most, 1..4096 */
  int seed_by_position;      /* 0, or 1: seed entries counted by position */
  int64_t max_position;      /* the last position of the context */
  const int64_t* out_cache_loc; int64_t loc_stride;  /* [S] (strided views allowed) */
  const int64_t* positions;  int64_t pos_stride;      /* [S] */
  const void* ids_in;        int64_t ids_stride;      /* [S] token ids, or NULL */
  int ids_in_bytes;          /* 4 or 8: int32 or int64 ids_in */
  const int32_t* seed;       int64_t seed_stride;     /* [S][K], or NULL */
  int64_t* slots;            /* [W] */
  int64_t* positions_out;    /* [W] */
  int32_t* indptr;           /* [W + 1] */
  int32_t* req_ids;          /* [W] */
  int32_t* topk_out;         /* [W * K + 1]: with a seed */
  int32_t* ids;              /* [W], or NULL (needs ids_in) */
  int32_t* ctx_len;          /* [W], or NULL */
} mk2_step_args;

int mk2_step_rows_launch(const mk2_step_args* args, mk2_stream_t stream);

/* seed row s (s < rows) := the keys of step row rows_of[s], topk[indptr[src] ..<
 * indptr[src + 1]], then -1 up to k.  Replaces tables.write_seed
 * (glm53/tables.py:134-167). */
int mk2_write_seed_launch(const int32_t* topk, const int32_t* indptr, int32_t* seed, int64_t seed_stride,
                          const int32_t* rows_of, int rows, int k, mk2_stream_t stream);

/* ------------------------------------------------------------------ misc */
const char* mk2_last_error(void);
int mk2_abi_version(void);

/* Matrix-core operand self-test: one 16x16 tile product per mode, for the layout
 * checks of the test suite (no counterpart in the reference).  mode 0: bf16 x bf16
 * over K=128 (a, b: bf16 [16][128]); mode 1: E2M1 x E4M3 over K=128 with E8M0
 * scales (a: [16][64 B], sa: [16][4], b: [16][128 B], sb: [16][4]); mode 2: E4M3
 * widened to bf16 x bf16 (a: [16][128 B] E4M3, b: bf16 [16][128]).  d: f32
 * [16][16], d[i][j] = sum_k A[i][k] B[j][k]. */
int mk2_selftest_mfma(int mode, const void* a, const void* sa, const void* b,
                      const void* sb, float* d, mk2_stream_t stream);

/* Measurement probes (no counterpart in the reference; used by bench.py --probes and
 * the GPU tests to evidence two design rules of the persistent layer).
 *
 * mk2_probe_stream_read: one 512-thread workgroup a CU streams `bytes` from src with
 * 16-byte loads, 8 in flight a lane (the layer's launch shape); bytes must be a
 * positive multiple of mk2_probe_stream_unit() (CUs x 64 KiB; 0 when the device
 * cannot be queried).  sink: one device word, practically never written.
 *
 * mk2_probe_handoff: a litmus of the hand-off rules across XCDs, `rounds` rounds of
 * one workgroup a CU handing data to workgroups on other XCDs.  mode 0: write-once
 * data, device-coherent stores, counter, plain loads; 1: the same with two producers
 * a 128-B line; 2: a line polled device-coherently while partly published, its late
 * half read with plain loads; 3: as 2, read with device-coherent loads.  The entry
 * point clears buf, flags and result itself (hipMemsetAsync: not for graph capture).
 * result[0] = mismatched words, result[1] = bounded waits that gave up (each spins at
 * most `spin` polls).  Buffer sizes from mk2_probe_handoff_bytes. */
size_t mk2_probe_stream_unit(void);
int mk2_probe_stream_read(const void* src, size_t bytes, uint32_t* sink, mk2_stream_t stream);
int mk2_probe_handoff_bytes(int rounds, size_t* buf_bytes, size_t* flag_bytes);
int mk2_probe_handoff(int mode, uint32_t* buf, size_t buf_bytes, int* flags, size_t flag_bytes, int* result,
                      int rounds, int spin, mk2_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MK2_H */
