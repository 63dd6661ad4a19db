// Device helpers of the K2 kernels: CDNA4 (gfx950) matrix-core operands, number
// formats and wavefront reductions.  Every kernel in this library includes it.
//
// Operand convention (one 64-lane wavefront, 16x16 MFMA tiles):
//   A (16 rows x K): lane l owns row l % 16 and the K slice of lane group l / 16.
//   B (K x 16 cols): lane l owns column l % 16 and the same K slice.
//   D (16 x 16 f32): lane l holds D[4 * (l / 16) + i][l % 16], i = 0..3.
// For v_mfma_scale_f32_16x16x128_f8f6f4 an E2M1 operand (low 4 dwords) holds
// k = 32g .. 32g+31 in group g; an E4M3 operand (8 dwords) holds k = 16g .. 16g+15 in
// dwords 0-3 and k = 64+16g .. 64+16g+15 in dwords 4-7.  The E8M0 a lane supplies
// scales the 32-block k = 32g .. 32g+31 of its row (A) or column (B) in both cases
// (measured with mk2_selftest_mfma).
// For v_mfma_f32_16x16x32_bf16 it is 8 bf16; a 128-k block is fed as four steps
// s = 0..3 where lane group g supplies k = 32g + 8s .. +7, so one lane reads 32
// consecutive k of its row (the dot product is order-free over k as long as A and
// B use the same map).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint16_t bf16_t;  // storage type of bf16 in memory

#define MK2_WAVE 64
#define MK2_DEV __device__ __forceinline__

namespace mk2 {

// ----------------------------------------------------------------- bf16 / f32
MK2_DEV float bf16_to_f32(bf16_t v) { return __uint_as_float(((uint32_t)v) << 16); }
// f32 -> bf16, round to nearest even: one v_cvt_pk_bf16_f32 (gfx950) a pair
MK2_DEV bf16_t f32_to_bf16(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }
MK2_DEV uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}
// two f32 that are exactly representable in bf16 -> packed pair (truncation is exact)
MK2_DEV uint32_t pack_bf16x2_exact(float lo, float hi) {
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
}

// ----------------------------------------------------------------- E4M3 / E2M1
// 4 E4M3 bytes of a dword -> 4 f32 (exact)
MK2_DEV void e4m3x4_to_f32(uint32_t w, float* o) {
  f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
  f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
  o[0] = a.x; o[1] = a.y; o[2] = b.x; o[3] = b.y;
}
// 8 E4M3 bytes (two dwords) -> 8 bf16: one scaled conversion (x 1.0) a pair, exact
// (an E4M3 value has 4 significant bits and an exponent bf16 holds)
MK2_DEV bf16x8 e4m3x8_to_bf16(uint32_t w0, uint32_t w1) {
  i32x4 r;
  r[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false));
  r[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true));
  r[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false));
  r[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true));
  return __builtin_bit_cast(bf16x8, r);
}
// 8 E2M1 codes (one dword, element 0 in the low nibble) times 2^(code - 127) -> 8 bf16.
// Exact: an E2M1 value times a power of two has at most 2 significant bits.
MK2_DEV bf16x8 e2m1x8_to_bf16(uint32_t w, float scale) {
  i32x4 r;
  r[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0));
  r[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1));
  r[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2));
  r[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3));
  return __builtin_bit_cast(bf16x8, r);
}
MK2_DEV float e8m0_to_f32(uint32_t code) { return __uint_as_float((code & 0xFFu) << 23); }

// f32 -> E4M3 byte, clamped to +-448, round to nearest even
MK2_DEV uint32_t f32_to_e4m3(float v) {
  v = fminf(fmaxf(v, -448.0f), 448.0f);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, 0.0f, 0, false) & 0xFFu;
}
MK2_DEV uint32_t f32x4_to_e4m3x4(float a, float b, float c, float d) {
  a = fminf(fmaxf(a, -448.0f), 448.0f);
  b = fminf(fmaxf(b, -448.0f), 448.0f);
  c = fminf(fmaxf(c, -448.0f), 448.0f);
  d = fminf(fmaxf(d, -448.0f), 448.0f);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// E8M0 code of an MXFP8 activation block: ceil-pow2 exponent of amax * f32(1/448),
// clamped to [1, 254] (the rule of the reference's quant_mxfp8).
MK2_DEV uint32_t mxfp8_scale_code(float amax) {
  uint32_t bits = __float_as_uint(amax * (1.0f / 448.0f));
  int e = (int)((bits >> 23) & 0xFFu) + ((bits & 0x7FFFFFu) != 0u ? 1 : 0);
  e = e < 1 ? 1 : (e > 254 ? 254 : e);
  return (uint32_t)e;
}
// exact 1 / 2^(code - 127) for code in [1, 254]
MK2_DEV float e8m0_inverse(uint32_t code) {
  int e = 254 - (int)code;  // biased exponent of the reciprocal
  if (e >= 1) return __uint_as_float((uint32_t)e << 23);
  return __uint_as_float(0x00400000u);  // code 254: 2^-127 (subnormal)
}

// ----------------------------------------------------------------- MFMA
MK2_DEV f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// A = 32 E2M1 (low 4 dwords of a), B = 32 E4M3; scale bytes selected by SA / SB
template <int SA, int SB>
MK2_DEV f32x4 mfma_fp4_fp8(i32x8 a, i32x8 b, f32x4 c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 4, 0, SA, sa, SB, sb);
}
// the same product with both operands in one format: FMT 0 = E4M3 (8 dwords each),
// 4 = E2M1 (the low 4 dwords); E8M0 scale bytes from byte 0 of sa / sb
template <int FMT>
MK2_DEV f32x4 mfma_same(i32x8 a, i32x8 b, f32x4 c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FMT, FMT, 0, sa, 0, sb);
}
constexpr int E8M0_ONE = 127;

// ----------------------------------------------------------------- activation quant
// MXFP4 activations, AITER's round-up rule (the reference's e8m0_roundup): the E8M0
// code of the smallest power of two >= amax * f32(1/6), at most 254 (0 for amax = 0)
MK2_DEV uint32_t mxfp4_act_code(float amax) {
  const uint32_t b = ((__float_as_uint(amax * (1.0f / 6.0f)) + 0x7FFFFFu) >> 23) & 0xFFu;
  return b < 254u ? b : 254u;
}
// 8 f32 over the E8M0 scale `code` -> 8 E2M1 codes in a dword (element 0 in the low
// nibble), rounded to nearest even and saturating at 6 by the hardware conversion
MK2_DEV uint32_t f32x8_to_e2m1x8(const float* f, uint32_t code) {
  const float sc = __uint_as_float(code ? code << 23 : 0x00400000u);  // 2^(code - 127)
  uint32_t w = 0;
  w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, f[0], f[1], sc, 0);
  w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, f[2], f[3], sc, 1);
  w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, f[4], f[5], sc, 2);
  w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, f[6], f[7], sc, 3);
  return w;
}
// 2 f32 over the E8M0 scale `code` -> 2 E2M1 codes in the low byte (element 0 in the low
// nibble), as f32x8_to_e2m1x8
MK2_DEV uint32_t f32x2_to_e2m1x2(float a, float b, uint32_t code) {
  const float sc = __uint_as_float(code ? code << 23 : 0x00400000u);
  return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, a, b, sc, 0) & 0xFFu;
}
// E8M0 of a 32-dim group of index queries quantized to MXFP4 (the reference's
// quantize_fp4_indexer_row, deepseek_v41/gfx950/attention/index_query.py:283-291): the
// smallest power of two >= max(amax / 6, 1e-4), the quotient rounded to f32 first,
// clamped to [1, 254]
MK2_DEV uint32_t fp4_query_code(float amax) {
  const uint32_t b = __float_as_uint(fmaxf(amax / 6.0f, 1.0e-4f));
  const uint32_t e = ((b >> 23) & 0xFFu) + ((b & 0x7FFFFFu) != 0u);
  return e < 1u ? 1u : (e > 254u ? 254u : e);
}
// FP8 per-128 block scale (the reference's quant_scaled): scale = amax * f32(1/448)
// and the multiplier 448 / amax (IEEE here, where the reference takes the hardware
// reciprocal); 1 and 1 for an all-zero block
MK2_DEV void fp8_block_scale(float amax, float* scale, float* inv) {
  const bool nz = amax > 0.f;
  *scale = nz ? amax * (1.0f / 448.0f) : 1.0f;
  *inv = nz ? 448.0f / amax : 1.0f;
}

// ----------------------------------------------------------------- reductions

// DPP lane moves within a 16-lane row (no LDS traffic): quad_perm [1,0,3,2] and
// [2,3,0,1], row_half_mirror (lane i <-> 7-i of each half row), row_mirror (i <-> 15-i)
template <int CTRL>
MK2_DEV float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;
// reduce over the 16 lanes of a lane row (lanes with equal l / 16); every lane of the
// row gets the result: quads first, then half rows, then the row
MK2_DEV float row16_max(float v) {
  v = fmaxf(v, dpp_f32<DPP_XOR1>(v));
  v = fmaxf(v, dpp_f32<DPP_XOR2>(v));
  v = fmaxf(v, dpp_f32<DPP_HALF_MIRROR>(v));
  return fmaxf(v, dpp_f32<DPP_MIRROR>(v));
}
MK2_DEV float row16_sum(float v) {
  v += dpp_f32<DPP_XOR1>(v);
  v += dpp_f32<DPP_XOR2>(v);
  v += dpp_f32<DPP_HALF_MIRROR>(v);
  return v + dpp_f32<DPP_MIRROR>(v);
}
// whole-wave reductions, the result in every lane: row totals by DPP, then lane 15's
// row total into rows 1 and 3 (row_bcast:15) and lane 31's into rows 2 and 3
// (row_bcast:31), so that row 3 holds the total; read from lane 63
template <int CTRL, int ROWS>
MK2_DEV float dpp_rows_f32(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                               CTRL, ROWS, 0xF, false));
}
constexpr int DPP_BCAST15 = 0x142, DPP_BCAST31 = 0x143;
constexpr int DPP_SHR1 = 0x111, DPP_SHR2 = 0x112, DPP_SHR4 = 0x114, DPP_SHR8 = 0x118;
template <int CTRL, int ROWS>
MK2_DEV int dpp_i32(int v) {  // lanes without a source (or outside ROWS) read 0
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xF, false);
}
// the sum over a 16-lane row, in every lane of the row
MK2_DEV int row16_sum_i32(int v) {
  v += dpp_i32<DPP_XOR1, 0xF>(v);
  v += dpp_i32<DPP_XOR2, 0xF>(v);
  v += dpp_i32<DPP_HALF_MIRROR, 0xF>(v);
  return v + dpp_i32<DPP_MIRROR, 0xF>(v);
}
// inclusive scan over the wave: shifts within each 16-lane row, then each row's total
// carried up (row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3)
MK2_DEV int wave_incl_scan(int v) {
  v += dpp_i32<DPP_SHR1, 0xF>(v);
  v += dpp_i32<DPP_SHR2, 0xF>(v);
  v += dpp_i32<DPP_SHR4, 0xF>(v);
  v += dpp_i32<DPP_SHR8, 0xF>(v);
  v += dpp_i32<DPP_BCAST15, 0xA>(v);
  v += dpp_i32<DPP_BCAST31, 0xC>(v);
  return v;
}
MK2_DEV float wave_sum(float v) {
  v = row16_sum(v);
  v += dpp_rows_f32<DPP_BCAST15, 0xA>(0.f, v);
  v += dpp_rows_f32<DPP_BCAST31, 0xC>(0.f, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
MK2_DEV float wave_max(float v) {
  v = row16_max(v);
  v = fmaxf(v, dpp_rows_f32<DPP_BCAST15, 0xA>(-INFINITY, v));
  v = fmaxf(v, dpp_rows_f32<DPP_BCAST31, 0xC>(-INFINITY, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// order-preserving u32 of f32 bits: larger keys rank first
// max(x, 0) as one integer max on the bits (a negative float is a negative int); no
// NaN quieting
MK2_DEV float relu_bits(float x) { return __int_as_float(max(__float_as_int(x), 0)); }
// v + (v of the lane 16 apart, xor) and v + (v of the lane 32 apart, xor), by the
// row-swapping permutes
MK2_DEV float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
MK2_DEV float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
MK2_DEV float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// lane i reads lane i + N of its 16-lane row (0 past the row's end)
template <int N>
MK2_DEV uint32_t dpp_shl(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x100 + N, 0xF, 0xF, false);
}
MK2_DEV uint32_t radix_key(float f) {
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

MK2_DEV float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// a 16-byte piece of a stream read once a launch (weights, index keys, latent-KV
// rows).  A plain load: the nontemporal form measured 0.8 us slower a layer (the
// layer at 8 rows, same-box A/B).
MK2_DEV uint4 ld_stream16(const void* p) { return *(const uint4*)p; }

// ----------------------------------------------------------------- hand-off memory
// Data that one workgroup hands to another inside a launch.  The L2 of one XCD is not
// coherent with the others for plain accesses, so:
//  - producers store with device-coherent stores (relaxed agent-scope atomic stores:
//    sc1, write-through), drain them (s_waitcnt) and only then publish a counter;
//  - consumers read PUBLISHED data -- written once per launch and read only after its
//    counter was seen -- with plain loads (ldp_*).  A launch starts with invalidated
//    caches and nothing on any XCD reads such data before it is published, so the
//    first read of a line misses the L2 and fetches the stored value;
//  - data built by device atomics (histograms) is read device-coherently (ld_dev_*),
//    and so is any line that a reader polled before all of it was published (the
//    top-k chunk counts): a plain load there could hit a copy taken between two
//    producers' stores.
// No cache write-back or invalidate is needed (an agent-scope fence costs both, for
// the whole L2).
#define MK2_DEV_LD(T, p) __hip_atomic_load((const T*)(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
#define MK2_DEV_ST(T, p, v) __hip_atomic_store((T*)(p), (T)(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
MK2_DEV int ld_dev_i32(const int* p) { return MK2_DEV_LD(int, p); }
MK2_DEV uint32_t ldp_u8(const void* p) { return *(const uint8_t*)p; }
MK2_DEV uint32_t ldp_u16(const void* p) { return *(const uint16_t*)p; }
MK2_DEV uint32_t ldp_u32(const void* p) { return *(const uint32_t*)p; }
MK2_DEV int ldp_i32(const int* p) { return *p; }
MK2_DEV float ldp_f32(const float* p) { return *p; }
MK2_DEV uint2 ldp_8(const void* p) { return *(const uint2*)p; }
MK2_DEV uint4 ldp_16(const void* p) { return *(const uint4*)p; }
MK2_DEV float4 ldp_f32x4(const float* p) { return *(const float4*)p; }
MK2_DEV void st_dev_u8(void* p, uint32_t v) { MK2_DEV_ST(uint8_t, p, v); }
MK2_DEV void st_dev_u16(void* p, uint32_t v) { MK2_DEV_ST(uint16_t, p, v); }
MK2_DEV void st_dev_u32(void* p, uint32_t v) { MK2_DEV_ST(uint32_t, p, v); }
MK2_DEV void st_dev_i32(int* p, int v) { MK2_DEV_ST(int, p, v); }
MK2_DEV void st_dev_f32(float* p, float v) { MK2_DEV_ST(float, p, v); }
MK2_DEV void st_dev_8(void* p, uint2 v) { MK2_DEV_ST(uint64_t, p, ((uint64_t)v.y << 32) | v.x); }
MK2_DEV void st_dev_16(void* p, uint4 v) {
  MK2_DEV_ST(uint64_t, p, ((uint64_t)v.y << 32) | v.x);
  MK2_DEV_ST(uint64_t, (uint64_t*)p + 1, ((uint64_t)v.w << 32) | v.z);
}
// the dependency wait a stage runs after issuing the loads of its static weights (the
// persistent launch waits on a counter there; a stand-alone kernel has nothing to wait
// for)
// a stage's dependency wait: true once satisfied, false when the launch is failing
// (the stage then returns at once, every thread alike)
struct NoWait {
  MK2_DEV bool operator()() const { return true; }
};
// a stage's optional progress marks (the persistent launch's timeline stamps)
struct NoMark {
  MK2_DEV void operator()(int) const {}
};

// every memory access of this thread has completed (stores are device-visible)
MK2_DEV void drain_memory() { __builtin_amdgcn_s_waitcnt(0); }

// ------------------------------------------------------------------ wait deadlines
// A dependency wait inside a persistent launch gives up once its deadline has passed
// on the constant 100 MHz s_memrealtime clock, counted from its first poll round that
// found the dependency unmet (a wait met at once reads no clock).  The differences are
// 32-bit ticks, so a deadline is at most MK2_MAX_WAIT_US.  A deadline, unlike a poll
// count, does not stretch when the polls slow down under contention.
constexpr uint32_t WAIT_TICKS_PER_US = 100;
constexpr uint32_t DEFAULT_WAIT_TICKS = 1000000u * WAIT_TICKS_PER_US;  // one second
struct WaitClock {
  uint32_t t0 = 0;
  bool started = false;
  // false on the first call (which starts the clock), then whether `ticks` have passed
  MK2_DEV bool expired(uint32_t ticks) {
    const uint32_t now = (uint32_t)__builtin_amdgcn_s_memrealtime();
    if (!started) {
      started = true;
      t0 = now;
      return false;
    }
    return now - t0 > ticks;
  }
};
// the ticks of a host-given deadline in microseconds (0: the default, one second)
inline uint32_t wait_ticks_of(int wait_us) {
  return wait_us > 0 ? (uint32_t)wait_us * WAIT_TICKS_PER_US : DEFAULT_WAIT_TICKS;
}

// ----------------------------------------------------------------- tagged hand-offs
// A 32-bit value one workgroup hands to another inside a persistent launch can travel
// with the launch's tag in the same 8-byte word, (tag << 32) | value, stored
// device-coherently.  The consumer polls the word itself until it carries its
// launch's tag: one memory round trip, with no store drain on the producer, no
// counter and no second load.  Tags grow by one a launch and are never 0, so on a
// workspace whose tagged regions hold only tagged words of earlier launches (a
// workspace zero-filled before its first launch and used for one shape) a stale word
// never matches; where the regions may hold other bytes (a scratch array shared by
// shapes whose layouts differ) the caller clears them before each launch.  Between stream-ordered
// kernels (one kernel a stage) the stream publishes the words: tag 0, read unchecked.
struct TagPoll {
  uint32_t tag;         // this launch's tag; 0: stream-ordered, no checking
  uint32_t wait_ticks;  // a wait's deadline (WaitClock ticks)
  int* err;             // the launch's sticky error word (set on giving up, seen by every poller)
};
MK2_DEV void st_pair(uint64_t* p, uint32_t v, uint32_t tag) {
  MK2_DEV_ST(uint64_t, p, ((uint64_t)tag << 32) | v);
}
MK2_DEV uint64_t ld_pair(const uint64_t* p) { return MK2_DEV_LD(uint64_t, p); }
MK2_DEV uint32_t pair_value(uint64_t w) { return (uint32_t)w; }
MK2_DEV bool pair_ready(uint64_t w, const TagPoll& tp) { return tp.tag == 0 || (uint32_t)(w >> 32) == tp.tag; }
// one wave's verdict after a poll round: all lanes ready (true), or keep polling; past
// the wait's deadline or on another poller's error the launch is failing: *bad = true
MK2_DEV bool poll_done(bool ready, int polls, WaitClock& wc, const TagPoll& tp, bool* bad) {
  if (__ballot(!ready) == 0) return true;
  if (wc.expired(tp.wait_ticks) || ((polls & 31) == 0 && tp.err && ld_dev_i32(tp.err))) {
    if ((threadIdx.x & 63) == 0 && tp.err) atomicOr(tp.err, 1);
    *bad = true;
    return true;
  }
  return false;
}

// the sync block at the start of a layer workspace: the persistent launch's counters
// (one a 128-byte line) and, in its last line, the launch epoch (the last tag used),
// which no reset or clear touches
constexpr int SYNC_INTS = 8192;
constexpr int SYNC_EPOCH = SYNC_INTS - 32;

}  // namespace mk2
