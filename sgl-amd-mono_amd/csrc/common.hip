// Error text, ABI version and the matrix-core operand self-test.
#include "mk2_device.h"
#include "mk2_host.h"

namespace mk2 {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}
void clear_error() { g_err[0] = 0; }

// one 16x16 tile over K = 128 in the library's operand convention
__global__ __launch_bounds__(64) void k_selftest(int mode, const uint8_t* a, const uint8_t* sa,
                                                 const uint8_t* b, const uint8_t* sb, float* d) {
  const int lane = threadIdx.x, r = lane & 15, g = lane >> 4;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (mode == 0 || mode == 2) {
    bf16x8 av[4], bv[4];
    const uint4* bs = (const uint4*)(b + r * 256 + g * 64);
    for (int q = 0; q < 4; ++q) bv[q] = __builtin_bit_cast(bf16x8, bs[q]);
    if (mode == 0) {
      const uint4* as = (const uint4*)(a + r * 256 + g * 64);
      for (int q = 0; q < 4; ++q) av[q] = __builtin_bit_cast(bf16x8, as[q]);
    } else {
      const uint4* as = (const uint4*)(a + r * 128 + g * 32);
      uint4 u0 = as[0], u1 = as[1];
      av[0] = e4m3x8_to_bf16(u0.x, u0.y);
      av[1] = e4m3x8_to_bf16(u0.z, u0.w);
      av[2] = e4m3x8_to_bf16(u1.x, u1.y);
      av[3] = e4m3x8_to_bf16(u1.z, u1.w);
    }
    for (int q = 0; q < 4; ++q) acc = mfma_bf16(av[q], bv[q], acc);
  } else {
    uint4 ua = *(const uint4*)(a + r * 64 + g * 16);
    i32x8 av = {(int)ua.x, (int)ua.y, (int)ua.z, (int)ua.w, 0, 0, 0, 0};
    uint4 u0 = *(const uint4*)(b + r * 128 + g * 16), u1 = *(const uint4*)(b + r * 128 + 64 + g * 16);
    i32x8 bv = {(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
    acc = mfma_fp4_fp8<0, 0>(av, bv, acc, sa[r * 4 + g], sb[r * 4 + g]);
  }
  for (int i = 0; i < 4; ++i) d[(4 * g + i) * 16 + r] = acc[i];
}

}  // namespace mk2

using namespace mk2;

extern "C" const char* mk2_last_error(void) { return g_err; }
extern "C" int mk2_abi_version(void) { return MK2_ABI_VERSION; }

extern "C" int mk2_selftest_mfma(int mode, const void* a, const void* sa, const void* b,
                                 const void* sb, float* d, mk2_stream_t stream) {
  clear_error();
  MK2_REQUIRE(mode >= 0 && mode <= 2, "selftest: mode must be 0, 1 or 2");
  MK2_REQUIRE(a && b && d, "selftest: a, b and d must be set");
  MK2_REQUIRE(mode != 1 || (sa && sb), "selftest: mode 1 needs both scale arrays");
  k_selftest<<<1, 64, 0, (hipStream_t)stream>>>(mode, (const uint8_t*)a, (const uint8_t*)sa,
                                                 (const uint8_t*)b, (const uint8_t*)sb, d);
  return check_launch("selftest");
}
