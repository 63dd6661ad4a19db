// Measurement probes behind two design rules of the persistent layer (no counterpart in
// the reference): the streaming-read ceiling of HBM in the layer's launch shape, and a
// litmus of the hand-off rules (device-coherent stores, counters, plain or
// device-coherent loads) across the eight XCDs' L2 caches.  Every wait is bounded.
#include "mk2_device.h"
#include "mk2_host.h"

namespace mk2 {

// One 512-thread workgroup a CU; wave w of workgroup g reads its own contiguous
// per_wave KiB with 8 loads of 16 B a lane in flight (one 1-KiB piece a load).
__global__ void __launch_bounds__(512) k_probe_stream(const uint4* src, size_t per_wave_kib, uint32_t* sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint4* p = src + (size_t)(blockIdx.x * 8 + wave) * per_wave_kib * 64;
  uint32_t acc = 0;
  for (size_t i = 0; i < per_wave_kib; i += 8) {
    uint4 v[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) v[d] = ld_stream16(p + (i + d) * 64 + lane);
#pragma unroll
    for (int d = 0; d < 8; ++d) acc ^= v[d].x + v[d].y + v[d].z + v[d].w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;  // keeps the loads; practically never stores
}

constexpr int kLitmusWords = 2048;  // a consumer's region a round: 64 lines of 128 B
constexpr int kFlagStride = 32;     // one flag a 128-B line

// a bounded wait of one thread; false on a spin-out or when another wait already failed
MK2_DEV bool probe_wait(const int* flag, int above, int* result, int spin) {
  for (int n = 0; ld_dev_i32(flag) <= above; ++n) {
    if (n > spin || ((n & 31) == 0 && ld_dev_i32(result + 1))) {
      atomicAdd(result + 1, 1);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

MK2_DEV uint32_t probe_word(int round, int owner, int k) { return (uint32_t)(round * 7919 + owner * 131 + k) | 1u; }

// Workgroup b produces for consumers c1 = b + 37 and c2 = b + 91 (mod G): with
// workgroups dealt round-robin over the 8 XCDs, producer and consumer sit on
// different XCDs.  Each round uses fresh regions (the hand-off data is written once).
//  mode 0: c1's whole region from b; the consumer waits on b's counter, then reads
//          with plain loads (the layer's rule for published data);
//  mode 1: two producers a line: b writes c1's even 64-B halves and c2's odd halves;
//          the consumer waits for both counters, then reads with plain loads;
//  mode 2/3: a line polled while partly published: b writes the first 64 B of each of
//          c1's lines; c1 polls those words device-coherently, then signals; b's
//          partner (the producer of c2) waits for that signal, writes the other 64 B
//          of c2's lines and bumps a counter; the consumer waits on it and reads the
//          late halves with plain loads (mode 2) or device-coherent loads (mode 3:
//          the layer's rule for such lines).
__global__ void __launch_bounds__(256) k_probe_handoff(int mode, uint32_t* buf, int* flags, int* result, int rounds,
                                                       int spin) {
  const int G = gridDim.x, b = blockIdx.x, t = threadIdx.x;
  const int c1 = (b + 37) % G, c2 = (b + 91) % G;
  const int p1 = (b + G - 37) % G, p2 = (b + G - 91) % G;
  int* cnt_a = flags;                             // [G] first hand-off counters
  int* cnt_b = flags + (size_t)G * kFlagStride;   // [G] second hand-off counters
  int* ack = flags + (size_t)2 * G * kFlagStride; // [G] "polled" signals (modes 2, 3)
  __shared__ int ok;
  int errors = 0;
  for (int i = 0; i < rounds; ++i) {
    uint32_t* region = buf + (size_t)i * G * kLitmusWords;
    if (mode == 0) {
      uint32_t* dst = region + (size_t)c1 * kLitmusWords;
      for (int k = t; k < kLitmusWords; k += 256) st_dev_u32(dst + k, probe_word(i, b, k));
    } else if (mode == 1) {
      for (int k = t; k < kLitmusWords; k += 256) {
        const int c = ((k >> 4) & 1) ? c2 : c1;
        st_dev_u32(region + (size_t)c * kLitmusWords + k, probe_word(i, 0, k));
      }
    } else {
      for (int k = t; k < kLitmusWords / 2; k += 256) {
        const int w = (k >> 4) * 32 + (k & 15);  // first 64 B of each line
        st_dev_u32(region + (size_t)c1 * kLitmusWords + w, probe_word(i, 0, w));
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0) {
      if (mode < 2) __hip_atomic_fetch_add(cnt_a + (size_t)b * kFlagStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok = 1;
    }
    __syncthreads();
    const uint32_t* mine = region + (size_t)b * kLitmusWords;
    if (mode < 2) {
      if (t == 0) {
        bool fine = probe_wait(cnt_a + (size_t)p1 * kFlagStride, i, result, spin);
        if (mode == 1) fine = fine && probe_wait(cnt_a + (size_t)p2 * kFlagStride, i, result, spin);
        ok = fine;
      }
      __syncthreads();
      if (!ok) break;
      for (int k = t; k < kLitmusWords; k += 256) {
        const uint32_t want = mode == 0 ? probe_word(i, p1, k) : probe_word(i, 0, k);
        errors += ldp_u32(mine + k) != want;
      }
      continue;
    }
    // modes 2, 3: poll the early halves of my 64 lines (one lane a line)
    if (t < 64) {
      const int w = t * 32 + (t & 15);
      const uint32_t want = probe_word(i, 0, w);
      int n = 0;
      while ((uint32_t)MK2_DEV_LD(uint32_t, mine + w) != want) {
        if (++n > spin || ((n & 31) == 0 && ld_dev_i32(result + 1))) {
          atomicAdd(result + 1, 1);
          ok = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    __syncthreads();
    if (!ok) break;
    if (t == 0) __hip_atomic_fetch_add(ack + (size_t)b * kFlagStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // as the producer of c2's late halves: wait until c2 has polled its lines
    if (t == 0) ok = probe_wait(ack + (size_t)c2 * kFlagStride, i, result, spin);
    __syncthreads();
    if (!ok) break;
    for (int k = t; k < kLitmusWords / 2; k += 256) {
      const int w = (k >> 4) * 32 + 16 + (k & 15);  // last 64 B of each line
      st_dev_u32(region + (size_t)c2 * kLitmusWords + w, probe_word(i, 1, w));
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0) {
      __hip_atomic_fetch_add(cnt_b + (size_t)b * kFlagStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok = probe_wait(cnt_b + (size_t)p2 * kFlagStride, i, result, spin);
    }
    __syncthreads();
    if (!ok) break;
    for (int k = t; k < kLitmusWords / 2; k += 256) {
      const int w = (k >> 4) * 32 + 16 + (k & 15);
      const uint32_t got = mode == 2 ? ldp_u32(mine + w) : (uint32_t)MK2_DEV_LD(uint32_t, mine + w);
      errors += got != probe_word(i, 1, w);
    }
  }
  if (errors) atomicAdd(result, errors);
}

static int probe_cus(int* g) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(g, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      *g <= 0)
    return set_error(MK2_ELAUNCH, "probe: cannot read the device's CU count");
  return MK2_OK;
}

}  // namespace mk2

extern "C" size_t mk2_probe_stream_unit(void) {
  int g = 0;
  if (mk2::probe_cus(&g)) return 0;
  return (size_t)g * 8 * 8 * 1024;
}

extern "C" int mk2_probe_stream_read(const void* src, size_t bytes, uint32_t* sink, mk2_stream_t stream) {
  mk2::clear_error();
  int g = 0;
  if (int e = mk2::probe_cus(&g)) return e;
  const size_t unit = (size_t)g * 8 * 8 * 1024;
  MK2_REQUIRE(src && sink, "probe_stream_read: null pointer");
  MK2_REQUIRE(bytes >= unit && bytes % unit == 0, "probe_stream_read: bytes (%zu) must be a positive multiple of %zu",
              bytes, unit);
  MK2_REQUIRE(((uintptr_t)src & 15) == 0, "probe_stream_read: src must be 16-byte aligned");
  hipLaunchKernelGGL(mk2::k_probe_stream, dim3(g), dim3(512), 0, (hipStream_t)stream, (const uint4*)src,
                     bytes / ((size_t)g * 8 * 1024), sink);
  return mk2::check_launch("k_probe_stream");
}

extern "C" int mk2_probe_handoff_bytes(int rounds, size_t* buf_bytes, size_t* flag_bytes) {
  mk2::clear_error();
  int g = 0;
  if (int e = mk2::probe_cus(&g)) return e;
  MK2_REQUIRE(rounds > 0 && buf_bytes && flag_bytes, "probe_handoff_bytes: bad arguments");
  *buf_bytes = (size_t)rounds * g * mk2::kLitmusWords * 4;
  *flag_bytes = (size_t)3 * g * mk2::kFlagStride * 4;
  return MK2_OK;
}

extern "C" int mk2_probe_handoff(int mode, uint32_t* buf, size_t buf_bytes, int* flags, size_t flag_bytes, int* result,
                                 int rounds, int spin, mk2_stream_t stream) {
  mk2::clear_error();
  size_t need_buf = 0, need_flags = 0;
  if (int e = mk2_probe_handoff_bytes(rounds, &need_buf, &need_flags)) return e;
  MK2_REQUIRE(mode >= 0 && mode <= 3, "probe_handoff: mode %d is not 0..3", mode);
  MK2_REQUIRE(buf && flags && result, "probe_handoff: null pointer");
  MK2_REQUIRE(buf_bytes >= need_buf && flag_bytes >= need_flags, "probe_handoff: buffers too small");
  MK2_REQUIRE(spin > 0 && spin <= (1 << 22), "probe_handoff: spin %d out of (0, 4194304]", spin);
  int g = 0;
  if (int e = mk2::probe_cus(&g)) return e;
  hipStream_t s = (hipStream_t)stream;
  if (hipMemsetAsync(buf, 0, need_buf, s) != hipSuccess || hipMemsetAsync(flags, 0, need_flags, s) != hipSuccess ||
      hipMemsetAsync(result, 0, 2 * sizeof(int), s) != hipSuccess)
    return mk2::set_error(MK2_ELAUNCH, "probe_handoff: clearing the buffers failed");
  hipLaunchKernelGGL(mk2::k_probe_handoff, dim3(g), dim3(256), 0, s, mode, buf, flags, result, rounds, spin);
  return mk2::check_launch("k_probe_handoff");
}
