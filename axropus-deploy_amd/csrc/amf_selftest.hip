// amf_selftest.hip - libamf_selftest.so: device-side checks of the codec
// building blocks that the save kernels inline, for the GPU test suite.
// Test infrastructure, not part of the drop-in C ABI (include/amf_selftest.h).
//
// The FP8 save kernels encode with f32x4_to_e4m3 (amf_kernel_util.h), which
// on gfx950 is the v_cvt_pk_fp8_f32 instruction.  The checks here pin that
// instruction two ways: against the portable bit-level encoder e4m3_from_f32
// (amf_device.h) on every fp32 value the kernels can hand it, and as a plain
// encoder over caller-chosen inputs that the tests compare with an
// independent CPU encoder.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/amf_selftest.h"
#include "amf_kernel_util.h"

namespace {

using amf::f32x4_to_e4m3;

// 448.0f: the largest e4m3fn magnitude; the save kernels clamp every
// quotient to [-448, 448] before encoding.
constexpr uint32_t kMaxBits = 0x43E00000u;

__global__ __launch_bounds__(256) void e4m3_sweep_kernel(uint32_t n_quads,
                                                         unsigned long long* bad,
                                                         uint32_t* first_bad) {
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t q = blockIdx.x * blockDim.x + threadIdx.x; q < n_quads; q += stride) {
#pragma unroll
    for (int sgn = 0; sgn < 2; ++sgn) {
      float x[4];
      uint32_t want = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t u = q * 4u + (uint32_t)e;
        if (u > kMaxBits) u = kMaxBits;
        u |= sgn ? 0x80000000u : 0u;
        x[e] = amf::u2f(u);
        want |= amf::e4m3_from_f32(x[e]) << (8 * e);
      }
      const uint32_t got = f32x4_to_e4m3(x);
      if (got != want) {
        const unsigned long long k = atomicAdd(bad, 1ull);
        if (k < AMF_SELFTEST_MAX_REPORT) {
          first_bad[3 * k] = q * 4u | (sgn ? 0x80000000u : 0u);
          first_bad[3 * k + 1] = want;
          first_bad[3 * k + 2] = got;
        }
      }
    }
  }
}

__global__ __launch_bounds__(256) void e4m3_encode_kernel(const float* __restrict__ x,
                                                          uint8_t* __restrict__ codes,
                                                          int64_t n) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t i = q * 4;
  if (i >= n) return;
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = (i + e < n) ? x[i + e] : 0.0f;
  const uint32_t w = f32x4_to_e4m3(v);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (i + e < n) codes[i + e] = (uint8_t)(w >> (8 * e));
}

}  // namespace

extern "C" int amf_selftest_e4m3_sweep(unsigned long long* mismatches, uint32_t* first_bad) {
  if (!mismatches || !first_bad) return -1;
  unsigned long long* d_bad = nullptr;
  uint32_t* d_first = nullptr;
  const size_t first_bytes = 3 * AMF_SELFTEST_MAX_REPORT * sizeof(uint32_t);
  hipError_t e = hipMalloc(&d_bad, sizeof(unsigned long long));
  if (e == hipSuccess) e = hipMalloc(&d_first, first_bytes);
  if (e == hipSuccess) e = hipMemset(d_bad, 0, sizeof(unsigned long long));
  if (e == hipSuccess) e = hipMemset(d_first, 0, first_bytes);
  if (e == hipSuccess) {
    const uint32_t n_quads = kMaxBits / 4u + 1u;  // covers 0 .. kMaxBits inclusive
    e4m3_sweep_kernel<<<16384, 256>>>(n_quads, d_bad, d_first);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess)
    e = hipMemcpy(mismatches, d_bad, sizeof(unsigned long long), hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(first_bad, d_first, first_bytes, hipMemcpyDeviceToHost);
  if (d_bad) (void)hipFree(d_bad);
  if (d_first) (void)hipFree(d_first);
  return e == hipSuccess ? 0 : (int)e;
}

extern "C" int amf_selftest_e4m3_encode(const float* x, uint8_t* codes, int64_t n, void* stream) {
  if (n < 0 || (n > 0 && (!x || !codes))) return -1;
  if (n == 0) return 0;
  const int64_t quads = (n + 3) / 4;
  const int64_t blocks = (quads + 255) / 256;
  if (blocks > 0x7FFFFFFF) return -1;
  e4m3_encode_kernel<<<(unsigned)blocks, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      x, codes, n);
  return (int)hipGetLastError();
}
