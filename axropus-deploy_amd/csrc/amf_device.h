// amf_device.h - scalar conversion helpers shared by the gfx950 kernels.
//
// Every helper is plain integer/float code, so the same definitions also
// compile as host C++ (g++).  The GPU tests check them against the oracle's
// independent encoders through the kernels and libamf_selftest.so, which also
// sweeps the e4m3 encoder against gfx950's conversion instruction.  Rounding
// is fixed by the functions themselves; kernels are compiled with
// -ffp-contract=off so that no multiply/add pair is silently fused.
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__) || defined(__HIP__)
#include <hip/hip_runtime.h>
#define AMF_HD __host__ __device__ __forceinline__
#else
#define AMF_HD static inline
#endif

namespace amf {

AMF_HD uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
AMF_HD float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// ---- bf16 / fp16 ----------------------------------------------------------

AMF_HD float bf16_to_f32(uint32_t b) { return u2f(b << 16); }

// fp32 -> bf16 bits, round to nearest even; NaN -> quiet NaN with the sign.
// (Same contract as PyTorch's CPU Tensor.to(torch.bfloat16).)
AMF_HD uint32_t f32_to_bf16_bits_sw(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) | 0x40u) & 0xFFFFu;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// ---- FP8 e4m3fn (OCP: bias 7, no infinities, S.1111.111 = NaN, max 448) ----

// fp32 -> e4m3fn code, round to nearest even with subnormals.  Magnitudes
// above 464 (including inf and NaN) give the NaN code S.1111.111, matching
// PyTorch's Tensor.to(torch.float8_e4m3fn) (c10 fp8e4m3fn_from_fp32_value).
AMF_HD uint32_t e4m3_from_f32(float f) {
  uint32_t u = f2u(f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x43E80000u) return sign | 0x7Fu;  // > 464.0, inf, NaN
  if (a < 0x3C800000u) {                     // < 2^-6: subnormal step 2^-9
    float r = __builtin_rintf(u2f(a) * 512.0f);
    return sign | (uint32_t)r;               // r == 8 is the smallest normal
  }
  // Normal: rebias the exponent (127 -> 7) and round the 23-bit mantissa to
  // 3 bits, ties to even; a carry moves into the exponent field.
  uint32_t odd = (a >> 20) & 1u;
  return sign | ((a - (120u << 23) + 0x7FFFFu + odd) >> 20);
}

// e4m3fn code -> fp32 (exact).  NaN codes give a quiet NaN.
AMF_HD float f32_from_e4m3(uint32_t c) {
  uint32_t sign = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xFu;
  uint32_t m = c & 7u;
  if (e == 0) return u2f(sign | f2u((float)m * 0.001953125f));  // m * 2^-9
  if ((c & 0x7Fu) == 0x7Fu) return u2f(sign | 0x7FC00000u);
  return u2f(sign | ((e + 120u) << 23) | (m << 20));
}

// Two e4m3 codes (bits 0-7 and 8-15 of `pair`) -> the fp16 bit patterns of
// code_value * 2^-8.  e4m3's exponent bias (7) is 8 below fp16's (15), so the
// 7 magnitude bits drop into the fp16 exponent/mantissa fields unchanged and
// e4m3 subnormals land on fp16 subnormals: the fp16 value is exact.  A caller
// multiplies the widened value by scale * 256, which gives the same fp32
// rounding as code_value * scale (power-of-two rescaling is exact).  Only the
// NaN codes differ (they decode to 480 * scale instead of NaN); the encoder
// never produces them from finite inputs.
AMF_HD uint32_t e4m3x2_to_f16x2_scaled(uint32_t pair) {
  uint32_t mag = ((pair & 0x007Fu) << 7) | ((pair & 0x7F00u) << 15);
  uint32_t sgn = ((pair & 0x0080u) << 8) | ((pair & 0x8000u) << 16);
  return mag | sgn;
}

}  // namespace amf
