// amf_kernel_util.h - device-side building blocks shared by the codec and
// decode kernels: 16-element cache-row loads/stores, fp8/bf16/fp16
// conversions and division helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/amf_hip.h"
#include "amf_device.h"

namespace amf {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---- restore work mapping ------------------------------------------------------
// The FP8 and INT4-sym restores write whole pages at block-table-chosen
// places.  Their grid is 1-D: workgroup id runs on XCD id % 8 (round-robin
// dispatch), and xcd_page_work gives XCD x the contiguous eighth x of the
// plane-major (plane, page) list, so each XCD's in-flight pages come from one
// or two planes instead of from every plane.  The FP8 restore is launched
// with kRestoreLdsPad bytes of (unused) dynamic LDS, which holds a CU to
// three of its workgroups: fewer pages in flight per XCD, still enough bytes
// in flight for the HBM (the INT4 restores, which write four times what they
// read, lose with the pad).
constexpr unsigned kRestoreLdsPad = 52u << 10;

struct PageWork {
  int64_t j;   // position in the gathered sequence
  int plane;
  bool valid;  // false for the up to 7 padding workgroups
};

__host__ __device__ inline int64_t xcd_page_items_per_xcd(int64_t n_pages, int n_planes) {
  return (n_pages * n_planes + 7) / 8;
}

__device__ __forceinline__ PageWork xcd_page_work(int64_t n_pages, int n_planes) {
  const int64_t id = blockIdx.x;
  const int64_t w = (id & 7) * xcd_page_items_per_xcd(n_pages, n_planes) + (id >> 3);
  PageWork r;
  r.valid = w < n_pages * n_planes;
  r.plane = (int)(w / n_pages);
  r.j = w - (int64_t)r.plane * n_pages;
  return r;
}

inline dim3 xcd_page_grid(int64_t n_pages, int n_planes) {
  return dim3((unsigned)(8 * xcd_page_items_per_xcd(n_pages, n_planes)));
}

// ---- streaming loads / stores -------------------------------------------------
// Data read or written once per launch (codes, restored pages) goes through
// these; AMF_USE_NT selects the non-temporal cache policy.
#ifndef AMF_USE_NT
#define AMF_USE_NT 1
#endif

// Loads a restore lane keeps in flight before its stores.
#ifndef AMF_RESTORE_UNROLL
#define AMF_RESTORE_UNROLL 4
#endif

template <typename T>
__device__ __forceinline__ T ld_stream(const T* p) {
#if AMF_USE_NT
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

template <typename T>
__device__ __forceinline__ void st_stream(const T& v, T* p) {
#if AMF_USE_NT
  __builtin_nontemporal_store(v, p);
#else
  *p = v;
#endif
}

// ---- cache element <-> fp32 -------------------------------------------------

// Low / high 16-bit halves of a dword as fp32, for a bf16 or fp16 cache.
template <bool BF16>
__device__ __forceinline__ float half_lo(uint32_t w) {
  if constexpr (BF16) {
    return u2f(w << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
  }
}
template <bool BF16>
__device__ __forceinline__ float half_hi(uint32_t w) {
  if constexpr (BF16) {
    return u2f(w & 0xFFFF0000u);
  } else {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
}

// Keeps an fp32 value materialised: without it the compiler may fold a
// preceding multiply into the fp16 conversion (v_fma_mix*_f16 with a +0
// addend), which rounds once instead of fp32-then-fp16 and turns -0 into +0.
__device__ __forceinline__ void keep_f32(float& x) { asm("" : "+v"(x)); }

// Two fp32 -> one dword of cache elements, round to nearest even
// (v_cvt_pk_bf16_f32 for bf16, v_cvt_f16_f32 for fp16).
template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (!BF16) {
    keep_f32(a);
    keep_f32(b);
  }
  if constexpr (BF16) {
    uint32_t lo = __builtin_bit_cast(uint16_t, (__bf16)a);
    uint32_t hi = __builtin_bit_cast(uint16_t, (__bf16)b);
    return lo | (hi << 16);
  } else {
    uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)a);
    uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)b);
    return lo | (hi << 16);
  }
}

// 8 cache elements (one 16-byte vector) -> fp32.
template <bool BF16>
__device__ __forceinline__ void unpack8(const u32x4& v, float* x) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = half_lo<BF16>(v[i]);
    x[2 * i + 1] = half_hi<BF16>(v[i]);
  }
}

template <bool BF16>
__device__ __forceinline__ u32x4 pack8(const float* x) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack2<BF16>(x[2 * i], x[2 * i + 1]);
  return r;
}

// ---- cache elements of any AMF_DTYPE_* tag ----------------------------------

// Bytes per element of a cache dtype tag.
template <int DT>
__host__ __device__ constexpr int elem_bytes() {
  return DT == AMF_DTYPE_F32 ? 4 : 2;
}

// Eight consecutive cache elements at byte address p (aligned to 8 elements)
// -> fp32: one 16-byte vector for bf16/fp16, two for fp32.
template <int DT>
__device__ __forceinline__ void load8(const uint8_t* p, float* x) {
  if constexpr (DT == AMF_DTYPE_F32) {
    const f32x4 a = reinterpret_cast<const f32x4*>(p)[0];
    const f32x4 b = reinterpret_cast<const f32x4*>(p)[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = a[i];
      x[4 + i] = b[i];
    }
  } else {
    unpack8<DT == AMF_DTYPE_BF16>(*reinterpret_cast<const u32x4*>(p), x);
  }
}

// load8 for data read once (non-temporal loads where enabled): each load
// instruction of a wave covers whole cache lines when lanes take consecutive
// 8-element chunks.
template <int DT>
__device__ __forceinline__ void load8_stream(const uint8_t* p, float* x) {
  if constexpr (DT == AMF_DTYPE_F32) {
    const f32x4 a = ld_stream(reinterpret_cast<const f32x4*>(p));
    const f32x4 b = ld_stream(reinterpret_cast<const f32x4*>(p) + 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = a[i];
      x[4 + i] = b[i];
    }
  } else {
    unpack8<DT == AMF_DTYPE_BF16>(ld_stream(reinterpret_cast<const u32x4*>(p)), x);
  }
}

// fp32 -> eight cache elements at byte address p (streaming store; bf16/fp16
// round to nearest even).
template <int DT>
__device__ __forceinline__ void store8(uint8_t* p, const float* x) {
  if constexpr (DT == AMF_DTYPE_F32) {
    st_stream(f32x4{x[0], x[1], x[2], x[3]}, reinterpret_cast<f32x4*>(p));
    st_stream(f32x4{x[4], x[5], x[6], x[7]}, reinterpret_cast<f32x4*>(p) + 1);
  } else {
    st_stream(pack8<DT == AMF_DTYPE_BF16>(x), reinterpret_cast<u32x4*>(p));
  }
}

// ---- fp8 e4m3fn -------------------------------------------------------------

// Four e4m3 codes (one dword) -> fp32, exact.  Uses gfx950's OCP-format
// v_cvt_pk_f32_fp8 when AMF_FP8_HW_DECODE is set, otherwise the fp16
// widening trick of e4m3x2_to_f16x2_scaled with an explicit 2^8 rescale.
__device__ __forceinline__ void e4m3x4_to_f32(uint32_t w, float* out) {
#if AMF_FP8_HW_DECODE
  f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  out[0] = a[0];
  out[1] = a[1];
  out[2] = b[0];
  out[3] = b[1];
#else
  uint32_t lo = e4m3x2_to_f16x2_scaled(w & 0xFFFFu);
  uint32_t hi = e4m3x2_to_f16x2_scaled(w >> 16);
  out[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(lo & 0xFFFFu)) * 256.0f;
  out[1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(lo >> 16)) * 256.0f;
  out[2] = (float)__builtin_bit_cast(_Float16, (uint16_t)(hi & 0xFFFFu)) * 256.0f;
  out[3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(hi >> 16)) * 256.0f;
#endif
}

// Four fp32 (already clamped to [-448, 448]) -> four e4m3fn codes in a dword.
__device__ __forceinline__ uint32_t f32x4_to_e4m3(const float* x) {
#if AMF_FP8_HW_ENCODE
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], w, true);
  return (uint32_t)w;
#else
  return e4m3_from_f32(x[0]) | (e4m3_from_f32(x[1]) << 8) | (e4m3_from_f32(x[2]) << 16) |
         (e4m3_from_f32(x[3]) << 24);
#endif
}

// ---- division ---------------------------------------------------------------

// x / b rounded to nearest even (IEEE) for b > 0.  rb must be the correctly
// rounded reciprocal RN(1/b).  With AMF_MARKSTEIN_DIV the quotient comes from
// Markstein's sequence q = RN(x*rb), r = x - b*q (exact via fma),
// q' = RN(q + r*rb), which returns RN(x/b) for normal operands when rb is
// RN(1/b) (Markstein 1990; Muller et al., Handbook of Floating-Point
// Arithmetic, Thm. 4.10).  The sum q + r*rb turns x = -0 into +0, so the
// sign of x (the sign of the quotient, b being positive) is put back.
// Otherwise the compiler's correctly rounded divide.
__device__ __forceinline__ float div_rn(float x, float b, float rb) {
#if AMF_MARKSTEIN_DIV
  float q = x * rb;
  float r = __builtin_fmaf(-q, b, x);
  return __builtin_copysignf(__builtin_fmaf(r, rb, q), x);
#else
  (void)rb;
  return x / b;
#endif
}

// ---- small reductions -------------------------------------------------------

__device__ __forceinline__ float wave_max_xor(float v, int width) {
  for (int o = width / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, width));
  return v;
}

}  // namespace amf
