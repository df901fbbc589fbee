// amf_internal.h - host-side plumbing shared by the libamf_hip.so sources:
// per-thread error text, argument checks and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/amf_hip.h"

namespace amf {

// Records `code` with a printf-style message for amf_last_error() and returns
// it, so call sites read `return fail(AMF_ERR_INVALID_ARG, "...")`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the calling thread's error text; returns AMF_OK.
int ok();

// Checks hipGetLastError() after a launch.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(int64_t v) { return (v & 15) == 0; }

// Cache element size in bytes for an AMF_DTYPE_* tag; 0 if not a cache dtype
// the codecs accept (bf16, fp16, fp32).
inline int cache_elem_bytes(int32_t dtype) {
  if (dtype == AMF_DTYPE_BF16 || dtype == AMF_DTYPE_F16) return 2;
  return dtype == AMF_DTYPE_F32 ? 4 : 0;
}

// Runs the statements after `dt` with `constexpr int DT` bound to the cache
// dtype tag `dt` (validated beforehand by check_codec_geometry).
#define AMF_WITH_DTYPE(dt, ...)                                       \
  do {                                                                \
    if ((dt) == AMF_DTYPE_BF16) {                                     \
      constexpr int DT = AMF_DTYPE_BF16;                              \
      __VA_ARGS__;                                                    \
    } else if ((dt) == AMF_DTYPE_F16) {                               \
      constexpr int DT = AMF_DTYPE_F16;                               \
      __VA_ARGS__;                                                    \
    } else {                                                          \
      constexpr int DT = AMF_DTYPE_F32;                               \
      __VA_ARGS__;                                                    \
    }                                                                 \
  } while (0)

// Per-tensor FP8 save workspace (words): the n_groups absmax slots, then,
// on a 128-byte line boundary, kFp8CoopClusters + 1 lines per group for the
// single-read kernel's cross-workgroup exchange.
constexpr int kFp8CoopClusters = 32;
constexpr int kFp8CoopLineWords = 32;
inline int64_t fp8_tensor_sync_offset(int64_t n_groups) {
  return (n_groups + kFp8CoopLineWords - 1) / kFp8CoopLineWords * kFp8CoopLineWords;
}
inline int64_t fp8_tensor_workspace_words(int64_t n_groups) {
  return fp8_tensor_sync_offset(n_groups) + n_groups * (kFp8CoopClusters + 1) * kFp8CoopLineWords;
}

// Common validation of the paged-geometry arguments of the codec entry points.
int check_codec_geometry(const char* who, const uint64_t* cache_planes,
                         int64_t cache_page_stride, int32_t cache_dtype,
                         const int32_t* block_ids, int64_t pool_pages,
                         const uint64_t* code_planes, const uint64_t* param_planes,
                         int32_t n_planes, int64_t n_pages, int32_t block_size,
                         int32_t num_heads, int32_t head_dim);

}  // namespace amf
