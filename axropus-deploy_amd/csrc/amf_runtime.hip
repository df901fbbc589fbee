// amf_runtime.hip - version, error reporting and argument validation of the
// libamf_hip.so C ABI.  Error convention after korith_c_api/korith.h:10-20
// (negative return on failure) with a thread-local message instead of stderr.
#include <stdarg.h>
#include <stdio.h>

#include "amf_internal.h"

namespace amf {

static thread_local char g_last_error[512];

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_last_error[0] = '\0';
  return AMF_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(AMF_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

int check_codec_geometry(const char* who, const uint64_t* cache_planes,
                         int64_t cache_page_stride, int32_t cache_dtype,
                         const int32_t* block_ids, int64_t pool_pages,
                         const uint64_t* code_planes, const uint64_t* param_planes,
                         int32_t n_planes, int64_t n_pages, int32_t block_size,
                         int32_t num_heads, int32_t head_dim) {
  (void)block_ids;
  if (!cache_planes || !code_planes || !param_planes)
    return fail(AMF_ERR_INVALID_ARG, "%s: null plane array", who);
  if (n_planes <= 0 || n_planes > 65535 || n_pages < 0)
    return fail(AMF_ERR_INVALID_ARG, "%s: bad n_planes=%d / n_pages=%lld", who, n_planes,
                (long long)n_pages);
  if (block_size <= 0 || num_heads <= 0 || head_dim <= 0)
    return fail(AMF_ERR_INVALID_ARG, "%s: bad geometry bs=%d H=%d D=%d", who, block_size,
                num_heads, head_dim);
  const int es = cache_elem_bytes(cache_dtype);
  if (es == 0)
    return fail(AMF_ERR_UNSUPPORTED, "%s: cache dtype %d is not bf16/fp16/fp32", who, cache_dtype);
  if (head_dim % 32 != 0)
    return fail(AMF_ERR_UNSUPPORTED, "%s: head_dim %d is not a multiple of 32", who, head_dim);
  int64_t page_elems = (int64_t)block_size * num_heads * head_dim;
  if (cache_page_stride < page_elems * es || !aligned16(cache_page_stride))
    return fail(AMF_ERR_INVALID_ARG, "%s: cache page stride %lld < page bytes %lld or unaligned",
                who, (long long)cache_page_stride, (long long)(page_elems * es));
  if (pool_pages <= 0 || pool_pages > 0x7FFFFFFF)
    return fail(AMF_ERR_INVALID_ARG, "%s: bad pool_pages %lld", who, (long long)pool_pages);
  if (n_pages > 0x7FFFFFFF) return fail(AMF_ERR_UNSUPPORTED, "%s: n_pages too large", who);
  return ok();
}

}  // namespace amf

extern "C" int amf_abi_version(void) { return AMF_ABI_VERSION; }

extern "C" const char* amf_last_error(void) { return amf::g_last_error; }

extern "C" int64_t amf_quant_workspace_bytes(int32_t format, int32_t n_planes,
                                             int32_t planes_per_scale, int32_t head_dim) {
  if (n_planes <= 0 || planes_per_scale <= 0) return 0;
  const int64_t n_groups = (n_planes + planes_per_scale - 1) / planes_per_scale;
  switch (format) {
    case AMF_FMT_FP8_E4M3: return amf::fp8_tensor_workspace_words(n_groups) * (int64_t)sizeof(float);
    case AMF_FMT_INT4_SYM: return n_groups * (int64_t)head_dim * (int64_t)sizeof(float);
    default: return 0;
  }
}

// ---- prefix keys (host) -------------------------------------------------------
// FNV-1a with the store's offset basis 1469598103934665603 (core/amf_store.cpp:27,
// amf_kv_manager.py:38) and the 64-bit FNV prime.

namespace {
constexpr uint64_t kFnvOffset = 1469598103934665603ull;
constexpr uint64_t kFnvPrime = 1099511628211ull;
}  // namespace

extern "C" uint64_t amf_fnv1a64(const void* data, int64_t n_bytes, uint64_t h) {
  const uint8_t* p = static_cast<const uint8_t*>(data);
  for (int64_t i = 0; i < n_bytes; ++i) h = (h ^ p[i]) * kFnvPrime;
  return h;
}

extern "C" uint64_t amf_hash_tokens(const int32_t* tokens, int64_t n_tokens) {
  uint64_t h = kFnvOffset;
  for (int64_t i = 0; i < n_tokens; ++i) h = (h ^ (uint64_t)(uint32_t)tokens[i]) * kFnvPrime;
  return h;
}
