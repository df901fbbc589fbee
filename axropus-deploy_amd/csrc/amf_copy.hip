// amf_copy.hip - raw paged gather / scatter (bit copies of whole pages).
//
// Replaces the advanced-index copies k_all[ids] and k_all[ids] = src of
// korith_vllm_ext/compressed_vram_pool.py:491-504, 599-606 and
// korith_vllm_ext/amf_kv_manager.py:311-318, 505-523.
//
// One workgroup moves one page of one plane: grid = (pages, planes).  The
// block id is wave-uniform (scalar load); every lane moves 16-byte vectors,
// UNROLL loads in flight before the matching stores, so a 4 KiB page is one
// trip of 256 lanes and a 32 KiB page four trips of two batches.
#include "amf_internal.h"
#include "amf_kernel_util.h"

namespace {

using amf::u32x4;
using amf::ld_stream;
using amf::st_stream;

constexpr int kThreads = 256;
constexpr int kUnroll = AMF_RESTORE_UNROLL;

__global__ __launch_bounds__(kThreads) void page_copy_kernel(
    const uint64_t* __restrict__ src_planes, int64_t src_stride, const int32_t* __restrict__ src_ids,
    int64_t src_pool, const uint64_t* __restrict__ dst_planes, int64_t dst_stride,
    const int32_t* __restrict__ dst_ids, int64_t dst_pool, int64_t n16, int32_t* err_flag) {
  const int64_t j = blockIdx.x;
  const int plane = blockIdx.y;
  const int64_t sp = src_ids ? (int64_t)src_ids[j] : j;
  const int64_t dp = dst_ids ? (int64_t)dst_ids[j] : j;
  if (sp < 0 || sp >= src_pool || dp < 0 || dp >= dst_pool) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  const u32x4* __restrict__ s =
      reinterpret_cast<const u32x4*>(src_planes[plane] + (uint64_t)(sp * src_stride));
  u32x4* __restrict__ d = reinterpret_cast<u32x4*>(dst_planes[plane] + (uint64_t)(dp * dst_stride));
  for (int64_t base = threadIdx.x; base < n16; base += kThreads * kUnroll) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int64_t k = base + (int64_t)u * kThreads;
      if (k < n16) v[u] = ld_stream(s + k);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int64_t k = base + (int64_t)u * kThreads;
      if (k < n16) st_stream(v[u], d + k);
    }
  }
}

int launch_copy(const char* who, const uint64_t* src_planes, int64_t src_stride,
                const int32_t* src_ids, int64_t src_pool, const uint64_t* dst_planes,
                int64_t dst_stride, const int32_t* dst_ids, int64_t dst_pool, int32_t n_planes,
                int64_t n_pages, int64_t page_bytes, int32_t* err_flag, void* stream) {
  using namespace amf;
  if (!src_planes || !dst_planes) return fail(AMF_ERR_INVALID_ARG, "%s: null plane array", who);
  if (n_planes <= 0 || n_planes > 65535 || n_pages < 0 || n_pages > 0x7FFFFFFF)
    return fail(AMF_ERR_INVALID_ARG, "%s: bad n_planes=%d n_pages=%lld", who, n_planes,
                (long long)n_pages);
  if (page_bytes <= 0 || !aligned16(page_bytes) || !aligned16(src_stride) ||
      !aligned16(dst_stride) || src_stride < page_bytes || dst_stride < page_bytes)
    return fail(AMF_ERR_INVALID_ARG,
                "%s: page_bytes=%lld and strides (%lld, %lld) must be positive multiples of 16 "
                "with stride >= page_bytes",
                who, (long long)page_bytes, (long long)src_stride, (long long)dst_stride);
  if (src_pool <= 0 || dst_pool <= 0)
    return fail(AMF_ERR_INVALID_ARG, "%s: pool_pages must be positive", who);
  if (n_pages == 0) return ok();
  dim3 grid((unsigned)n_pages, (unsigned)n_planes);
  page_copy_kernel<<<grid, kThreads, 0, as_stream(stream)>>>(
      src_planes, src_stride, src_ids, src_pool, dst_planes, dst_stride, dst_ids, dst_pool,
      page_bytes / 16, err_flag);
  return check_launch(who);
}

}  // namespace

extern "C" int amf_kv_gather_pages(const uint64_t* cache_planes, int64_t cache_page_stride,
                                   const int32_t* block_ids, int64_t pool_pages,
                                   const uint64_t* out_planes, int64_t out_page_stride,
                                   int32_t n_planes, int64_t n_pages, int64_t page_bytes,
                                   int32_t* err_flag, void* stream) {
  return launch_copy("amf_kv_gather_pages", cache_planes, cache_page_stride, block_ids,
                     pool_pages, out_planes, out_page_stride, nullptr, INT64_MAX, n_planes,
                     n_pages, page_bytes, err_flag, stream);
}

extern "C" int amf_kv_scatter_pages(const uint64_t* in_planes, int64_t in_page_stride,
                                    const uint64_t* cache_planes, int64_t cache_page_stride,
                                    const int32_t* block_ids, int64_t pool_pages,
                                    int32_t n_planes, int64_t n_pages, int64_t page_bytes,
                                    int32_t* err_flag, void* stream) {
  return launch_copy("amf_kv_scatter_pages", in_planes, in_page_stride, nullptr, INT64_MAX,
                     cache_planes, cache_page_stride, block_ids, pool_pages, n_planes, n_pages,
                     page_bytes, err_flag, stream);
}
