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

// ---------------------------------------------------------------- slots --
//
// Token-slot form of the same copy: the unit is one token row (H*D elements,
// row_bytes bytes) of a cache plane addressed by a vLLM slot id, slot =
// block * block_size + offset.  The cache row sits at
//   plane + (slot / block_size) * page_stride + (slot % block_size) * row_bytes
// and the dense side row r at plane + r * row_stride.
//
// A row is LPR lanes wide (the power of two >= row_bytes / 16, at most a
// wave), so one wave moves 64 / LPR rows at once and a short row (256 B for
// 2 heads x 64 x bf16) still fills the wave; kRowUnroll rows per lane group
// keep several 16-byte loads in flight before their stores.
constexpr int kRowUnroll = 4;

template <int LPR>
__global__ __launch_bounds__(kThreads) void slot_copy_kernel(
    const uint64_t* __restrict__ src_planes, const int64_t* __restrict__ src_slots,
    int64_t src_page_stride, int32_t src_block, int64_t src_rows,
    const uint64_t* __restrict__ dst_planes, const int64_t* __restrict__ dst_slots,
    int64_t dst_page_stride, int32_t dst_block, int64_t dst_rows, int64_t n_rows,
    int64_t row_bytes, int32_t* err_flag) {
  constexpr int kRowsPerTrip = kThreads / LPR;
  const int sub = threadIdx.x % LPR;
  const int grp = threadIdx.x / LPR;
  const int plane = blockIdx.y;
  const char* sbase = reinterpret_cast<const char*>(src_planes[plane]);
  char* dbase = reinterpret_cast<char*>(dst_planes[plane]);
  const int n16 = (int)(row_bytes / 16);
  const int64_t step = (int64_t)gridDim.x * kRowsPerTrip * kRowUnroll;
  for (int64_t r0 = (int64_t)blockIdx.x * kRowsPerTrip * kRowUnroll; r0 < n_rows; r0 += step) {
    const u32x4* s[kRowUnroll];
    u32x4* d[kRowUnroll];
    bool live[kRowUnroll];
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t r = r0 + (int64_t)u * kRowsPerTrip + grp;
      live[u] = false;
      s[u] = nullptr;
      d[u] = nullptr;
      if (r < n_rows) {
        const int64_t ss = src_slots ? src_slots[r] : r;
        const int64_t ds = dst_slots ? dst_slots[r] : r;
        if (ss < 0 || ss >= src_rows || ds < 0 || ds >= dst_rows) {
          if (sub == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
        } else {
          live[u] = true;
          s[u] = reinterpret_cast<const u32x4*>(
              sbase + (ss / src_block) * src_page_stride + (ss % src_block) * row_bytes);
          d[u] = reinterpret_cast<u32x4*>(dbase + (ds / dst_block) * dst_page_stride +
                                          (ds % dst_block) * row_bytes);
        }
      }
    }
    for (int k = sub; k < n16; k += LPR) {
      u32x4 v[kRowUnroll];
#pragma unroll
      for (int u = 0; u < kRowUnroll; ++u)
        if (live[u]) v[u] = ld_stream(s[u] + k);
#pragma unroll
      for (int u = 0; u < kRowUnroll; ++u)
        if (live[u]) st_stream(v[u], d[u] + k);
    }
  }
}

struct SlotSide {
  const uint64_t* planes;
  const int64_t* slots;  // nullptr: dense rows 0..n_rows-1
  int64_t page_stride;   // bytes between pages (dense side: the row stride)
  int32_t block;         // rows per page (dense side: 1)
  int64_t rows;          // rows addressable in each plane
};

int launch_slots(const char* who, SlotSide src, SlotSide dst, int32_t n_planes, int64_t n_rows,
                 int64_t row_bytes, int32_t* err_flag, void* stream) {
  using namespace amf;
  if (!src.planes || !dst.planes) return fail(AMF_ERR_INVALID_ARG, "%s: null plane array", who);
  if (n_planes <= 0 || n_planes > 65535 || n_rows < 0)
    return fail(AMF_ERR_INVALID_ARG, "%s: bad n_planes=%d n_slots=%lld", who, n_planes,
                (long long)n_rows);
  if (row_bytes <= 0 || !aligned16(row_bytes) || row_bytes / 16 > 0x7FFFFFFF)
    return fail(AMF_ERR_INVALID_ARG, "%s: row_bytes=%lld must be a positive multiple of 16", who,
                (long long)row_bytes);
  for (const SlotSide* side : {&src, &dst}) {
    if (side->block <= 0 || side->rows <= 0)
      return fail(AMF_ERR_INVALID_ARG, "%s: block_size and pool_slots must be positive", who);
    if (!aligned16(side->page_stride) || side->page_stride < (int64_t)side->block * row_bytes)
      return fail(AMF_ERR_INVALID_ARG,
                  "%s: page stride %lld must be a multiple of 16 holding %d rows of %lld bytes",
                  who, (long long)side->page_stride, side->block, (long long)row_bytes);
  }
  if (n_rows == 0) return ok();
  const int64_t n16 = row_bytes / 16;
  int lpr = 1;
  while (lpr < n16 && lpr < 64) lpr *= 2;
  const int64_t rows_per_block = (int64_t)(kThreads / lpr) * kRowUnroll;
  const int64_t blocks = (n_rows + rows_per_block - 1) / rows_per_block;
  dim3 grid((unsigned)std::min<int64_t>(blocks, 1 << 20), (unsigned)n_planes);
  hipStream_t s = as_stream(stream);
#define AMF_SLOT_LAUNCH(L)                                                                     \
  slot_copy_kernel<L><<<grid, kThreads, 0, s>>>(src.planes, src.slots, src.page_stride,        \
                                                src.block, src.rows, dst.planes, dst.slots,    \
                                                dst.page_stride, dst.block, dst.rows, n_rows,  \
                                                row_bytes, err_flag)
  switch (lpr) {
    case 1: AMF_SLOT_LAUNCH(1); break;
    case 2: AMF_SLOT_LAUNCH(2); break;
    case 4: AMF_SLOT_LAUNCH(4); break;
    case 8: AMF_SLOT_LAUNCH(8); break;
    case 16: AMF_SLOT_LAUNCH(16); break;
    case 32: AMF_SLOT_LAUNCH(32); break;
    default: AMF_SLOT_LAUNCH(64); break;
  }
#undef AMF_SLOT_LAUNCH
  return check_launch(who);
}

}  // namespace

extern "C" int amf_kv_gather_slots(const uint64_t* cache_planes, int64_t cache_page_stride,
                                   int32_t block_size, const int64_t* slot_mapping,
                                   int64_t pool_slots, const uint64_t* out_planes,
                                   int64_t out_row_stride, int32_t n_planes, int64_t n_slots,
                                   int64_t row_bytes, int32_t* err_flag, void* stream) {
  if (!slot_mapping && n_slots > 0)
    return amf::fail(AMF_ERR_INVALID_ARG, "amf_kv_gather_slots: null slot_mapping");
  return launch_slots("amf_kv_gather_slots",
                      {cache_planes, slot_mapping, cache_page_stride, block_size, pool_slots},
                      {out_planes, nullptr, out_row_stride, 1, INT64_MAX}, n_planes, n_slots,
                      row_bytes, err_flag, stream);
}

extern "C" int amf_kv_scatter_slots(const uint64_t* in_planes, int64_t in_row_stride,
                                    const uint64_t* cache_planes, int64_t cache_page_stride,
                                    int32_t block_size, const int64_t* slot_mapping,
                                    int64_t pool_slots, int32_t n_planes, int64_t n_slots,
                                    int64_t row_bytes, int32_t* err_flag, void* stream) {
  if (!slot_mapping && n_slots > 0)
    return amf::fail(AMF_ERR_INVALID_ARG, "amf_kv_scatter_slots: null slot_mapping");
  return launch_slots("amf_kv_scatter_slots", {in_planes, nullptr, in_row_stride, 1, INT64_MAX},
                      {cache_planes, slot_mapping, cache_page_stride, block_size, pool_slots},
                      n_planes, n_slots, row_bytes, err_flag, stream);
}

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
