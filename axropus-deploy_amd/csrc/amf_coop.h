// amf_coop.h - the work map, loads and launch sizing of the single-read
// per-tensor FP8 save: a cooperative grid walks the scale groups in order
// and holds each workgroup's share of a group in registers from load to
// store, while the group's absmax is exchanged between workgroups.
//
// Work map: a scale group is pps planes of n_pages pages.  Workgroup b holds
// pages b, b + G, b + 2G, ... of the group (G workgroups, at most ppw pages
// each); its lanes hold CPT 16-byte chunks of each page (tid + 256 m), so
// page addresses are workgroup-uniform and a lane's chunks of a page are
// 4 KiB apart.  Exchange lines: per group, kCoopClusters + 1 lines of 128
// bytes (kLineWords words), each on its own line because device-scope
// atomics on one line serialize; workgroup b reports to cluster
// b % kCoopClusters, the last line is the group's root.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <map>
#include <mutex>
#include <utility>

#include "amf_internal.h"
#include "amf_kernel_util.h"

namespace amf {

constexpr int kCoopChunks = 16;   // 16-byte chunks per lane per register buffer
constexpr int kCoopThreads = 256;
constexpr uint32_t kCoopSpinLimit = 1u << 20;  // polls before a wait gives up
constexpr int kCoopClusters = kFp8CoopClusters;
constexpr int kLineWords = kFp8CoopLineWords;
constexpr uint32_t kReady = 0x80000000u;  // above every non-negative float's bits

struct CoopGeom {
  const uint64_t* cache_planes;
  int64_t cache_stride;
  const int32_t* block_ids;
  int64_t pool;
  int64_t n_pages;
  int64_t group_pages;  // pps * n_pages
  int pps;
  int n_groups;
  int ppw;              // pages per workgroup per group
  uint32_t spin_limit;  // polls before a wait gives up (coop_spin_limit())
  int32_t* err_flag;
};

// kCoopSpinLimit, or AMF_COOP_SPIN_LIMIT from the environment (read once):
// the tests set it to 0 to drive every wait down its give-up path, which
// must leave the kernel to finish normally with its group scales poisoned.
inline uint32_t coop_spin_limit() {
  static const uint32_t limit = [] {
    const char* e = getenv("AMF_COOP_SPIN_LIMIT");
    return e ? (uint32_t)strtoul(e, nullptr, 10) : kCoopSpinLimit;
  }();
  return limit;
}

// AMF_NO_COOP set to a non-zero value in the environment (read once) turns
// the cooperative launches off: per-tensor FP8 saves then take the two-pass
// kernels.  For processes that cannot have a cooperative launch (a profiler
// that does not survive one, a caller capturing into a graph).
inline bool coop_disabled() {
  static const bool off = [] {
    const char* e = getenv("AMF_NO_COOP");
    return e && strtol(e, nullptr, 10) != 0;
  }();
  return off;
}

__device__ __forceinline__ uint32_t* coop_line(uint32_t* sync, int gi, int k) {
  return sync + ((int64_t)gi * (kCoopClusters + 1) + k) * kLineWords;
}

// Page i of this workgroup in group gi: its plane and gathered position,
// whether it exists, and whether it also has an in-range block id (sp).
struct CoopPage {
  bool exists;
  bool ok;
  int plane;
  int64_t j;
  int64_t sp;
};

__device__ __forceinline__ CoopPage coop_page(const CoopGeom& a, int gi, int i) {
  CoopPage r;
  const int64_t pg = blockIdx.x + (int64_t)i * gridDim.x;
  r.exists = i < a.ppw && pg < a.group_pages;
  r.ok = r.exists;
  r.plane = 0;
  r.j = 0;
  r.sp = -1;
  if (r.exists) {
    const int pl = (int)(pg / a.n_pages);
    r.plane = gi * a.pps + pl;
    r.j = pg - (int64_t)pl * a.n_pages;
    r.sp = a.block_ids ? (int64_t)a.block_ids[r.j] : r.j;
    r.ok = r.sp >= 0 && r.sp < a.pool;
  }
  return r;
}

// Loads the workgroup's pages of group gi; absent pages and pages whose
// block id is out of range read as zero (and are never stored).
template <int CPT>
__device__ __forceinline__ void coop_load(const CoopGeom& a, int gi, u32x4 (&buf)[kCoopChunks]) {
#pragma unroll
  for (int i = 0; i < kCoopChunks / CPT; ++i) {
    const CoopPage q = coop_page(a, gi, i);
    if (q.ok) {
      const u32x4* src = reinterpret_cast<const u32x4*>(
          reinterpret_cast<const uint8_t*>(a.cache_planes[q.plane]) + q.sp * a.cache_stride);
#pragma unroll
      for (int m = 0; m < CPT; ++m)
        buf[i * CPT + m] = ld_stream(src + threadIdx.x + kCoopThreads * m);
    } else {
#pragma unroll
      for (int m = 0; m < CPT; ++m) buf[i * CPT + m] = u32x4{0u, 0u, 0u, 0u};
      if (q.exists && threadIdx.x == 0 && a.err_flag) atomicOr(a.err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    }
  }
}

// |x| of a bf16 / fp16 element as its 16-bit pattern with the sign cleared:
// for non-NaN values these order as the magnitudes do; NaN patterns (above
// the infinity pattern) become 0, as fmaxf drops NaN in the two-pass kernels.
template <int DT>
__device__ __forceinline__ uint32_t abs_bits16(uint32_t h) {
  constexpr uint32_t kInf = DT == AMF_DTYPE_BF16 ? 0x7F80u : 0x7C00u;
  const uint32_t a = h & 0x7FFFu;
  return a > kInf ? 0u : a;
}

// Workgroups of a cooperative kernel that the current device keeps resident
// at once (0: no cooperative launch).  Queried once per (device, kernel).
inline int coop_blocks(const void* fn) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, int> cache;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(dev, fn);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int coop = 0, cus = 0, per_cu = 0;
  hipError_t e = hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kCoopThreads, 0);
  if (e != hipSuccess) (void)hipGetLastError();
  const int blocks = (e == hipSuccess && coop) ? per_cu * cus : 0;
  cache[key] = blocks;
  return blocks;
}

// Smallest scale group (bytes of cache read) worth the cooperative path: a
// smaller group's exchange costs more than its second read.
constexpr int64_t kCoopMinGroupBytes = 4ll << 20;

}  // namespace amf
