// amf_fp8.hip - FP8 e4m3fn codec of the compressed VRAM pool, fused with the
// paged gather (save) and the paged scatter (restore).
//
// Replaces, per layer of compressed_vram_pool.py:481-508 / 579-606, the torch
// op chains of FP8E4M3Codec.compress / decompress_to
// (korith_vllm_ext/codecs/amf_codec.py:182-222): one pass over HBM instead of
// gather -> stack -> abs/amax -> float -> divide -> clamp -> cast.
//
// Work split: one 256-lane workgroup per (page, plane).  A page is n_rows =
// block_size * num_heads rows of head_dim elements; lane `tid` owns the
// 16-element column chunk (tid % (head_dim/16)) of rows tid / (head_dim/16),
// + rows_per_iter, ...  Code chunks are 16-byte loads/stores, cache chunks two
// 16-byte vectors.
#include "amf_coop.h"
#include "amf_internal.h"
#include "amf_kernel_util.h"

namespace {

using namespace amf;

constexpr int kThreads = 256;
constexpr int kMaxRowsPerLane = 16;  // page rows a lane may keep in registers on save

// The floor clamp_min_(1e-8) applies in the tensor's own dtype
// (amf_codec.py:183): bf16(1e-8) (these bits), fp16(1e-8) = 0, fp32(1e-8).
constexpr uint32_t kBf16FloorBits = 0x322C0000u;
constexpr float kFp8Max = 448.0f;

struct PageGeom {
  int n_rows;        // block_size * num_heads
  int head_dim;
  int num_heads;
  int cpr_log2;      // log2(head_dim / 16)
  int head_const;    // rows_per_iter % num_heads == 0: a lane's head never changes
  int pps;           // planes per scale group (per-tensor format)
};

__device__ __forceinline__ int lane_col(const PageGeom& g) { return threadIdx.x & ((1 << g.cpr_log2) - 1); }
__device__ __forceinline__ int lane_row0(const PageGeom& g) { return threadIdx.x >> g.cpr_log2; }
__device__ __forceinline__ int rows_per_iter(const PageGeom& g) { return kThreads >> g.cpr_log2; }

template <int DT>
__device__ __forceinline__ float tensor_floor() {
  if constexpr (DT == AMF_DTYPE_BF16) {
    return u2f(kBf16FloorBits);
  } else if constexpr (DT == AMF_DTYPE_F16) {
    return 0.0f;
  } else {
    return 1e-8f;
  }
}

template <bool BF16>
constexpr int dtype_of() {
  return BF16 ? AMF_DTYPE_BF16 : AMF_DTYPE_F16;
}

// ---------------------------------------------------------------- restore --

// One lane = one 8-element chunk (8 code bytes in, one 16-byte vector of
// cache elements out), so each wave-wide store covers 1 KiB contiguously and
// every cache line is written whole.  The chunk's head is fixed per lane when
// 2048 elements (one workgroup pass) span whole rows of heads.
template <int DT, bool PER_TENSOR>
__global__ __launch_bounds__(kThreads) void fp8_dequant_scatter_kernel(
    const uint64_t* __restrict__ code_planes, const uint64_t* __restrict__ param_planes,
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, int64_t n_pages, int n_planes,
    PageGeom g, int32_t* err_flag) {
  const PageWork pw = xcd_page_work(n_pages, n_planes);
  if (!pw.valid) return;
  const int64_t j = pw.j;
  const int plane = pw.plane;
  const int64_t dp = block_ids ? (int64_t)block_ids[j] : j;
  if (dp < 0 || dp >= pool) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  const int page_elems = g.n_rows * g.head_dim;
  const int n8 = page_elems >> 3;
  const uint8_t* __restrict__ codes =
      reinterpret_cast<const uint8_t*>(code_planes[plane]) + j * (int64_t)page_elems;
  const float* __restrict__ params = reinterpret_cast<const float*>(param_planes[plane]);
  uint8_t* __restrict__ out = reinterpret_cast<uint8_t*>(cache_planes[plane]) + dp * cache_stride;
  const float* __restrict__ page_scales = params + j * g.num_heads;
  const int tid = threadIdx.x;
  float s_fixed = 0.0f;
  if (PER_TENSOR)
    s_fixed = params[plane & 1];
  else if (g.head_const)
    s_fixed = page_scales[((tid * 8) / g.head_dim) % g.num_heads];

  constexpr int U = AMF_RESTORE_UNROLL;
  for (int base = tid; base < n8; base += U * kThreads) {
    u32x2 c[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = base + u * kThreads;
      if (k < n8) c[u] = ld_stream(reinterpret_cast<const u32x2*>(codes) + k);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = base + u * kThreads;
      if (k < n8) {
        const float s = (PER_TENSOR || g.head_const)
                            ? s_fixed
                            : page_scales[((k * 8) / g.head_dim) % g.num_heads];
        float x[8];
        e4m3x4_to_f32(c[u][0], x);
        e4m3x4_to_f32(c[u][1], x + 4);
#pragma unroll
        for (int q = 0; q < 8; ++q) x[q] = x[q] * s;
        store8<DT>(out + (int64_t)k * (8 * elem_bytes<DT>()), x);
      }
    }
  }
}

// ------------------------------------------------------------------- save --

// Per-tensor absmax (first of the three per-tensor save kernels): each
// workgroup folds a strided set of one plane's pages, then sends its max to
// the scale group's slot ws[plane / pps] by one integer atomic max on the
// non-negative float's bit pattern.  All groups' slots share a cache line, so
// the workgroup count (kAbsBlocks over all planes) bounds the atomics that
// line serializes.  A page's rows are contiguous: it is read as a flat run of
// 16-byte vectors, kAbsUnroll of them in flight per lane before any is
// reduced.
constexpr int kAbsUnroll = 8;
constexpr int kAbsBlocks = 2048;

template <int DT>
__device__ __forceinline__ float absmax16(const u32x4& v, float m) {
  if constexpr (DT == AMF_DTYPE_F32) {
#pragma unroll
    for (int q = 0; q < 4; ++q) m = fmaxf(m, fabsf(u2f(v[q])));
  } else {
    float x[8];
    unpack8<DT == AMF_DTYPE_BF16>(v, x);
#pragma unroll
    for (int q = 0; q < 8; ++q) m = fmaxf(m, fabsf(x[q]));
  }
  return m;
}

template <int DT>
__global__ __launch_bounds__(kThreads) void fp8_absmax_kernel(
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, int64_t n_pages, PageGeom g,
    uint32_t* ws, int32_t* err_flag) {
  const int plane = blockIdx.y;
  const int n16 = g.n_rows * g.head_dim * elem_bytes<DT>() / 16;
  float m = 0.0f;
  for (int64_t j = blockIdx.x; j < n_pages; j += gridDim.x) {
    const int64_t sp = block_ids ? (int64_t)block_ids[j] : j;
    if (sp < 0 || sp >= pool) {
      if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
      continue;
    }
    const u32x4* __restrict__ src = reinterpret_cast<const u32x4*>(
        reinterpret_cast<const uint8_t*>(cache_planes[plane]) + sp * cache_stride);
    for (int base = threadIdx.x; base < n16; base += kThreads * kAbsUnroll) {
      u32x4 v[kAbsUnroll];
#pragma unroll
      for (int u = 0; u < kAbsUnroll; ++u) {
        const int k = base + u * kThreads;
        if (k < n16) v[u] = ld_stream(src + k);
      }
#pragma unroll
      for (int u = 0; u < kAbsUnroll; ++u)
        if (base + u * kThreads < n16) m = absmax16<DT>(v[u], m);
    }
  }
  m = wave_max_xor(m, 64);
  __shared__ uint32_t s_max;
  if (threadIdx.x == 0) s_max = 0;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) atomicMax(&s_max, f2u(m));
  __syncthreads();
  if (threadIdx.x == 0) atomicMax(ws + plane / g.pps, s_max);
}

__global__ void fill_u32_kernel(uint32_t* p, int n, uint32_t v) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Scale of the per-tensor format from the layer absmax, exactly as
// amf_codec.py:182-191 computes it: absmax clamped to the dtype's 1e-8 floor,
// divided by 448 (double division then rounding to fp32 equals one fp32
// division since 53 >= 2*24 + 2).
template <int DT>
__device__ __forceinline__ float tensor_scale_from(uint32_t amax_bits) {
  return fmaxf(u2f(amax_bits), tensor_floor<DT>()) / kFp8Max;
}

// Writes each scale group's sidecar [k_scale, v_scale, q_scale, prob_scale]
// = [s, s, 1, 1] (FP8ScaleSidecar(k_scale=scale, v_scale=scale),
// amf_codec.py:200) from the first plane of the group.
template <int DT>
__global__ void fp8_tensor_finalize_kernel(const uint64_t* __restrict__ param_planes,
                                           const uint32_t* __restrict__ ws, int n_planes, int pps) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_planes && i % pps == 0) {
    float* sc = reinterpret_cast<float*>(param_planes[i]);
    const float s = tensor_scale_from<DT>(ws[i / pps]);
    sc[0] = s;
    sc[1] = s;
    sc[2] = 1.0f;
    sc[3] = 1.0f;
  }
}

// Per-tensor save in one read of the cache.  The two-pass form (absmax
// kernel, then a quantize kernel that reads every page again) moves two
// reads and a write through HBM.  Here a cooperative grid (every workgroup
// resident) walks the scale groups in order and keeps its share of a group
// in registers from the load to the store: the group's absmax is one atomic
// max per workgroup into ws[group], a per-group arrival counter says when
// every workgroup has contributed, and only then are the held values
// quantized and stored.  Two register buffers alternate, so the next group's
// loads are in flight while a workgroup waits on the current group's count.
// The exchange is a two-level tree, because device-scope atomics on one
// cache line serialize (one line for the whole grid cost about 20 us per
// group): workgroup b reports to cluster b % kCoopClusters, each cluster's
// last arrival forwards the cluster's max to the group's root line, and the
// root's last arrival writes the group's max with a ready bit into every
// cluster's line, where that cluster's workgroups poll for it.  Each
// cluster and root keeps its words on its own 128-byte line.
// Workgroup b holds pages b, b + G, b + 2G, ... of a group (G workgroups,
// at most kCoopChunks / CPT pages each); its lanes hold CPT 16-byte chunks
// of each page (tid + 256 m), so page addresses are workgroup-uniform.  The
// host takes this path only when a group fits the grid; others take the
// two-pass kernels.
struct CoopArgs {
  CoopGeom geo;
  const uint64_t* code_planes;
  int64_t page_elems;
  uint32_t* ws;         // [n_groups] absmax bits, written by each group's root
  // Per group, kCoopClusters + 1 lines, zeroed before the launch.  Cluster
  // line k: [0] arrivals, [1] max bits, [2] the group's max | kReady once
  // complete.  Root line: [0] clusters complete, [1] max bits.
  uint32_t* sync;
};

// The absmax works on the 16-bit patterns (abs_bits16): not converting to
// fp32 here also keeps the compiler from holding converted copies of the
// buffer until the store.
template <int DT>
__device__ __forceinline__ uint32_t absmax_bits16(const u32x4& v, uint32_t m) {
#pragma unroll
  for (int q = 0; q < 4; ++q)
    m = max(m, max(abs_bits16<DT>(v[q] & 0xFFFFu), abs_bits16<DT>(v[q] >> 16)));
  return m;
}

// Reports the buffer's absmax for group gi.  Lane 0 folds it into its
// cluster's max, waits for that atomic to complete, then counts itself in;
// each atomic is device-scope, performed where every XCD sees it.  The
// cluster's last arrival (its count returns cluster size - 1, so every other
// member's max is already in) forwards the cluster max to the root the same
// way, and the root's last arrival publishes the group's max to ws[gi] and
// to every cluster line.  The codes a workgroup stored need not be visible
// to others, so no release fence (an L2 write-back) is taken.
template <int DT>
__device__ __forceinline__ void coop_arrive(const CoopArgs& a, int gi,
                                            const u32x4 (&buf)[kCoopChunks], uint32_t* s_max) {
  uint32_t mb = 0;
#pragma unroll
  for (int k = 0; k < kCoopChunks; ++k) mb = absmax_bits16<DT>(buf[k], mb);
  float m;
  if constexpr (DT == AMF_DTYPE_BF16)
    m = u2f(mb << 16);
  else
    m = (float)__builtin_bit_cast(_Float16, (uint16_t)mb);
  m = wave_max_xor(m, 64);
  if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = f2u(m);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t b = s_max[0];
#pragma unroll
    for (int w = 1; w < kCoopThreads / 64; ++w) b = b > s_max[w] ? b : s_max[w];
    const int G = (int)gridDim.x;
    const int k = (int)blockIdx.x % kCoopClusters;
    const int n_clusters = G < kCoopClusters ? G : kCoopClusters;
    const uint32_t members = (uint32_t)((G - k + kCoopClusters - 1) / kCoopClusters);
    uint32_t* cl = coop_line(a.sync, gi, k);
    __hip_atomic_fetch_max(cl + 1, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the max has completed before the count moves
    if (__hip_atomic_fetch_add(cl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        members - 1) {
      const uint32_t cm = __hip_atomic_load(cl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      uint32_t* root = coop_line(a.sync, gi, kCoopClusters);
      __hip_atomic_fetch_max(root + 1, cm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      if (__hip_atomic_fetch_add(root, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
          (uint32_t)n_clusters - 1) {
        const uint32_t gm =
            __hip_atomic_load(root + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_max(a.ws + gi, gm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int c = 0; c < n_clusters; ++c)
          __hip_atomic_store(coop_line(a.sync, gi, c) + 2, gm | kReady, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// Waits (lane 0, bounded) for group gi's max on this workgroup's cluster
// line and returns it to the whole workgroup.  Every workgroup of a
// cooperative launch is resident, so the max arrives; the bound only keeps a
// broken launch from spinning forever.  A workgroup whose wait runs out
// raises AMF_ERRFLAG_SYNC, waits no more (no workgroup spins longer than one
// bound in a launch), and raises the group's absmax slot to +inf, so the
// scale written for that group is infinite and a restore of it yields
// inf/NaN rather than plausible values.
__device__ __forceinline__ uint32_t coop_wait(const CoopArgs& a, int gi, uint32_t* s_bits,
                                              bool& gave_up) {
  if (threadIdx.x == 0) {
    const uint32_t* go = coop_line(a.sync, gi, (int)blockIdx.x % kCoopClusters) + 2;
    uint32_t v = __hip_atomic_load(go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t spins = 0;
    while (!gave_up && !(v & kReady)) {
      if (++spins > a.geo.spin_limit) {
        if (a.geo.err_flag) atomicOr(a.geo.err_flag, AMF_ERRFLAG_SYNC);
        gave_up = true;
      }
      __builtin_amdgcn_s_sleep(2);
      v = __hip_atomic_load(go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!(v & kReady))
      __hip_atomic_fetch_max(a.ws + gi, 0x7F800000u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_bits = v & ~kReady;
  }
  __syncthreads();
  const uint32_t bits = *s_bits;
  __syncthreads();  // s_bits is reused by the next group
  return bits;
}

template <int DT, int CPT>
__device__ __forceinline__ void coop_store(const CoopArgs& a, int gi,
                                           const u32x4 (&buf)[kCoopChunks], uint32_t amax_bits) {
  const float am = fmaxf(u2f(amax_bits), tensor_floor<DT>());
  const float tdiv = (am == 0.0f) ? 1e-12f : am / kFp8Max;
  const float trcp = 1.0f / tdiv;
#pragma unroll
  for (int i = 0; i < kCoopChunks / CPT; ++i) {
    const CoopPage q = coop_page(a.geo, gi, i);
    if (!q.ok) continue;
    u32x2* codes = reinterpret_cast<u32x2*>(reinterpret_cast<uint8_t*>(a.code_planes[q.plane]) +
                                            q.j * a.page_elems);
#pragma unroll
    for (int m = 0; m < CPT; ++m) {
      float x[8];
      unpack8<DT == AMF_DTYPE_BF16>(buf[i * CPT + m], x);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        x[e] = fminf(fmaxf(div_rn(x[e], tdiv, trcp), -kFp8Max), kFp8Max);
      u32x2 cw;
      cw[0] = f32x4_to_e4m3(x);
      cw[1] = f32x4_to_e4m3(x + 4);
      st_stream(cw, codes + threadIdx.x + kCoopThreads * m);
    }
  }
}

template <int DT, int CPT>
__global__ __launch_bounds__(kCoopThreads) void fp8_tensor_coop_kernel(CoopArgs a) {
  __shared__ uint32_t s_max[kCoopThreads / 64];
  __shared__ uint32_t s_bits;
  bool gave_up = false;  // lane 0's: a wait ran out of its bound
  u32x4 b0[kCoopChunks], b1[kCoopChunks];
  const int ng = a.geo.n_groups;
  coop_load<CPT>(a.geo, 0, b0);
  coop_arrive<DT>(a, 0, b0, s_max);
  if (ng > 1) coop_load<CPT>(a.geo, 1, b1);
  // Groups in pairs so that each buffer is a fixed register array.  A group
  // is reported as soon as the previous group's max is known (its loads were
  // issued before that wait), ahead of the previous group's stores, so the
  // report never waits on store completion.  Every workgroup takes the same
  // branches (they depend on n_groups only).
  for (int gi = 0; gi < ng; gi += 2) {
    const uint32_t m0 = coop_wait(a, gi, &s_bits, gave_up);
    if (gi + 1 < ng) coop_arrive<DT>(a, gi + 1, b1, s_max);
    coop_store<DT, CPT>(a, gi, b0, m0);
    if (gi + 2 < ng) coop_load<CPT>(a.geo, gi + 2, b0);
    if (gi + 1 >= ng) break;
    const uint32_t m1 = coop_wait(a, gi + 1, &s_bits, gave_up);
    if (gi + 2 < ng) coop_arrive<DT>(a, gi + 2, b0, s_max);
    coop_store<DT, CPT>(a, gi + 1, b1, m1);
    if (gi + 3 < ng) coop_load<CPT>(a.geo, gi + 3, b1);
  }
}

// Per-(page, head) save without a workgroup barrier: a head's bs x head_dim
// block belongs to one half-wave (32 lanes), each lane holding CPL 8-element
// chunks of it in registers, so the head's absmax is a 32-lane shuffle
// reduction and each half-wave quantizes as soon as its own loads land.
// Chunk c of a head is token c / (head_dim / 8), dims 8 (c % (head_dim / 8))
// ..+7: 16 consecutive lanes read one 256-byte row (bf16, head_dim 128).
// A workgroup takes 8 heads per pass.
template <int DT, int CPL>
__global__ __launch_bounds__(kThreads) void fp8_ph_quant_gather_kernel(
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, const uint64_t* __restrict__ code_planes,
    const uint64_t* __restrict__ param_planes, PageGeom g, int32_t* err_flag) {
  const int64_t j = blockIdx.x;
  const int plane = blockIdx.y;
  const int64_t sp = block_ids ? (int64_t)block_ids[j] : j;
  if (sp < 0 || sp >= pool) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  const int H = g.num_heads, D = g.head_dim;
  const int64_t page_elems = (int64_t)g.n_rows * D;
  const uint8_t* __restrict__ src =
      reinterpret_cast<const uint8_t*>(cache_planes[plane]) + sp * cache_stride;
  uint8_t* __restrict__ codes = reinterpret_cast<uint8_t*>(code_planes[plane]) + j * page_elems;
  float* __restrict__ params = reinterpret_cast<float*>(param_planes[plane]) + j * H;
  const int lh = threadIdx.x & 31;
  const int cpr = D >> 3;  // chunks per token row of one head
  for (int h = (int)(threadIdx.x >> 5); h < H; h += kThreads / 32) {
    int64_t off[CPL];
    float x[CPL][8];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = lh + 32 * i;
      off[i] = ((int64_t)(c / cpr) * H + h) * D + (c % cpr) * 8;
      load8_stream<DT>(src + off[i] * elem_bytes<DT>(), x[i]);
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i)
#pragma unroll
      for (int q = 0; q < 8; ++q) m = fmaxf(m, fabsf(x[i][q]));
    m = wave_max_xor(m, 32);
    // scale = max(absmax, 1e-8) / 448, stored per (page, head).
    const float b = fmaxf(m, 1e-8f) / kFp8Max;
    const float rb = 1.0f / b;
    if (lh == 0) params[h] = b;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
#pragma unroll
      for (int q = 0; q < 8; ++q)
        x[i][q] = fminf(fmaxf(div_rn(x[i][q], b, rb), -kFp8Max), kFp8Max);
      u32x2 c;
      c[0] = f32x4_to_e4m3(x[i]);
      c[1] = f32x4_to_e4m3(x[i] + 4);
      st_stream(c, reinterpret_cast<u32x2*>(codes + off[i]));
    }
  }
}

// Per-tensor save, pass 2 (after fp8_absmax_kernel): one lane = CPL
// 8-element chunks kThreads apart, so each load instruction of a wave covers
// 1 KiB of whole lines (non-temporal: read once) and each code store 512
// contiguous bytes.  Same arithmetic as fp8_quant_gather_kernel<PER_TENSOR>.
template <int DT, int CPL>
__global__ __launch_bounds__(kThreads) void fp8_tensor_quant_kernel(
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, const uint64_t* __restrict__ code_planes,
    PageGeom g, const uint32_t* __restrict__ ws, int32_t* err_flag) {
  const int64_t j = blockIdx.x;
  const int plane = blockIdx.y;
  const int64_t sp = block_ids ? (int64_t)block_ids[j] : j;
  if (sp < 0 || sp >= pool) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  const int64_t page_elems = (int64_t)g.n_rows * g.head_dim;
  const uint8_t* __restrict__ src =
      reinterpret_cast<const uint8_t*>(cache_planes[plane]) + sp * cache_stride;
  u32x2* __restrict__ codes =
      reinterpret_cast<u32x2*>(reinterpret_cast<uint8_t*>(code_planes[plane]) + j * page_elems);
  float x[CPL][8];
#pragma unroll
  for (int i = 0; i < CPL; ++i)
    load8_stream<DT>(src + (int64_t)(threadIdx.x + i * kThreads) * (8 * elem_bytes<DT>()), x[i]);
  const float a = fmaxf(u2f(ws[plane / g.pps]), tensor_floor<DT>());
  // amf_codec.py:191 divides by max(scale, 1e-12); only a zero absmax (an
  // fp16 cache, whose floor rounds to 0) reaches that clamp.
  const float b = (a == 0.0f) ? 1e-12f : a / kFp8Max;
  const float rb = 1.0f / b;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
#pragma unroll
    for (int q = 0; q < 8; ++q) x[i][q] = fminf(fmaxf(div_rn(x[i][q], b, rb), -kFp8Max), kFp8Max);
    u32x2 c;
    c[0] = f32x4_to_e4m3(x[i]);
    c[1] = f32x4_to_e4m3(x[i] + 4);
    st_stream(c, codes + threadIdx.x + i * kThreads);
  }
}

template <bool BF16, bool PER_TENSOR, int R>
__global__ __launch_bounds__(kThreads) void fp8_quant_gather_kernel(
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, const uint64_t* __restrict__ code_planes,
    const uint64_t* __restrict__ param_planes, PageGeom g, const uint32_t* __restrict__ ws,
    int32_t* err_flag) {
  const int64_t j = blockIdx.x;
  const int plane = blockIdx.y;
  const int64_t sp = block_ids ? (int64_t)block_ids[j] : j;
  __shared__ uint32_t s_amax[256];
  const bool bad = sp < 0 || sp >= pool;
  if (bad) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  const int64_t page_elems = (int64_t)g.n_rows * g.head_dim;
  const uint8_t* __restrict__ src =
      reinterpret_cast<const uint8_t*>(cache_planes[plane]) + sp * cache_stride;
  uint8_t* __restrict__ codes = reinterpret_cast<uint8_t*>(code_planes[plane]) + j * page_elems;
  float* __restrict__ params = reinterpret_cast<float*>(param_planes[plane]);

  const int col = lane_col(g), rpi = rows_per_iter(g), r0 = lane_row0(g);
  const int cpr = 1 << g.cpr_log2;
  if (!PER_TENSOR) {
    for (int h = threadIdx.x; h < g.num_heads; h += kThreads) s_amax[h] = 0;
    __syncthreads();
  }

  // Load this lane's rows (at most R; chosen on the host).
  u32x4 v[R][2];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int row = r0 + k * rpi;
    if (row < g.n_rows) {
      const u32x4* p =
          reinterpret_cast<const u32x4*>(src + 2 * ((int64_t)row * g.head_dim + col * 16));
      v[k][0] = p[0];
      v[k][1] = p[1];
    }
  }

  if (!PER_TENSOR) {
    // Per-(page, head) absmax: reduce a row's chunks across its cpr lanes,
    // then one LDS atomic max per row.
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int row = r0 + k * rpi;
      if (k * rpi >= g.n_rows) break;  // uniform: no lane has this row
      float x[16];
      float m = 0.0f;
      if (row < g.n_rows) {
        unpack8<BF16>(v[k][0], x);
        unpack8<BF16>(v[k][1], x + 8);
#pragma unroll
        for (int q = 0; q < 16; ++q) m = fmaxf(m, fabsf(x[q]));
      }
      m = wave_max_xor(m, cpr);
      if (col == 0 && row < g.n_rows) atomicMax(&s_amax[row % g.num_heads], f2u(m));
    }
    __syncthreads();
    // scale = max(absmax, 1e-8) / 448, stored per (page, head).
    for (int h = threadIdx.x; h < g.num_heads; h += kThreads)
      params[j * g.num_heads + h] = fmaxf(u2f(s_amax[h]), 1e-8f) / kFp8Max;
  }

  float tdiv = 0.0f, trcp = 0.0f;
  if (PER_TENSOR) {
    const float a = fmaxf(u2f(ws[plane / g.pps]), tensor_floor<dtype_of<BF16>()>());
    // amf_codec.py:191 divides by max(scale, 1e-12); only a zero absmax (an
    // fp16 cache, whose floor rounds to 0) reaches that clamp.
    tdiv = (a == 0.0f) ? 1e-12f : a / kFp8Max;
    trcp = 1.0f / tdiv;
  }

#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int row = r0 + k * rpi;
    if (row < g.n_rows) {
      float b = tdiv, rb = trcp;
      if (!PER_TENSOR) {
        b = fmaxf(u2f(s_amax[row % g.num_heads]), 1e-8f) / kFp8Max;
        rb = 1.0f / b;
      }
      float x[16];
      unpack8<BF16>(v[k][0], x);
      unpack8<BF16>(v[k][1], x + 8);
#pragma unroll
      for (int q = 0; q < 16; ++q) x[q] = fminf(fmaxf(div_rn(x[q], b, rb), -kFp8Max), kFp8Max);
      u32x4 c;
#pragma unroll
      for (int q = 0; q < 4; ++q) c[q] = f32x4_to_e4m3(x + 4 * q);
      st_stream(
          c, reinterpret_cast<u32x4*>(codes + (int64_t)row * g.head_dim + col * 16));
    }
  }
}

// Save of pages larger than the register-resident kernel holds, and of fp32
// caches: the page is read twice (per-(page, head) absmax, then codes; the
// second read hits in cache).  One lane = one 8-element chunk per step;
// head_dim % 16 == 0, so a chunk never straddles rows.  Same arithmetic as
// fp8_quant_gather_kernel.
template <int DT, bool PER_TENSOR>
__global__ __launch_bounds__(kThreads) void fp8_quant_gather_looped_kernel(
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, const uint64_t* __restrict__ code_planes,
    const uint64_t* __restrict__ param_planes, PageGeom g, const uint32_t* __restrict__ ws,
    int32_t* err_flag) {
  constexpr int ES = elem_bytes<DT>();
  const int64_t j = blockIdx.x;
  const int plane = blockIdx.y;
  const int64_t sp = block_ids ? (int64_t)block_ids[j] : j;
  __shared__ uint32_t s_amax[kThreads];
  if (sp < 0 || sp >= pool) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  const int64_t page_elems = (int64_t)g.n_rows * g.head_dim;
  const int64_t n8 = page_elems >> 3;
  const uint8_t* __restrict__ src =
      reinterpret_cast<const uint8_t*>(cache_planes[plane]) + sp * cache_stride;
  uint8_t* __restrict__ codes = reinterpret_cast<uint8_t*>(code_planes[plane]) + j * page_elems;
  float* __restrict__ params = reinterpret_cast<float*>(param_planes[plane]);
  if (!PER_TENSOR) {
    for (int h = threadIdx.x; h < g.num_heads; h += kThreads) s_amax[h] = 0;
    __syncthreads();
    for (int64_t k = threadIdx.x; k < n8; k += kThreads) {
      float x[8];
      load8<DT>(src + k * (8 * ES), x);
      float m = 0.0f;
#pragma unroll
      for (int q = 0; q < 8; ++q) m = fmaxf(m, fabsf(x[q]));
      atomicMax(&s_amax[(int)((k * 8 / g.head_dim) % g.num_heads)], f2u(m));
    }
    __syncthreads();
    for (int h = threadIdx.x; h < g.num_heads; h += kThreads)
      params[j * g.num_heads + h] = fmaxf(u2f(s_amax[h]), 1e-8f) / kFp8Max;
  }
  float tdiv = 0.0f, trcp = 0.0f;
  if (PER_TENSOR) {
    const float a = fmaxf(u2f(ws[plane / g.pps]), tensor_floor<DT>());
    tdiv = (a == 0.0f) ? 1e-12f : a / kFp8Max;
    trcp = 1.0f / tdiv;
  }
  for (int64_t k = threadIdx.x; k < n8; k += kThreads) {
    float b = tdiv, rb = trcp;
    if (!PER_TENSOR) {
      b = fmaxf(u2f(s_amax[(int)((k * 8 / g.head_dim) % g.num_heads)]), 1e-8f) / kFp8Max;
      rb = 1.0f / b;
    }
    float x[8];
    load8<DT>(src + k * (8 * ES), x);
#pragma unroll
    for (int q = 0; q < 8; ++q) x[q] = fminf(fmaxf(div_rn(x[q], b, rb), -kFp8Max), kFp8Max);
    u32x2 c;
    c[0] = f32x4_to_e4m3(x);
    c[1] = f32x4_to_e4m3(x + 4);
    st_stream(c, reinterpret_cast<u32x2*>(codes) + k);
  }
}

int make_geom(const char* who, int32_t block_size, int32_t num_heads, int32_t head_dim,
              int32_t pps, PageGeom* g) {
  if (head_dim % 16 != 0) return fail(AMF_ERR_UNSUPPORTED, "%s: head_dim %% 16 != 0", who);
  const int cpr = head_dim / 16;
  if (cpr > kThreads || (cpr & (cpr - 1)) != 0)
    return fail(AMF_ERR_UNSUPPORTED, "%s: head_dim/16 = %d must be a power of two <= %d", who,
                cpr, kThreads);
  g->n_rows = block_size * num_heads;
  g->head_dim = head_dim;
  g->num_heads = num_heads;
  g->cpr_log2 = __builtin_ctz(cpr);
  // Restore passes advance 8 * kThreads elements; save passes kThreads / cpr rows.
  g->head_const = ((kThreads * 8) % (head_dim * num_heads)) == 0 &&
                  ((kThreads / cpr) % num_heads) == 0;
  g->pps = pps > 0 ? pps : 1;
  return ok();
}

// The cooperative kernel for a cache dtype and chunks per page row (CPT),
// or nullptr for combinations it does not cover.
const void* coop_kernel(int dt, int cpt) {
#define AMF_COOP(D, C) reinterpret_cast<const void*>(&fp8_tensor_coop_kernel<D, C>)
#define AMF_COOP_CPT(D)                                               \
  switch (cpt) {                                                      \
    case 1: return AMF_COOP(D, 1);                                    \
    case 2: return AMF_COOP(D, 2);                                    \
    case 4: return AMF_COOP(D, 4);                                    \
    case 8: return AMF_COOP(D, 8);                                    \
    case 16: return AMF_COOP(D, 16);                                  \
    default: return nullptr;                                          \
  }
  if (dt == AMF_DTYPE_BF16) { AMF_COOP_CPT(AMF_DTYPE_BF16) }
  if (dt == AMF_DTYPE_F16) { AMF_COOP_CPT(AMF_DTYPE_F16) }
  return nullptr;
#undef AMF_COOP_CPT
#undef AMF_COOP
}

constexpr int kCoopNotTaken = 1;

// Per-tensor save through fp8_tensor_coop_kernel when the device supports a
// cooperative launch, a page row of chunks maps onto the workgroup (the
// page's 16-byte chunks are 256 * CPT, CPT a power of two <= kCoopChunks)
// and a scale group fits the grid.  Returns AMF_OK after the launch,
// kCoopNotTaken to leave the call to the two-pass kernels (nothing
// launched), or an error code.  ws must hold the zeroed absmax slots and
// arrival counters.
int try_tensor_coop(int32_t dt, const uint64_t* cache_planes, int64_t cache_page_stride,
                    const int32_t* block_ids, int64_t pool_pages, const uint64_t* code_planes,
                    int64_t n_pages, const PageGeom& g, int n_groups, uint32_t* ws,
                    int32_t* err_flag, hipStream_t s) {
  if (coop_disabled() || !aligned16(cache_page_stride)) return kCoopNotTaken;
  const int64_t page_elems = (int64_t)g.n_rows * g.head_dim;
  const int64_t chunks_pp = page_elems / 8;  // head_dim % 16 == 0: whole 16-byte chunks
  if (chunks_pp % kCoopThreads != 0) return kCoopNotTaken;
  const int cpt = (int)(chunks_pp / kCoopThreads);
  const void* fn = coop_kernel(dt, cpt);
  if (!fn) return kCoopNotTaken;
  const int64_t group_pages = (int64_t)g.pps * n_pages;
  if (group_pages * chunks_pp * 16 < kCoopMinGroupBytes) return kCoopNotTaken;
  const int blocks = coop_blocks(fn);
  if (blocks <= 0) return kCoopNotTaken;
  const int64_t ppw = (group_pages + blocks - 1) / blocks;
  if (ppw > kCoopChunks / cpt) return kCoopNotTaken;
  // No workgroup without a page: an idle one still takes part in every
  // group's exchange (512 pages per group: 308 us at 512 workgroups against
  // 333 us at 768).  Evening out the pages per workgroup beyond that (512
  // workgroups of 2 pages instead of 768 of 1 or 2) is slower: fewer reads
  // in flight.
  const int grid = (int)std::min<int64_t>(blocks, group_pages);
  CoopArgs a;
  a.geo.cache_planes = cache_planes;
  a.geo.cache_stride = cache_page_stride;
  a.geo.block_ids = block_ids;
  a.geo.pool = pool_pages;
  a.geo.n_pages = n_pages;
  a.geo.group_pages = group_pages;
  a.geo.pps = g.pps;
  a.geo.n_groups = n_groups;
  a.geo.ppw = (int)ppw;
  a.geo.spin_limit = coop_spin_limit();
  a.geo.err_flag = err_flag;
  a.code_planes = code_planes;
  a.page_elems = page_elems;
  a.ws = ws;
  a.sync = ws + fp8_tensor_sync_offset(n_groups);
  void* args[] = {&a};
  const hipError_t e =
      hipLaunchCooperativeKernel(fn, dim3((unsigned)grid), dim3(kCoopThreads), args, 0, s);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return kCoopNotTaken;
  }
  return ok();
}

}  // namespace

extern "C" int amf_fp8_dequant_scatter(int32_t format, const uint64_t* code_planes,
                                       const uint64_t* param_planes, const uint64_t* cache_planes,
                                       int64_t cache_page_stride, int32_t cache_dtype,
                                       const int32_t* block_ids, int64_t pool_pages,
                                       int32_t n_planes, int64_t n_pages, int32_t block_size,
                                       int32_t num_heads, int32_t head_dim, int32_t* err_flag,
                                       void* stream) {
  const char* who = "amf_fp8_dequant_scatter";
  if (format != AMF_FMT_FP8_E4M3 && format != AMF_FMT_FP8_E4M3_PH)
    return fail(AMF_ERR_INVALID_ARG, "%s: format %d is not an FP8 format", who, format);
  int rc = check_codec_geometry(who, cache_planes, cache_page_stride, cache_dtype, block_ids,
                                pool_pages, code_planes, param_planes, n_planes, n_pages,
                                block_size, num_heads, head_dim);
  if (rc) return rc;
  PageGeom g;
  if ((rc = make_geom(who, block_size, num_heads, head_dim, 1, &g))) return rc;
  if (n_pages == 0) return ok();
  if (n_pages * n_planes > 0x7FFFFFF0ll)
    return fail(AMF_ERR_UNSUPPORTED, "%s: %lld pages x %d planes exceed one launch", who,
                (long long)n_pages, n_planes);
  const dim3 grid = xcd_page_grid(n_pages, n_planes);
  hipStream_t s = as_stream(stream);
  const bool pt = format == AMF_FMT_FP8_E4M3;
#define AMF_LAUNCH(T)                                                                       \
  fp8_dequant_scatter_kernel<DT, T><<<grid, kThreads, kRestoreLdsPad, s>>>(                 \
      code_planes, param_planes, cache_planes, cache_page_stride, block_ids, pool_pages,     \
      n_pages, n_planes, g, err_flag)
  AMF_WITH_DTYPE(cache_dtype, if (pt) AMF_LAUNCH(true); else AMF_LAUNCH(false));
#undef AMF_LAUNCH
  return check_launch(who);
}

extern "C" int amf_fp8_quant_gather(int32_t format, const uint64_t* cache_planes,
                                    int64_t cache_page_stride, int32_t cache_dtype,
                                    const int32_t* block_ids, int64_t pool_pages,
                                    const uint64_t* code_planes, const uint64_t* param_planes,
                                    int32_t n_planes, int32_t planes_per_scale, int64_t n_pages,
                                    int32_t block_size, int32_t num_heads, int32_t head_dim,
                                    float* workspace,
                                    int64_t workspace_bytes, int32_t* err_flag, void* stream) {
  const char* who = "amf_fp8_quant_gather";
  if (format != AMF_FMT_FP8_E4M3 && format != AMF_FMT_FP8_E4M3_PH)
    return fail(AMF_ERR_INVALID_ARG, "%s: format %d is not an FP8 format", who, format);
  int rc = check_codec_geometry(who, cache_planes, cache_page_stride, cache_dtype, block_ids,
                                pool_pages, code_planes, param_planes, n_planes, n_pages,
                                block_size, num_heads, head_dim);
  if (rc) return rc;
  const bool pt = format == AMF_FMT_FP8_E4M3;
  if (pt && (planes_per_scale <= 0 || n_planes % planes_per_scale != 0))
    return fail(AMF_ERR_INVALID_ARG, "%s: planes_per_scale %d does not divide n_planes %d", who,
                planes_per_scale, n_planes);
  PageGeom g;
  if ((rc = make_geom(who, block_size, num_heads, head_dim, planes_per_scale, &g))) return rc;
  const int rpi = kThreads >> g.cpr_log2;
  // Pages that fit lanes' registers take the single-read kernel; larger pages
  // and fp32 caches the two-read one.
  const bool looped = cache_dtype == AMF_DTYPE_F32 || g.n_rows > rpi * kMaxRowsPerLane;
  if (format == AMF_FMT_FP8_E4M3_PH && num_heads > kThreads)
    return fail(AMF_ERR_UNSUPPORTED, "%s: num_heads > %d", who, kThreads);
  const int64_t need = amf_quant_workspace_bytes(format, n_planes, planes_per_scale, head_dim);
  if (pt && (!workspace || workspace_bytes < need))
    return fail(AMF_ERR_WORKSPACE, "%s: per-tensor format needs %lld workspace bytes", who,
                (long long)need);
  if (n_pages == 0) return ok();
  hipStream_t s = as_stream(stream);
  dim3 grid((unsigned)n_pages, (unsigned)n_planes);
  uint32_t* ws = reinterpret_cast<uint32_t*>(workspace);
  const int n_groups = n_planes / g.pps;
  if (pt) {
    // ws: n_groups absmax slots, then the single-read kernel's cluster lines.
    const int n_words = (int)fp8_tensor_workspace_words(n_groups);
    fill_u32_kernel<<<(n_words + 255) / 256, 256, 0, s>>>(ws, n_words, 0u);
    rc = try_tensor_coop(cache_dtype, cache_planes, cache_page_stride, block_ids, pool_pages,
                         code_planes, n_pages, g, n_groups, ws, err_flag, s);
    if (rc != kCoopNotTaken) {
      if (rc != AMF_OK) return rc;
      AMF_WITH_DTYPE(cache_dtype, fp8_tensor_finalize_kernel<DT>
                     <<<(n_planes + 255) / 256, 256, 0, s>>>(param_planes, ws, n_planes, g.pps));
      return check_launch(who);
    }
    const int64_t per_plane = std::max<int64_t>(
        1, std::min<int64_t>(n_pages, (kAbsBlocks + n_planes - 1) / n_planes));
    dim3 agrid((unsigned)per_plane, (unsigned)n_planes);
    AMF_WITH_DTYPE(cache_dtype,
                   fp8_absmax_kernel<DT><<<agrid, kThreads, 0, s>>>(
                       cache_planes, cache_page_stride, block_ids, pool_pages, n_pages, g, ws,
                       err_flag));
  }
  // Per-tensor pass 2: pages of 1-16 chunks of 8 elements per lane take the
  // register-resident whole-line kernel.
  const int64_t page_chunks = (int64_t)g.n_rows * head_dim / 8;
  const int64_t tcpl = page_chunks % kThreads == 0 ? page_chunks / kThreads : 0;
  if (pt && cache_dtype != AMF_DTYPE_F32 &&
      (tcpl == 1 || tcpl == 2 || tcpl == 4 || tcpl == 8 || tcpl == 16)) {
#define AMF_LAUNCH(C)                                                                          \
  AMF_WITH_DTYPE(cache_dtype, fp8_tensor_quant_kernel<DT, C><<<grid, kThreads, 0, s>>>(        \
                                  cache_planes, cache_page_stride, block_ids, pool_pages,      \
                                  code_planes, g, ws, err_flag))
    if (tcpl == 1) AMF_LAUNCH(1);
    else if (tcpl == 2) AMF_LAUNCH(2);
    else if (tcpl == 4) AMF_LAUNCH(4);
    else if (tcpl == 8) AMF_LAUNCH(8);
    else AMF_LAUNCH(16);
#undef AMF_LAUNCH
    AMF_WITH_DTYPE(cache_dtype, fp8_tensor_finalize_kernel<DT>
                   <<<(n_planes + 255) / 256, 256, 0, s>>>(param_planes, ws, n_planes, g.pps));
    return check_launch(who);
  }
  const int64_t head_chunks = (int64_t)(g.n_rows / g.num_heads) * head_dim / 8;
  const int cpl = (int)(head_chunks / 32);
  if (!pt && cache_dtype != AMF_DTYPE_F32 && head_chunks % 32 == 0 &&
      (cpl == 2 || cpl == 4 || cpl == 8 || cpl == 16)) {
#define AMF_LAUNCH(C)                                                                          \
  AMF_WITH_DTYPE(cache_dtype, fp8_ph_quant_gather_kernel<DT, C><<<grid, kThreads, 0, s>>>(     \
                                  cache_planes, cache_page_stride, block_ids, pool_pages,      \
                                  code_planes, param_planes, g, err_flag))
    if (cpl == 2) AMF_LAUNCH(2);
    else if (cpl == 4) AMF_LAUNCH(4);
    else if (cpl == 8) AMF_LAUNCH(8);
    else AMF_LAUNCH(16);
#undef AMF_LAUNCH
    return check_launch(who);
  }
  if (looped) {
#define AMF_LAUNCH(T)                                                                         \
  fp8_quant_gather_looped_kernel<DT, T><<<grid, kThreads, 0, s>>>(                            \
      cache_planes, cache_page_stride, block_ids, pool_pages, code_planes, param_planes, g, ws, \
      err_flag)
    AMF_WITH_DTYPE(cache_dtype, if (pt) AMF_LAUNCH(true); else AMF_LAUNCH(false));
#undef AMF_LAUNCH
  } else {
    const int rows = (g.n_rows + rpi - 1) / rpi;
    const bool bf16 = cache_dtype == AMF_DTYPE_BF16;
#define AMF_LAUNCH(B, T, R)                                                                   \
  fp8_quant_gather_kernel<B, T, R><<<grid, kThreads, 0, s>>>(cache_planes, cache_page_stride,  \
                                                             block_ids, pool_pages,            \
                                                             code_planes, param_planes, g, ws, \
                                                             err_flag)
#define AMF_LAUNCH_R(B, T)                 \
  if (rows <= 1) AMF_LAUNCH(B, T, 1);      \
  else if (rows <= 2) AMF_LAUNCH(B, T, 2); \
  else if (rows <= 4) AMF_LAUNCH(B, T, 4); \
  else if (rows <= 8) AMF_LAUNCH(B, T, 8); \
  else AMF_LAUNCH(B, T, 16)
    if (bf16 && pt) { AMF_LAUNCH_R(true, true); }
    else if (bf16) { AMF_LAUNCH_R(true, false); }
    else if (pt) { AMF_LAUNCH_R(false, true); }
    else { AMF_LAUNCH_R(false, false); }
#undef AMF_LAUNCH_R
#undef AMF_LAUNCH
  }
  if (pt)
    AMF_WITH_DTYPE(cache_dtype, fp8_tensor_finalize_kernel<DT>
                   <<<(n_planes + 255) / 256, 256, 0, s>>>(param_planes, ws, n_planes, g.pps));
  return check_launch(who);
}
