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
    const int32_t* __restrict__ block_ids, int64_t pool, PageGeom g, int32_t* err_flag) {
  const int64_t j = blockIdx.x;
  const int plane = blockIdx.y;
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
        if (k < n16) v[u] = src[k];
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
      load8<DT>(src + off[i] * elem_bytes<DT>(), x[i]);
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
  dim3 grid((unsigned)n_pages, (unsigned)n_planes);
  hipStream_t s = as_stream(stream);
  const bool pt = format == AMF_FMT_FP8_E4M3;
#define AMF_LAUNCH(T)                                                                      \
  fp8_dequant_scatter_kernel<DT, T><<<grid, kThreads, 0, s>>>(                             \
      code_planes, param_planes, cache_planes, cache_page_stride, block_ids, pool_pages, g, \
      err_flag)
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
    fill_u32_kernel<<<(n_groups + 255) / 256, 256, 0, s>>>(ws, n_groups, 0u);
    const int64_t per_plane = std::max<int64_t>(
        1, std::min<int64_t>(n_pages, (kAbsBlocks + n_planes - 1) / n_planes));
    dim3 agrid((unsigned)per_plane, (unsigned)n_planes);
    AMF_WITH_DTYPE(cache_dtype,
                   fp8_absmax_kernel<DT><<<agrid, kThreads, 0, s>>>(
                       cache_planes, cache_page_stride, block_ids, pool_pages, n_pages, g, ws,
                       err_flag));
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
