// amf_int4.hip - INT4 codecs of the compressed VRAM pool, fused with the
// paged gather (save) and paged scatter (restore).
//
// Formats (layouts in include/amf_hip.h):
//  - AMF_FMT_INT4_SYM_BLOCK: INT4PerBlockCodec on a page tensor
//    (korith_vllm_ext/codecs/amf_codec.py:358-447): the page is the 16-token
//    axis padded to the codec's 128-token block, so one scale per (plane,
//    page) over every head.
//  - AMF_FMT_INT4_SYM: INT4PerChannelCodec (amf_codec.py:305-343): one scale
//    per head_dim channel over a whole layer, K and V together.
//  - AMF_FMT_INT4_ASYM_G32: asymmetric 32-dim groups, fp16 (scale, zero).
// Nibble order of the symmetric formats follows _pack_int4 / _unpack_int4
// (amf_codec.py:502-539): element 2i in the low nibble, u = q + 8.
#include "amf_internal.h"
#include "amf_kernel_util.h"

namespace {

using namespace amf;

constexpr int kThreads = 256;
constexpr float kSymMax = 7.0f;
constexpr float kAsymLevels = 15.0f;

// Nibble n (0..7) of a dword, as fp32.
__device__ __forceinline__ float nib(uint32_t w, int n) {
  return (float)__builtin_amdgcn_ubfe(w, 4 * n, 4);
}

// ------------------------------------------------------------ symmetric ----

struct SymGeom {
  int n_rows;     // block_size * num_heads
  int head_dim;
  int cpr_log2;   // log2(head_dim / 32): 32-element chunks per row
  int pps;        // planes per scale group (per-channel format)
};

__device__ __forceinline__ int sym_col(const SymGeom& g) { return threadIdx.x & ((1 << g.cpr_log2) - 1); }
__device__ __forceinline__ int sym_row0(const SymGeom& g) { return threadIdx.x >> g.cpr_log2; }
__device__ __forceinline__ int sym_rpi(const SymGeom& g) { return kThreads >> g.cpr_log2; }

// 32 cache elements at byte address `p` -> fp32.
template <int DT>
__device__ __forceinline__ void load32(const uint8_t* p, float* x) {
#pragma unroll
  for (int q = 0; q < 4; ++q) load8<DT>(p + q * (8 * elem_bytes<DT>()), x + 8 * q);
}

// Code words a sym-restore lane keeps in flight before its stores.
#ifndef AMF_SYM_RESTORE_UNROLL
#define AMF_SYM_RESTORE_UNROLL AMF_RESTORE_UNROLL
#endif

// CHANNEL = false: INT4_SYM_BLOCK (params: [n_pages] fp16);
// CHANNEL = true : INT4_SYM       (params: [head_dim] fp16 per scale group).
// One lane = one 8-element chunk (4 code bytes in, one 16-byte vector out):
// wave-wide stores cover 1 KiB contiguously.  A page of more than 8 passes
// of the workgroup is cut into `parts` workgroups of whole passes (a dense
// tensor's page can hold millions of elements).
template <int DT, bool CHANNEL>
__global__ __launch_bounds__(kThreads) void int4_sym_dequant_scatter_kernel(
    const uint64_t* __restrict__ code_planes, const uint64_t* __restrict__ param_planes,
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, int64_t n_pages, int n_planes,
    int parts, SymGeom g, int32_t* err_flag) {
  const PageWork pw = xcd_page_work(n_pages * parts, n_planes);
  if (!pw.valid) return;
  const int64_t j = pw.j / parts;
  const int part = (int)(pw.j % parts);
  const int plane = pw.plane;
  const int64_t dp = block_ids ? (int64_t)block_ids[j] : j;
  if (dp < 0 || dp >= pool) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  const int page_elems = g.n_rows * g.head_dim;
  const int n8 = page_elems >> 3;
  // this workgroup's chunks: [k_begin, k_end), k_begin a multiple of kThreads
  const int span = (n8 + parts - 1) / parts;
  const int k_begin = part * ((span + kThreads - 1) / kThreads * kThreads);
  const int k_end = min(n8, k_begin + (span + kThreads - 1) / kThreads * kThreads);
  const uint32_t* __restrict__ codes =
      reinterpret_cast<const uint32_t*>(code_planes[plane]) + j * (int64_t)n8;
  const _Float16* __restrict__ params = reinterpret_cast<const _Float16*>(param_planes[plane]);
  uint8_t* __restrict__ out = reinterpret_cast<uint8_t*>(cache_planes[plane]) + dp * cache_stride;
  const int tid = threadIdx.x;
  const float s_page = CHANNEL ? 0.0f : (float)params[j];
  // Channel scales of this lane's 8 dims; fixed while 8 * kThreads is a
  // multiple of head_dim (checked on the host).
  float s_ch[8];
  if (CHANNEL) {
    const int d0 = (tid * 8) % g.head_dim;
#pragma unroll
    for (int q = 0; q < 8; ++q) s_ch[q] = (float)params[d0 + q];
  }
  constexpr int U = AMF_SYM_RESTORE_UNROLL;
  for (int base = k_begin + tid; base < k_end; base += U * kThreads) {
    uint32_t c[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = base + u * kThreads;
      if (k < k_end) c[u] = ld_stream(codes + k);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = base + u * kThreads;
      if (k < k_end) {
        float x[8];
#pragma unroll
        for (int n = 0; n < 8; ++n) x[n] = (nib(c[u], n) - 8.0f) * (CHANNEL ? s_ch[n] : s_page);
        store8<DT>(out + (int64_t)k * (8 * elem_bytes<DT>()), x);
      }
    }
  }
}

// INT4_SYM_BLOCK save: page absmax -> scale -> codes; the page stays in
// registers.  One lane = CPL 8-element chunks kThreads apart, so each load
// instruction of a wave covers 1 KiB of whole lines (non-temporal: read once)
// and each code store 256 contiguous bytes.
template <bool BF16, int CPL>
__global__ __launch_bounds__(kThreads) void int4_symblock_quant_gather_kernel(
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, const uint64_t* __restrict__ code_planes,
    const uint64_t* __restrict__ param_planes, SymGeom g, int32_t* err_flag) {
  const int64_t j = blockIdx.x;
  const int plane = blockIdx.y;
  const int64_t sp = block_ids ? (int64_t)block_ids[j] : j;
  if (sp < 0 || sp >= pool) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  const int n8 = (int)((int64_t)g.n_rows * g.head_dim / 8);
  const u32x4* __restrict__ src = reinterpret_cast<const u32x4*>(
      reinterpret_cast<const uint8_t*>(cache_planes[plane]) + sp * cache_stride);
  uint32_t* __restrict__ codes = reinterpret_cast<uint32_t*>(code_planes[plane]) + j * n8;
  _Float16* __restrict__ params = reinterpret_cast<_Float16*>(param_planes[plane]);

  u32x4 v[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int k = threadIdx.x + i * kThreads;
    if (k < n8) v[i] = ld_stream(src + k);
  }
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    if (threadIdx.x + i * kThreads < n8) {
      float x[8];
      unpack8<BF16>(v[i], x);
#pragma unroll
      for (int n = 0; n < 8; ++n) m = fmaxf(m, fabsf(x[n]));
    }
  }
  m = wave_max_xor(m, 64);
  __shared__ float s_wmax[kThreads / 64];
  if ((threadIdx.x & 63) == 0) s_wmax[threadIdx.x >> 6] = m;
  __syncthreads();
  float amax = s_wmax[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) amax = fmaxf(amax, s_wmax[w]);
  // amf_codec.py:392-394: absmax.clamp_min(1e-8) / 7 in fp32.
  const float scale = fmaxf(amax, 1e-8f) / kSymMax;
  const float rscale = 1.0f / scale;
  if (threadIdx.x == 0) params[j] = (_Float16)scale;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int k = threadIdx.x + i * kThreads;
    if (k < n8) {
      float x[8];
      unpack8<BF16>(v[i], x);
      uint32_t w = 0;
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        float qv = __builtin_rintf(div_rn(x[n], scale, rscale));
        qv = fminf(fmaxf(qv, -8.0f), 7.0f);
        w |= (uint32_t)((int)qv + 8) << (4 * n);
      }
      st_stream(w, codes + k);
    }
  }
}

// INT4_SYM_BLOCK save of pages larger than the register-resident kernel
// holds, and of fp32 caches: the page absmax in a first read, the codes in a
// second (which hits in cache).  One lane = one 8-element chunk per step.
// Same arithmetic as int4_symblock_quant_gather_kernel.
template <int DT>
__global__ __launch_bounds__(kThreads) void int4_symblock_quant_looped_kernel(
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, const uint64_t* __restrict__ code_planes,
    const uint64_t* __restrict__ param_planes, SymGeom g, int32_t* err_flag) {
  constexpr int ES = elem_bytes<DT>();
  const int64_t j = blockIdx.x;
  const int plane = blockIdx.y;
  const int64_t sp = block_ids ? (int64_t)block_ids[j] : j;
  if (sp < 0 || sp >= pool) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  const int64_t n8 = (int64_t)g.n_rows * g.head_dim / 8;
  const uint8_t* __restrict__ src =
      reinterpret_cast<const uint8_t*>(cache_planes[plane]) + sp * cache_stride;
  uint32_t* __restrict__ codes = reinterpret_cast<uint32_t*>(code_planes[plane]) + j * n8;
  _Float16* __restrict__ params = reinterpret_cast<_Float16*>(param_planes[plane]);
  float m = 0.0f;
  for (int64_t k = threadIdx.x; k < n8; k += kThreads) {
    float x[8];
    load8<DT>(src + k * (8 * ES), x);
#pragma unroll
    for (int n = 0; n < 8; ++n) m = fmaxf(m, fabsf(x[n]));
  }
  m = wave_max_xor(m, 64);
  __shared__ float s_wmax[kThreads / 64];
  if ((threadIdx.x & 63) == 0) s_wmax[threadIdx.x >> 6] = m;
  __syncthreads();
  float amax = s_wmax[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) amax = fmaxf(amax, s_wmax[w]);
  const float scale = fmaxf(amax, 1e-8f) / kSymMax;
  const float rscale = 1.0f / scale;
  if (threadIdx.x == 0) params[j] = (_Float16)scale;
  for (int64_t k = threadIdx.x; k < n8; k += kThreads) {
    float x[8];
    load8<DT>(src + k * (8 * ES), x);
    uint32_t w = 0;
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      float qv = __builtin_rintf(div_rn(x[n], scale, rscale));
      qv = fminf(fmaxf(qv, -8.0f), 7.0f);
      w |= (uint32_t)((int)qv + 8) << (4 * n);
    }
    st_stream(w, codes + k);
  }
}

// INT4_SYM save, pass 1: per-channel absmax over a scale group.  One lane =
// one 8-element chunk, as in pass 2 (kThreads * 8 is a multiple of head_dim,
// so a lane's 8 channels stay fixed): every load instruction of a wave covers
// 1 KiB of whole lines, and a page's chunks are all in flight at once.  Each
// workgroup folds a strided set of pages, reduces the lanes that share
// channels (shuffles, then an LDS table), and issues one global atomic max
// per channel into ws[group][head_dim].
constexpr int kAbsmaxUnroll = 8;

template <int DT>
__global__ __launch_bounds__(kThreads) void int4_channel_absmax_kernel(
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, int64_t n_pages, SymGeom g,
    uint32_t* ws, int32_t* err_flag) {
  const int plane = blockIdx.y;
  __shared__ uint32_t s_max[1024];
  for (int d = threadIdx.x; d < g.head_dim; d += kThreads) s_max[d] = 0;
  const int n8 = (int)((int64_t)g.n_rows * g.head_dim / 8);
  float m[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) m[q] = 0.0f;
  for (int64_t j = blockIdx.x; j < n_pages; j += gridDim.x) {
    const int64_t sp = block_ids ? (int64_t)block_ids[j] : j;
    if (sp < 0 || sp >= pool) {
      if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
      continue;
    }
    const uint8_t* src = reinterpret_cast<const uint8_t*>(cache_planes[plane]) + sp * cache_stride;
    for (int base = threadIdx.x; base < n8; base += kThreads * kAbsmaxUnroll) {
      float x[kAbsmaxUnroll][8];
#pragma unroll
      for (int u = 0; u < kAbsmaxUnroll; ++u) {
        const int k = base + u * kThreads;
        if (k < n8) load8_stream<DT>(src + (int64_t)k * (8 * elem_bytes<DT>()), x[u]);
      }
#pragma unroll
      for (int u = 0; u < kAbsmaxUnroll; ++u) {
        if (base + u * kThreads < n8) {
#pragma unroll
          for (int q = 0; q < 8; ++q) m[q] = fmaxf(m[q], fabsf(x[u][q]));
        }
      }
    }
  }
  // Lanes lane, lane + L, lane + 2L, ... of a wave (L = head_dim / 8 chunks
  // per row) hold the same channels.
  const int lpr = g.head_dim / 8;
#pragma unroll
  for (int q = 0; q < 8; ++q)
    for (int o = 32; o >= lpr; o >>= 1) m[q] = fmaxf(m[q], __shfl_xor(m[q], o));
  __syncthreads();  // s_max cleared
  if ((threadIdx.x & 63) < lpr) {
    const int d0 = (threadIdx.x * 8) % g.head_dim;
#pragma unroll
    for (int q = 0; q < 8; ++q) atomicMax(&s_max[d0 + q], f2u(m[q]));
  }
  __syncthreads();
  for (int d = threadIdx.x; d < g.head_dim; d += kThreads)
    atomicMax(ws + (int64_t)(plane / g.pps) * g.head_dim + d, s_max[d]);
}

__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// INT4_SYM save, pass 2: one lane = one 8-element chunk (16 bytes of bf16 in,
// one 4-byte code word out), so a wave stores 256 contiguous bytes.  Chunk k
// covers channels (8 k) % head_dim ..+7 and k advances by kThreads, a
// multiple of head_dim / 8: a lane's 8 channels, and so its scales and
// reciprocals, stay fixed for the whole page.
#ifndef AMF_CHAN_UNROLL
#define AMF_CHAN_UNROLL 4
#endif
constexpr int kChanUnroll = AMF_CHAN_UNROLL;

template <int DT>
__global__ __launch_bounds__(kThreads) void int4_channel_quant_gather_kernel(
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, const uint64_t* __restrict__ code_planes,
    const uint64_t* __restrict__ param_planes, SymGeom g, const uint32_t* __restrict__ ws,
    int32_t* err_flag) {
  const int64_t j = blockIdx.x;
  const int plane = blockIdx.y;
  // The group's fp16 scales (amf_codec.py:312-313), written once per group
  // by its first plane's first page.
  if (j == 0 && plane % g.pps == 0) {
    _Float16* p = reinterpret_cast<_Float16*>(param_planes[plane]);
    const uint32_t* gw = ws + (int64_t)(plane / g.pps) * g.head_dim;
    for (int d = threadIdx.x; d < g.head_dim; d += kThreads)
      p[d] = (_Float16)(fmaxf(u2f(gw[d]), 1e-8f) / kSymMax);
  }
  const int64_t sp = block_ids ? (int64_t)block_ids[j] : j;
  if (sp < 0 || sp >= pool) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  const int64_t page_elems = (int64_t)g.n_rows * g.head_dim;
  const int n8 = (int)(page_elems / 8);
  const uint8_t* __restrict__ src =
      reinterpret_cast<const uint8_t*>(cache_planes[plane]) + sp * cache_stride;
  uint32_t* __restrict__ codes =
      reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(code_planes[plane]) + j * (page_elems / 2));
  const int d0 = (threadIdx.x * 8) % g.head_dim;
  const uint32_t* lw = ws + (int64_t)(plane / g.pps) * g.head_dim + d0;
  float sc[8], rc[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    sc[q] = fmaxf(u2f(lw[q]), 1e-8f) / kSymMax;  // amf_codec.py:312-313
    rc[q] = 1.0f / sc[q];
  }
  for (int base = threadIdx.x; base < n8; base += kThreads * kChanUnroll) {
    float x[kChanUnroll][8];
#pragma unroll
    for (int u = 0; u < kChanUnroll; ++u) {
      const int k = base + u * kThreads;
      if (k < n8) load8_stream<DT>(src + (int64_t)k * (8 * elem_bytes<DT>()), x[u]);
    }
#pragma unroll
    for (int u = 0; u < kChanUnroll; ++u) {
      const int k = base + u * kThreads;
      if (k < n8) {
        uint32_t w = 0;
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          float qv = __builtin_rintf(div_rn(x[u][n], sc[n], rc[n]));
          qv = fminf(fmaxf(qv, -8.0f), 7.0f);
          w |= (uint32_t)((int)qv + 8) << (4 * n);
        }
        st_stream(w, codes + k);
      }
    }
  }
}

// ----------------------------------------------------------- asymmetric ----
//
// Page geometry: block_size 16, G = head_dim / 32 groups.  Per (page, head):
// K codes [16][D/2], K params [16][G]; V codes tiled dim-major, V params [G][16].

struct AsymGeom {
  int num_heads;
  int head_dim;
  int groups;          // head_dim / 32
  int hb_code_bytes;   // 16 * head_dim / 2   (one (page, head) code block)
  int hb_param_words;  // 16 * groups
};

// Group quantizer: min / max over 32 values, then
// scale = max(mx - mn, 1e-8) / 15 and q = clamp(rint((x - mn) / scale), 0, 15).
struct AsymParams {
  float mn, scale, rscale;
};

__device__ __forceinline__ AsymParams asym_params(const float* x) {
  float mn = x[0], mx = x[0];
#pragma unroll
  for (int n = 1; n < 32; ++n) {
    mn = fminf(mn, x[n]);
    mx = fmaxf(mx, x[n]);
  }
  AsymParams p;
  p.mn = mn;
  p.scale = fmaxf(mx - mn, 1e-8f) / kAsymLevels;
  p.rscale = 1.0f / p.scale;
  return p;
}

__device__ __forceinline__ uint32_t asym_code(float x, const AsymParams& p) {
  float q = __builtin_rintf(div_rn(x - p.mn, p.scale, p.rscale));
  q = fminf(fmaxf(q, 0.0f), kAsymLevels);
  return (uint32_t)q;
}

__device__ __forceinline__ uint32_t asym_param_word(const AsymParams& p) {
  uint32_t s = __builtin_bit_cast(uint16_t, (_Float16)p.scale);
  uint32_t z = __builtin_bit_cast(uint16_t, (_Float16)p.mn);
  return s | (z << 16);
}

__device__ __forceinline__ float param_scale(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
}
__device__ __forceinline__ float param_zero(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// Restore of one page of one plane; even planes are K, odd planes V (tiled
// layout).  Items:
//  K: (head, token, group): 16 code bytes + 1 param word -> 32 outputs of a row
//  V: (head, 8-dim block, token half): 32 code bytes + 8 param words ->
//     8 tokens x 8 dims.
#ifndef AMF_ASYM_K_UNROLL
#define AMF_ASYM_K_UNROLL 4
#endif
constexpr int kKUnroll = AMF_ASYM_K_UNROLL;

template <int DT>
__global__ __launch_bounds__(kThreads) void int4_asym_dequant_scatter_kernel(
    const uint64_t* __restrict__ code_planes, const uint64_t* __restrict__ param_planes,
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, AsymGeom g, int32_t* err_flag) {
  // A (page, plane) grid, page-major: all XCDs work on one plane at a time,
  // which measured faster here than the XCD-contiguous map of the other
  // restores (1.025 vs 1.065 ms at 32 layers x 2048 pages).
  const int64_t j = blockIdx.x;
  const int plane = blockIdx.y;
  const bool is_v = (plane & 1) != 0;
  const int64_t dp = block_ids ? (int64_t)block_ids[j] : j;
  if (dp < 0 || dp >= pool) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  const int H = g.num_heads, D = g.head_dim, G = g.groups;
  const uint8_t* __restrict__ codes = reinterpret_cast<const uint8_t*>(code_planes[plane]) +
                                      j * (int64_t)H * g.hb_code_bytes;
  const uint32_t* __restrict__ params = reinterpret_cast<const uint32_t*>(param_planes[plane]) +
                                        j * (int64_t)H * g.hb_param_words;
  uint8_t* __restrict__ out = reinterpret_cast<uint8_t*>(cache_planes[plane]) + dp * cache_stride;

  if (!is_v) {
    // Items (token, head, 8-dim block) in cache order: lane k writes the k-th
    // 16-byte vector of the page, reads 4 code bytes and its group's param word.
    // kKUnroll items per lane have their code and param loads in flight
    // before any is converted.
    const int kpr = D / 8;  // 8-dim blocks per row
    const int n_items = 16 * H * kpr;
    for (int it0 = threadIdx.x; it0 < n_items; it0 += kThreads * kKUnroll) {
      uint32_t c[kKUnroll], pw[kKUnroll];
#pragma unroll
      for (int u = 0; u < kKUnroll; ++u) {
        const int it = it0 + u * kThreads;
        if (it < n_items) {
          const int kk = it % kpr;
          const int th = it / kpr;  // token * H + head
          const int t = th / H, h = th % H;
          const int ht = h * 16 + t;
          c[u] = ld_stream(reinterpret_cast<const uint32_t*>(codes + (int64_t)ht * (D / 2)) + kk);
          pw[u] = params[ht * G + (kk >> 2)];
        }
      }
#pragma unroll
      for (int u = 0; u < kKUnroll; ++u) {
        const int it = it0 + u * kThreads;
        if (it < n_items) {
          const float s = param_scale(pw[u]), z = param_zero(pw[u]);
          float x[8];
#pragma unroll
          for (int n = 0; n < 8; ++n) x[n] = nib(c[u], n) * s + z;
          store8<DT>(out + (int64_t)it * (8 * elem_bytes<DT>()), x);
        }
      }
    }
  } else {
    const int nb = D / 8;
    const int n_items = H * nb * 2;
    for (int it = threadIdx.x; it < n_items; it += kThreads) {
      const int th = it & 1;
      const int b = (it >> 1) % nb;
      const int h = (it >> 1) / nb;
      const u32x4* cp =
          reinterpret_cast<const u32x4*>(codes + (int64_t)h * g.hb_code_bytes + 64 * b + 32 * th);
      const u32x4 c0 = ld_stream(cp);
      const u32x4 c1 = ld_stream(cp + 1);
      const uint32_t w[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
      const u32x4* pp = reinterpret_cast<const u32x4*>(params + h * g.hb_param_words +
                                                       (b >> 2) * 16 + 8 * th);
      const u32x4 p0 = pp[0], p1 = pp[1];
      const uint32_t pw[8] = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float s = param_scale(pw[i]), z = param_zero(pw[i]);
        float x[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = nib(w[k], i) * s + z;
        const int t = 8 * th + i;
        store8<DT>(out + elem_bytes<DT>() * ((int64_t)(t * H + h) * D + 8 * b), x);
      }
    }
  }
}

// Save of one page of a K plane: items (head, token, group) read 64 cache
// bytes, write 16 code bytes and one param word.
#ifndef AMF_ASYM_KSAVE_UNROLL
#define AMF_ASYM_KSAVE_UNROLL 2
#endif
constexpr int kKSaveUnroll = AMF_ASYM_KSAVE_UNROLL;
template <int DT>
__device__ __forceinline__ void asym_quant_k(const uint8_t* __restrict__ src,
                                             uint8_t* __restrict__ codes,
                                             uint32_t* __restrict__ params, const AsymGeom& g) {
  const int H = g.num_heads, D = g.head_dim, G = g.groups;
  const int n_items = 16 * H * G;
  // Items in cache order (token, head, group) so the loads are contiguous;
  // kKSaveUnroll items per lane are loaded before any is quantized.
  for (int it0 = threadIdx.x; it0 < n_items; it0 += kThreads * kKSaveUnroll) {
    float x[kKSaveUnroll][32];
#pragma unroll
    for (int u = 0; u < kKSaveUnroll; ++u) {
      const int it = it0 + u * kThreads;
      if (it < n_items)
        load32<DT>(src + elem_bytes<DT>() * ((int64_t)(it / G) * D + 32 * (it % G)), x[u]);
    }
#pragma unroll
    for (int u = 0; u < kKSaveUnroll; ++u) {
      const int it = it0 + u * kThreads;
      if (it < n_items) {
        const int gi = it % G;
        const int th = it / G;  // token * H + head
        const int t = th / H, h = th % H;
        const AsymParams p = asym_params(x[u]);
        u32x4 c;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t w = 0;
#pragma unroll
          for (int n = 0; n < 8; ++n) w |= asym_code(x[u][8 * q + n], p) << (4 * n);
          c[q] = w;
        }
        const int ht = h * 16 + t;
        st_stream(c, reinterpret_cast<u32x4*>(codes + (int64_t)ht * (D / 2) + 16 * gi));
        params[ht * G + gi] = asym_param_word(p);
      }
    }
  }
}

// Save of one page of a V plane.  Groups run along head_dim while the code
// tiles run along tokens: phase 1 computes every group's (mn, scale) into LDS
// tables, phase 2 builds the 8-token x 8-dim tiles.  STAGED copies the page
// into LDS first (when it fits); otherwise both phases read the page from
// global memory, where the second read hits in cache.
constexpr int kAsymLdsBytes = 64 * 1024;
#ifndef AMF_ASYM_STAGE_UNROLL
#define AMF_ASYM_STAGE_UNROLL 8
#endif
constexpr int kStageUnroll = AMF_ASYM_STAGE_UNROLL;

template <int DT, bool STAGED>
__device__ __forceinline__ void asym_quant_v(const uint8_t* __restrict__ src,
                                             uint8_t* __restrict__ codes,
                                             uint32_t* __restrict__ params, const AsymGeom& g,
                                             uint8_t* lds) {
  constexpr int ES = elem_bytes<DT>();
  const int H = g.num_heads, D = g.head_dim, G = g.groups;
  const int page_bytes = STAGED ? 16 * H * D * ES : 0;
  // phase 0: page -> LDS (cache layout)
  if (STAGED) {
    // kStageUnroll vectors per lane in flight before they are stored to LDS.
    for (int o0 = threadIdx.x * 16; o0 < page_bytes; o0 += kThreads * 16 * kStageUnroll) {
      u32x4 v[kStageUnroll];
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int o = o0 + u * kThreads * 16;
        if (o < page_bytes) v[u] = ld_stream(reinterpret_cast<const u32x4*>(src + o));
      }
#pragma unroll
      for (int u = 0; u < kStageUnroll; ++u) {
        const int o = o0 + u * kThreads * 16;
        if (o < page_bytes) *reinterpret_cast<u32x4*>(lds + o) = v[u];
      }
    }
  }
  const uint8_t* data = STAGED ? lds : src;
  float* s_mn = reinterpret_cast<float*>(lds + page_bytes);          // [H][G][16]
  float* s_sc = s_mn + 16 * H * G;                                   // [H][G][16]
  float* s_rc = s_sc + 16 * H * G;                                   // [H][G][16]
  __syncthreads();
  const int n_groups = 16 * H * G;
  for (int it = threadIdx.x; it < n_groups; it += kThreads) {
    // it = (head, group, token): params are written in V order.
    const int t = it & 15;
    const int hg = it >> 4;
    const int h = hg / G, gi = hg % G;
    float x[32];
    load32<DT>(data + ES * ((t * H + h) * D + 32 * gi), x);
    const AsymParams p = asym_params(x);
    s_mn[it] = p.mn;
    s_sc[it] = p.scale;
    s_rc[it] = p.rscale;
    params[it] = asym_param_word(p);
  }
  __syncthreads();
  const int nb = D / 8;
  const int n_items = H * nb * 2;
  for (int it = threadIdx.x; it < n_items; it += kThreads) {
    const int th = it & 1;
    const int b = (it >> 1) % nb;
    const int h = (it >> 1) / nb;
    uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = 8 * th + i;
      const int pi = (h * G + (b >> 2)) * 16 + t;
      AsymParams p;
      p.mn = s_mn[pi];
      p.scale = s_sc[pi];
      p.rscale = s_rc[pi];
      float x[8];
      load8<DT>(data + ES * ((t * H + h) * D + 8 * b), x);
#pragma unroll
      for (int k = 0; k < 8; ++k) w[k] |= asym_code(x[k], p) << (4 * i);
    }
    u32x4* cp = reinterpret_cast<u32x4*>(codes + (int64_t)h * g.hb_code_bytes + 64 * b + 32 * th);
    st_stream(u32x4{w[0], w[1], w[2], w[3]}, cp);
    st_stream(u32x4{w[4], w[5], w[6], w[7]}, cp + 1);
  }
}

template <int DT, bool STAGED>
__global__ __launch_bounds__(kThreads) void int4_asym_quant_gather_kernel(
    const uint64_t* __restrict__ cache_planes, int64_t cache_stride,
    const int32_t* __restrict__ block_ids, int64_t pool, const uint64_t* __restrict__ code_planes,
    const uint64_t* __restrict__ param_planes, AsymGeom g, int32_t* err_flag) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int64_t j = blockIdx.x;
  const int plane = blockIdx.y;
  const int64_t sp = block_ids ? (int64_t)block_ids[j] : j;
  if (sp < 0 || sp >= pool) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  const int H = g.num_heads;
  const uint8_t* __restrict__ src =
      reinterpret_cast<const uint8_t*>(cache_planes[plane]) + sp * cache_stride;
  uint8_t* __restrict__ codes =
      reinterpret_cast<uint8_t*>(code_planes[plane]) + j * (int64_t)H * g.hb_code_bytes;
  uint32_t* __restrict__ params =
      reinterpret_cast<uint32_t*>(param_planes[plane]) + j * (int64_t)H * g.hb_param_words;
  if ((plane & 1) == 0) {
    if (STAGED) {
      // The page enters LDS by whole-line non-temporal loads (1 KiB per wave
      // instruction); the items' 64-byte reads then come from LDS.  Reading
      // the items straight from memory splits every line over four load
      // instructions, which the non-temporal policy would fetch repeatedly.
      const int page_bytes = 16 * H * g.head_dim * elem_bytes<DT>();
      for (int o0 = threadIdx.x * 16; o0 < page_bytes; o0 += kThreads * 16 * kStageUnroll) {
        u32x4 v[kStageUnroll];
#pragma unroll
        for (int u = 0; u < kStageUnroll; ++u) {
          const int o = o0 + u * kThreads * 16;
          if (o < page_bytes) v[u] = ld_stream(reinterpret_cast<const u32x4*>(src + o));
        }
#pragma unroll
        for (int u = 0; u < kStageUnroll; ++u) {
          const int o = o0 + u * kThreads * 16;
          if (o < page_bytes) *reinterpret_cast<u32x4*>(lds + o) = v[u];
        }
      }
      __syncthreads();
      asym_quant_k<DT>(lds, codes, params, g);
    } else {
      asym_quant_k<DT>(src, codes, params, g);
    }
  } else {
    asym_quant_v<DT, STAGED>(src, codes, params, g, lds);
  }
}

int check_int4_format(const char* who, int32_t format) {
  if (format != AMF_FMT_INT4_SYM_BLOCK && format != AMF_FMT_INT4_SYM &&
      format != AMF_FMT_INT4_ASYM_G32)
    return fail(AMF_ERR_INVALID_ARG, "%s: format %d is not an INT4 format", who, format);
  return ok();
}

int make_sym_geom(const char* who, int32_t block_size, int32_t num_heads, int32_t head_dim,
                  int32_t pps, SymGeom* g) {
  const int cpr = head_dim / 32;
  if (cpr > kThreads || (cpr & (cpr - 1)) != 0)
    return fail(AMF_ERR_UNSUPPORTED, "%s: head_dim/32 = %d must be a power of two <= %d", who,
                cpr, kThreads);
  g->n_rows = block_size * num_heads;
  g->head_dim = head_dim;
  g->cpr_log2 = __builtin_ctz(cpr);
  g->pps = pps > 0 ? pps : 1;
  return ok();
}

// lds_staged: LDS of the V save with the page staged (the page in the cache
// dtype + three fp32 tables of 16*H*G entries); lds_tables: the tables alone.
int make_asym_geom(const char* who, int32_t block_size, int32_t num_heads, int32_t head_dim,
                   int32_t elem_size, int32_t n_planes, AsymGeom* g, size_t* lds_staged,
                   size_t* lds_tables) {
  if (block_size != 16)
    return fail(AMF_ERR_UNSUPPORTED, "%s: INT4_ASYM_G32 needs block_size 16 (got %d)", who,
                block_size);
  if (n_planes % 2 != 0)
    return fail(AMF_ERR_INVALID_ARG, "%s: INT4_ASYM_G32 needs (K, V) plane pairs", who);
  g->num_heads = num_heads;
  g->head_dim = head_dim;
  g->groups = head_dim / 32;
  g->hb_code_bytes = 16 * head_dim / 2;
  g->hb_param_words = 16 * g->groups;
  *lds_tables = (size_t)3 * 4 * 16 * num_heads * g->groups;
  *lds_staged = (size_t)16 * num_heads * head_dim * elem_size + *lds_tables;
  if (*lds_tables > (size_t)kAsymLdsBytes)
    return fail(AMF_ERR_UNSUPPORTED, "%s: %d heads x %d dims exceed the LDS parameter tables", who,
                num_heads, head_dim);
  return ok();
}

}  // namespace

extern "C" int amf_int4_dequant_scatter(int32_t format, const uint64_t* code_planes,
                                        const uint64_t* param_planes, const uint64_t* cache_planes,
                                        int64_t cache_page_stride, int32_t cache_dtype,
                                        const int32_t* block_ids, int64_t pool_pages,
                                        int32_t n_planes, int64_t n_pages, int32_t block_size,
                                        int32_t num_heads, int32_t head_dim, int32_t* err_flag,
                                        void* stream) {
  const char* who = "amf_int4_dequant_scatter";
  int rc = check_int4_format(who, format);
  if (rc) return rc;
  rc = check_codec_geometry(who, cache_planes, cache_page_stride, cache_dtype, block_ids,
                            pool_pages, code_planes, param_planes, n_planes, n_pages, block_size,
                            num_heads, head_dim);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
  if (n_pages * n_planes > 0x7FFFFFF0ll)
    return fail(AMF_ERR_UNSUPPORTED, "%s: %lld pages x %d planes exceed one launch", who,
                (long long)n_pages, n_planes);
  if (format == AMF_FMT_INT4_ASYM_G32) {
    AsymGeom g;
    size_t lds_staged, lds_tables;
    if ((rc = make_asym_geom(who, block_size, num_heads, head_dim, cache_elem_bytes(cache_dtype),
                             n_planes, &g, &lds_staged, &lds_tables)))
      return rc;
    if (n_pages == 0) return ok();
    AMF_WITH_DTYPE(cache_dtype,
                   int4_asym_dequant_scatter_kernel<DT>
                   <<<dim3((unsigned)n_pages, (unsigned)n_planes), kThreads, 0, s>>>(
                       code_planes, param_planes, cache_planes, cache_page_stride, block_ids,
                       pool_pages, g, err_flag));
    return check_launch(who);
  }
  SymGeom g;
  if ((rc = make_sym_geom(who, block_size, num_heads, head_dim, 1, &g))) return rc;
  const bool ch = format == AMF_FMT_INT4_SYM;
  if (ch && (8 * kThreads) % head_dim != 0)
    return fail(AMF_ERR_UNSUPPORTED, "%s: head_dim %d must divide %d", who, head_dim, 8 * kThreads);
  if (n_pages == 0) return ok();
  // pages beyond 8 workgroup passes are split over workgroups of 8 passes
  const int64_t n8 = (int64_t)g.n_rows * g.head_dim / 8;
  const int parts = (int)std::max<int64_t>(1, n8 / (8 * kThreads));
  if (n_pages * parts * n_planes > 0x7FFFFFF0ll)
    return fail(AMF_ERR_UNSUPPORTED, "%s: %lld pages x %d parts x %d planes exceed one launch",
                who, (long long)n_pages, parts, n_planes);
  const dim3 sgrid = xcd_page_grid(n_pages * parts, n_planes);
#define AMF_LAUNCH(C)                                                                        \
  int4_sym_dequant_scatter_kernel<DT, C><<<sgrid, kThreads, 0, s>>>(                          \
      code_planes, param_planes, cache_planes, cache_page_stride, block_ids, pool_pages,      \
      n_pages, n_planes, parts, g, err_flag)
  AMF_WITH_DTYPE(cache_dtype, if (ch) AMF_LAUNCH(true); else AMF_LAUNCH(false));
#undef AMF_LAUNCH
  return check_launch(who);
}

extern "C" int amf_int4_quant_gather(int32_t format, const uint64_t* cache_planes,
                                     int64_t cache_page_stride, int32_t cache_dtype,
                                     const int32_t* block_ids, int64_t pool_pages,
                                     const uint64_t* code_planes, const uint64_t* param_planes,
                                     int32_t n_planes, int32_t planes_per_scale, int64_t n_pages,
                                     int32_t block_size, int32_t num_heads, int32_t head_dim,
                                     float* workspace,
                                     int64_t workspace_bytes, int32_t* err_flag, void* stream) {
  const char* who = "amf_int4_quant_gather";
  int rc = check_int4_format(who, format);
  if (rc) return rc;
  rc = check_codec_geometry(who, cache_planes, cache_page_stride, cache_dtype, block_ids,
                            pool_pages, code_planes, param_planes, n_planes, n_pages, block_size,
                            num_heads, head_dim);
  if (rc) return rc;
  const bool bf16 = cache_dtype == AMF_DTYPE_BF16;
  hipStream_t s = as_stream(stream);
  dim3 grid((unsigned)n_pages, (unsigned)n_planes);
  if (format == AMF_FMT_INT4_ASYM_G32) {
    AsymGeom g;
    size_t lds_staged, lds_tables;
    if ((rc = make_asym_geom(who, block_size, num_heads, head_dim, cache_elem_bytes(cache_dtype),
                             n_planes, &g, &lds_staged, &lds_tables)))
      return rc;
    if (n_pages == 0) return ok();
    const bool staged = lds_staged <= (size_t)kAsymLdsBytes;
#define AMF_LAUNCH(ST)                                                                         \
  int4_asym_quant_gather_kernel<DT, ST><<<grid, kThreads, ST ? lds_staged : lds_tables, s>>>(  \
      cache_planes, cache_page_stride, block_ids, pool_pages, code_planes, param_planes, g, \
      err_flag)
    AMF_WITH_DTYPE(cache_dtype, if (staged) AMF_LAUNCH(true); else AMF_LAUNCH(false));
#undef AMF_LAUNCH
    return check_launch(who);
  }
  if (format == AMF_FMT_INT4_SYM &&
      (planes_per_scale <= 0 || n_planes % planes_per_scale != 0))
    return fail(AMF_ERR_INVALID_ARG, "%s: planes_per_scale %d does not divide n_planes %d", who,
                planes_per_scale, n_planes);
  SymGeom g;
  if ((rc = make_sym_geom(who, block_size, num_heads, head_dim, planes_per_scale, &g))) return rc;
  if (n_pages == 0) return ok();
  if (format == AMF_FMT_INT4_SYM_BLOCK) {
    const int64_t n8 = (int64_t)g.n_rows * g.head_dim / 8;
    const int64_t cpl = (n8 + kThreads - 1) / kThreads;  // chunks per lane
    // Pages that fit lanes' registers (up to 32 chunks of 8 elements per lane)
    // take the single-read kernel; larger pages and fp32 caches the two-read one.
    if (cpl > 32 || cache_dtype == AMF_DTYPE_F32) {
      AMF_WITH_DTYPE(cache_dtype, int4_symblock_quant_looped_kernel<DT><<<grid, kThreads, 0, s>>>(
                                      cache_planes, cache_page_stride, block_ids, pool_pages,
                                      code_planes, param_planes, g, err_flag));
      return check_launch(who);
    }
#define AMF_LAUNCH(B, C)                                                                        \
  int4_symblock_quant_gather_kernel<B, C><<<grid, kThreads, 0, s>>>(                            \
      cache_planes, cache_page_stride, block_ids, pool_pages, code_planes, param_planes, g, \
      err_flag)
#define AMF_LAUNCH_R(B)                     \
  if (cpl <= 1) AMF_LAUNCH(B, 1);           \
  else if (cpl <= 2) AMF_LAUNCH(B, 2);      \
  else if (cpl <= 4) AMF_LAUNCH(B, 4);      \
  else if (cpl <= 8) AMF_LAUNCH(B, 8);      \
  else if (cpl <= 16) AMF_LAUNCH(B, 16);    \
  else AMF_LAUNCH(B, 32)
    if (bf16) { AMF_LAUNCH_R(true); } else { AMF_LAUNCH_R(false); }
#undef AMF_LAUNCH_R
#undef AMF_LAUNCH
    return check_launch(who);
  }
  // AMF_FMT_INT4_SYM: absmax pass, then the quant pass (which also writes the fp16 scales).
  if (head_dim > 1024) return fail(AMF_ERR_UNSUPPORTED, "%s: head_dim > 1024", who);
  const int64_t need = amf_quant_workspace_bytes(format, n_planes, planes_per_scale, head_dim);
  if (!workspace || workspace_bytes < need)
    return fail(AMF_ERR_WORKSPACE, "%s: needs %lld workspace bytes", who, (long long)need);
  uint32_t* ws = reinterpret_cast<uint32_t*>(workspace);
  const int64_t n_ws = need / 4;
  fill_u32_kernel<<<(unsigned)((n_ws + 255) / 256), 256, 0, s>>>(ws, n_ws, 0u);
#ifndef AMF_ABSMAX_WGS
#define AMF_ABSMAX_WGS 64
#endif
  dim3 rgrid((unsigned)(n_pages < AMF_ABSMAX_WGS ? n_pages : AMF_ABSMAX_WGS), (unsigned)n_planes);
  AMF_WITH_DTYPE(cache_dtype, int4_channel_absmax_kernel<DT><<<rgrid, kThreads, 0, s>>>(
                                  cache_planes, cache_page_stride, block_ids, pool_pages, n_pages,
                                  g, ws, err_flag));
  AMF_WITH_DTYPE(cache_dtype, int4_channel_quant_gather_kernel<DT><<<grid, kThreads, 0, s>>>(
                                  cache_planes, cache_page_stride, block_ids, pool_pages,
                                  code_planes, param_planes, g, ws, err_flag));
  return check_launch(who);
}
