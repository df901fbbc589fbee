// amf_attn.hip - dense scaled-dot-product attention over plain K/V rows, or
// over INT4_SYM codes dequantized in registers: the positional path of
// int4_decode_attention.
//
// Computes out = softmax(q k^T * scale + mask) v for every query row, the
// result of korith_vllm_ext/kernels/dispatch.py:117-143 (fallback_fp16_kernel,
// which the reference's dispatch returns for every format on every device),
// in fp32 with one rounding to the output dtype at the end.  GQA is accepted
// (num_q_heads a multiple of num_kv_heads); the reference's matmul broadcast
// allows only equal head counts or a single KV head.
//
// Split path (head_dim 64, 128 or 256, a caller workspace): flash decoding.
// The KV tokens of a row are cut into splits sized so that the launch has
// about kSplitWaves waves; one wave per (up to 4 query heads of a GQA group,
// split) streams its tokens in batches of wave loads, each K/V row loaded
// (and dequantized) once for all its heads.  A K or V row is D / 8 lanes
// wide (16-byte loads, 8 elements per lane), so one wave load covers
// 64 / (D / 8) whole rows; the score of a token is a reduction over its
// row's lanes, the online softmax runs per lane on its rows' scores, and the
// PV product accumulates 8 dims per lane and head.  Each split leaves (max,
// sum, acc[D]) per head in the workspace and a merge kernel combines a row's
// splits with an LSE rescale.  The waves of one KV head's group run on one
// XCD, so what they share is read from HBM about once.  INT4_SYM K/V at
// head_dim 128 with bf16 / fp16 queries and no mask take an MFMA form of the
// split kernel (int4_sym_attn_mfma_kernel, described where it is defined)
// with the same splits, partials and merge.
//
// Single-pass path (other head dims, kv_len 0, or no workspace): one
// workgroup (4 waves) per query row.  Wave w takes the 64-token chunks w,
// w+4, w+8, ...; lane l scores token chunk_base + l against the query held in
// LDS, the wave keeps an online softmax (running max and sum), and the PV
// product is lane-parallel over head_dim with the chunk's probabilities
// broadcast by readlane.  The four partial (max, sum, acc) triples are merged
// through LDS.
#include <math.h>

#include <algorithm>

#include "amf_internal.h"
#include "amf_kernel_util.h"

namespace {

using amf::u32x4;
using amf::f32x4;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxD = 256;
constexpr int kAccPerLane = kMaxD / 64;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* mask;
  int64_t ms0, ms1, ms2, ms3;  // mask strides over (batch, q head, q row, kv token)
  void* out;
  int64_t batch;
  int32_t num_q_heads, num_kv_heads;
  int64_t q_len, kv_len;
  int32_t head_dim;
  float scale;
  // INT4_SYM K/V (split path only): k and v point at packed codes (element
  // 8 w + n of a row in nibble n of code word w), these at the fp16
  // per-channel scales [head_dim].
  const _Float16* k_scales;
  const _Float16* v_scales;
};

template <int DT>
__device__ __forceinline__ float elem(const void* p, int64_t i) {
  if constexpr (DT == AMF_DTYPE_F32) {
    return static_cast<const float*>(p)[i];
  } else {
    const uint16_t h = static_cast<const uint16_t*>(p)[i];
    if constexpr (DT == AMF_DTYPE_BF16) {
      return amf::u2f((uint32_t)h << 16);
    } else {
      return (float)__builtin_bit_cast(_Float16, h);
    }
  }
}

// Eight consecutive elements starting at element i (i a multiple of 8, row
// bases 16-byte aligned: checked on the host).
template <int DT>
__device__ __forceinline__ void elem8(const void* p, int64_t i, float (&x)[8]) {
  if constexpr (DT == AMF_DTYPE_F32) {
    const f32x4* q = reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
    const f32x4 a = q[0], b = q[1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
    const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p) + i);
    constexpr bool BF = DT == AMF_DTYPE_BF16;
    x[0] = amf::half_lo<BF>(w.x); x[1] = amf::half_hi<BF>(w.x);
    x[2] = amf::half_lo<BF>(w.y); x[3] = amf::half_hi<BF>(w.y);
    x[4] = amf::half_lo<BF>(w.z); x[5] = amf::half_hi<BF>(w.z);
    x[6] = amf::half_lo<BF>(w.w); x[7] = amf::half_hi<BF>(w.w);
  }
}

template <int OUT_DT>
__device__ __forceinline__ void store_out(void* out, int64_t i, float x) {
  if constexpr (OUT_DT == AMF_DTYPE_F32) {
    static_cast<float*>(out)[i] = x;
  } else if constexpr (OUT_DT == AMF_DTYPE_BF16) {
    static_cast<uint16_t*>(out)[i] = __builtin_bit_cast(uint16_t, (__bf16)x);
  } else {
    amf::keep_f32(x);
    static_cast<uint16_t*>(out)[i] = __builtin_bit_cast(uint16_t, (_Float16)x);
  }
}

__device__ __forceinline__ float wave_sum(float x) {
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

template <int DT, int OUT_DT, bool VEC8>
__global__ __launch_bounds__(kThreads) void dense_attn_kernel(AttnArgs a) {
  __shared__ float q_s[kMaxD];
  __shared__ float m_s[kWaves], l_s[kWaves];
  __shared__ float acc_s[kWaves][kMaxD];

  const int64_t row = blockIdx.x;  // (b, h, tq) flattened
  const int64_t tq = row % a.q_len;
  const int64_t bh = row / a.q_len;
  const int h = (int)(bh % a.num_q_heads);
  const int64_t b = bh / a.num_q_heads;
  const int hkv = h / (a.num_q_heads / a.num_kv_heads);
  const int D = a.head_dim;
  const int64_t T = a.kv_len;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

  for (int d = tid; d < D; d += kThreads) q_s[d] = elem<DT>(a.q, row * D + d);
  __syncthreads();

  const int64_t kv_base = (b * a.num_kv_heads + hkv) * T;  // first token row of this (b, hkv)
  const float* mrow = a.mask ? a.mask + b * a.ms0 + (int64_t)h * a.ms1 + tq * a.ms2 : nullptr;

  float m_run = -INFINITY, l_run = 0.0f;
  float acc[kAccPerLane];
#pragma unroll
  for (int j = 0; j < kAccPerLane; ++j) acc[j] = 0.0f;

  for (int64_t t0 = (int64_t)w * 64; t0 < T; t0 += (int64_t)kWaves * 64) {
    const int64_t t = t0 + lane;
    float s = -INFINITY;
    if (t < T) {
      const int64_t kr = (kv_base + t) * D;
      float dot = 0.0f;
      if constexpr (VEC8) {
        for (int d = 0; d < D; d += 8) {
          float x[8];
          elem8<DT>(a.k, kr + d, x);
#pragma unroll
          for (int e = 0; e < 8; ++e) dot = fmaf(q_s[d + e], x[e], dot);
        }
      } else {
        for (int d = 0; d < D; ++d) dot = fmaf(q_s[d], elem<DT>(a.k, kr + d), dot);
      }
      s = dot * a.scale;
      if (mrow) s += mrow[t * a.ms3];
      s *= kLog2e;
    }
    float m_chunk = s;
    for (int off = 32; off > 0; off >>= 1) m_chunk = fmaxf(m_chunk, __shfl_xor(m_chunk, off));
    const float m_new = fmaxf(m_run, m_chunk);
    if (m_new == -INFINITY) continue;  // every score so far is -inf (wave-uniform)
    const float alpha = exp2f(m_run - m_new);
    const float p = (s == -INFINITY) ? 0.0f : exp2f(s - m_new);
    l_run = l_run * alpha + wave_sum(p);
#pragma unroll
    for (int j = 0; j < kAccPerLane; ++j) acc[j] *= alpha;
    const int n = (int)min<int64_t>(64, T - t0);
    for (int tt = 0; tt < n; ++tt) {
      const float pt = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), tt));
      const int64_t vr = (kv_base + t0 + tt) * D;
#pragma unroll
      for (int j = 0; j < kAccPerLane; ++j) {
        const int d = lane + 64 * j;
        if (d < D) acc[j] = fmaf(pt, elem<DT>(a.v, vr + d), acc[j]);
      }
    }
    m_run = m_new;
  }

  if (lane == 0) {
    m_s[w] = m_run;
    l_s[w] = l_run;
  }
#pragma unroll
  for (int j = 0; j < kAccPerLane; ++j) {
    const int d = lane + 64 * j;
    if (d < D) acc_s[w][d] = acc[j];
  }
  __syncthreads();

  for (int d = tid; d < D; d += kThreads) {
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) M = fmaxf(M, m_s[i]);
    float num = 0.0f, den = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int i = 0; i < kWaves; ++i) {
        if (m_s[i] == -INFINITY) continue;
        const float f = exp2f(m_s[i] - M);
        num = fmaf(acc_s[i][d], f, num);
        den = fmaf(l_s[i], f, den);
      }
    }
    // T == 0: empty softmax, empty sum -> 0 (as matmul over a zero-length
    // axis); a row whose scores are all -inf -> NaN (as softmax gives).
    const float o = (T == 0) ? 0.0f : num / den;
    store_out<OUT_DT>(a.out, row * D + d, o);
  }
}

// ---------------------------------------------------------- split path --

#ifndef AMF_DENSE_SPLIT_WAVES
#define AMF_DENSE_SPLIT_WAVES 2048
#endif
#ifndef AMF_DENSE_MIN_CHUNKS
#define AMF_DENSE_MIN_CHUNKS 1
#endif
constexpr int64_t kSplitWaves = AMF_DENSE_SPLIT_WAVES;  // waves one launch aims for
constexpr int64_t kMinChunks = AMF_DENSE_MIN_CHUNKS;     // 64-token chunks per split, at least
constexpr int kPartPad = 4;            // a split partial: acc[D], m, l, 2 pad (16-byte rows)
constexpr int64_t kXcds = 8;           // XCDs of the chip, dealt workgroups round-robin

// Query heads one wave of the split kernel serves: up to 4 of a GQA group
// of G, so that it loads (and for INT4 dequantizes) each K/V row once for
// all of them.
inline int heads_per_wave(int32_t num_q_heads, int32_t num_kv_heads) {
  const int G = num_q_heads / num_kv_heads;
  return G % 4 == 0 ? 4 : G % 2 == 0 ? 2 : 1;
}

// Splits per row and tokens per split (a multiple of 64) for `rows` query
// rows, hpw of them per wave, over kv_len tokens: about kSplitWaves waves
// in all, at least kMinChunks and at most all 64-token chunks per split.
inline void dense_splits(int64_t rows, int hpw, int64_t kv_len, int64_t* n_splits,
                         int64_t* split_tokens) {
  const int64_t chunks = (kv_len + 63) / 64;
  const int64_t wave_rows = rows / hpw;
  int64_t n = (kSplitWaves + wave_rows - 1) / wave_rows;
  n = std::min<int64_t>(n, (chunks + kMinChunks - 1) / kMinChunks);
  n = std::max<int64_t>(1, std::min<int64_t>(n, chunks));
  const int64_t per = (chunks + n - 1) / n;  // chunks per split
  *split_tokens = per * 64;
  *n_splits = (chunks + per - 1) / per;
}

inline bool split_head_dim(int32_t D) { return D == 64 || D == 128 || D == 256; }

// Sum over the LPR lanes of a row group (lanes LPR g .. LPR g + LPR - 1).
template <int LPR>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (LPR == 16) {
    // DPP rotates within 16-lane rows: every lane of the row gets the sum
    int v = __builtin_bit_cast(int, x);
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false));
    v = __builtin_bit_cast(int, x);
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false));
    v = __builtin_bit_cast(int, x);
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x122, 0xF, 0xF, false));
    v = __builtin_bit_cast(int, x);
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x121, 0xF, 0xF, false));
    return x;
  } else {
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) x += __shfl_xor(x, o);
    return x;
  }
}

// Sum / max over the row groups (lanes with the same lane % LPR).
template <int LPR>
__device__ __forceinline__ float across_groups_sum(float x) {
#pragma unroll
  for (int o = LPR; o < 64; o <<= 1) x += __shfl_xor(x, o);
  return x;
}
template <int LPR>
__device__ __forceinline__ float across_groups_max(float x) {
#pragma unroll
  for (int o = LPR; o < 64; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

// INT4 = true: K and V are INT4_SYM codes, dequantized as the codec's restore
// does, (code - 8) * scale in fp32 rounded to DT (the dtype the restore would
// write and q's dtype), so the scores see the values a decompressed tensor
// holds.  (code - 8) * s is taken as fma(code, s, -8 s): the exact product
// fits fp32 (4 + 11 bits), so the single rounding of the fma is exact too.
// The nibbles go to bytes first (even elements in w & 0x0F0F0F0F, odd ones
// in (w >> 4) & 0x0F0F0F0F), so that v_cvt_f32_ubyte0..3 convert them; the
// empty asm keeps the compiler from folding that back into a bit-field
// extract per element.
template <int DT>
__device__ __forceinline__ float round_to(float y) {
  if constexpr (DT == AMF_DTYPE_BF16) {
    return (float)(__bf16)y;
  } else if constexpr (DT == AMF_DTYPE_F16) {
    amf::keep_f32(y);
    return (float)(_Float16)y;
  } else {
    return y;
  }
}

// The 8 exact products (code - 8) * scale of one code word, before rounding.
__device__ __forceinline__ void int4_sym_vals(uint32_t w, const float (&s)[8], const float (&z)[8],
                                              float (&y)[8]) {
  uint32_t ev = w & 0x0F0F0F0Fu, od = (w >> 4) & 0x0F0F0F0Fu;
  asm("" : "+v"(ev));
  asm("" : "+v"(od));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    y[2 * i] = __builtin_fmaf((float)((ev >> (8 * i)) & 0xFFu), s[2 * i], z[2 * i]);
    y[2 * i + 1] = __builtin_fmaf((float)((od >> (8 * i)) & 0xFFu), s[2 * i + 1], z[2 * i + 1]);
  }
}

// a.lo * b.lo + a.hi * b.hi + c for two bf16 or fp16 pairs (fp32 products
// and sum).
template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (DT == AMF_DTYPE_BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b),
                                  c, false);
}

// One lane's 8 elements of a K/V row as loaded (lane c of a row group holds
// dims 8c .. 8c + 7 of a head_dim-D row): a code word for INT4, else 16
// (bf16/fp16) or 32 (fp32) bytes.  decode() gives them as fp32; pairs()
// (bf16/fp16 only) as four DT pairs, elements 2i and 2i + 1 in word i.
template <int DT, bool INT4>
struct RawRow {  // bf16 / fp16
  u32x4 w;
  static __device__ __forceinline__ RawRow load(const void* base, int64_t r, int c, int D) {
    return RawRow{*reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + r * D +
                                                  8 * c)};
  }
  __device__ __forceinline__ void decode(const float (&)[8], const float (&)[8],
                                         float (&x)[8]) const {
    amf::unpack8<DT == AMF_DTYPE_BF16>(w, x);
  }
  __device__ __forceinline__ void pairs(const float (&)[8], const float (&)[8],
                                        uint32_t (&pr)[4]) const {
    pr[0] = w.x;
    pr[1] = w.y;
    pr[2] = w.z;
    pr[3] = w.w;
  }
};

template <>
struct RawRow<AMF_DTYPE_F32, false> {
  f32x4 lo, hi;
  static __device__ __forceinline__ RawRow load(const void* base, int64_t r, int c, int D) {
    const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + r * D + 8 * c);
    return RawRow{p[0], p[1]};
  }
  __device__ __forceinline__ void decode(const float (&)[8], const float (&)[8],
                                         float (&x)[8]) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = lo[e];
      x[4 + e] = hi[e];
    }
  }
};

template <int DT>
struct RawRow<DT, true> {
  uint32_t w;
  static __device__ __forceinline__ RawRow load(const void* base, int64_t r, int c, int D) {
    return RawRow{static_cast<const uint32_t*>(base)[r * (D / 8) + c]};
  }
  __device__ __forceinline__ void decode(const float (&s)[8], const float (&z)[8],
                                         float (&x)[8]) const {
    float y[8];
    int4_sym_vals(w, s, z, y);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = round_to<DT>(y[e]);
  }
  __device__ __forceinline__ void pairs(const float (&s)[8], const float (&z)[8],
                                        uint32_t (&pr)[4]) const {
    float y[8];
    int4_sym_vals(w, s, z, y);
    // round to nearest even, as decode() and the restore do
#pragma unroll
    for (int i = 0; i < 4; ++i) pr[i] = amf::pack2<DT == AMF_DTYPE_BF16>(y[2 * i], y[2 * i + 1]);
  }
};

#ifndef AMF_DENSE_BATCH
#define AMF_DENSE_BATCH 8
#endif

// One wave per (query rows of GH heads of a GQA group, split).  LPR =
// head_dim / 8 lanes per K/V row, TPS = 64 / LPR rows per wave load; lane
// (g = lane / LPR, c = lane % LPR) holds elements 8c .. 8c + 7 of the GH
// query rows and, in step i of a batch, of K/V row t0 + TPS i + g, which it
// loads (and for INT4 dequantizes) once for all GH heads.
//
// Workgroup order: a unit is (b, KV head, tq, split), served by G / GH
// waves (G = Hq / Hkv).  Workgroups are dealt to the 8 XCDs round-robin by
// id, so unit u goes to XCD u % 8 and its waves take consecutive slots
// there: they share one L2.
template <int DT, int LPR, bool INT4, int GH>
__global__ __launch_bounds__(64) void dense_attn_split_kernel(AttnArgs a, float* part,
                                                              int64_t split_tokens,
                                                              int64_t n_splits, int64_t units) {
  constexpr int TPS = 64 / LPR;
  // Steps of a batch: its K (and, for INT4, V) loads are all issued before
  // the first is used.
  constexpr int SB = LPR < AMF_DENSE_BATCH ? LPR : AMF_DENSE_BATCH;
  constexpr int BT = TPS * SB;  // tokens per batch, divides 64
  using Raw = RawRow<DT, INT4>;
  const int lane = threadIdx.x, g = lane / LPR, c = lane % LPR;
  const int G = a.num_q_heads / a.num_kv_heads;
  const int W = G / GH;  // waves per unit
  const int64_t id = blockIdx.x, slot = id / kXcds;
  const int r = (int)(slot % W);
  const int64_t u = (slot / W) * kXcds + id % kXcds;
  if (u >= units) return;
  const int64_t split = u % n_splits, rest = u / n_splits;
  const int64_t tq = rest % a.q_len, bkv = rest / a.q_len;
  const int hkv = (int)(bkv % a.num_kv_heads);
  const int64_t b = bkv / a.num_kv_heads;
  const int h0 = hkv * G + r * GH;  // first of this wave's query heads
  const int D = 8 * LPR;
  const int64_t T = a.kv_len;
  const int64_t t_begin = split * split_tokens, t_end = min(T, t_begin + split_tokens);
  const int64_t kv_base = (b * a.num_kv_heads + hkv) * T;
  const float qs = a.scale * kLog2e;
  // query row of head h0 + j: (b, h0 + j, tq) flattened
  auto qrow = [&](int j) { return (b * a.num_q_heads + h0 + j) * a.q_len + tq; };

  // bf16 / fp16: scores are v_dot2 products of K pairs and the query's own
  // pairs, scaled afterwards; fp32: fma chains on the pre-scaled query.
  constexpr bool PK = DT != AMF_DTYPE_F32;
  float q[PK ? 1 : GH][8];
  uint32_t qp[PK ? GH : 1][4];
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    if constexpr (PK) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.q) +
                                                      qrow(j) * D + 8 * c);
      qp[j][0] = v.x;
      qp[j][1] = v.y;
      qp[j][2] = v.z;
      qp[j][3] = v.w;
    } else {
      elem8<DT>(a.q, qrow(j) * D + 8 * c, q[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) q[j][e] *= qs;
    }
  }
  // this lane's 8 channels' scales s and -8 s (INT4)
  float ksc[8], kz[8], vsc[8], vz[8];
  if constexpr (INT4) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ksc[e] = (float)a.k_scales[8 * c + e];
      vsc[e] = (float)a.v_scales[8 * c + e];
      kz[e] = -8.0f * ksc[e];
      vz[e] = -8.0f * vsc[e];
    }
  }
  float m_run[GH], l_run[GH];  // l_run: this lane's row group's tokens
  float acc[GH][8];
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    m_run[j] = -INFINITY;
    l_run[j] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.0f;
  }

  for (int64_t t0 = t_begin; t0 < t_end; t0 += BT) {
    Raw kr[SB];
    Raw vr[INT4 ? SB : 1];
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      const int64_t t = t0 + TPS * i + g;
      kr[i] = Raw::load(a.k, kv_base + (t < t_end ? t : t_begin), c, D);
    }
    if constexpr (INT4) {
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const int64_t t = t0 + TPS * i + g;
        vr[i] = Raw::load(a.v, kv_base + (t < t_end ? t : t_begin), c, D);
      }
    }
    float sc[GH][SB];
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      if constexpr (PK) {
        uint32_t kp[4];
        kr[i].pairs(ksc, kz, kp);
#pragma unroll
        for (int j = 0; j < GH; ++j) {
          float d = dot2<DT>(kp[0], qp[j][0], 0.0f);
          d = dot2<DT>(kp[1], qp[j][1], d);
          d = dot2<DT>(kp[2], qp[j][2], d);
          d = dot2<DT>(kp[3], qp[j][3], d);
          sc[j][i] = group_sum<LPR>(d) * qs;
        }
      } else {
        float x[8];
        kr[i].decode(ksc, kz, x);
#pragma unroll
        for (int j = 0; j < GH; ++j) {
          float d = q[j][0] * x[0];
#pragma unroll
          for (int e = 1; e < 8; ++e) d = fmaf(q[j][e], x[e], d);
          sc[j][i] = group_sum<LPR>(d);
        }
      }
    }
    if (a.mask) {  // additive mask, per head
#pragma unroll
      for (int j = 0; j < GH; ++j) {
        const float* mrow = a.mask + b * a.ms0 + (int64_t)(h0 + j) * a.ms1 + tq * a.ms2;
#pragma unroll
        for (int i = 0; i < SB; ++i) {
          const int64_t t = t0 + TPS * i + g;
          sc[j][i] = fmaf(mrow[(t < t_end ? t : t_begin) * a.ms3], kLog2e, sc[j][i]);
        }
      }
    }
    float m_new[GH];
    bool live = false;
#pragma unroll
    for (int j = 0; j < GH; ++j) {
#pragma unroll
      for (int i = 0; i < SB; ++i)
        if (t0 + TPS * i + g >= t_end) sc[j][i] = -INFINITY;
      float mc = sc[j][0];
#pragma unroll
      for (int i = 1; i < SB; ++i) mc = fmaxf(mc, sc[j][i]);
      mc = across_groups_max<LPR>(mc);
      m_new[j] = fmaxf(m_run[j], mc);
      live = live || m_new[j] != -INFINITY;
    }
    if (!live) continue;  // every score so far is -inf for every head (wave-uniform)
#pragma unroll
    for (int j = 0; j < GH; ++j) {
      // a head with every score so far -inf keeps l = 0, acc = 0
      const float alpha = m_new[j] == -INFINITY ? 1.0f : exp2f(m_run[j] - m_new[j]);
      l_run[j] *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[j][e] *= alpha;
    }
    Raw vd[INT4 ? 1 : SB];
    if constexpr (!INT4) {
      // dense V: loaded after the scores, all SB loads in flight together
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const int64_t t = t0 + TPS * i + g;
        vd[i] = Raw::load(a.v, kv_base + (t < t_end ? t : t_begin), c, D);
      }
    }
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      float x[8];
      if constexpr (INT4)
        vr[i].decode(vsc, vz, x);
      else
        vd[i].decode(vsc, vz, x);
#pragma unroll
      for (int j = 0; j < GH; ++j) {
        const float p = sc[j][i] == -INFINITY ? 0.0f : exp2f(sc[j][i] - m_new[j]);
        l_run[j] += p;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[j][e] = fmaf(p, x[e], acc[j][e]);
      }
    }
#pragma unroll
    for (int j = 0; j < GH; ++j) m_run[j] = m_new[j];
  }
  // the row groups hold disjoint tokens: add them up
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    const float l = across_groups_sum<LPR>(l_run[j]);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = across_groups_sum<LPR>(acc[j][e]);
    float* pr = part + (qrow(j) * n_splits + split) * (int64_t)(D + kPartPad);
    if (g == 0) {
      *reinterpret_cast<f32x4*>(pr + 8 * c) = f32x4{o[0], o[1], o[2], o[3]};
      *reinterpret_cast<f32x4*>(pr + 8 * c + 4) = f32x4{o[4], o[5], o[6], o[7]};
    }
    if (lane == 0) {
      pr[D] = m_run[j];
      pr[D + 1] = l;
    }
  }
}

// ---- INT4_SYM split kernel on MFMA tiles (head_dim 128, bf16/fp16 q, no mask) ----
//
// The INT4_SYM scales are per channel, so they fold into the query and the
// output: score = sum_d (q_d s_d) c_d - 8 sum_d q_d s_d and
// out_d = s_d sum_t p_t (c_td - 8) / l, with c the raw codes.  The codes
// enter v_mfma_f32_16x16x32_f16 as exact fp16 subnormals (c 2^-24; the high
// nibble of a byte pair comes out x16 and its partner operand carries 1/16),
// q s (exact in fp32: 8 or 11 by 11 bits) as an fp16 hi + lo pair that holds
// it exactly after a per-wave power-of-two scaling, and p as an fp16 hi + lo
// pair (22 bits).  The scores and PV sums are so exact products accumulated
// in fp32: attention over the exactly dequantized K/V, where the codec's
// restore rounds them to the cache dtype first.
//
// QK^T tile: rows = the wave's GH query heads (of 16; the other rows repeat
// row 0 and their scores are masked), k = 32 dims, columns = 16 tokens.  Lane (token lo, slice hi) loads 16 bytes of its
// token's code row, dims 32 hi .. 32 hi + 31, and word st of them is its B
// operand of k-step st (dims 32 hi + 8 st + 0..7); the query operand follows
// the same dim order.  PV needs tokens along k: an MFMA of the V codes (A:
// row = token, k = the 32 dims of word m of every slice) against a constant
// 0/1 selector (B: column c = one of 16 of those dims) transposes them, so
// lane (dim c, r) receives tokens 4 r .. 4 r + 3 of the tile as exact fp32
// (c - 8) 2^-24 (the -8 from the accumulator input), and the two 16-token
// tiles of a chunk give the 8 tokens of its PV k-slice, converted back to
// fp16 exactly.  Output dim of (word m, selector half h, column c):
// 32 (2 h + c / 8) + 8 m + c % 8.
constexpr float kNegBigAttn = -1.0e30f;
constexpr float kRescaleSlackAttn = 8.0f;  // p <= 2^8 between rescales

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma_f16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pk_f16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((amf::f32x2){a, b}, f16x2_t));
}

// 8 nibbles of w as fp16 subnormals in the operand order
// [n0 n4 n1 n5 n2 n6 n3 n7]: even nibbles c 2^-24, odd ones 16 c 2^-24.
__host__ __device__ constexpr int nib_of_k16(int k) { return (k >> 1) + 4 * (k & 1); }
__host__ __device__ constexpr bool k16_x16(int k) { return (k & 2) != 0; }
__device__ __forceinline__ u32x4 nib8_to_f16_sub(uint32_t w) {
  const uint32_t w8 = w >> 8;
  return u32x4{w & 0x000F000Fu, w & 0x00F000F0u, w8 & 0x000F000Fu, w8 & 0x00F000F0u};
}

__device__ __forceinline__ float row_max16(float x) {
  int v = __builtin_bit_cast(int, x);
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false)));
  v = __builtin_bit_cast(int, x);
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false)));
  v = __builtin_bit_cast(int, x);
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x122, 0xF, 0xF, false)));
  v = __builtin_bit_cast(int, x);
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x121, 0xF, 0xF, false)));
  return x;
}

template <int DT>
__device__ __forceinline__ float qelem(uint32_t w, int half) {
  const uint16_t b = (uint16_t)(half ? w >> 16 : w & 0xFFFFu);
  if constexpr (DT == AMF_DTYPE_BF16) return amf::u2f((uint32_t)b << 16);
  else return (float)__builtin_bit_cast(_Float16, b);
}

template <int DT, int GH>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3)))
void int4_sym_attn_mfma_kernel(AttnArgs a, float* part,
                                                                int64_t split_tokens,
                                                                int64_t n_splits, int64_t units) {
  constexpr int D = 128;
  static_assert(GH >= 1 && GH <= 16, "heads per wave: the 16 rows of the tile");
  __shared__ __attribute__((aligned(16))) float p_lds[16][32];
  const int lane = threadIdx.x, lo = lane & 15, hi = lane >> 4;
  const int G = a.num_q_heads / a.num_kv_heads;
  const int W = G / GH;
  const int64_t id = blockIdx.x, slot = id / kXcds;
  const int r = (int)(slot % W);
  const int64_t u = (slot / W) * kXcds + id % kXcds;
  if (u >= units) return;
  const int64_t split = u % n_splits, rest = u / n_splits;
  const int64_t tq = rest % a.q_len, bkv = rest / a.q_len;
  const int hkv = (int)(bkv % a.num_kv_heads);
  const int64_t b = bkv / a.num_kv_heads;
  const int h0 = hkv * G + r * GH;
  const int64_t T = a.kv_len;
  const int64_t t_begin = split * split_tokens, t_end = min(T, t_begin + split_tokens);
  const int64_t kv_base = (b * a.num_kv_heads + hkv) * T;
  auto qrow = [&](int j) { return (b * a.num_q_heads + h0 + j) * a.q_len + tq; };
  const float scl = a.scale * kLog2e;

  // lane (lo, hi): 16 code bytes of token t0 + 16 j + lo, dims 32 hi .. + 31;
  // the first chunk's are in flight while the query operand is built.  (The
  // host keeps kv_len D / 2 below 2^32: 32-bit offsets from the row's base.)
  const uint8_t* kcodes = static_cast<const uint8_t*>(a.k) + kv_base * (D / 2);
  const uint8_t* vcodes = static_cast<const uint8_t*>(a.v) + kv_base * (D / 2);
  auto row_off = [&](int64_t t) {
    return (uint32_t)(t < t_end ? t : t_begin) * (uint32_t)(D / 2) + 16u * hi;
  };
  auto load = [&](u32x4 (&kx)[2], u32x4 (&vx)[2], int64_t t0) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      kx[j] = *reinterpret_cast<const u32x4*>(kcodes + row_off(t0 + 16 * j + lo));
      vx[j] = *reinterpret_cast<const u32x4*>(vcodes + row_off(t0 + 16 * j + lo));
    }
  };
  u32x4 kc[2], vc[2];
  load(kc, vc, t_begin);

  // ---- query operand: x = q s over this lane's 32 dims (row lo) ----
  // Rows GH .. 15 repeat row 0: they leave the maximum alone and their
  // scores are masked below.
  const int qr = lo < GH ? lo : 0;
  float x[32];
  {
    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + qrow(qr) * D + 32 * hi;
    const uint16_t* sp = reinterpret_cast<const uint16_t*>(a.k_scales) + 32 * hi;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4 qw = *reinterpret_cast<const u32x4*>(qp + 8 * v);
      const u32x4 sw = *reinterpret_cast<const u32x4*>(sp + 8 * v);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float qv = qelem<DT>(qw[e >> 1], e & 1);
        const float sv = qelem<AMF_DTYPE_F16>(sw[e >> 1], e & 1);
        x[8 * v + e] = qv * sv;
      }
    }
  }
  float qsum = 0.0f, xmax = 0.0f;
#pragma unroll
  for (int d = 0; d < 32; ++d) {
    qsum += x[d];
    xmax = fmaxf(xmax, fabsf(x[d]));
  }
  qsum += __shfl_xor(qsum, 16);
  qsum += __shfl_xor(qsum, 32);
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) xmax = fmaxf(xmax, __shfl_xor(xmax, o));
  // scale so that the largest |q s| lands in [2^14, 2^15): hi and lo then
  // hold every q s above 2^-24 of it exactly
  const int xexp = (int)((amf::f2u(xmax) >> 23) & 0xFFu);
  const int qe = (xexp > 0 && xexp < 255) ? min(max(xexp - 127 - 14, -100), 100) : 0;
  const float down = __builtin_ldexpf(1.0f, -qe);
  u32x4 qa_hi[4], qa_lo[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      float v[2], h[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int i = 2 * jj + t;
        v[t] = x[8 * st + nib_of_k16(i)] * (down * (k16_x16(i) ? 0.0625f : 1.0f));
      }
      const uint32_t hp = pk_f16(v[0], v[1]);
      h[0] = amf::half_lo<false>(hp);
      h[1] = amf::half_hi<false>(hp);
      qa_hi[st][jj] = hp;
      qa_lo[st][jj] = pk_f16(v[0] - h[0], v[1] - h[1]);
    }
  }
  // scores: (MFMA sum) 2^(24 + qe) - 8 sum_d q_d s_d, times scale log2(e)
  const float c1 = __builtin_ldexpf(scl, 24 + qe);
  float c2[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) c2[e] = -8.0f * scl * __shfl(qsum, 4 * hi + e);

  // ---- transpose selectors: column c takes dim 32 (2 h + c / 8) + 8 m + c % 8 ----
  u32x4 sel[2];
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      float v[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int i = 2 * jj + t;
        const bool on = hi == 2 * h2 + (lo >> 3) && nib_of_k16(i) == (lo & 7);
        v[t] = on ? (k16_x16(i) ? 0.0625f : 1.0f) : 0.0f;
      }
      sel[h2][jj] = pk_f16(v[0], v[1]);
    }
  }
  float vsc[4][2];  // V scale of each output dim of this lane
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2)
      vsc[m][h2] = (float)a.v_scales[32 * (2 * h2 + (lo >> 3)) + 8 * m + (lo & 7)];

  // the first chunk sets them: every split holds at least one token
  float m_run[4], l_run[4];
  f32x4 acc[4][2];

  // One chunk on the codes in kc / vc, loading the next one into kn / vn.
  // The first chunk of the split starts the running max, sums and
  // accumulators.
  auto chunk = [&](auto first_c, int64_t t0, u32x4 (&kn)[2], u32x4 (&vn)[2]) {
    constexpr bool first = decltype(first_c)::value;
    if (t0 + 32 < t_end) load(kn, vn, t0 + 32);
    // QK^T: two 16-token tiles, hi and lo query parts against one code operand
    float xs[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4 cs = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const u32x4 kb = nib8_to_f16_sub(kc[j][st]);
        cs = mfma_f16(qa_hi[st], kb, cs);
        cs = mfma_f16(qa_lo[st], kb, cs);
      }
      const bool valid = t0 + 16 * j + lo < t_end;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        xs[j][e] = (valid && 4 * hi + e < GH) ? fmaf(cs[e], c1, c2[e]) : -INFINITY;
    }
    // online softmax per head row (lanes of one 16-lane row share it): the
    // reference max moves only when a score exceeds it by the slack
    if constexpr (first) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        m_run[e] = fmaxf(kNegBigAttn, row_max16(fmaxf(xs[0][e], xs[1][e])));
        l_run[e] = 0.0f;
      }
    } else {
    bool up = false;
#pragma unroll
    for (int e = 0; e < 4; ++e) up = up || fmaxf(xs[0][e], xs[1][e]) > m_run[e] + kRescaleSlackAttn;
    if (__any(up)) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float m_new = fmaxf(m_run[e], row_max16(fmaxf(xs[0][e], xs[1][e])));
        const float alpha = __builtin_amdgcn_exp2f(m_run[e] - m_new);
        l_run[e] *= alpha;
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) acc[m][h2][e] *= alpha;
        m_run[e] = m_new;
      }
    }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p = __builtin_amdgcn_exp2f(xs[j][e] - m_run[e]);
        l_run[e] += p;
        p_lds[4 * hi + e][16 * j + lo] = p;
      }
    __builtin_amdgcn_wave_barrier();
    // PV weights in the A layout: row lo, k-slice hi = tokens 4 hi .. + 3 and
    // 16 + 4 hi .. + 3, as fp16 hi + lo
    u32x4 pa_hi, pa_lo;
    {
      const f32x4 p0 = *reinterpret_cast<const f32x4*>(&p_lds[lo][4 * hi]);
      const f32x4 p1 = *reinterpret_cast<const f32x4*>(&p_lds[lo][16 + 4 * hi]);
      const float pv[8] = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const uint32_t hp = pk_f16(pv[2 * jj], pv[2 * jj + 1]);
        pa_hi[jj] = hp;
        pa_lo[jj] = pk_f16(pv[2 * jj] - amf::half_lo<false>(hp),
                           pv[2 * jj + 1] - amf::half_hi<false>(hp));
      }
    }
    __builtin_amdgcn_wave_barrier();
    // V codes transposed by the selectors, then PV
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const u32x4 av0 = nib8_to_f16_sub(vc[0][m]), av1 = nib8_to_f16_sub(vc[1][m]);
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        // centred codes: the accumulator starts at -8 2^-24, so the PV sums
        // take c - 8 (exact in fp16) and the output needs no - 8 l term,
        // which would cancel most of an average over many tokens
        const f32x4 z = {-0x1p-21f, -0x1p-21f, -0x1p-21f, -0x1p-21f};
        const f32x4 t0v = mfma_f16(av0, sel[h2], z);
        const f32x4 t1v = mfma_f16(av1, sel[h2], z);
        const u32x4 bv = {pk_f16(t0v[0], t0v[1]), pk_f16(t0v[2], t0v[3]),
                          pk_f16(t1v[0], t1v[1]), pk_f16(t1v[2], t1v[3])};
        const f32x4 a0 = first ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : acc[m][h2];
        acc[m][h2] = mfma_f16(pa_hi, bv, a0);
        acc[m][h2] = mfma_f16(pa_lo, bv, acc[m][h2]);
      }
    }
  };
  u32x4 kn[2], vn[2];
  auto next = [&] {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      kc[j] = kn[j];
      vc[j] = vn[j];
    }
  };
  chunk(std::true_type{}, t_begin, kn, vn);
  for (int64_t t0 = t_begin + 32; t0 < t_end; t0 += 32) {
    next();
    chunk(std::false_type{}, t0, kn, vn);
  }
  // ---- the split's partials: o_d = s_d sum p (c - 8), m, l per head ----
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int head = 4 * hi + e;
    const float l = group_sum<16>(l_run[e]);
    if (head < GH) {
      float* pr = part + (qrow(head) * n_splits + split) * (int64_t)(D + kPartPad);
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
          pr[32 * (2 * h2 + (lo >> 3)) + 8 * m + (lo & 7)] = vsc[m][h2] * (acc[m][h2][e] * 0x1p24f);
      if (lo == 0) {
        pr[D] = m_run[e];
        pr[D + 1] = l;
      }
    }
  }
}

// One workgroup of kMergeWaves waves per query row:
// out = sum_k 2^(m_k - M) acc_k / sum_k 2^(m_k - M) l_k.  Every wave finds M
// and the denominator over all splits, wave 0 puts the split weights in LDS;
// wave w then sums the splits w, w + kMergeWaves, ..., lane (phase, quad)
// taking the f32x4 quad `quad` of every P-th of them (P = 256 / D phases).
// The accumulator loads of its first kMergeBatch splits per lane do not
// depend on the weights and are issued first, in flight with the (m, l)
// loads.  Phases are added by shuffles, waves through LDS.
constexpr int kMaxSplits = 4096;
constexpr int kMergeWaves = 4;
constexpr int kMergeBatch = 16;  // accumulator loads per lane in flight
static_assert(kSplitWaves <= kMaxSplits, "dense_splits gives at most kSplitWaves splits");

template <int OUT_DT, int D>
__global__ __launch_bounds__(64 * kMergeWaves) void dense_attn_merge_kernel(AttnArgs a,
                                                                          const float* part,
                                                                          int64_t n_splits) {
  constexpr int Q = D / 4, P = 64 / Q, STRIDE = D + kPartPad, S = P * kMergeWaves;
  __shared__ float f_s[kMaxSplits];
  __shared__ __attribute__((aligned(16))) float o_s[kMergeWaves][D];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = blockIdx.x;
  const int ns = (int)n_splits;
  const float* pr = part + row * n_splits * (int64_t)STRIDE;
  const int quad = lane % Q, phase = lane / Q;
  const int k0 = wv * P + phase;  // this lane's splits: k0, k0 + S, ...
  f32x4 x[kMergeBatch];
#pragma unroll
  for (int i = 0; i < kMergeBatch; ++i) {
    const int k = k0 + S * i;
    x[i] = k < ns ? *reinterpret_cast<const f32x4*>(pr + (int64_t)k * STRIDE + 4 * quad)
                  : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  // (m, l) of splits lane, lane + 64, ...: the first in registers
  float m0 = -INFINITY, l0 = 0.0f;
  if (lane < ns) {
    const amf::f32x2 ml = *reinterpret_cast<const amf::f32x2*>(pr + (int64_t)lane * STRIDE + D);
    m0 = ml[0];
    l0 = ml[1];
  }
  float M = m0;
  for (int k = lane + 64; k < ns; k += 64) M = fmaxf(M, pr[(int64_t)k * STRIDE + D]);
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
  // every wave finds the denominator; wave 0 writes the weights
  float den = 0.0f;
  if (lane < ns) {
    const float f = (M == -INFINITY || m0 == -INFINITY) ? 0.0f : exp2f(m0 - M);
    den = l0 * f;
    if (wv == 0) f_s[lane] = f;
  }
  for (int k = lane + 64; k < ns; k += 64) {
    const float mk = pr[(int64_t)k * STRIDE + D];
    const float f = (M == -INFINITY || mk == -INFINITY) ? 0.0f : exp2f(mk - M);
    den = fmaf(pr[(int64_t)k * STRIDE + D + 1], f, den);
    if (wv == 0) f_s[k] = f;
  }
  for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o);
  __syncthreads();
  f32x4 o4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < kMergeBatch; ++i) {
    const int k = k0 + S * i;
    const float f = k < ns ? f_s[k] : 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) o4[e] = fmaf(x[i][e], f, o4[e]);
  }
  for (int k = k0 + S * kMergeBatch; k < ns; k += S) {
    const f32x4 y = *reinterpret_cast<const f32x4*>(pr + (int64_t)k * STRIDE + 4 * quad);
    const float f = f_s[k];
#pragma unroll
    for (int e = 0; e < 4; ++e) o4[e] = fmaf(y[e], f, o4[e]);
  }
#pragma unroll
  for (int o = Q; o < 64; o <<= 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) o4[e] += __shfl_xor(o4[e], o);
  }
  if (phase == 0) *reinterpret_cast<f32x4*>(&o_s[wv][4 * quad]) = o4;
  __syncthreads();
  // a row whose scores are all -inf: 0 / 0 = NaN, as softmax gives
  if (wv == 0 && phase == 0) {
    f32x4 t = *reinterpret_cast<const f32x4*>(&o_s[0][4 * quad]);
#pragma unroll
    for (int w = 1; w < kMergeWaves; ++w) {
      const f32x4 u = *reinterpret_cast<const f32x4*>(&o_s[w][4 * quad]);
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] += u[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) store_out<OUT_DT>(a.out, row * D + 4 * quad + e, t[e] / den);
  }
}

// Workgroups of the split launch: units (b, KV head, query row, split)
// rounded up to the XCD count, times the waves per unit.
inline int64_t split_grid(int64_t rows, int64_t n_splits, int32_t num_q_heads,
                          int32_t num_kv_heads, int64_t* units) {
  const int64_t G = num_q_heads / num_kv_heads;
  *units = rows / G * n_splits;
  return (*units + kXcds - 1) / kXcds * kXcds * (G / heads_per_wave(num_q_heads, num_kv_heads));
}

template <int DT, bool INT4, int GH>
void launch_split_gh(const AttnArgs& a, float* part, int64_t split_tokens, int64_t n_splits,
                     dim3 grid, int64_t units, hipStream_t st) {
  if (a.head_dim == 64)
    dense_attn_split_kernel<DT, 8, INT4, GH>
        <<<grid, 64, 0, st>>>(a, part, split_tokens, n_splits, units);
  else if (a.head_dim == 128)
    dense_attn_split_kernel<DT, 16, INT4, GH>
        <<<grid, 64, 0, st>>>(a, part, split_tokens, n_splits, units);
  else
    dense_attn_split_kernel<DT, 32, INT4, GH>
        <<<grid, 64, 0, st>>>(a, part, split_tokens, n_splits, units);
}

void launch_merge(const AttnArgs& a, int32_t out_dtype, int64_t rows, const float* part,
                  int64_t n_splits, hipStream_t st) {
  const dim3 mgrid((unsigned)rows);
#define AMF_MERGE(OUT)                                                                            \
  if (a.head_dim == 64)                                                                           \
    dense_attn_merge_kernel<OUT, 64><<<mgrid, 64 * kMergeWaves, 0, st>>>(a, part, n_splits);      \
  else if (a.head_dim == 128)                                                                     \
    dense_attn_merge_kernel<OUT, 128><<<mgrid, 64 * kMergeWaves, 0, st>>>(a, part, n_splits);     \
  else                                                                                            \
    dense_attn_merge_kernel<OUT, 256><<<mgrid, 64 * kMergeWaves, 0, st>>>(a, part, n_splits)
  if (out_dtype == AMF_DTYPE_F32) {
    AMF_MERGE(AMF_DTYPE_F32);
  } else if (out_dtype == AMF_DTYPE_BF16) {
    AMF_MERGE(AMF_DTYPE_BF16);
  } else {
    AMF_MERGE(AMF_DTYPE_F16);
  }
#undef AMF_MERGE
}

template <int DT, bool INT4>
void launch_split(const AttnArgs& a, int32_t out_dtype, int64_t rows, float* part,
                  int64_t split_tokens, int64_t n_splits, hipStream_t st) {
  int64_t units = 0;
  const dim3 grid((unsigned)split_grid(rows, n_splits, a.num_q_heads, a.num_kv_heads, &units));
  const int gh = heads_per_wave(a.num_q_heads, a.num_kv_heads);
  if (gh == 4)
    launch_split_gh<DT, INT4, 4>(a, part, split_tokens, n_splits, grid, units, st);
  else if (gh == 2)
    launch_split_gh<DT, INT4, 2>(a, part, split_tokens, n_splits, grid, units, st);
  else
    launch_split_gh<DT, INT4, 1>(a, part, split_tokens, n_splits, grid, units, st);
  launch_merge(a, out_dtype, rows, part, n_splits, st);
}

// The INT4_SYM split on MFMA tiles (head_dim 128, bf16 / fp16 queries, no
// mask), with the same splits, partials and merge as launch_split.
template <int DT>
void launch_int4_mfma(const AttnArgs& a, int32_t out_dtype, int64_t rows, float* part,
                      int64_t split_tokens, int64_t n_splits, hipStream_t st) {
  // Up to 16 heads of a GQA group per wave (the tile's rows), the largest
  // power of two dividing the group: one wave reads a unit's codes for all
  // of them.  The splits are those of the workspace (dense_splits).
  const int G = a.num_q_heads / a.num_kv_heads;
  const int gh = G % 16 == 0 ? 16 : G % 8 == 0 ? 8 : G % 4 == 0 ? 4 : G % 2 == 0 ? 2 : 1;
  const int64_t units = rows / G * n_splits;
  const dim3 grid((unsigned)((units + kXcds - 1) / kXcds * kXcds * (G / gh)));
  const dim3 block(64);
#define AMF_INT4_MFMA(GH) \
  int4_sym_attn_mfma_kernel<DT, GH><<<grid, block, 0, st>>>(a, part, split_tokens, n_splits, units)
  if (gh == 16)
    AMF_INT4_MFMA(16);
  else if (gh == 8)
    AMF_INT4_MFMA(8);
  else if (gh == 4)
    AMF_INT4_MFMA(4);
  else if (gh == 2)
    AMF_INT4_MFMA(2);
  else
    AMF_INT4_MFMA(1);
#undef AMF_INT4_MFMA
  launch_merge(a, out_dtype, rows, part, n_splits, st);
}

template <int DT, int OUT_DT>
void launch_typed(const AttnArgs& a, bool vec8, int64_t rows, hipStream_t st) {
  if (vec8)
    dense_attn_kernel<DT, OUT_DT, true><<<dim3((unsigned)rows), kThreads, 0, st>>>(a);
  else
    dense_attn_kernel<DT, OUT_DT, false><<<dim3((unsigned)rows), kThreads, 0, st>>>(a);
}

template <int DT>
void launch_out(const AttnArgs& a, int32_t out_dtype, bool vec8, int64_t rows, hipStream_t st) {
  if (out_dtype == AMF_DTYPE_F32)
    launch_typed<DT, AMF_DTYPE_F32>(a, vec8, rows, st);
  else if (out_dtype == AMF_DTYPE_BF16)
    launch_typed<DT, AMF_DTYPE_BF16>(a, vec8, rows, st);
  else
    launch_typed<DT, AMF_DTYPE_F16>(a, vec8, rows, st);
}

bool is_dtype(int32_t t) {
  return t == AMF_DTYPE_F16 || t == AMF_DTYPE_F32 || t == AMF_DTYPE_BF16;
}

// Shape and dtype checks shared by the dense and INT4_SYM entry points.
int check_attn_args(const char* who, int32_t dtype, int32_t out_dtype, int64_t batch,
                    int32_t num_q_heads, int32_t num_kv_heads, int64_t q_len, int64_t kv_len,
                    int32_t head_dim) {
  using namespace amf;
  if (!is_dtype(dtype) || !is_dtype(out_dtype))
    return fail(AMF_ERR_INVALID_ARG, "%s: bad dtype %d / out_dtype %d", who, dtype, out_dtype);
  if (batch < 0 || q_len < 0 || kv_len < 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads != 0)
    return fail(AMF_ERR_INVALID_ARG,
                "%s: bad shape batch=%lld q_len=%lld kv_len=%lld heads=%d/%d (q heads must be a "
                "multiple of kv heads)",
                who, (long long)batch, (long long)q_len, (long long)kv_len, num_q_heads,
                num_kv_heads);
  if (head_dim <= 0 || head_dim > kMaxD)
    return fail(AMF_ERR_UNSUPPORTED, "%s: head_dim %d outside [1, %d]", who, head_dim, kMaxD);
  if (batch > 0x7FFFFFFF || q_len > 0x7FFFFFFF ||
      (batch > 0 && q_len > 0x7FFFFFFF / batch) || batch * q_len * num_q_heads > 0x7FFFFFFF)
    return fail(AMF_ERR_UNSUPPORTED, "%s: batch %lld x %d heads x %lld rows exceed one launch",
                who, (long long)batch, num_q_heads, (long long)q_len);
  return ok();
}

}  // namespace

extern "C" int64_t amf_dense_attn_workspace_bytes(int64_t batch, int32_t num_q_heads,
                                                  int32_t num_kv_heads, int64_t q_len,
                                                  int64_t kv_len, int32_t head_dim) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      q_len <= 0 || kv_len <= 0 || !split_head_dim(head_dim) || batch > 0x7FFFFFFF ||
      q_len > 0x7FFFFFFF)
    return 0;
  const int64_t rows = batch * num_q_heads * q_len;
  if (rows > 0x7FFFFFFF) return 0;
  int64_t n_splits = 1, split_tokens = 64;
  dense_splits(rows, heads_per_wave(num_q_heads, num_kv_heads), kv_len, &n_splits, &split_tokens);
  // The split launch has at most rows * n_splits + 8 * num_q_heads
  // workgroups; a shape beyond one launch takes the single-pass kernel.
  if (rows > (0x7FFFFFFF - kXcds * num_q_heads) / n_splits) return 0;
  return rows * n_splits * (int64_t)(head_dim + kPartPad) * (int64_t)sizeof(float);
}

extern "C" int amf_dense_attn(const void* q, const void* k, const void* v, int32_t dtype,
                              const float* mask, int64_t mask_stride_b, int64_t mask_stride_h,
                              int64_t mask_stride_q, int64_t mask_stride_t, void* out,
                              int32_t out_dtype, int64_t batch, int32_t num_q_heads,
                              int32_t num_kv_heads, int64_t q_len, int64_t kv_len,
                              int32_t head_dim, float softmax_scale, void* workspace,
                              int64_t workspace_bytes, void* stream) {
  using namespace amf;
  const char* who = "amf_dense_attn";
  if (!q || !out || (kv_len > 0 && (!k || !v)))
    return fail(AMF_ERR_INVALID_ARG, "%s: null q/k/v/out", who);
  int rc = check_attn_args(who, dtype, out_dtype, batch, num_q_heads, num_kv_heads, q_len,
                           kv_len, head_dim);
  if (rc) return rc;
  const int64_t rows = batch * num_q_heads * q_len;
  if (rows == 0) return ok();
  const int esize = dtype == AMF_DTYPE_F32 ? 4 : 2;
  const bool vec8 = head_dim % 8 == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0 &&
                    ((int64_t)head_dim * esize) % 16 == 0;
  AttnArgs a{q, k, v, mask, mask_stride_b, mask_stride_h, mask_stride_q, mask_stride_t, out,
             batch, num_q_heads, num_kv_heads, q_len, kv_len, head_dim,
             softmax_scale, nullptr, nullptr};
  hipStream_t st = as_stream(stream);
  const int64_t need =
      amf_dense_attn_workspace_bytes(batch, num_q_heads, num_kv_heads, q_len, kv_len, head_dim);
  if (need > 0 && vec8 && ((uintptr_t)q % 16) == 0 && workspace && workspace_bytes >= need &&
      ((uintptr_t)workspace % 16) == 0) {
    int64_t n_splits = 1, split_tokens = 64;
    dense_splits(rows, heads_per_wave(num_q_heads, num_kv_heads), kv_len, &n_splits,
                 &split_tokens);
    float* part = static_cast<float*>(workspace);
    if (dtype == AMF_DTYPE_F32)
      launch_split<AMF_DTYPE_F32, false>(a, out_dtype, rows, part, split_tokens, n_splits, st);
    else if (dtype == AMF_DTYPE_BF16)
      launch_split<AMF_DTYPE_BF16, false>(a, out_dtype, rows, part, split_tokens, n_splits, st);
    else
      launch_split<AMF_DTYPE_F16, false>(a, out_dtype, rows, part, split_tokens, n_splits, st);
    return check_launch(who);
  }
  if (dtype == AMF_DTYPE_F32)
    launch_out<AMF_DTYPE_F32>(a, out_dtype, vec8, rows, st);
  else if (dtype == AMF_DTYPE_BF16)
    launch_out<AMF_DTYPE_BF16>(a, out_dtype, vec8, rows, st);
  else
    launch_out<AMF_DTYPE_F16>(a, out_dtype, vec8, rows, st);
  return check_launch(who);
}

extern "C" int amf_int4_sym_dense_attn(const void* q, int32_t dtype, const void* k_codes,
                                       const uint16_t* k_scales, const void* v_codes,
                                       const uint16_t* v_scales, const float* mask,
                                       int64_t mask_stride_b, int64_t mask_stride_h,
                                       int64_t mask_stride_q, int64_t mask_stride_t, void* out,
                                       int32_t out_dtype, int64_t batch, int32_t num_q_heads,
                                       int32_t num_kv_heads, int64_t q_len, int64_t kv_len,
                                       int32_t head_dim, float softmax_scale, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  using namespace amf;
  const char* who = "amf_int4_sym_dense_attn";
  if (!q || !out || (kv_len > 0 && (!k_codes || !v_codes || !k_scales || !v_scales)))
    return fail(AMF_ERR_INVALID_ARG, "%s: null q/codes/scales/out", who);
  int rc = check_attn_args(who, dtype, out_dtype, batch, num_q_heads, num_kv_heads, q_len,
                           kv_len, head_dim);
  if (rc) return rc;
  if (!split_head_dim(head_dim))
    return fail(AMF_ERR_UNSUPPORTED, "%s: head_dim %d (64, 128 or 256 only)", who, head_dim);
  if (((uintptr_t)q % 16) != 0 || ((uintptr_t)k_codes % 4) != 0 || ((uintptr_t)v_codes % 4) != 0 ||
      ((uintptr_t)k_scales % 2) != 0 || ((uintptr_t)v_scales % 2) != 0)
    return fail(AMF_ERR_INVALID_ARG, "%s: q must be 16-byte, codes 4-byte aligned", who);
  const int64_t rows = batch * num_q_heads * q_len;
  if (rows == 0) return ok();
  AttnArgs a{q, k_codes, v_codes, mask, mask_stride_b, mask_stride_h, mask_stride_q,
             mask_stride_t, out, batch, num_q_heads, num_kv_heads, q_len, kv_len, head_dim,
             softmax_scale, reinterpret_cast<const _Float16*>(k_scales),
             reinterpret_cast<const _Float16*>(v_scales)};
  hipStream_t st = as_stream(stream);
  if (kv_len == 0) {  // an empty softmax: zeros, no K/V read
    if (dtype == AMF_DTYPE_F32)
      launch_out<AMF_DTYPE_F32>(a, out_dtype, false, rows, st);
    else if (dtype == AMF_DTYPE_BF16)
      launch_out<AMF_DTYPE_BF16>(a, out_dtype, false, rows, st);
    else
      launch_out<AMF_DTYPE_F16>(a, out_dtype, false, rows, st);
    return check_launch(who);
  }
  const int64_t need =
      amf_dense_attn_workspace_bytes(batch, num_q_heads, num_kv_heads, q_len, kv_len, head_dim);
  if (need == 0)
    return fail(AMF_ERR_UNSUPPORTED, "%s: %lld query rows exceed one launch", who,
                (long long)rows);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace % 16) != 0)
    return fail(AMF_ERR_WORKSPACE, "%s: needs %lld workspace bytes (16-byte aligned)", who,
                (long long)need);
  int64_t n_splits = 1, split_tokens = 64;
  dense_splits(rows, heads_per_wave(num_q_heads, num_kv_heads), kv_len, &n_splits,
               &split_tokens);
  float* part = static_cast<float*>(workspace);
  // the MFMA kernel addresses a (batch, KV head) row of codes with 32-bit offsets
  const bool mfma = head_dim == 128 && !mask && dtype != AMF_DTYPE_F32 &&
                    kv_len < ((int64_t)1 << 32) / 64;
  if (mfma && dtype == AMF_DTYPE_BF16)
    launch_int4_mfma<AMF_DTYPE_BF16>(a, out_dtype, rows, part, split_tokens, n_splits, st);
  else if (mfma)
    launch_int4_mfma<AMF_DTYPE_F16>(a, out_dtype, rows, part, split_tokens, n_splits, st);
  else if (dtype == AMF_DTYPE_F32)
    launch_split<AMF_DTYPE_F32, true>(a, out_dtype, rows, part, split_tokens, n_splits, st);
  else if (dtype == AMF_DTYPE_BF16)
    launch_split<AMF_DTYPE_BF16, true>(a, out_dtype, rows, part, split_tokens, n_splits, st);
  else
    launch_split<AMF_DTYPE_F16, true>(a, out_dtype, rows, part, split_tokens, n_splits, st);
  return check_launch(who);
}
