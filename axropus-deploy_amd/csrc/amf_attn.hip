// amf_attn.hip - dense scaled-dot-product attention over plain (already
// dequantized) K/V rows: the positional path of int4_decode_attention.
//
// Computes out = softmax(q k^T * scale + mask) v for every query row, the
// result of korith_vllm_ext/kernels/dispatch.py:117-143 (fallback_fp16_kernel,
// which the reference's dispatch returns for every format on every device),
// in fp32 with one rounding to the output dtype at the end.  GQA is accepted
// (num_q_heads a multiple of num_kv_heads); the reference's matmul broadcast
// allows only equal head counts or a single KV head.
//
// One workgroup (4 waves) per query row.  Wave w takes the 64-token chunks
// w, w+4, w+8, ...; lane l scores token chunk_base + l against the query held
// in LDS, the wave keeps an online softmax (running max and sum), and the PV
// product is lane-parallel over head_dim with the chunk's probabilities
// broadcast by readlane.  The four partial (max, sum, acc) triples are merged
// through LDS.
#include <math.h>

#include "amf_internal.h"
#include "amf_kernel_util.h"

namespace {

using amf::u32x4;
using amf::f32x4;

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

}  // namespace

extern "C" int amf_dense_attn(const void* q, const void* k, const void* v, int32_t dtype,
                              const float* mask, int64_t mask_stride_b, int64_t mask_stride_h,
                              int64_t mask_stride_q, int64_t mask_stride_t, void* out,
                              int32_t out_dtype, int64_t batch, int32_t num_q_heads,
                              int32_t num_kv_heads, int64_t q_len, int64_t kv_len,
                              int32_t head_dim, float softmax_scale, void* stream) {
  using namespace amf;
  const char* who = "amf_dense_attn";
  if (!q || !out || (kv_len > 0 && (!k || !v)))
    return fail(AMF_ERR_INVALID_ARG, "%s: null q/k/v/out", who);
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
  const int64_t rows = batch * num_q_heads * q_len;
  if (rows > 0x7FFFFFFF)
    return fail(AMF_ERR_UNSUPPORTED, "%s: %lld query rows exceed one launch", who,
                (long long)rows);
  if (rows == 0) return ok();
  const int esize = dtype == AMF_DTYPE_F32 ? 4 : 2;
  const bool vec8 = head_dim % 8 == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0 &&
                    ((int64_t)head_dim * esize) % 16 == 0;
  AttnArgs a{q, k, v, mask, mask_stride_b, mask_stride_h, mask_stride_q, mask_stride_t, out,
             batch, num_q_heads, num_kv_heads, q_len, kv_len, head_dim,
             softmax_scale};
  hipStream_t st = as_stream(stream);
  if (dtype == AMF_DTYPE_F32)
    launch_out<AMF_DTYPE_F32>(a, out_dtype, vec8, rows, st);
  else if (dtype == AMF_DTYPE_BF16)
    launch_out<AMF_DTYPE_BF16>(a, out_dtype, vec8, rows, st);
  else
    launch_out<AMF_DTYPE_F16>(a, out_dtype, vec8, rows, st);
  return check_launch(who);
}
