// amf_decode.hip - paged GQA decode attention reading AMF_FMT_INT4_ASYM_G32
// KV pages with fused dequantization (split-K "flash decoding" + LSE merge).
//
// Replaces int4_decode_attention (korith_vllm_ext/int4_decode_attention.py:6-9
// -> kernels/dispatch.py:117-143: full decompress then matmul/softmax/matmul)
// and the never-dispatched CUDA kernel it stood for
// (korith_vllm_ext/kernels/int4_decode_attention.cu:39-177: one CTA per
// (batch, head), serial online softmax over 128-token tiles).  This kernel
// adds paging (block tables), GQA and split-K.
//
// Work (MFMA path, "stream-K"): the units (sequence, KV head, 32-token
// chunk), sequence-major, are cut into G equal shares, G = the waves the
// device keeps resident at once, one share per wave, so every wave streams
// about the same number of chunks and the grid runs in one round whatever
// the mix of context lengths.  A wave walks its share pair by pair; within a
// (sequence, KV head) it streams chunks of 32 tokens (two 16-token pages)
// through a small per-wave LDS ring by non-temporal LDS DMA, keeping per
// query head of the GQA group a running max m (log2 domain), sum l and an
// unnormalised output.  A pair held by one wave is finished in place; a pair
// shared by several leaves one partial per wave (slot 0 of the wave for the
// segment its share starts with, slot 1 for the one it ends with), and a
// second kernel merges them with an LSE rescale.  The VALU path keeps fixed
// splits of split_tokens tokens, one wave per (sequence, KV head, split).
//
// Dequantisation is folded into the dot products.  With K = s*c + z per
// (token, 32-dim group):
//   q.k = sum_g [ s_g * sum_{d in g} q_d c_d + z_g * sum_{d in g} q_d ].
// Codes enter the matrix cores as exact fp16 subnormals c * 2^-24 (a nibble
// masked in place; a high nibble comes out as 16 c * 2^-24 and the other
// operand carries the 1/16), so no code bias enters the constant term.
//
// MFMA path (v_mfma_f32_16x16x32_f16, 64 lanes, lane = 16 * hi + lo):
//  QK^T  computed as S^T[(r,g), t] = sum_k A[(r,g), k] B[k, t] where A holds
//        q of head r restricted to group g (zero elsewhere: block structure),
//        as fp16 scaled per wave by a power of two, and B the 16 tokens'
//        codes; four k-steps of 32 dims.  Lane (t = lo, j = hi) then owns
//        C[(r = j, g = 0..3), t] and folds the four groups itself, so every
//        output is useful.
//  PV    O[(r,g), d] = sum_t W[(r,g), t] c_{t,d} with W = p * s_g(t) as one
//        fp16 per weight where an error budget on the rounding of those
//        weights and the chunk's V scales allow (pv_single_ok), otherwise
//        (and for AMF_DECODE_MFMA_PRECISE) as a bf16 hi + lo pair against the
//        codes as the exact bf16 128 + c (v_mfma_f32_16x16x32_bf16, the bias
//        folded into the constant term); the V pages are stored dim-major in
//        8x8 tiles, so a lane's B operand (8 tokens of one dim) is one dword
//        of a contiguous 32-byte run.  Only the row of each output column's
//        own group is used.
// VALU path: the same data flow with fp32 FMAs (kept for the MFMA-vs-VALU
// comparison and as a second implementation).
#include <algorithm>
#include <map>
#include <mutex>

#include "amf_internal.h"
#include "amf_kernel_util.h"

// Decode attention is held to a tolerance, not to the codecs' exact
// operation sequence: let multiplies and adds fuse into FMAs here.
#pragma clang fp contract(fast)

namespace {

using namespace amf;

constexpr int kD = 128;          // head_dim
constexpr int kBS = 16;          // tokens per page
constexpr int kHBCodes = 1024;   // code bytes of one (page, head) block
constexpr int kHBParams = 64;    // param words of one (page, head) block
constexpr int kPartStride = kD + 4;  // split partial: D accumulators, m, l, 2 pad (16-byte rows)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));

struct DecodeArgs {
  const uint16_t* q;
  void* out;
  const uint8_t* kc;
  const uint32_t* kp;
  const uint8_t* vc;
  const uint32_t* vp;
  int64_t pool_pages;
  const int32_t* block_tables;
  int bt_stride;
  const int32_t* context_lens;
  int num_q_heads;
  int num_kv_heads;
  int split_tokens;
  int max_splits;
  int max_context_len;
  int head_fast;         // grid order, see work_head
  int pv16;              // fp16 PV tiles where the V scales allow (else bf16 hi/lo throughout)
  float qk_scale_log2;  // softmax_scale * log2(e)
  float* ws;
  int32_t* err_flag;
  int out_dtype;
  int num_seqs;
  int stream_k;          // MFMA path: waves take equal shares of the (sequence, KV head, chunk) space
  int sk_waves;          // grid size of the stream-K decode launch
  int64_t* sk_meta;      // stream-K: units before each sequence [num_seqs], then all units
};

// ---- lane helpers -----------------------------------------------------------

__device__ __forceinline__ float dpp_ror(float v, int n) {
  // row_ror:n (rotate within each row of 16 lanes): dpp_ctrl 0x120 + n.
  int x = __builtin_bit_cast(int, v);
  switch (n) {
    case 8: x = __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false); break;
    case 4: x = __builtin_amdgcn_update_dpp(0, x, 0x124, 0xF, 0xF, false); break;
    case 2: x = __builtin_amdgcn_update_dpp(0, x, 0x122, 0xF, 0xF, false); break;
    default: x = __builtin_amdgcn_update_dpp(0, x, 0x121, 0xF, 0xF, false); break;
  }
  return __builtin_bit_cast(float, x);
}

__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp_ror(v, 8));
  v = fmaxf(v, dpp_ror(v, 4));
  v = fmaxf(v, dpp_ror(v, 2));
  v = fmaxf(v, dpp_ror(v, 1));
  return v;
}

__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_ror(v, 8);
  v += dpp_ror(v, 4);
  v += dpp_ror(v, 2);
  v += dpp_ror(v, 1);
  return v;
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// 8 nibbles of w (nibble i in bits 4i..4i+3) -> 8 bf16 values 128 + c as an
// MFMA operand.  bf16(128 + c) = 0x4300 | c: the code is the low byte and 0x43
// the high byte, so two masks and four byte permutes build the operand.  The
// element order is k = [n0 n2 n4 n6 n1 n3 n5 n7] (kNibOfK below); the other
// operand of the product is laid out in the same order.
constexpr float kCodeBias = 128.0f;
// The PV accumulators hold O * kPvScale: fp16 subnormal codes are c * 2^-24
// (x16 for odd tokens) against fp16 weights 16 w (w for odd tokens).
constexpr float kPvScale = 0x1p-20f;
// fp16 bit patterns bounding the V scales of the fp16 PV path: [2^-10, 255].
constexpr uint32_t kF16ScaleMinBits = 0x1400u;  // 2^-10
constexpr uint32_t kF16ScaleMaxBits = 0x4BC0u;  // 15.5

__device__ __forceinline__ u32x4 nib8_to_bf16_128c(uint32_t w) {
  const uint32_t ev = w & 0x0F0F0F0Fu;          // bytes: n0 n2 n4 n6
  const uint32_t od = (w >> 4) & 0x0F0F0F0Fu;   // bytes: n1 n3 n5 n7
  const uint32_t k43 = 0x43434343u;
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(k43, ev, 0x04010400u);  // n0, n2
  r[1] = __builtin_amdgcn_perm(k43, ev, 0x04030402u);  // n4, n6
  r[2] = __builtin_amdgcn_perm(k43, od, 0x04010400u);  // n1, n3
  r[3] = __builtin_amdgcn_perm(k43, od, 0x04030402u);  // n5, n7
  return r;
}

// Nibble index held by operand element k of nib8_to_bf16_128c, and the
// operand element holding nibble e.
__host__ __device__ constexpr int nib_of_k(int k) { return k < 4 ? 2 * k : 2 * (k - 4) + 1; }
__host__ __device__ constexpr int k_of_nib(int e) { return (e & 1) ? 4 + (e >> 1) : (e >> 1); }

__device__ __forceinline__ f32x4 mfma_bf16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t bf16_bits(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}

// Two fp32 values as one packed bf16 pair (RNE, one v_cvt_pk_bf16_f32).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

// Two fp32 values as one packed fp16 pair (RNE, one v_cvt_pk_f16_f32).
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ uint32_t pk_f16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, f16x2_t));
}

__device__ __forceinline__ f32x4 mfma_f16(const u32x4& a, const u32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// 8 nibbles of w (tokens 0..7 of one V dim) -> fp16 PV operand in the k
// order [t0 t4 t1 t5 t2 t6 t3 t7], as subnormals: even tokens c * 2^-24, odd
// tokens 16 c * 2^-24 (the nibble left where it sits; the matching weights
// carry 1/16).  Exact inputs, no bias term; five ops per 8 codes.
// Nibble (dimension of the 8) held by operand element k of nib8_to_f16_sub,
// and whether that element comes out x16 (a high nibble of its byte pair).
__host__ __device__ constexpr int nib_of_k16(int k) { return (k >> 1) + 4 * (k & 1); }
__host__ __device__ constexpr bool k16_x16(int k) { return (k & 2) != 0; }

__device__ __forceinline__ u32x4 nib8_to_f16_sub(uint32_t w) {
  const uint32_t w8 = w >> 8;
  return u32x4{w & 0x000F000Fu, w & 0x00F000F0u, w8 & 0x000F000Fu, w8 & 0x00F000F0u};
}

// (a, b) as a bf16 hi pair plus the bf16 pair of what the hi parts leave
// (a - hi_a, b - hi_b, exact in fp32): about 16 significant bits each.
__device__ __forceinline__ void pk_bf16_hilo(float a, float b, uint32_t* hi, uint32_t* lo) {
  const uint32_t h = pk_bf16(a, b);
  *hi = h;
  *lo = pk_bf16(a - u2f(h << 16), b - u2f(h & 0xFFFF0000u));
}

__device__ __forceinline__ float pscale(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
}
__device__ __forceinline__ float pzero(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// One v_fma_mix_f32 with an fp16 operand taken from h's high or low half
// (converted exactly; one rounding), in place: acc += hi(h) * x, or
// x *= lo(h).  Written out because the compiler converts a param it uses
// twice and then issues a separate fma for each use.  The result goes to the
// register of a value the compiler has just written (acc's or x's): an
// inline-asm write into a register that an MFMA still reads as its
// accumulator input needs wait states the compiler inserts only for its own
// instructions.  For the same reason no operand may be an MFMA result.
__device__ __forceinline__ void fma_mix_hi_acc(float& acc, uint32_t h, float x) {
  asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(h), "v"(x));
}
__device__ __forceinline__ void mul_mix_lo_inplace(float& x, uint32_t h) {
  asm("v_fma_mix_f32 %0, %1, %0, 0 op_sel_hi:[1,0,0]" : "+v"(x) : "v"(h));
}

// Query element as fp32 (bf16 or fp16 storage).
template <bool QBF16>
__device__ __forceinline__ float qval(uint16_t b) {
  if constexpr (QBF16) return u2f((uint32_t)b << 16);
  else return (float)__builtin_bit_cast(_Float16, b);
}

template <bool QBF16>
__device__ __forceinline__ uint16_t oval(float x) {
  if constexpr (QBF16) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  } else {
    keep_f32(x);
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
}

struct SplitRange {
  int begin, end;  // token range of this split; begin >= end: nothing to do
};

// Context length of sequence s, clamped to what the block table and the
// launch (max_context_len, which sized the grid and the workspace) cover.
__device__ __forceinline__ int clamp_context(const DecodeArgs& a, int s) {
  int ctx = a.context_lens[s];
  const int max_tok = min(a.bt_stride * kBS, a.max_context_len);
  if (ctx > max_tok || ctx < 0) {
    if (threadIdx.x == 0 && a.err_flag) atomicOr(a.err_flag, AMF_ERRFLAG_CONTEXT);
    ctx = ctx < 0 ? 0 : max_tok;
  }
  return ctx;
}

// ---- stream-K work map (MFMA path) ----------------------------------------
// Units are (sequence, KV head, 32-token chunk), sequence-major; wave w of G
// takes units [w C / G, (w + 1) C / G) of the C in all.  A (sequence, KV head)
// spanned by several waves is merged from their partials: slot 0 of a wave
// holds the segment its share starts with, slot 1 the one it ends with.

// Chunks of sequence s (its context clamped as clamp_context does).
__device__ __forceinline__ int64_t sk_chunks(const DecodeArgs& a, int s) {
  int ctx = a.context_lens[s];
  const int max_tok = min(a.bt_stride * kBS, a.max_context_len);
  ctx = ctx < 0 ? 0 : min(ctx, max_tok);
  return (ctx + 31) / 32;
}

// A wave-uniform value the compiler cannot prove uniform, moved to SGPRs.
__device__ __forceinline__ int64_t uni64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ int uni32(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// C: units of all sequences (every lane gets it).
__device__ __forceinline__ int64_t sk_total_units(const DecodeArgs& a, int n_seqs) {
  const int lane = threadIdx.x & 63;
  int64_t t = 0;
  for (int i = lane; i < n_seqs; i += 64) t += sk_chunks(a, i);
  return uni64(wave_sum_i64(t) * a.num_kv_heads);
}

// Sequence s holding unit u0 < C, and the units P before it.
__device__ __forceinline__ void sk_locate(const DecodeArgs& a, int n_seqs, int64_t u0, int* s_out,
                                          int64_t* p_out) {
  const int lane = threadIdx.x & 63;
  int64_t before = 0;
  for (int s0 = 0; s0 < n_seqs; s0 += 64) {
    const int64_t n = s0 + lane < n_seqs ? sk_chunks(a, s0 + lane) * a.num_kv_heads : 0;
    int64_t incl = n;  // inclusive prefix over the lanes
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t y = __shfl_up(incl, o);
      if (lane >= o) incl += y;
    }
    const uint64_t hit = __ballot(before + incl > u0);
    if (hit) {
      const int l = __builtin_ctzll(hit);
      *s_out = uni32(s0 + l);
      *p_out = uni64(before + __shfl(incl - n, l));
      return;
    }
    before = uni64(before + __shfl(incl, 63));
  }
  *s_out = n_seqs;
  *p_out = before;
}

// Wave holding unit u: the largest w with w C / G <= u.
__device__ __forceinline__ int64_t sk_wave_of(int64_t u, int64_t total, int64_t G) {
  return ((u + 1) * G - 1) / total;
}

// 8 output elements at element offset `row` of the output, in its dtype.
__device__ __forceinline__ void store_out8(const DecodeArgs& a, int64_t row, const float* y) {
  if (a.out_dtype == AMF_DTYPE_F32) {
    float* out = static_cast<float*>(a.out) + row;
    *reinterpret_cast<float4*>(out) = float4{y[0], y[1], y[2], y[3]};
    *reinterpret_cast<float4*>(out + 4) = float4{y[4], y[5], y[6], y[7]};
  } else {
    uint16_t* out = static_cast<uint16_t*>(a.out) + row;
    u32x4 v;
    if (a.out_dtype == AMF_DTYPE_BF16) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[i] = (uint32_t)oval<true>(y[2 * i]) | ((uint32_t)oval<true>(y[2 * i + 1]) << 16);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[i] = (uint32_t)oval<false>(y[2 * i]) | ((uint32_t)oval<false>(y[2 * i + 1]) << 16);
    }
    *reinterpret_cast<u32x4*>(out) = v;
  }
}

// Physical page of logical page `pi` (which must lie inside the context);
// out-of-range ids are reported and replaced by page 0 with ok = false.
__device__ __forceinline__ int64_t page_of(const DecodeArgs& a, const int32_t* bt, int pi,
                                           bool in_ctx, bool* ok) {
  if (!in_ctx) {
    *ok = false;
    return 0;
  }
  const int v = bt[pi];
  *ok = v >= 0 && (int64_t)v < a.pool_pages;
  if (!*ok && threadIdx.x == 0 && a.err_flag) atomicOr(a.err_flag, AMF_ERRFLAG_BLOCK_RANGE);
  return *ok ? (int64_t)v : 0;
}

// The chunks of a split stream through a per-wave LDS ring.  A slot holds
// the K codes of page 0 and 1 (1 KiB each, [0, 2048)), their V codes
// ([2048, 4096)) and the four 256-byte parameter blocks K0, K1, V0, V1
// ([4096, 5120)).  Each block arrives by one LDS DMA (global_load_lds_dwordx4,
// non-temporal: every line is read once, by one instruction); DMA lane L
// writes slot bytes [16 L, 16 L + 16), and its source address is chosen so
// that the compute lanes' reads (read_chunk_k, read_chunk_vc/vp) are consecutive 16-byte slots
// (no bank conflicts).  No load registers are held while a chunk is in
// flight, so a wave keeps several chunks in flight at any occupancy.
constexpr int kSlotBytes = 5120;

// One 16-byte LDS DMA per lane: lane i's 16 bytes at g land at lds + 16 i
// (lds wave-uniform), non-temporal.  Written as inline asm so that the
// compiler does not track it: it cannot tell which LDS bytes a DMA writes,
// and for a DMA it knows of it waits for every load in flight (vmcnt(0))
// before LDS accesses it cannot separate from it (p_lds, and the ring slot
// being read), which drains the ring each chunk.  dma_wait does the waiting
// instead; loads the compiler issues complete in order with these DMAs, so
// its own vmcnt waits stay valid (DMAs it does not count only make them
// wait longer).  Each DMA takes a wave-uniform base in SGPRs and the lane's
// 32-bit byte offset (the saddr form), so a chunk's addresses cost no VALU
// work; lane i's bytes land at LDS address m0 + 16 i (dwordx4) or + 4 i
// (dword).  One wait state separates the M0 write from the DMA.
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
               : : "v"(off), "s"(base), "s"(m0) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const void* base, uint32_t off, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1 nt"
               : : "v"(off), "s"(base), "s"(m0) : "memory", "m0");
}

// LDS address of a __shared__ byte (wave-uniform for the ring slots).
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)p;
}

// The lane's byte offsets into a chunk's blocks, fixed for the kernel.
struct DmaLane {
  uint32_t koff;  // K codes: compute lane (t = lo, j = hi) reads slot lane,
                  // bytes 64 t + 16 j .. + 15 of the (page, head) block
  uint32_t voff;  // V codes: compute lane (lo, hi) needs the 32 bytes
                  // 64 lo + 32 (hi & 1) of page hi >> 1, as halves j = 0, 1
                  // in slots lo + 16 (hi & 1) + 32 j of that page
  uint32_t poff;  // params: 4 bytes per lane of a 256-byte block
};
__device__ __forceinline__ DmaLane dma_lane(int lane) {
  const int lo = lane & 15, hi = lane >> 4;
  return DmaLane{(uint32_t)(lo * 64 + hi * 16), (uint32_t)(64 * lo + 32 * (hi & 1) + 16 * (hi >> 1)),
                 (uint32_t)(lane * 4)};
}

// The 8 DMAs of one chunk (pages pg0, pg1 of KV head h) into the slot at LDS
// address m0: K codes of both pages, V codes of both pages, then the four
// 256-byte param blocks (K0, K1, V0, V1) as they are.
constexpr int kDmasPerChunk = 8;
__device__ __forceinline__ void dma_chunk(const DecodeArgs& a, int64_t pg0, int64_t pg1, int h,
                                          const DmaLane& dl, uint32_t m0) {
  const int64_t H = a.num_kv_heads, hb0 = pg0 * H + h, hb1 = pg1 * H + h;
  lds_dma16(a.kc + hb0 * kHBCodes, dl.koff, m0);
  lds_dma16(a.kc + hb1 * kHBCodes, dl.koff, m0 + 1024);
  lds_dma16(a.vc + hb0 * kHBCodes, dl.voff, m0 + 2048);
  lds_dma16(a.vc + hb1 * kHBCodes, dl.voff, m0 + 3072);
  lds_dma4(a.kp + hb0 * kHBParams, dl.poff, m0 + 4096);
  lds_dma4(a.kp + hb1 * kHBParams, dl.poff, m0 + 4096 + 256);
  lds_dma4(a.vp + hb0 * kHBParams, dl.poff, m0 + 4096 + 512);
  lds_dma4(a.vp + hb1 * kHBParams, dl.poff, m0 + 4096 + 768);
}

// Operands of one chunk from its slot, in the MFMA lane layout.  K: codes
// and params of page u for lane (t = lo, j = hi).  V: codes of dim block lo
// for tokens 8 hi .. 8 hi + 7 (halves 0 and 1: dims 0-3 and 4-7 of the
// block), and the params of group lo % 4 for those tokens.
__device__ __forceinline__ void read_chunk_k(const uint8_t* slot, int lane, u32x4 (&kcode)[2],
                                             u32x4 (&kpar)[2]) {
  const int lo = lane & 15;
  kcode[0] = *reinterpret_cast<const u32x4*>(slot + lane * 16);
  kcode[1] = *reinterpret_cast<const u32x4*>(slot + 1024 + lane * 16);
  kpar[0] = *reinterpret_cast<const u32x4*>(slot + 4096 + lo * 16);
  kpar[1] = *reinterpret_cast<const u32x4*>(slot + 4096 + 256 + lo * 16);
}

__device__ __forceinline__ void read_chunk_vc(const uint8_t* slot, int lane, u32x4* vc0,
                                              u32x4* vc1) {
  const int lo = lane & 15, hi = lane >> 4;
  const uint8_t* vs = slot + 2048 + 1024 * (hi >> 1) + (lo + 16 * (hi & 1)) * 16;
  *vc0 = *reinterpret_cast<const u32x4*>(vs);
  *vc1 = *reinterpret_cast<const u32x4*>(vs + 512);
}

__device__ __forceinline__ void read_chunk_vp(const uint8_t* slot, int lane, u32x4* vp0,
                                              u32x4* vp1) {
  const int lo = lane & 15, hi = lane >> 4;
  const uint8_t* ps = slot + 4096 + 512 + 256 * (hi >> 1) + ((lo & 3) * 16 + 8 * (hi & 1)) * 4;
  *vp0 = *reinterpret_cast<const u32x4*>(ps);
  *vp1 = *reinterpret_cast<const u32x4*>(ps + 16);
}

// Waits until at most `newer` chunks' DMAs (issued after the one about to be
// read) are outstanding; vmcnt counts this wave's vector-memory instructions
// in issue order and the loop issues nothing else.  The compiler does not
// order LDS reads after LDS DMAs by itself, so the memory clobber also keeps
// the chunk's LDS reads below the wait.
template <int D>
__device__ __forceinline__ void dma_wait(int newer) {
  static_assert(D >= 2 && D <= 4, "ring depth");
  static_assert(kDmasPerChunk == 8, "the counts below are 8 per chunk");
  if (D >= 4 && newer >= 3) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
  else if (D >= 3 && newer >= 2) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  else if (newer >= 1) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Block-table entries of a split (at most 64 pages: split_tokens <= 1024),
// one per lane; chunk code reads them back with readlane (wave-uniform).
struct SplitPages {
  int v;            // this lane's physical page id (or -1)
  int first;        // logical page index of lane 0
  uint64_t okmask;  // bit i: lane i's page is in the context with a valid id
};

// Lane's raw block-table entry of split sp, read before the context length
// is known (so the two loads overlap); bounded by the table's row only.
__device__ __forceinline__ int split_table_entry(const DecodeArgs& a, const int32_t* bt, int sp) {
  const int first = sp * (a.split_tokens / kBS), lane = threadIdx.x & 63;
  return (lane < a.split_tokens / kBS && first + lane < a.bt_stride) ? bt[first + lane] : -1;
}

// The split's pages from the raw entries: entries past the context become
// -1 (never read); out-of-range ids inside it are reported and become -2
// (masked, never dereferenced).
__device__ __forceinline__ SplitPages split_pages(const DecodeArgs& a, int raw, int tok_begin,
                                                  int tok_end) {
  SplitPages sp;
  sp.first = tok_begin / kBS;
  const int n = (tok_end - tok_begin + kBS - 1) / kBS;
  // An empty asm that reads raw outside any lane branch: the compiler waits
  // for raw's load here, on every path.  Otherwise the wait sits in a branch
  // it cannot prove is taken, and it later waits for every load and DMA in
  // flight (vmcnt(0)) before it reuses raw's register, inside the chunk loop.
  asm volatile("" : : "v"(raw));
  int v = -1;
  if ((int)(threadIdx.x & 63) < n) {
    v = raw;
    if (v < 0 || (int64_t)v >= a.pool_pages) {
      if (a.err_flag) atomicOr(a.err_flag, AMF_ERRFLAG_BLOCK_RANGE);
      v = -2;
    }
  }
  sp.v = v;
  sp.okmask = __ballot(v >= 0);
  return sp;
}

// Physical page of logical page pi of the split, page 0 when it is outside
// the context or invalid (ok = false).
__device__ __forceinline__ int64_t split_page(const SplitPages& sp, int pi, bool* ok) {
  const int v = __builtin_amdgcn_readlane(sp.v, pi - sp.first);
  *ok = v >= 0;
  return v >= 0 ? (int64_t)v : 0;
}

// Work item of this wave.  With head_fast the grid is (num_kv_heads,
// max_splits, num_seqs): the KV heads of a split are neighbouring workgroups,
// so the codes of one page (all heads, contiguous) are read at about the same
// time; otherwise (more splits than grid.y allows) it is (max_splits,
// num_kv_heads, num_seqs).
__device__ __forceinline__ int work_head(const DecodeArgs& a) {
  return a.head_fast ? blockIdx.x : blockIdx.y;
}
__device__ __forceinline__ int work_split(const DecodeArgs& a) {
  return a.head_fast ? blockIdx.y : blockIdx.x;
}

// ============================================================== MFMA path ==

// One 32-token chunk of the MFMA kernel, in two steps: chunk_qk (QK^T and the
// online softmax, leaving the weights p in p_lds) and chunk_pv (PV).
#ifndef AMF_DECODE_RESCALE_SLACK
#define AMF_DECODE_RESCALE_SLACK 8.0f
#endif
constexpr float kRescaleSlack = AMF_DECODE_RESCALE_SLACK;  // log2 units

template <int R>
__device__ __forceinline__ void chunk_qk(
    const uint8_t* slot, const bool (&pok)[2], int c0, int tok_end, int lo, int hi,
    const u32x4 (&qa)[(R + 3) / 4][4], float qk_scale, const float (&qs_lds)[(R + 3) / 4][4][4],
    float (&m_run)[(R + 3) / 4], float (&l_run)[(R + 3) / 4],
    float (&corr)[(R + 3) / 4], float (&wsum)[(R + 3) / 4], float (&lsum)[(R + 3) / 4],
    f32x4 (&acc)[(R + 3) / 4][8], float (&p_lds)[(R + 3) / 4][2][4][16]) {
  constexpr int NT = (R + 3) / 4;
  const int lane = lo + 16 * hi;
  // K operands only; the V side is read from the slot just before the PV
  // product, so its registers are not live across QK^T and the softmax.
  u32x4 kcode[2], kpar[2];
  read_chunk_k(slot, lane, kcode, kpar);

  // ---- QK^T and online softmax ----
  float x[NT][2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    u32x4 kb[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) kb[st] = nib8_to_f16_sub(kcode[u][st]);
    float ks[4];
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) ks[gi] = pscale(kpar[u][gi]);
    const bool valid = pok[u] && (c0 + u * kBS + lo) < tok_end;
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      // the group sums of head 4T + hi's query (one LDS broadcast read)
      const float4 q4 = *reinterpret_cast<const float4*>(&qs_lds[T][hi][0]);
      const float qsum[4] = {q4.x, q4.y, q4.z, q4.w};
      f32x4 cacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st = 0; st < 4; ++st) cacc = mfma_f16(qa[T][st], kb[st], cacc);
      // One fma chain: the four scaled group sums (cacc, an MFMA result, is
      // read by compiler-visible operations only), then the zero-point terms
      // (the zeros read as fp16 from the high halves of the param words).
      float sc = ks[0] * cacc[0];
#pragma unroll
      for (int gi = 1; gi < 4; ++gi) sc = __builtin_fmaf(ks[gi], cacc[gi], sc);
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) fma_mix_hi_acc(sc, kpar[u][gi], qsum[gi]);
      x[T][u] = valid ? sc * qk_scale : -__builtin_inff();
    }
  }

  float p[NT][2];
#pragma unroll
  for (int T = 0; T < NT; ++T) {
    // Lazy rescale: the reference max moves only when a score exceeds it by
    // more than kRescaleSlack (p stays <= 2^kRescaleSlack), so the
    // accumulators are rescaled a few times per split, not every chunk.  A
    // lane compare and a wave vote decide that; the row maximum is only
    // taken when some score does exceed it.
    const float xm = fmaxf(x[T][0], x[T][1]);
    if (__any(xm > m_run[T] + kRescaleSlack)) {
      const float cm = row_max16(xm);
      const float m_new = fmaxf(m_run[T], cm);
      const float alpha = exp2_fast(m_run[T] - m_new);
      l_run[T] *= alpha;
#pragma unroll
      for (int b = 0; b < 8; ++b) acc[T][b] *= alpha;
      // corr, wsum and lsum live in the A layout: lane lo holds head 4T + lo/4.
      const float alpha_a = __shfl(alpha, 16 * (lo >> 2));
      corr[T] *= alpha_a;
      wsum[T] *= alpha_a;
      lsum[T] *= alpha_a;
      m_run[T] = m_new;
    }
    p[T][0] = exp2_fast(x[T][0] - m_run[T]);
    p[T][1] = exp2_fast(x[T][1] - m_run[T]);
    l_run[T] += p[T][0] + p[T][1];
    p_lds[T][0][hi][lo] = p[T][0];
    p_lds[T][1][hi][lo] = p[T][1];
  }
  __builtin_amdgcn_wave_barrier();
}

// ---- PV product: weights, the choice of their form ----
//
// The PV product is a 16x16x32 tile of weights (rows: head x group, k:
// tokens) times codes (k: tokens, columns: dims).  Codes 0-15 are exact in
// either input type; the weight w = p * s (p <= 2^8 after the lazy rescale,
// s the token's V scale of the row's group) is the rounded part.  All forms
// accumulate O * 2^-20 (restored by the partial write), so chunks of any
// form can share a split.
//  fp16: one fp16 per weight (relative error <= 2^-11), 16 w for even and w
//   for odd tokens against the codes as exact fp16 subnormals (c * 2^-24,
//   16 c * 2^-24 for odd tokens, see nib8_to_f16_sub); one MFMA per tile.
//  fp16 pair: the same operand plus a second, fp16 (x - hi) (about 22 bits;
//   a lo part below 2^-14 is off by at most 2^-25 absolute); two MFMAs per
//   tile on the same code operand.
//  bf16 pair: w * 2^-20 as a bf16 hi + lo pair (about 16 bits) against the
//   codes as the bf16 128 + c, so the zero-point term carries -128 s; two
//   MFMAs per tile.  Only for a chunk whose V scales leave [2^-10, 15.5] (then
//   fp16 weights could overflow, p <= 2^8, or lose their normal range); its
//   error is up to 2^-18 * 143 * s per unit of weight.
// Every chunk whose scales allow takes the fp16 form if the error bound
// below allows, else the fp16 pair; AMF_DECODE_MFMA_PRECISE takes the pair
// throughout.
//
// Centered codes.  The fp16 forms multiply the weights by the codes c in
// [0, 15] but account for them as c - 8 in [-8, 7]: each chunk subtracts
// 8 * (the sum of the weights exactly as the MFMA used them, the fp16
// values for the fp16 form) from the row-group's zero-point term and adds
// 8 s to each token's zero point instead (z + 8 s is exact in fp32).  The
// total is unchanged, but the weights' rounding error now meets |c - 8| <= 8
// instead of c <= 15.
//
// Error bound of the fp16 form.  Rounding w to fp16 is off by at most
// 2^-11 (w + 2^-14) (relative 2^-11 for a normal result, 2^-25 absolute for
// a subnormal one), so the fp16 weights move output element d of row (r, g)
// by at most 2^-11 * 8 * W / l, with centered codes |c - 8| <= 8, W the sum
// of w + 2^-14 over the row-group's fp16 weights and l the row's softmax sum
// (every chunk's tokens).  A chunk takes the fp16 form only if
// W <= kPv16Beta * l holds afterwards for every row-group of the GQA group;
// then that error is at most 2^-11 * 8 * kPv16Beta = 0.0146 for the finished
// row (both sides
// scale alike under the online rescale, l only grows and W only by accepted
// chunks) and for an LSE merge of such rows.  The check: lane (lo, hi) keeps
// its k-slice's shares of W and of l (the p of its tokens 8 hi .. 8 hi + 7 of
// every chunk); a chunk passes at once if every lane's W share stays within
// kPv16Beta times its l share, as the four lanes of a row-group then add up
// to W <= kPv16Beta * l; otherwise the shares are added across the k-slices
// and compared.  The weights' fp16 values stand in for w in W, and the l
// shares are summed in another order than l_run (off by 2^-11 and a few fp32
// ulps relative, inside the bound's rounding of 0.0146 to 0.015).
#ifndef AMF_DECODE_PV16_BETA
#define AMF_DECODE_PV16_BETA 3.75f
#endif
constexpr float kPv16Beta = AMF_DECODE_PV16_BETA;

// Sum of a lane's 8 fp16 PV weights as the MFMA takes them: pairs 0 and 2
// hold 16 w of even tokens, pairs 1 and 3 w of odd ones (fp16 products are
// exact in the fp32 sum).
__device__ __forceinline__ float f16_weight_sum(const f16x2_t (&h)[4]) {
  const f16x2_t k_even = {(_Float16)0.0625f, (_Float16)0.0625f}, k_odd = {(_Float16)1.0f,
                                                                          (_Float16)1.0f};
  float d = __builtin_amdgcn_fdot2(h[1], k_odd, 0.0f, false);
  d = __builtin_amdgcn_fdot2(h[3], k_odd, d, false);
  d = __builtin_amdgcn_fdot2(h[0], k_even, d, false);
  return __builtin_amdgcn_fdot2(h[2], k_even, d, false);
}

// Whether a chunk's V scales allow fp16 weights (0 or in [2^-10, 15.5]: no
// weight overflows fp16 with p <= 2^8, and every token with p >= 2^-4 has a
// normal weight): each lane checks the scale words of its 8 tokens, then the
// wave votes.
__device__ __forceinline__ bool pv_f16_range_ok(const u32x4& vp0, const u32x4& vp1) {
  uint32_t smax = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) smax = max(smax, max(vp0[e] & 0xFFFFu, vp1[e] & 0xFFFFu));
  return !__any(smax > kF16ScaleMaxBits || (smax != 0u && smax < kF16ScaleMinBits));
}

// Zeroes the V param words of the lane's tokens 8 hi .. 8 hi + 7 that lie
// outside the context or on a page with a bad id (their bytes may be
// anything), for a chunk that holds such tokens; the fp16 weight path then
// multiplies them by p = +0 with plain IEEE operations.
__device__ __forceinline__ void mask_vp_invalid(u32x4& vp0, u32x4& vp1, const bool (&pok)[2],
                                                int c0, int tok_end, int hi) {
  const int t0 = c0 + 8 * hi;
  const bool pg = pok[hi >> 1];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    vp0[e] = (pg && t0 + e < tok_end) ? vp0[e] : 0u;
    vp1[e] = (pg && t0 + 4 + e < tok_end) ? vp1[e] : 0u;
  }
}

// The chunk's fp16 PV operand in the A layout: lane (lo, hi) holds row-group
// (head 4T + lo/4, group lo%4) for tokens 8 hi .. 8 hi + 7 of the chunk, in
// the operand order [t0 t4 t1 t5 t2 t6 t3 t7], 16 w for even and w for odd
// tokens.  The zero-point sum p * (z + 8 s) goes to corr, the lane's p to
// lsum (its share of l), and wr returns the lane's fp16 weights summed as
// the MFMA takes them (w, with the 16 of even tokens divided out), for the
// centered-code correction and the error bound.  The param words of tokens
// outside the context are zero (mask_vp_invalid), and those tokens have
// p = +0 exactly (their score is -inf).
template <int R>
__device__ __forceinline__ void pv_weights_f16(const u32x4& vp0, const u32x4& vp1, int lo, int hi,
                                               float (&p_lds)[(R + 3) / 4][2][4][16],
                                               u32x4 (&a16)[(R + 3) / 4],
                                               float (&corr)[(R + 3) / 4],
                                               float (&lsum)[(R + 3) / 4],
                                               float (&wr)[(R + 3) / 4]) {
  constexpr int NT = (R + 3) / 4;
  const int vu = hi >> 1, vhalf = hi & 1;
  const uint32_t pw[8] = {vp0[0], vp0[1], vp0[2], vp0[3], vp1[0], vp1[1], vp1[2], vp1[3]};
  // per token: 16 s for even tokens, and the centered zero point z + 8 s
  float s16[8], z8[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    s16[e] = pscale(pw[e]) * 16.0f;
    z8[e] = pzero(pw[e]) + 8.0f * pscale(pw[e]);
  }
#pragma unroll
  for (int T = 0; T < NT; ++T) {
    const float4* pl = reinterpret_cast<const float4*>(&p_lds[T][vu][lo >> 2][8 * vhalf]);
    const float4 pa = pl[0], pb = pl[1];
    const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
    lsum[T] += ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
    float w[8];
    float cs = corr[T];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      cs = __builtin_fmaf(pv[e], z8[e], cs);
      if (e & 1) {
        w[e] = pv[e];
        mul_mix_lo_inplace(w[e], pw[e]);
      } else {
        w[e] = pv[e] * s16[e];
      }
    }
    f16x2_t h16[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h16[j] = __builtin_convertvector((f32x2_t){w[j], w[j + 4]}, f16x2_t);
      a16[T][j] = __builtin_bit_cast(uint32_t, h16[j]);
    }
    corr[T] = cs;
    wr[T] = f16_weight_sum(h16);
  }
}

// The error bound above for the chunk's fp16 weights (wr, the lane's sum of
// them); on yes, they join wsum (the lane's share of W).  lsum holds the
// lane's share of l (A layout, head 4T + lo/4).
template <int R>
__device__ __forceinline__ bool pv_single_ok(int lo, const float (&wr)[(R + 3) / 4],
                                             float (&wsum)[(R + 3) / 4],
                                             const float (&lsum)[(R + 3) / 4]) {
  constexpr int NT = (R + 3) / 4;
  float cand[NT];
  bool ok = true;
#pragma unroll
  for (int T = 0; T < NT; ++T) {
    // the lane's share so far, the chunk's weights and 8 * 2^-14
    cand[T] = wr[T] + (wsum[T] + 0x1p-11f);
    // rows past the GQA group carry scores of a zero query: never checked
    const bool row_used = 4 * T + (lo >> 2) < R;
    ok = ok && (!row_used || cand[T] <= kPv16Beta * lsum[T]);
  }
  if (__any(!ok)) {
    ok = true;
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      float wrow = cand[T] + __shfl_xor(cand[T], 16);
      wrow += __shfl_xor(wrow, 32);
      float lrow = lsum[T] + __shfl_xor(lsum[T], 16);
      lrow += __shfl_xor(lrow, 32);
      const bool row_used = 4 * T + (lo >> 2) < R;
      ok = ok && (!row_used || wrow <= kPv16Beta * lrow);
    }
    if (__any(!ok)) return false;
  }
#pragma unroll
  for (int T = 0; T < NT; ++T) wsum[T] = cand[T];
  return true;
}

// PV of one chunk with single fp16 weights.
template <int R>
__device__ __forceinline__ void chunk_pv_f16(const uint8_t* slot, int lane,
                                             const u32x4 (&a16)[(R + 3) / 4],
                                             f32x4 (&acc)[(R + 3) / 4][8]) {
  constexpr int NT = (R + 3) / 4;
  u32x4 vc0, vc1;
  read_chunk_vc(slot, lane, &vc0, &vc1);
  const uint32_t vw[8] = {vc0[0], vc0[1], vc0[2], vc0[3], vc1[0], vc1[1], vc1[2], vc1[3]};
  // Dim block outermost: one block's code operand is live at a time.
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const u32x4 vb = nib8_to_f16_sub(vw[b]);
#pragma unroll
    for (int T = 0; T < NT; ++T) acc[T][b] = mfma_f16(a16[T], vb, acc[T][b]);
  }
  __builtin_amdgcn_wave_barrier();
}

// The second half of a chunk's fp16 pair (after chunk_pv_f16 with the
// single weights, which are the pair's hi parts): lo = fp16(w - hi) from the
// weights in p_lds and the V params (masked as for pv_weights_f16) and the
// slot's V codes, its PV product, and 8 x its
// weights off the zero-point term (centered codes).  One 16-row tile at a
// time, so that one tile's operand is live (the code operand is rebuilt per
// tile).
template <int R>
__device__ __forceinline__ void chunk_pv_f16_lo(const uint8_t* slot, const u32x4& vp0,
                                                const u32x4& vp1, int lo, int hi,
                                                float (&p_lds)[(R + 3) / 4][2][4][16],
                                                float (&corr)[(R + 3) / 4],
                                                f32x4 (&acc)[(R + 3) / 4][8]) {
  constexpr int NT = (R + 3) / 4;
  const int lane = lo + 16 * hi;
  u32x4 vc0, vc1;
  read_chunk_vc(slot, lane, &vc0, &vc1);
  const uint32_t vw[8] = {vc0[0], vc0[1], vc0[2], vc0[3], vc1[0], vc1[1], vc1[2], vc1[3]};
  const uint32_t pw[8] = {vp0[0], vp0[1], vp0[2], vp0[3], vp1[0], vp1[1], vp1[2], vp1[3]};
  const int vu = hi >> 1, vhalf = hi & 1;
#pragma unroll
  for (int T = 0; T < NT; ++T) {
    const float4* pl = reinterpret_cast<const float4*>(&p_lds[T][vu][lo >> 2][8 * vhalf]);
    const float4 pa = pl[0], pb = pl[1];
    const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
    u32x4 al;
    f16x2_t l16[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // operand pair (t_j, t_{j+4}): 16 w for even tokens, w for odd ones
      const float sa = pscale(pw[j]), sb = pscale(pw[j + 4]);
      const float wa = pv[j] * ((j & 1) ? sa : sa * 16.0f);
      const float wb = pv[j + 4] * ((j & 1) ? sb : sb * 16.0f);
      const uint32_t h = pk_f16(wa, wb);
      l16[j] = __builtin_convertvector(
          (f32x2_t){wa - half_lo<false>(h), wb - half_hi<false>(h)}, f16x2_t);
      al[j] = __builtin_bit_cast(uint32_t, l16[j]);
    }
    corr[T] = __builtin_fmaf(-8.0f, f16_weight_sum(l16), corr[T]);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const u32x4 vb = nib8_to_f16_sub(vw[b]);
      acc[T][b] = mfma_f16(al, vb, acc[T][b]);
    }
  }
  __builtin_amdgcn_wave_barrier();
}

// PV of one chunk with bf16 hi + lo weights, from the V params (masked as for
// pv_weights_f16); the zero-point term carries the codes' bias, -128 s per
// token, besides the zero point p * z.
template <int R>
__device__ __forceinline__ void chunk_pv_bf16(const uint8_t* slot, const u32x4& vp0,
                                              const u32x4& vp1, int lo, int hi,
                                              float (&corr)[(R + 3) / 4],
                                              f32x4 (&acc)[(R + 3) / 4][8],
                                              float (&p_lds)[(R + 3) / 4][2][4][16]) {
  constexpr int NT = (R + 3) / 4;
  const int vu = hi >> 1, vhalf = hi & 1;
  u32x4 vc0, vc1;
  read_chunk_vc(slot, lo + 16 * hi, &vc0, &vc1);
  const uint32_t pw[8] = {vp0[0], vp0[1], vp0[2], vp0[3], vp1[0], vp1[1], vp1[2], vp1[3]};
  const uint32_t vw[8] = {vc0[0], vc0[1], vc0[2], vc0[3], vc1[0], vc1[1], vc1[2], vc1[3]};
  u32x4 ahi[NT], alo[NT];
#pragma unroll
  for (int T = 0; T < NT; ++T) {
    const float4* pl = reinterpret_cast<const float4*>(&p_lds[T][vu][lo >> 2][8 * vhalf]);
    const float4 pa = pl[0], pb = pl[1];
    const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
    float wk[8];
    float cs = corr[T];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float sv = pscale(pw[e]);
      wk[k_of_nib(e)] = pv[e] * (sv * kPvScale);
      cs = __builtin_fmaf(pv[e], pzero(pw[e]) - kCodeBias * sv, cs);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t h, l;
      pk_bf16_hilo(wk[2 * j], wk[2 * j + 1], &h, &l);
      ahi[T][j] = h;
      alo[T][j] = l;
    }
    corr[T] = cs;
  }
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const u32x4 vb = nib8_to_bf16_128c(vw[b]);
#pragma unroll
    for (int T = 0; T < NT; ++T) acc[T][b] = mfma_bf16(ahi[T], vb, acc[T][b]);
#pragma unroll
    for (int T = 0; T < NT; ++T) acc[T][b] = mfma_bf16(alo[T], vb, acc[T][b]);
  }
  __builtin_amdgcn_wave_barrier();
}



#ifndef AMF_DECODE_WAVES_PER_EU
#define AMF_DECODE_WAVES_PER_EU 2
#endif
#ifndef AMF_DECODE_WAVES_PER_EU_SMALL_GQA
#define AMF_DECODE_WAVES_PER_EU_SMALL_GQA 3
#endif

// D: chunks in the LDS ring (D - 1 in flight while one computes).
#ifndef AMF_DECODE_RING_SMALL_GQA
#define AMF_DECODE_RING_SMALL_GQA 2
#endif
#ifndef AMF_DECODE_RING_GQA8
#define AMF_DECODE_RING_GQA8 3
#endif
template <int R, bool QBF16, int D = (R > 4 ? AMF_DECODE_RING_GQA8 : AMF_DECODE_RING_SMALL_GQA)>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(
    R > 4 ? AMF_DECODE_WAVES_PER_EU : AMF_DECODE_WAVES_PER_EU_SMALL_GQA)))
void int4_decode_mfma_kernel(DecodeArgs a) {
  constexpr int NT = (R + 3) / 4;  // 16-row tiles of (head, group) pairs
  const int lane = threadIdx.x, lo = lane & 15, hi = lane >> 4;
  const int H = a.num_kv_heads;
  __shared__ __attribute__((aligned(16))) float p_lds[NT][2][4][16];
  __shared__ __attribute__((aligned(16))) uint8_t ring[D][kSlotBytes];
  const uint32_t ring_m0 = __builtin_amdgcn_readfirstlane(lds_addr(&ring[0][0]));
  const DmaLane dl = dma_lane(lane);
  __shared__ __attribute__((aligned(16))) float qs_lds[NT][4][4];  // query group sums

  // ---- this wave's share: units (sequence, KV head, 32-token chunk) in that
  // order, units [w C / G, (w + 1) C / G) for wave w of G ----
  const int64_t total = sk_total_units(a, a.num_seqs);
  // G <= C: every wave of the first G gets at least one unit, so the waves
  // spanning a pair all hold a part of it (the rest exit).
  const int64_t G = min((int64_t)a.sk_waves, total), w = blockIdx.x;
  if (w >= G) return;
  // The merge finds a pair's waves from the units before its sequence, which
  // the wave holding the sequence's first unit records, and from the total.
  if (w == 0 && lane == 0) a.sk_meta[a.num_seqs] = total;
  const int64_t u0 = uni64(w * total / G), u1 = uni64((w + 1) * total / G);
  if (u0 >= u1) return;
  int s = 0;
  int64_t P = 0;  // units before sequence s
  sk_locate(a, a.num_seqs, u0, &s, &P);
  int64_t u = u0;
  while (u < u1) {
    const int ctx = uni32(clamp_context(a, s));
    const int nch_s = (ctx + 31) / 32;
    if (u >= P + (int64_t)H * nch_s) {  // past this sequence (or an empty one)
      P += (int64_t)H * nch_s;
      ++s;
      continue;
    }
    if (u == P && lane == 0) a.sk_meta[s] = P;
    const int h = uni32((int)((u - P) / nch_s));
    const int64_t pair0 = uni64(P + (int64_t)h * nch_s), pair1 = pair0 + nch_s;
    const int64_t seg_end = uni64(min(u1, pair1));
    const int c_a = uni32((int)(u - pair0)), c_b = uni32((int)(seg_end - pair0));
    const int32_t* bt = a.block_tables + (int64_t)s * a.bt_stride;
    const uint16_t* qh = a.q + ((int64_t)s * a.num_q_heads + (int64_t)h * R) * kD;

    // ---- Q operands (constant for the wave) ----
    // Every lane loads (rows past the GQA group clamped to its last row) and
    // the lanes a value does not belong to zero it afterwards: loads under a
    // lane condition would each wait for the one before.
    u32x4 qraw[NT][5];
  #pragma unroll
    for (int T = 0; T < NT; ++T) {
      const int r = 4 * T + (lo >> 2), g = lo & 3;
      const uint16_t* qr = qh + (r < R ? r : R - 1) * kD;
  #pragma unroll
      for (int st = 0; st < 4; ++st)
        qraw[T][st] = *reinterpret_cast<const u32x4*>(qr + 32 * hi + 8 * st);
      qraw[T][4] = *reinterpret_cast<const u32x4*>(qr + 32 * g + 8 * hi);
    }
    // The QK^T tiles are fp16: K codes as exact subnormals c * 2^-24
    // (nib8_to_f16_sub) against the query scaled by 2^-qe, qe chosen per wave
    // so that its largest |q| lands in [2^14, 2^15): every bf16 or fp16 query
    // element above 2^-24 of that maximum converts exactly.  The scores are
    // then scaled back by 2^(24 + qe) (folded into qk_scale, and the zero-point
    // sums qsum are scaled by 2^-(24 + qe) to match).
    float qmax = 0.0f;
  #pragma unroll
    for (int T = 0; T < NT; ++T)
  #pragma unroll
      for (int st = 0; st < 4; ++st)
  #pragma unroll
        for (int i = 0; i < 4; ++i)
          qmax = fmaxf(qmax, fmaxf(fabsf(qval<QBF16>((uint16_t)(qraw[T][st][i] & 0xFFFFu))),
                                   fabsf(qval<QBF16>((uint16_t)(qraw[T][st][i] >> 16)))));
    qmax = wave_max_xor(qmax, 64);
    // floor(log2(qmax)) - 14 for a normal finite qmax; 0 otherwise (a zero, a
    // subnormal-only or a non-finite query keeps its own values)
    const int qexp = (int)((f2u(qmax) >> 23) & 0xFFu);
    const int qe = (qexp > 0 && qexp < 255) ? min(max(qexp - 127 - 14, -100), 100) : 0;
    const float q_down = __builtin_ldexpf(1.0f, -qe);
    const float qk_scale = a.qk_scale_log2 * __builtin_ldexpf(1.0f, 24 + qe);
    const float qsum_down = __builtin_ldexpf(1.0f, -24 - qe);
    u32x4 qa[NT][4];
  #pragma unroll
    for (int T = 0; T < NT; ++T) {
      const int r = 4 * T + (lo >> 2), g = lo & 3;
      // A operand of k-step st: row (r, g) holds q[r][32 g + 8 st + e] on the
      // lanes whose k-slice (hi) is group g.
      const bool mine = r < R && g == hi;
  #pragma unroll
      for (int st = 0; st < 4; ++st) {
        // Elements in the k order of nib8_to_f16_sub, the x16 ones divided by 16.
        const u32x4 raw = qraw[T][st];
        float xq[8];
  #pragma unroll
        for (int i = 0; i < 4; ++i) {
          xq[2 * i] = qval<QBF16>((uint16_t)(raw[i] & 0xFFFFu)) * q_down;
          xq[2 * i + 1] = qval<QBF16>((uint16_t)(raw[i] >> 16)) * q_down;
        }
        u32x4 v;
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e0 = xq[nib_of_k16(2 * j)] * (k16_x16(2 * j) ? 0.0625f : 1.0f);
          const float e1 = xq[nib_of_k16(2 * j + 1)] * (k16_x16(2 * j + 1) ? 0.0625f : 1.0f);
          v[j] = mine ? pk_f16(e0, e1) : 0u;
        }
        qa[T][st] = v;
      }
      // Qsum[r][g] = sum of q[r][32 g .. 32 g + 31]: lanes (lo, hi) add 8 of
      // them, a cross-row sum completes it, and row hi = 0 stores it for the
      // QK^T step, where lane (t, j) reads the four groups of head 4T + j.
      float part = 0.0f;
  #pragma unroll
      for (int i = 0; i < 4; ++i)
        part += qval<QBF16>((uint16_t)(qraw[T][4][i] & 0xFFFFu)) +
                qval<QBF16>((uint16_t)(qraw[T][4][i] >> 16));
      part = r < R ? part : 0.0f;
      part += __shfl_xor(part, 16);
      part += __shfl_xor(part, 32);
      if (hi == 0) qs_lds[T][lo >> 2][lo & 3] = part * qsum_down;
    }
    __builtin_amdgcn_wave_barrier();


    float m_run[NT], l_run[NT], corr[NT], wsum[NT], lsum[NT];
    f32x4 acc[NT][8];
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      m_run[T] = kNegBig;
      l_run[T] = 0.0f;
      corr[T] = 0.0f;
      wsum[T] = 0.0f;
      lsum[T] = 0.0f;
#pragma unroll
      for (int b = 0; b < 8; ++b) acc[T][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // Pieces of at most 32 chunks (64 pages: one block-table entry per lane).
    for (int pc = c_a; pc < c_b; pc += 32) {
      const int tok_begin = pc * 32;
      const int tok_end = min(ctx, min(c_b, pc + 32) * 32);
      const int pfirst = tok_begin / kBS, pn = (tok_end - tok_begin + kBS - 1) / kBS;
      const int bt_raw = (lane < pn && pfirst + lane < a.bt_stride) ? bt[pfirst + lane] : -1;
      // Ring pipeline: chunks c + 1 .. c + D - 1 are in flight while chunk c
      // computes.
      const SplitPages spg = split_pages(a, bt_raw, tok_begin, tok_end);
      const int nch = (tok_end - tok_begin + 31) / 32;
      const int pi0 = tok_begin / kBS;
      auto issue = [&](int c) {
        bool ok;
        const int64_t p0 = split_page(spg, pi0 + 2 * c, &ok);
        const int64_t p1 = split_page(spg, pi0 + 2 * c + 1, &ok);
        dma_chunk(a, p0, p1, h, dl, ring_m0 + (uint32_t)((c % D) * kSlotBytes));
      };
    #pragma unroll
      for (int k = 0; k + 1 < D; ++k)
        if (k < nch) issue(k);
      auto qk = [&](int c, bool (&pok)[2]) {
        dma_wait<D>(min(D - 1, nch - 1 - c));
        pok[0] = (spg.okmask >> (pi0 - spg.first + 2 * c)) & 1;
        pok[1] = (spg.okmask >> (pi0 - spg.first + 2 * c + 1)) & 1;
        chunk_qk<R>(ring[c % D], pok, tok_begin + 32 * c, tok_end, lo, hi, qa, qk_scale, qs_lds,
                    m_run, l_run, corr, wsum, lsum, acc, p_lds);
      };
      // Chunks take fp16 weights, single where the error bound allows
      // (pv_single_ok) and paired elsewhere, until one whose V scales fp16
      // cannot take; from that chunk on the piece finishes on bf16 pairs (a
      // second loop, so that each loop keeps its own register footprint).
      // The chunk's V params, those of tokens outside the context zeroed.
      auto load_vp = [&](int c, const bool (&pok)[2], u32x4& vp0, u32x4& vp1) {
        read_chunk_vp(ring[c % D], lane, &vp0, &vp1);
        if (!(pok[0] && pok[1] && tok_begin + 32 * c + 32 <= tok_end))
          mask_vp_invalid(vp0, vp1, pok, tok_begin + 32 * c, tok_end, hi);
      };
      int c = 0;
      bool pending = false;  // chunk c has had QK^T and the softmax, not PV
      u32x4 pvp0, pvp1;      // and these V params
      for (; c < nch; ++c) {
        if (c + D - 1 < nch) issue(c + D - 1);
        bool pok[2];
        qk(c, pok);
        u32x4 vp0, vp1;
        load_vp(c, pok, vp0, vp1);
        if (!pv_f16_range_ok(vp0, vp1)) {
          pending = true;
          pvp0 = vp0;
          pvp1 = vp1;
          break;
        }
        u32x4 a16[NT];
        float wr[NT];
        pv_weights_f16<R>(vp0, vp1, lo, hi, p_lds, a16, corr, lsum, wr);
        // centered codes: 8 x the weights the MFMA takes come off the zero-point term
        const bool single = a.pv16 && pv_single_ok<R>(lo, wr, wsum, lsum);
#pragma unroll
        for (int T = 0; T < NT; ++T) corr[T] = __builtin_fmaf(-8.0f, wr[T], corr[T]);
        chunk_pv_f16<R>(ring[c % D], lane, a16, acc);
        if (!single) {
          // the params again (their registers are not kept across the PV)
          u32x4 wp0, wp1;
          load_vp(c, pok, wp0, wp1);
          chunk_pv_f16_lo<R>(ring[c % D], wp0, wp1, lo, hi, p_lds, corr, acc);
        }
      }
      for (; c < nch; ++c) {
        if (!pending) {
          if (c + D - 1 < nch) issue(c + D - 1);
          bool pok[2];
          qk(c, pok);
          load_vp(c, pok, pvp0, pvp1);
        }
        pending = false;
        chunk_pv_bf16<R>(ring[c % D], pvp0, pvp1, lo, hi, corr, acc, p_lds);
      }
    }

    // ---- the segment's result: the output itself when the wave holds the
    // whole (sequence, KV head), else a partial (unnormalised O, m, l) in
    // its slot: 0 for the share's first segment, 1 for its last ----
    const bool owned = c_a == 0 && c_b == nch_s;
    const int slot = u == u0 ? 0 : 1;
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      const float l_tot = row_sum16(l_run[T]);
      float cf = corr[T];
      cf += __shfl_xor(cf, 16);
      cf += __shfl_xor(cf, 32);
      const int gsel = lo >> 2;  // group of dims 8 lo .. 8 lo + 7
      const float cv = __shfl(cf, 4 * hi + gsel);
      const int r = 4 * T + hi;
      if (r < R) {
        float o[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const f32x4 t = acc[T][b];
          const float v = gsel == 0 ? t[0] : gsel == 1 ? t[1] : gsel == 2 ? t[2] : t[3];
          o[b] = __builtin_fmaf(v, 1.0f / kPvScale, cv);
        }
        if (owned) {
          // as the merge does for one split: its weight exp2(m - m) = 1
          const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
          const int64_t row = ((int64_t)s * a.num_q_heads + (int64_t)h * R + r) * kD + 8 * lo;
          float y[8];
#pragma unroll
          for (int b = 0; b < 8; ++b) y[b] = o[b] * inv;
          store_out8(a, row, y);
        } else {
          float* base = a.ws + ((w * 2 + slot) * R + r) * kPartStride;
          *reinterpret_cast<float4*>(base + 8 * lo) = float4{o[0], o[1], o[2], o[3]};
          *reinterpret_cast<float4*>(base + 8 * lo + 4) = float4{o[4], o[5], o[6], o[7]};
          if (lo == 0) {
            base[kD] = m_run[T];
            base[kD + 1] = l_tot;
          }
        }
      }
    }
    u = seg_end;
  }
}

// ============================================================== VALU path ==

template <int R, bool QBF16>
__global__ __launch_bounds__(64) void int4_decode_valu_kernel(DecodeArgs a) {
  static_assert(R <= 4, "VALU path: at most 4 query heads per KV head");
  const int sp = work_split(a), h = work_head(a), s = blockIdx.z;
  const int lane = threadIdx.x, lo = lane & 15, hi = lane >> 4;
  const int ctx = clamp_context(a, s);
  const int tok_begin = sp * a.split_tokens;
  if (tok_begin >= ctx) return;
  const int tok_end = min(ctx, tok_begin + a.split_tokens);
  const int32_t* bt = a.block_tables + (int64_t)s * a.bt_stride;
  const int H = a.num_kv_heads;
  const uint16_t* qh = a.q + ((int64_t)s * a.num_q_heads + (int64_t)h * R) * kD;

  // QK layout: lane (t = lo, j = hi) owns K dims 32 j .. 32 j + 31 (group j).
  float qr[R][32], qs[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    qs[r] = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4 raw = *reinterpret_cast<const u32x4*>(qh + r * kD + 32 * hi + 8 * v);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        qr[r][8 * v + 2 * i] = qval<QBF16>((uint16_t)(raw[i] & 0xFFFFu));
        qr[r][8 * v + 2 * i + 1] = qval<QBF16>((uint16_t)(raw[i] >> 16));
      }
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) qs[r] += qr[r][i];
  }

  float m_run = kNegBig, l_run = 0.0f;      // head hi (rows of the score layout)
  float accv[R][8], zacc[R];                // PV layout: lane (n = lo, j' = hi)
#pragma unroll
  for (int r = 0; r < R; ++r) {
    zacc[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) accv[r][k] = 0.0f;
  }
  __shared__ __attribute__((aligned(16))) float p_lds[2][4][16];

  for (int c0 = tok_begin; c0 < tok_end; c0 += 32) {
    const int pi0 = c0 / kBS;
    bool pok[2];
    int64_t pg[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) pg[u] = page_of(a, bt, pi0 + u, (pi0 + u) * kBS < tok_end, &pok[u]);

    float x[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t hb = pg[u] * H + h;
      const u32x4 kc = *reinterpret_cast<const u32x4*>(a.kc + hb * kHBCodes + lo * 64 + hi * 16);
      const uint32_t kw = a.kp[hb * kHBParams + lo * 4 + hi];
      const float ks = pscale(kw), kz = pzero(kw);
      float c[32];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
        for (int n = 0; n < 8; ++n) c[8 * q4 + n] = (float)__builtin_amdgcn_ubfe(kc[q4], 4 * n, 4);
      float sr[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) d = __builtin_fmaf(qr[r][i], c[i], d);
        float part = ks * d + kz * qs[r];
        part += __shfl_xor(part, 16);
        part += __shfl_xor(part, 32);
        sr[r] = part;
      }
      const float mine = hi == 0 ? sr[0] : hi == 1 ? sr[1] : hi == 2 ? sr[2] : sr[3];
      const bool valid = pok[u] && (c0 + u * kBS + lo) < tok_end && hi < R;
      x[u] = valid ? mine * a.qk_scale_log2 : -__builtin_inff();
    }
    const float cm = row_max16(fmaxf(x[0], x[1]));
    const float m_new = fmaxf(m_run, cm);
    if (__any(m_new > m_run)) {
      const float alpha = exp2_fast(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float ar = __shfl(alpha, 16 * r);
        zacc[r] *= ar;
#pragma unroll
        for (int k = 0; k < 8; ++k) accv[r][k] *= ar;
      }
      m_run = m_new;
    }
    const float p0 = exp2_fast(x[0] - m_run), p1 = exp2_fast(x[1] - m_run);
    l_run += p0 + p1;
    p_lds[0][hi][lo] = p0;
    p_lds[1][hi][lo] = p1;
    __builtin_amdgcn_wave_barrier();

    // PV layout: lane (n = lo, j' = hi): dims 8 n .. 8 n + 7, tokens 8 j' .. 8 j' + 7.
    const int vu = hi >> 1, vhalf = hi & 1;
    const int64_t vhb = pg[vu] * H + h;
    const u32x4* vcp = reinterpret_cast<const u32x4*>(a.vc + vhb * kHBCodes + 64 * lo + 32 * vhalf);
    const u32x4 vc0 = vcp[0], vc1 = vcp[1];
    const uint32_t vw[8] = {vc0[0], vc0[1], vc0[2], vc0[3], vc1[0], vc1[1], vc1[2], vc1[3]};
    const u32x4* vpp =
        reinterpret_cast<const u32x4*>(a.vp + vhb * kHBParams + (lo >> 2) * 16 + 8 * vhalf);
    const u32x4 vp0 = vpp[0], vp1 = vpp[1];
    const uint32_t pw[8] = {vp0[0], vp0[1], vp0[2], vp0[3], vp1[0], vp1[1], vp1[2], vp1[3]};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool valid = pok[vu] && (c0 + 8 * hi + e) < tok_end;
      const float sv = pscale(pw[e]), zv = pzero(pw[e]);
      float cv[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) cv[k] = (float)__builtin_amdgcn_ubfe(vw[k], 4 * e, 4);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        // A token outside the context has p = 0, but its param words may hold
        // any bytes (0 * inf = NaN): select, do not multiply, them away.
        const float pr = p_lds[vu][r][8 * vhalf + e];
        const float w = valid ? pr * sv : 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) accv[r][k] = __builtin_fmaf(w, cv[k], accv[r][k]);
        zacc[r] = valid ? __builtin_fmaf(pr, zv, zacc[r]) : zacc[r];
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  const float l_tot = row_sum16(l_run);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float o[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float v = accv[r][k] + zacc[r];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      o[k] = v;
    }
    const float mr = __shfl(m_run, 16 * r), lr = __shfl(l_tot, 16 * r);
    if (hi == 0) {
      float* base = a.ws + (((int64_t)s * a.num_q_heads + (int64_t)h * R + r) * a.max_splits + sp) *
                               kPartStride;
      *reinterpret_cast<float4*>(base + 8 * lo) = float4{o[0], o[1], o[2], o[3]};
      *reinterpret_cast<float4*>(base + 8 * lo + 4) = float4{o[4], o[5], o[6], o[7]};
      if (lo == 0) {
        base[kD] = mr;
        base[kD + 1] = lr;
      }
    }
  }
}

// ================================================================ merge ====

// Stream-K merge: one wave per (query head, sequence).  The pair's parts are
// the slots of waves wf..wl (the first one's slot 1 when its share began in
// an earlier pair), found from the units before the sequence (sk_meta, written
// by the decode launch) with the decode's own share arithmetic; a pair one
// wave held was finished by it.  Lane k reads (m, l) of part k; lane (half, c)
// reads dims 4c .. 4c + 3 of parts half, half + 2, ...; the first kSkPre of
// those are loaded with the (m, l) words, before the maximum is known, so the
// merge waits on memory once for up to 2 kSkPre parts.  A map entry that
// this call's decode launch did not write raises AMF_ERRFLAG_SYNC (the
// output is then invalid) and is never used as an address.
constexpr int kSkPre = 8;

template <int OUT_DTYPE>
__global__ __launch_bounds__(64) void int4_decode_merge_sk_kernel(DecodeArgs a) {
  const int qhd = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
  const int half = lane >> 5, c = lane & 31;
  const int R = a.num_q_heads / a.num_kv_heads;
  // context length and the map are independent loads; an empty sequence
  // (no units) never reads its map entry's value
  const int64_t nch = sk_chunks(a, s);
  const int64_t P = a.sk_meta[s], total = a.sk_meta[a.num_seqs];
  float L = 0.0f;
  float4 o = {0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t H = a.num_kv_heads;
  // a map entry outside [0, total - H nch] (not written by this call's decode
  // launch) is reported and leaves zeros instead of reading outside the slots
  const bool map_ok = P >= 0 && total > 0 && P <= total - H * nch;
  if (nch > 0 && !map_ok && lane == 0 && a.err_flag) atomicOr(a.err_flag, AMF_ERRFLAG_SYNC);
  if (nch > 0 && map_ok) {
    const int64_t G = min((int64_t)a.sk_waves, total);  // as the decode launch uses it
    const int64_t pair0 = P + (int64_t)(qhd / R) * nch;
    const int64_t wf = sk_wave_of(pair0, total, G);
    const int64_t wl = sk_wave_of(pair0 + nch - 1, total, G);
    if (wf == wl) return;  // one wave held the whole pair and wrote the output
    const int n_sp = (int)(wl - wf + 1);
    const bool first_slot1 = wf * total / G < pair0;
    const float* base = a.ws + (wf * 2 * R + qhd % R) * kPartStride;
    auto part = [&](int k) -> const float* {
      const int slot = (k == 0 && first_slot1) ? 1 : 0;
      return base + (int64_t)((2 * k + slot) * R) * kPartStride;
    };
    // accumulators of parts half, half + 2, ... (rows clamped into the pair's
    // parts; a clamped row is loaded but never added)
    float4 pre[kSkPre];
#pragma unroll
    for (int j = 0; j < kSkPre; ++j)
      pre[j] = *reinterpret_cast<const float4*>(part(min(half + 2 * j, n_sp - 1)) + 4 * c);
    float m0 = kNegBig, l0 = 0.0f;
    if (lane < n_sp) {
      const float2 ml = *reinterpret_cast<const float2*>(part(lane) + kD);
      m0 = ml.x;
      l0 = ml.y;
    }
    float M = m0;
    for (int k = lane + 64; k < n_sp; k += 64) M = fmaxf(M, part(k)[kD]);
    M = wave_max_xor(M, 64);
    for (int k0 = 0; k0 < n_sp; k0 += 64) {
      float wk = 0.0f;
      if (k0 + lane < n_sp) {
        float mk = m0, lk = l0;
        if (k0 != 0) {
          const float2 ml = *reinterpret_cast<const float2*>(part(k0 + lane) + kD);
          mk = ml.x;
          lk = ml.y;
        }
        wk = exp2_fast(mk - M);
        L += wk * lk;
      }
      const int cnt = min(64, n_sp - k0);
      int j0 = 0;
      if (k0 == 0) {
#pragma unroll
        for (int j = 0; j < kSkPre; ++j) {
          const float wj = __shfl(wk, half + 2 * j);  // every lane shuffles
          if (half + 2 * j < cnt) {
            o.x += wj * pre[j].x;
            o.y += wj * pre[j].y;
            o.z += wj * pre[j].z;
            o.w += wj * pre[j].w;
          }
        }
        j0 = 2 * kSkPre;
      }
#pragma unroll 4
      for (int j = j0; j < cnt; j += 2) {
        const int jj = j + half;
        const float wj = __shfl(wk, min(jj, 63));
        if (jj < cnt) {
          const float4 v = *reinterpret_cast<const float4*>(part(k0 + jj) + 4 * c);
          o.x += wj * v.x;
          o.y += wj * v.y;
          o.z += wj * v.z;
          o.w += wj * v.w;
        }
      }
    }
    o.x += __shfl_xor(o.x, 32);
    o.y += __shfl_xor(o.y, 32);
    o.z += __shfl_xor(o.z, 32);
    o.w += __shfl_xor(o.w, 32);
    for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off);
  }
  if (half != 0) return;
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  const int64_t row = ((int64_t)s * a.num_q_heads + qhd) * kD;
  if constexpr (OUT_DTYPE == AMF_DTYPE_F32) {
    float* out = static_cast<float*>(a.out) + row;
    *reinterpret_cast<float4*>(out + 4 * c) = float4{o.x * inv, o.y * inv, o.z * inv, o.w * inv};
  } else {
    constexpr bool BF = OUT_DTYPE == AMF_DTYPE_BF16;
    uint16_t* out = static_cast<uint16_t*>(a.out) + row;
    const uint32_t p0 = (uint32_t)oval<BF>(o.x * inv) | ((uint32_t)oval<BF>(o.y * inv) << 16);
    const uint32_t p1 = (uint32_t)oval<BF>(o.z * inv) | ((uint32_t)oval<BF>(o.w * inv) << 16);
    *reinterpret_cast<uint2*>(out + 4 * c) = uint2{p0, p1};
  }
}

// Split merge (fixed splits of the VALU path): one workgroup of four waves
// per (query head, sequence):
// O = sum_i 2^(m_i - M) acc_i / L, written as OUT_DTYPE (an AMF_DTYPE_* tag).
// Thread t reads (m, l) of split t once (and of splits t + 256, ... when
// there are more) and the weights are shared through LDS.  For the
// accumulators, lane (half, c) of wave w reads dims 4c .. 4c + 3 of splits
// w + 4 half, w + 4 half + 8, ...: a wave load covers two whole splits and
// several are in flight; the halves and then the waves are summed at the end.
constexpr int kMergeThreads = 256;
constexpr int kMergeWaves = kMergeThreads / 64;
constexpr int kMergePre = 8;  // splits per thread loaded up front (64 per workgroup)

template <int OUT_DTYPE>
__global__ __launch_bounds__(kMergeThreads) void int4_decode_merge_kernel(DecodeArgs a) {
  __shared__ float wgt[kMergeThreads];
  __shared__ __attribute__((aligned(16))) float red[kMergeWaves][kD];
  __shared__ float sred[kMergeWaves];
  const int qhd = blockIdx.x, s = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int half = lane >> 5, c = lane & 31;
  const int ctx = clamp_context(a, s);
  const int n_sp = (ctx + a.split_tokens - 1) / a.split_tokens;
  const float* base = a.ws + ((int64_t)s * a.num_q_heads + qhd) * a.max_splits * kPartStride;
  auto part = [&](int k) -> const float* { return base + (int64_t)k * kPartStride; };
  // The accumulators of this thread's first kMergePre splits are loaded
  // together with the (m, l) words, before the maximum is known, so the merge
  // waits on memory once (rows clamped into the sequence's splits; a clamped
  // row is loaded but never added).
  const int k_first = w + kMergeWaves * half;
  float4 pre[kMergePre];
#pragma unroll
  for (int j = 0; j < kMergePre; ++j) {
    const int k = max(min(k_first + 2 * kMergeWaves * j, n_sp - 1), 0);
    pre[j] = *reinterpret_cast<const float4*>(part(k) + 4 * c);
  }
  float m0 = kNegBig, l0 = 0.0f;  // (m, l) of split tid, kept for the weights
  if (tid < n_sp) {
    const float2 ml = *reinterpret_cast<const float2*>(part(tid) + kD);
    m0 = ml.x;
    l0 = ml.y;
  }
  float M = m0;
  for (int i = tid + kMergeThreads; i < n_sp; i += kMergeThreads)
    M = fmaxf(M, part(i)[kD]);
  M = wave_max_xor(M, 64);
  if (lane == 0) sred[w] = M;
  __syncthreads();
  M = sred[0];
#pragma unroll
  for (int i = 1; i < kMergeWaves; ++i) M = fmaxf(M, sred[i]);
  float L = 0.0f;
  float4 o = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int i0 = 0; i0 < n_sp; i0 += kMergeThreads) {
    __syncthreads();  // sred / wgt of the previous pass are consumed
    const int i = i0 + tid;
    float wi = 0.0f;
    if (i < n_sp) {
      float mi = m0, li = l0;
      if (i0 != 0) {
        const float2 ml = *reinterpret_cast<const float2*>(part(i) + kD);
        mi = ml.x;
        li = ml.y;
      }
      wi = exp2_fast(mi - M);
      L += wi * li;
    }
    wgt[tid] = wi;
    __syncthreads();
    const int cnt = min(kMergeThreads, n_sp - i0);
    int k_from = k_first;
    if (i0 == 0) {
#pragma unroll
      for (int j = 0; j < kMergePre; ++j) {
        const int k = k_first + 2 * kMergeWaves * j;
        if (k < cnt) {
          const float wk = wgt[k];
          o.x += wk * pre[j].x;
          o.y += wk * pre[j].y;
          o.z += wk * pre[j].z;
          o.w += wk * pre[j].w;
        }
      }
      k_from += 2 * kMergeWaves * kMergePre;
    }
#pragma unroll 4
    for (int k = k_from; k < cnt; k += 2 * kMergeWaves) {
      const float wk = wgt[k];
      const float4 v =
          *reinterpret_cast<const float4*>(part(i0 + k) + 4 * c);
      o.x += wk * v.x;
      o.y += wk * v.y;
      o.z += wk * v.z;
      o.w += wk * v.w;
    }
  }
  o.x += __shfl_xor(o.x, 32);
  o.y += __shfl_xor(o.y, 32);
  o.z += __shfl_xor(o.z, 32);
  o.w += __shfl_xor(o.w, 32);
  for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off);
  __syncthreads();
  if (lane == 0) sred[w] = L;
  if (half == 0) *reinterpret_cast<float4*>(&red[w][4 * c]) = o;
  __syncthreads();
  if (w != 0 || half != 0) return;
  L = sred[0];
  o = *reinterpret_cast<const float4*>(&red[0][4 * c]);
#pragma unroll
  for (int i = 1; i < kMergeWaves; ++i) {
    L += sred[i];
    const float4 r = *reinterpret_cast<const float4*>(&red[i][4 * c]);
    o.x += r.x;
    o.y += r.y;
    o.z += r.z;
    o.w += r.w;
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  const int64_t row = ((int64_t)s * a.num_q_heads + qhd) * kD;
  if constexpr (OUT_DTYPE == AMF_DTYPE_F32) {
    float* out = static_cast<float*>(a.out) + row;
    *reinterpret_cast<float4*>(out + 4 * c) = float4{o.x * inv, o.y * inv, o.z * inv, o.w * inv};
  } else {
    constexpr bool BF = OUT_DTYPE == AMF_DTYPE_BF16;
    uint16_t* out = static_cast<uint16_t*>(a.out) + row;
    const uint32_t p0 = (uint32_t)oval<BF>(o.x * inv) | ((uint32_t)oval<BF>(o.y * inv) << 16);
    const uint32_t p1 = (uint32_t)oval<BF>(o.z * inv) | ((uint32_t)oval<BF>(o.w * inv) << 16);
    *reinterpret_cast<uint2*>(out + 4 * c) = uint2{p0, p1};
  }
}

// Split size: a multiple of 32 tokens in [256, 1024] chosen so that about
// kTargetWaves waves of work exist when every sequence is max_context_len
// long, with at most kMaxSplitsPerSeq splits per sequence.
#ifndef AMF_DECODE_TARGET_WAVES
#define AMF_DECODE_TARGET_WAVES 16384
#endif
constexpr int64_t kTargetWaves = AMF_DECODE_TARGET_WAVES;
constexpr int kMaxSplitTokens = 1024;  // 64 pages: one block-table entry per lane
#ifndef AMF_DECODE_MIN_SPLIT
#define AMF_DECODE_MIN_SPLIT 256
#endif
constexpr int kMinSplitTokens = AMF_DECODE_MIN_SPLIT;
#ifndef AMF_DECODE_MAX_SPLITS
#define AMF_DECODE_MAX_SPLITS 128
#endif
constexpr int kMaxSplitsPerSeq = AMF_DECODE_MAX_SPLITS;  // bounds the merge's reads of partials

int choose_split(int32_t num_seqs, int32_t num_kv_heads, int32_t max_context_len) {
  const int64_t work = (int64_t)num_seqs * num_kv_heads * (max_context_len > 0 ? max_context_len : 1);
  int64_t split = (work + kTargetWaves - 1) / kTargetWaves;
  const int64_t per_seq = ((int64_t)max_context_len + kMaxSplitsPerSeq - 1) / kMaxSplitsPerSeq;
  if (split < per_seq) split = per_seq;
  split = (split + 31) / 32 * 32;
  if (split < kMinSplitTokens) split = kMinSplitTokens;
  if (split > kMaxSplitTokens) split = kMaxSplitTokens;
  return (int)split;
}

// ---- scratch for the entry point that allocates nothing -----------------------
// One array per device that loads the library, held until the process ends.
// Host code never passes `scratch` itself to a kernel (in host code the name is
// a stand-in, not a device address): scratch_address() asks the runtime for
// the current device's copy once and keeps it.
constexpr int64_t kDecodeScratchBytes = 64ll << 20;
static __device__ __align__(256) uint8_t scratch[kDecodeScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Address of the current device's scratch (looked up on the first call on
// that device, with it current), or nullptr with the error recorded.
void* scratch_address(const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fail(AMF_ERR_RUNTIME, "%s: hipGetDevice failed: %s", who, hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    fail(AMF_ERR_UNSUPPORTED, "%s: device %d beyond the %d this library tracks", who, dev,
         kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fail(AMF_ERR_RUNTIME, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev,
           hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

// Waves of one stream-K decode launch: as many as the device keeps resident
// at once (occupancy of the kernel x compute units), the larger of the bf16-
// and fp16-query kernels of the group size; 0 when the runtime cannot say.
template <int R>
int sk_waves_for() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  static std::mutex mu;
  static std::map<int, int> cache;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int ncu = 0;
  if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      ncu <= 0)
    return 0;
  int best = 0;
  for (const void* fn : {reinterpret_cast<const void*>(&int4_decode_mfma_kernel<R, true>),
                         reinterpret_cast<const void*>(&int4_decode_mfma_kernel<R, false>)}) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, 64, 0) != hipSuccess) return 0;
    best = std::max(best, nb);
  }
  const int g = std::max(1, best) * ncu;
  cache[dev] = g;
  return g;
}

int sk_waves(int R) {
  switch (R) {
    case 1: return sk_waves_for<1>();
    case 2: return sk_waves_for<2>();
    case 4: return sk_waves_for<4>();
    default: return sk_waves_for<8>();
  }
}

}  // namespace

extern "C" int64_t amf_int4_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                                   int32_t num_kv_heads, int32_t head_dim,
                                                   int32_t max_context_len) {
  if (num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim != kD) return 0;
  const int split = choose_split(num_seqs, num_kv_heads, max_context_len);
  const int64_t max_splits = (max_context_len + split - 1) / split;
  // split partials of the VALU path; two partial slots per wave of the MFMA path
  const int64_t split_bytes = (int64_t)num_seqs * num_q_heads * (max_splits > 0 ? max_splits : 1) *
                              kPartStride * (int64_t)sizeof(float);
  const int R = num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 ? num_q_heads / num_kv_heads
                                                                     : 1;
  // stream-K: two partial slots per resident wave, then the map of sequence
  // starts (num_seqs + 1 int64)
  const int64_t sk_bytes =
      (R == 1 || R == 2 || R == 4 || R == 8)
          ? (int64_t)sk_waves(R) * 2 * R * kPartStride * (int64_t)sizeof(float) +
                ((int64_t)num_seqs + 1) * (int64_t)sizeof(int64_t)
          : 0;
  return std::max(split_bytes, sk_bytes);
}


extern "C" int amf_int4_paged_decode_attn(const void* q, int32_t q_dtype, void* out,
                                          int32_t out_dtype,
                                          const void* k_codes, const void* k_params,
                                          const void* v_codes, const void* v_params,
                                          int64_t pool_pages, const int32_t* block_tables,
                                          int32_t block_table_stride, const int32_t* context_lens,
                                          int32_t num_seqs, int32_t num_q_heads,
                                          int32_t num_kv_heads, int32_t head_dim,
                                          int32_t block_size, int32_t max_context_len,
                                          float softmax_scale, void* workspace,
                                          int64_t workspace_bytes, int32_t algo,
                                          int32_t* err_flag, void* stream) {
  const char* who = "amf_int4_paged_decode_attn";
  if (!q || !out || !k_codes || !k_params || !v_codes || !v_params || !block_tables ||
      !context_lens)
    return fail(AMF_ERR_INVALID_ARG, "%s: null pointer argument", who);
  if (q_dtype != AMF_DTYPE_BF16 && q_dtype != AMF_DTYPE_F16)
    return fail(AMF_ERR_UNSUPPORTED, "%s: q dtype %d is not bf16/fp16", who, q_dtype);
  if (out_dtype != AMF_DTYPE_BF16 && out_dtype != AMF_DTYPE_F16 && out_dtype != AMF_DTYPE_F32)
    return fail(AMF_ERR_UNSUPPORTED, "%s: out dtype %d is not bf16/fp16/fp32", who, out_dtype);
  if (head_dim != kD || block_size != kBS)
    return fail(AMF_ERR_UNSUPPORTED, "%s: needs head_dim %d and block_size %d (got %d, %d)", who,
                kD, kBS, head_dim, block_size);
  if (num_seqs < 0 || num_seqs > 65535 || num_kv_heads <= 0 || num_kv_heads > 65535 ||
      num_q_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return fail(AMF_ERR_INVALID_ARG, "%s: bad head counts q=%d kv=%d or num_seqs=%d", who,
                num_q_heads, num_kv_heads, num_seqs);
  const int R = num_q_heads / num_kv_heads;
  if (R != 1 && R != 2 && R != 4 && R != 8)
    return fail(AMF_ERR_UNSUPPORTED, "%s: GQA group %d not in {1,2,4,8}", who, R);
  if (pool_pages <= 0 || block_table_stride <= 0 || max_context_len < 0)
    return fail(AMF_ERR_INVALID_ARG, "%s: bad pool_pages / block_table_stride / max_context_len",
                who);
  if ((int64_t)max_context_len > (int64_t)block_table_stride * kBS)
    return fail(AMF_ERR_INVALID_ARG, "%s: max_context_len %d exceeds the block table (%d pages)",
                who, max_context_len, block_table_stride);
  if (algo != AMF_DECODE_AUTO && algo != AMF_DECODE_VALU && algo != AMF_DECODE_MFMA &&
      algo != AMF_DECODE_MFMA_PRECISE)
    return fail(AMF_ERR_INVALID_ARG, "%s: bad algo %d", who, algo);
  if (algo == AMF_DECODE_VALU && R > 4)
    return fail(AMF_ERR_UNSUPPORTED, "%s: the VALU path handles GQA groups up to 4", who);
  const int64_t need =
      amf_int4_decode_workspace_bytes(num_seqs, num_q_heads, num_kv_heads, head_dim, max_context_len);
  if (!workspace || workspace_bytes < need)
    return fail(AMF_ERR_WORKSPACE, "%s: needs %lld workspace bytes", who, (long long)need);
  if (num_seqs == 0) return ok();

  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.out = out;
  a.kc = static_cast<const uint8_t*>(k_codes);
  a.kp = static_cast<const uint32_t*>(k_params);
  a.vc = static_cast<const uint8_t*>(v_codes);
  a.vp = static_cast<const uint32_t*>(v_params);
  a.pool_pages = pool_pages;
  a.block_tables = block_tables;
  a.bt_stride = block_table_stride;
  a.context_lens = context_lens;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.split_tokens = choose_split(num_seqs, num_kv_heads, max_context_len);
  a.max_context_len = max_context_len;
  const int max_splits = (max_context_len + a.split_tokens - 1) / a.split_tokens;
  a.max_splits = max_splits > 0 ? max_splits : 1;
  a.head_fast = max_splits <= 65535;
  const float scale = softmax_scale > 0.0f ? softmax_scale : 1.0f / sqrtf((float)head_dim);
  a.qk_scale_log2 = scale * kLog2e;
  a.pv16 = algo != AMF_DECODE_MFMA_PRECISE;
  a.ws = static_cast<float*>(workspace);
  a.err_flag = err_flag;
  a.out_dtype = out_dtype;
  a.num_seqs = num_seqs;
  a.stream_k = algo != AMF_DECODE_VALU;
  a.sk_waves = a.stream_k ? sk_waves(R) : 0;
  if (a.stream_k && a.sk_waves <= 0)
    return fail(AMF_ERR_RUNTIME, "%s: could not size the decode grid (device occupancy query)", who);
  a.sk_meta = a.stream_k ? reinterpret_cast<int64_t*>(
                               static_cast<uint8_t*>(workspace) +
                               (int64_t)a.sk_waves * 2 * R * kPartStride * (int64_t)sizeof(float))
                         : nullptr;
  // Stream-K unit arithmetic stays in int64: units x waves < 2^62.
  if (a.stream_k && ((int64_t)max_context_len / 32 + 1) * num_seqs * num_kv_heads >
                        ((int64_t)1 << 62) / a.sk_waves)
    return fail(AMF_ERR_UNSUPPORTED, "%s: %d sequences x %d KV heads x %d tokens is too large", who,
                num_seqs, num_kv_heads, max_context_len);

  hipStream_t st = as_stream(stream);
  const bool bf16 = q_dtype == AMF_DTYPE_BF16;
  if (max_splits > 0) {
    const dim3 grid = a.head_fast
                          ? dim3((unsigned)num_kv_heads, (unsigned)max_splits, (unsigned)num_seqs)
                          : dim3((unsigned)max_splits, (unsigned)num_kv_heads, (unsigned)num_seqs);
    const bool valu = algo == AMF_DECODE_VALU;
#define AMF_LAUNCH(K, RR, B) K<RR, B><<<grid, 64, 0, st>>>(a)
#define AMF_LAUNCH_B(K, RR) \
  if (bf16) AMF_LAUNCH(K, RR, true); else AMF_LAUNCH(K, RR, false)
    if (valu) {
      if (R == 1) { AMF_LAUNCH_B(int4_decode_valu_kernel, 1); }
      else if (R == 2) { AMF_LAUNCH_B(int4_decode_valu_kernel, 2); }
      else { AMF_LAUNCH_B(int4_decode_valu_kernel, 4); }
    } else {
#undef AMF_LAUNCH
#define AMF_LAUNCH(K, RR, B) K<RR, B><<<dim3((unsigned)a.sk_waves), 64, 0, st>>>(a)
      if (R == 1) { AMF_LAUNCH_B(int4_decode_mfma_kernel, 1); }
      else if (R == 2) { AMF_LAUNCH_B(int4_decode_mfma_kernel, 2); }
      else if (R == 4) { AMF_LAUNCH_B(int4_decode_mfma_kernel, 4); }
      else { AMF_LAUNCH_B(int4_decode_mfma_kernel, 8); }
    }
#undef AMF_LAUNCH_B
#undef AMF_LAUNCH
  }
  dim3 mgrid((unsigned)num_q_heads, (unsigned)num_seqs);
  if (a.stream_k) {
    if (out_dtype == AMF_DTYPE_BF16)
      int4_decode_merge_sk_kernel<AMF_DTYPE_BF16><<<mgrid, 64, 0, st>>>(a);
    else if (out_dtype == AMF_DTYPE_F16)
      int4_decode_merge_sk_kernel<AMF_DTYPE_F16><<<mgrid, 64, 0, st>>>(a);
    else
      int4_decode_merge_sk_kernel<AMF_DTYPE_F32><<<mgrid, 64, 0, st>>>(a);
  } else if (out_dtype == AMF_DTYPE_BF16) {
    int4_decode_merge_kernel<AMF_DTYPE_BF16><<<mgrid, kMergeThreads, 0, st>>>(a);
  } else if (out_dtype == AMF_DTYPE_F16) {
    int4_decode_merge_kernel<AMF_DTYPE_F16><<<mgrid, kMergeThreads, 0, st>>>(a);
  } else {
    int4_decode_merge_kernel<AMF_DTYPE_F32><<<mgrid, kMergeThreads, 0, st>>>(a);
  }
  return check_launch(who);
}

extern "C" int amf_int4_paged_decode_attn_noalloc(
    const void* q, int32_t q_dtype, void* out, int32_t out_dtype, const void* k_codes,
    const void* k_params, const void* v_codes, const void* v_params, int64_t pool_pages,
    const int32_t* block_tables, int32_t block_table_stride, const int32_t* context_lens,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block_size, int32_t max_context_len, float softmax_scale, int32_t algo,
    int32_t* err_flag, void* stream) {
  const char* who = "amf_int4_paged_decode_attn_noalloc";
  const int64_t need = amf_int4_decode_workspace_bytes(num_seqs, num_q_heads, num_kv_heads,
                                                       head_dim, max_context_len);
  if (need > kDecodeScratchBytes)
    return fail(AMF_ERR_WORKSPACE,
                "%s: %lld bytes of split partials exceed the %lld-byte scratch (use "
                "amf_int4_paged_decode_attn with a workspace)",
                who, (long long)need, (long long)kDecodeScratchBytes);
  void* ws = scratch_address(who);
  if (!ws) return AMF_ERR_RUNTIME;
  return amf_int4_paged_decode_attn(q, q_dtype, out, out_dtype, k_codes, k_params, v_codes,
                                    v_params, pool_pages, block_tables, block_table_stride,
                                    context_lens, num_seqs, num_q_heads, num_kv_heads, head_dim,
                                    block_size, max_context_len, softmax_scale, ws,
                                    kDecodeScratchBytes, algo, err_flag, stream);
}
