/*
 * amf_hip.h - C ABI of libamf_hip.so, the gfx950 (MI355X) implementation of
 * the Axropus AMF KV-materialization hot path.
 *
 * Scope: paged gather/scatter between a vLLM-style paged KV cache and the AMF
 * VRAM tier, the FP8 (e4m3fn) and INT4 codecs of the compressed VRAM pool
 * (quantize-on-save, dequantize+scatter-on-restore), and paged GQA decode
 * attention that reads INT4 KV with fused dequantization.
 *
 * Conventions shared by every entry point
 * ---------------------------------------
 *  - All pointers except `stream` are DEVICE addresses; sizes are int64/int32.
 *  - A "plane" is one K or V array of one layer.  Plane arrays (`*_planes`)
 *    are device arrays of n_planes uint64 base addresses, normally ordered
 *    (K of layer 0, V of layer 0, K of layer 1, ...).  Page p of a cache plane
 *    starts at planes[i] + p * page_stride (bytes) and holds
 *    block_size * num_heads * head_dim elements in [token][head][dim] order
 *    (vLLM's [num_blocks, block_size, num_kv_heads, head_size] page).
 *  - `block_ids` (int32, device, n_pages entries) maps a position in the
 *    gathered sequence to a physical page of the cache.  NULL means the
 *    identity map (contiguous, unpaged source or destination).
 *  - Every page whose block id lies outside [0, pool_pages) is skipped (never
 *    read or written); the kernel then ORs AMF_ERRFLAG_BLOCK_RANGE into
 *    *err_flag when err_flag is not NULL.  Duplicate ids in a scatter target
 *    leave those pages holding one of the writers' values (unspecified which);
 *    nothing faults.
 *  - `stream` is a hipStream_t (NULL = default stream).  Every call is
 *    stream-ordered, allocates no device memory, keeps no state between
 *    calls and may be issued from any host thread.
 *  - Return value: AMF_OK (0) or a negative AMF_ERR_* code; the message for
 *    the calling thread's last failure is returned by amf_last_error().
 *    Nothing throws across this boundary.
 *
 * Interfaces replaced (reference file:line):
 *  - korith_vllm_ext/compressed_vram_pool.py:434-560  put_from_vllm gather+compress
 *  - korith_vllm_ext/compressed_vram_pool.py:562-608  restore_to_vllm decompress+scatter
 *  - korith_vllm_ext/amf_kv_manager.py:298-321, 488-523  raw page gather / scatter
 *  - korith_vllm_ext/codecs/amf_codec.py:174-222      FP8E4M3Codec compress/decompress_to
 *  - korith_vllm_ext/codecs/amf_codec.py:292-447      INT4PerChannelCodec / INT4PerBlockCodec
 *  - korith_vllm_ext/codecs/amf_codec.py:502-539      _pack_int4 / _unpack_int4
 *  - korith_vllm_ext/int4_decode_attention.py:6-9 -> kernels/dispatch.py:117-143
 *    (int4_decode_attention; the CUDA kernel it was meant to reach is
 *    korith_vllm_ext/kernels/int4_decode_attention.cu:39-213, bound at
 *    korith_vllm_ext/kernels/bindings.cpp:64-76)
 */
#ifndef AMF_HIP_H
#define AMF_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AMF_ABI_VERSION 3

/* ---- status codes ------------------------------------------------------ */
#define AMF_OK                  0
#define AMF_ERR_INVALID_ARG    (-1)  /* null pointer, negative size, bad enum */
#define AMF_ERR_UNSUPPORTED    (-2)  /* shape/format not implemented here */
#define AMF_ERR_LAUNCH         (-3)  /* the HIP runtime rejected a launch */
#define AMF_ERR_WORKSPACE      (-4)  /* workspace missing or too small */
#define AMF_ERR_FORMAT         (-5)  /* blob is not a valid AMFK snapshot */
#define AMF_ERR_MISMATCH       (-6)  /* snapshot does not fit the caller's KV tensors */
#define AMF_ERR_RUNTIME        (-7)  /* a HIP runtime call (allocation, copy, event) failed */

/* bits ORed into *err_flag by kernels */
#define AMF_ERRFLAG_BLOCK_RANGE 1    /* a block id was outside [0, pool_pages) */
#define AMF_ERRFLAG_CONTEXT     2    /* a context length exceeded its block table */
#define AMF_ERRFLAG_SYNC        4    /* a cross-workgroup wait gave up (that call's output is invalid) */

/* ---- element types: same numbering as the AMFK header dtype field
 *      (core/amf_direct_kv.h AmfKvDtype; amf_kv_manager.py:60-64) --------- */
#define AMF_DTYPE_F16   0
#define AMF_DTYPE_F32   1
#define AMF_DTYPE_BF16  2

/* ---- codec formats ------------------------------------------------------
 * Layouts are per plane; n_pages pages of one plane are contiguous.
 * Cache pages (cache_dtype AMF_DTYPE_BF16, AMF_DTYPE_F16 or AMF_DTYPE_F32)
 * are [block_size][num_heads][head_dim] row-major; head_dim is a multiple of
 * 32 (FP8: head_dim/16, INT4 symmetric: head_dim/32 a power of two).
 *
 * AMF_FMT_FP8_E4M3 (reference "fp8_e4m3", amf_codec.py:174-222)
 *   codes  : [n_pages][block_size][num_heads][head_dim] e4m3fn bytes
 *   params : the scale group's fp32 sidecar [k_scale, v_scale, q_scale,
 *            prob_scale] (FP8ScaleSidecar, amf_codec.py:62-94).  A scale
 *            group is `planes_per_scale` consecutive planes (2 = the K and V
 *            of one layer) whose param_planes entries all hold the address of
 *            that group's sidecar; save writes the group's scale to slots 0
 *            and 1 and 1.0 to slots 2 and 3; restore reads slot (plane & 1).
 *   scale  = max(absmax over the group, floor) / 448, floor = 1e-8 rounded
 *            to the cache dtype; code = e4m3fn_rne(clamp(x / scale, -448, 448))
 *            (division by 1e-12 when the floored absmax is 0);
 *   x'     = to_cache_dtype(fp32(code) * scale).
 * AMF_FMT_FP8_E4M3_PH (per-(page, head) scale; no reference counterpart)
 *   codes  : as AMF_FMT_FP8_E4M3
 *   params : [n_pages][num_heads] fp32 scales
 *   scale  = max(absmax over the page's block_size x head_dim values of that
 *            head, 1e-8f) / 448; codes and x' as above.
 * AMF_FMT_INT4_SYM_BLOCK (reference "int4_sym_block" on a page tensor,
 *   amf_codec.py:345-447): one fp16 scale per page over all heads
 *   codes  : [n_pages][block_size][num_heads][head_dim/2] bytes, byte i of a
 *            row = (u[2i+1] << 4) | u[2i], u = q + 8 (amf_codec.py:502-521)
 *   params : [n_pages] fp16; scale32 = max(absmax_page, 1e-8f) / 7,
 *            q = clamp(rint(x / scale32), -8, 7), stored fp16(scale32);
 *   x'     = to_cache_dtype(fp32(q) * fp32(fp16 scale)).
 * AMF_FMT_INT4_SYM (reference "int4_sym", amf_codec.py:292-343): one fp16
 *   scale per head_dim channel over a scale group of `planes_per_scale`
 *   planes (2 = K and V of a layer) whose param_planes entries all hold the
 *   address of the group's [head_dim] fp16 scales.
 *   codes as AMF_FMT_INT4_SYM_BLOCK; scale32_d = max(absmax_d, 1e-8f) / 7.
 * AMF_FMT_INT4_ASYM_G32 (no reference counterpart): asymmetric, one fp16
 *   (scale, zero) pair per (token, head, 32-dim group); G = head_dim / 32.
 *   Pages are head-major; within a (page, head) block of block_size = 16:
 *   K codes : [16 tokens][head_dim/2] bytes, byte i = dims 2i (low nibble)
 *             and 2i+1 (high nibble)
 *   V codes : dim-major tiles: for dim d and token t the nibble lives in
 *             byte 64*(d/8) + 32*(t/8) + 4*(d%8) + (t%8)/2, low nibble for
 *             even t.  (One 32-byte run = 8 tokens x 8 dims.)
 *   K params: [16 tokens][G] uint32, low half fp16 scale, high half fp16 zero
 *   V params: [G][16 tokens] uint32, same packing
 *   mn, mx  = min, max of the group (fp32);
 *   scale32 = max(mx - mn, 1e-8f) / 15;  q = clamp(rint((x - mn) / scale32), 0, 15);
 *   stored  (fp16(scale32), fp16(mn));   x' = to_cache_dtype(q * s16 + z16)
 *   with an unfused fp32 multiply then add.
 * All divisions are IEEE correctly rounded; rint rounds half to even.
 */
#define AMF_FMT_FP8_E4M3        1
#define AMF_FMT_FP8_E4M3_PH     2
#define AMF_FMT_INT4_SYM_BLOCK  3
#define AMF_FMT_INT4_SYM        4
#define AMF_FMT_INT4_ASYM_G32   5

/* ABI version of the loaded library (AMF_ABI_VERSION when it was built). */
int amf_abi_version(void);

/* Message describing the calling thread's last failed call ("" if none). */
const char* amf_last_error(void);

/* Bytes of fp32 workspace that amf_*_quant_gather needs for `format`
 * (cross-page reductions: AMF_FMT_FP8_E4M3 one absmax word per scale group,
 * padded to a 128-byte line, then 33 lines per group that the single-read
 * save exchanges its partial maxima through; AMF_FMT_INT4_SYM head_dim
 * slots per group); 0 for formats reduced within a page. */
int64_t amf_quant_workspace_bytes(int32_t format, int32_t n_planes, int32_t planes_per_scale,
                                  int32_t head_dim);

/* Raw paged gather (snapshot): out_planes[i] page j <- cache_planes[i] page
 * block_ids[j], for i < n_planes, j < n_pages; page_bytes bytes each (a
 * multiple of 16, all strides and bases 16-byte aligned).
 * Replaces k_all[block_ids] / v_all[block_ids] in
 * compressed_vram_pool.py:491-504 and amf_kv_manager.py:311-318. */
int amf_kv_gather_pages(const uint64_t* cache_planes, int64_t cache_page_stride,
                        const int32_t* block_ids, int64_t pool_pages,
                        const uint64_t* out_planes, int64_t out_page_stride,
                        int32_t n_planes, int64_t n_pages, int64_t page_bytes,
                        int32_t* err_flag, void* stream);

/* Raw paged scatter (restore): cache_planes[i] page block_ids[j] <-
 * in_planes[i] page j.  Replaces k_all[chunk_ids] = src in
 * compressed_vram_pool.py:599-606 and amf_kv_manager.py:505-523. */
int amf_kv_scatter_pages(const uint64_t* in_planes, int64_t in_page_stride,
                         const uint64_t* cache_planes, int64_t cache_page_stride,
                         const int32_t* block_ids, int64_t pool_pages,
                         int32_t n_planes, int64_t n_pages, int64_t page_bytes,
                         int32_t* err_flag, void* stream);

/* Token-slot gather (the connector's save): out_planes[i] row j <- the cache
 * row slot_mapping[j] of cache_planes[i], for i < n_planes, j < n_slots.  A
 * row is one token's H*D elements, row_bytes bytes (a multiple of 16).  Cache
 * slot s lives at plane + (s / block_size) * cache_page_stride
 * + (s % block_size) * row_bytes (rows contiguous within a page); dense row j
 * at out_planes[i] + j * out_row_stride.  slot_mapping: device int64 array of
 * n_slots slot ids in [0, pool_slots); others are skipped and flagged in
 * err_flag.
 * Replaces flat[:, slots, :, :] of korith_vllm_ext/amf_kv_connector.py:411-422. */
int amf_kv_gather_slots(const uint64_t* cache_planes, int64_t cache_page_stride,
                        int32_t block_size, const int64_t* slot_mapping, int64_t pool_slots,
                        const uint64_t* out_planes, int64_t out_row_stride,
                        int32_t n_planes, int64_t n_slots, int64_t row_bytes,
                        int32_t* err_flag, void* stream);

/* Token-slot scatter (the connector's load): the cache row slot_mapping[j]
 * of cache_planes[i] <- in_planes[i] row j.  Addressing as
 * amf_kv_gather_slots.  Replaces flat_cache[:, slots, ...] = kv_slice of
 * korith_vllm_ext/amf_kv_connector.py:374-385. */
int amf_kv_scatter_slots(const uint64_t* in_planes, int64_t in_row_stride,
                         const uint64_t* cache_planes, int64_t cache_page_stride,
                         int32_t block_size, const int64_t* slot_mapping, int64_t pool_slots,
                         int32_t n_planes, int64_t n_slots, int64_t row_bytes,
                         int32_t* err_flag, void* stream);

/* Save path: gather n_pages pages of each cache plane through block_ids and
 * quantize them into code_planes / param_planes in `format` (an AMF_FMT_FP8_*
 * value).  planes_per_scale (>= 1, dividing n_planes) groups planes for the
 * per-tensor format and is ignored otherwise.  workspace: device fp32
 * buffer of amf_quant_workspace_bytes() bytes (may be NULL when that is 0);
 * its contents on entry do not matter.  The per-tensor format reads the cache
 * once through a cooperative launch when the device supports it and a scale
 * group (planes_per_scale planes of n_pages pages, at least 4 MiB) fits the
 * resident grid, and twice (absmax kernel, then quantize kernel) otherwise
 * or when AMF_NO_COOP is set to a non-zero value in the environment (read
 * once; for processes that cannot have a cooperative launch, such as a
 * profiler session or graph capture); both give the same bytes.  A
 * cooperative wait that gives up (never in a
 * correct launch) raises AMF_ERRFLAG_SYNC and writes an infinite scale for
 * its group.
 * Replaces compressed_vram_pool.py:481-508 with FP8E4M3Codec.compress
 * (amf_codec.py:186-209). */
int amf_fp8_quant_gather(int32_t format,
                         const uint64_t* cache_planes, int64_t cache_page_stride,
                         int32_t cache_dtype, const int32_t* block_ids, int64_t pool_pages,
                         const uint64_t* code_planes, const uint64_t* param_planes,
                         int32_t n_planes, int32_t planes_per_scale, int64_t n_pages,
                         int32_t block_size, int32_t num_heads, int32_t head_dim,
                         float* workspace, int64_t workspace_bytes,
                         int32_t* err_flag, void* stream);

/* Restore path: dequantize n_pages pages of each plane and scatter them into
 * the cache pages block_ids[j].  Replaces compressed_vram_pool.py:579-606
 * with FP8E4M3Codec.decompress_to (amf_codec.py:211-222). */
int amf_fp8_dequant_scatter(int32_t format,
                            const uint64_t* code_planes, const uint64_t* param_planes,
                            const uint64_t* cache_planes, int64_t cache_page_stride,
                            int32_t cache_dtype, const int32_t* block_ids, int64_t pool_pages,
                            int32_t n_planes, int64_t n_pages,
                            int32_t block_size, int32_t num_heads, int32_t head_dim,
                            int32_t* err_flag, void* stream);

/* INT4 save path (format = AMF_FMT_INT4_*).  Replaces
 * compressed_vram_pool.py:481-508 with INT4PerBlockCodec.compress
 * (amf_codec.py:358-408) / INT4PerChannelCodec.compress (:305-330). */
int amf_int4_quant_gather(int32_t format,
                          const uint64_t* cache_planes, int64_t cache_page_stride,
                          int32_t cache_dtype, const int32_t* block_ids, int64_t pool_pages,
                          const uint64_t* code_planes, const uint64_t* param_planes,
                          int32_t n_planes, int32_t planes_per_scale, int64_t n_pages,
                          int32_t block_size, int32_t num_heads, int32_t head_dim,
                          float* workspace, int64_t workspace_bytes,
                          int32_t* err_flag, void* stream);

/* INT4 restore path.  Replaces compressed_vram_pool.py:579-606 with
 * INT4PerBlockCodec.decompress_to (amf_codec.py:410-447) /
 * INT4PerChannelCodec.decompress_to (:332-343). */
int amf_int4_dequant_scatter(int32_t format,
                             const uint64_t* code_planes, const uint64_t* param_planes,
                             const uint64_t* cache_planes, int64_t cache_page_stride,
                             int32_t cache_dtype, const int32_t* block_ids, int64_t pool_pages,
                             int32_t n_planes, int64_t n_pages,
                             int32_t block_size, int32_t num_heads, int32_t head_dim,
                             int32_t* err_flag, void* stream);

/* ---- paged GQA decode attention over AMF_FMT_INT4_ASYM_G32 pages --------
 * q, out     : [num_seqs][num_q_heads][head_dim]; q_dtype is AMF_DTYPE_BF16
 *              or AMF_DTYPE_F16, out_dtype one of those or AMF_DTYPE_F32
 * k_codes, k_params, v_codes, v_params : one layer's INT4_ASYM_G32 planes of
 *              pool_pages pages each (page strides implied by the geometry)
 * block_tables: [num_seqs][block_table_stride] int32; context_lens: [num_seqs]
 * Query head h attends KV head h / (num_q_heads / num_kv_heads).
 * max_context_len bounds every context_lens[i] (it sizes the grid: no
 * device-to-host sync); a sequence with context 0 gets zeros.
 * softmax_scale <= 0 selects 1/sqrt(head_dim).
 * workspace: split partials and, for the MFMA path, a map of the
 *              sequences' first work units (num_seqs + 1 int64);
 *              amf_int4_decode_workspace_bytes() bytes (it sizes the MFMA
 *              path for the current device's resident waves: call it with
 *              the device of the launch current).
 * algo: AMF_DECODE_AUTO (= AMF_DECODE_MFMA), AMF_DECODE_VALU,
 *       AMF_DECODE_MFMA (PV products on single fp16 weights for a 32-token
 *       chunk only while their rounding error stays provably within 0.015
 *       of the output, fp16 hi + lo pairs elsewhere, bf16 hi + lo pairs where
 *       a chunk's V scales leave [2^-10, 15.5]) or AMF_DECODE_MFMA_PRECISE
 *       (pairs throughout).
 * Supported: head_dim 128, block_size 16, num_q_heads / num_kv_heads in
 * {1, 2, 4, 8}; anything else returns AMF_ERR_UNSUPPORTED.
 * Replaces int4_decode_attention (int4_decode_attention.py:6-9 ->
 * dispatch.py:117-143), adding paging and GQA. */
#define AMF_DECODE_AUTO  0
#define AMF_DECODE_VALU  1
#define AMF_DECODE_MFMA  2
#define AMF_DECODE_MFMA_PRECISE 3

int64_t amf_int4_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                        int32_t num_kv_heads, int32_t head_dim,
                                        int32_t max_context_len);

int amf_int4_paged_decode_attn(const void* q, int32_t q_dtype, void* out, int32_t out_dtype,
                               const void* k_codes, const void* k_params,
                               const void* v_codes, const void* v_params,
                               int64_t pool_pages,
                               const int32_t* block_tables, int32_t block_table_stride,
                               const int32_t* context_lens,
                               int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                               int32_t head_dim, int32_t block_size,
                               int32_t max_context_len, float softmax_scale,
                               void* workspace, int64_t workspace_bytes,
                               int32_t algo, int32_t* err_flag, void* stream);

/* amf_int4_paged_decode_attn without the workspace arguments: the split
 * partials go to a scratch array inside the library (one 64 MiB array per GPU
 * that loads the library, held until the process ends), so the call makes no
 * device allocation of its own or through the caller.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc).  A call whose
 * partials (amf_int4_decode_workspace_bytes()) exceed 64 MiB returns
 * AMF_ERR_WORKSPACE before any launch.  Every call on a GPU shares that GPU's
 * array and it keeps the last call's contents: calls that overlap on one GPU
 * (different streams, or threads without ordering) race; order them on one
 * stream.  Arguments and results otherwise as amf_int4_paged_decode_attn. */
int amf_int4_paged_decode_attn_noalloc(const void* q, int32_t q_dtype, void* out,
                                       int32_t out_dtype, const void* k_codes,
                                       const void* k_params, const void* v_codes,
                                       const void* v_params, int64_t pool_pages,
                                       const int32_t* block_tables, int32_t block_table_stride,
                                       const int32_t* context_lens, int32_t num_seqs,
                                       int32_t num_q_heads, int32_t num_kv_heads,
                                       int32_t head_dim, int32_t block_size,
                                       int32_t max_context_len, float softmax_scale,
                                       int32_t algo, int32_t* err_flag, void* stream);

/* ---- prefix keys (host functions, no device work) ---------------------------
 * FNV-1a over bytes, continuing from hash h (pass AMF_FNV_OFFSET to start).
 * Replaces _fnv1a_bytes (amf_kv_manager.py:69-72; C++ hash_bytes of
 * core/amf_store.cpp). */
#define AMF_FNV_OFFSET 1469598103934665603ull
uint64_t amf_fnv1a64(const void* data, int64_t n_bytes, uint64_t h);

/* Prefix hash of a token sequence: one FNV-1a step per token on its 32-bit
 * value, h = (h ^ (uint32_t)tok) * prime from AMF_FNV_OFFSET.  Replaces
 * amf_hash_tokens (amf_kv_manager.py:75-81). */
uint64_t amf_hash_tokens(const int32_t* tokens, int64_t n_tokens);

/* ---- dense attention ---------------------------------------------------------
 * out = softmax(q k^T * softmax_scale + mask) v, per query row, computed in
 * fp32 and rounded once to out_dtype.  q [batch, num_q_heads, q_len, head_dim],
 * k and v [batch, num_kv_heads, kv_len, head_dim], out like q; all contiguous,
 * q/k/v of one dtype (AMF_DTYPE_*).  num_q_heads must be a multiple of
 * num_kv_heads (GQA; query head h reads KV head h / (num_q_heads/num_kv_heads)).
 * mask: NULL or fp32 additive mask read at
 *   b*mask_stride_b + h*mask_stride_h + i*mask_stride_q + t*mask_stride_t
 * (element strides; 0 broadcasts).  kv_len 0 gives zeros; a row whose scores
 * are all -inf gives NaN, as softmax does.  head_dim <= 256.
 * workspace: device scratch of workspace_bytes (16-byte aligned).  When it
 * holds amf_dense_attn_workspace_bytes(...) bytes (non-zero only for
 * head_dim 64, 128 or 256 and kv_len > 0) and q, k, v are 16-byte aligned,
 * the KV tokens of each row are split over many waves (flash decoding) and
 * merged by a second launch; otherwise (NULL, too small) one workgroup per
 * query row runs the whole row.  Both give the same result to fp32 rounding.
 * Calls sharing a workspace must be ordered on one stream.
 * Replaces the attention of fallback_fp16_kernel (kernels/dispatch.py:117-143),
 * which int4_decode_attention (int4_decode_attention.py:6-9) reaches for k/v
 * given as tensors or CompressedKV without a block table. */
int amf_dense_attn(const void* q, const void* k, const void* v, int32_t dtype,
                   const float* mask, int64_t mask_stride_b, int64_t mask_stride_h,
                   int64_t mask_stride_q, int64_t mask_stride_t,
                   void* out, int32_t out_dtype,
                   int64_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                   int64_t q_len, int64_t kv_len, int32_t head_dim,
                   float softmax_scale, void* workspace, int64_t workspace_bytes,
                   void* stream);

/* Workspace bytes amf_dense_attn needs for its split path at this shape; 0
 * when the shape takes the single-pass path (then pass NULL, 0). */
int64_t amf_dense_attn_workspace_bytes(int64_t batch, int32_t num_q_heads,
                                       int32_t num_kv_heads, int64_t q_len,
                                       int64_t kv_len, int32_t head_dim);

/* amf_dense_attn over INT4_SYM K and V without materialising them: k_codes
 * and v_codes [batch, num_kv_heads, kv_len, head_dim / 2] packed codes
 * (element 2i in the low nibble of byte i), k_scales and v_scales the fp16
 * per-channel scales [head_dim], as an AMF_FMT_INT4_SYM codec leaves them.
 * head_dim 128 with bf16 / fp16 q and no mask (the decode shape) runs on
 * MFMA tiles with the scales folded into the query and the output: attention
 * over the exactly dequantized K/V, (code - 8) * scale not rounded to dtype,
 * with exact products accumulated in fp32 (softmax weights to 22 bits).
 * Otherwise each element is dequantized as the codec's restore writes it
 * into a cache of dtype (q's dtype): (code - 8) * scale in fp32, rounded to
 * dtype, and the result equals amf_dense_attn over the restored K/V to fp32
 * summation order.  head_dim 64, 128 or 256; q 16-byte and codes 4-byte
 * aligned; the workspace of amf_dense_attn_workspace_bytes
 * (AMF_ERR_WORKSPACE without it).  kv_len 0 gives zeros.
 * Replaces the decompress_to + fallback_fp16_kernel pair that
 * int4_decode_attention (int4_decode_attention.py:6-9 ->
 * kernels/dispatch.py:117-152) runs for "int4_sym" CompressedKV k/v. */
int amf_int4_sym_dense_attn(const void* q, int32_t dtype, const void* k_codes,
                            const uint16_t* k_scales, const void* v_codes,
                            const uint16_t* v_scales, const float* mask,
                            int64_t mask_stride_b, int64_t mask_stride_h,
                            int64_t mask_stride_q, int64_t mask_stride_t,
                            void* out, int32_t out_dtype,
                            int64_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                            int64_t q_len, int64_t kv_len, int32_t head_dim,
                            float softmax_scale, void* workspace, int64_t workspace_bytes,
                            void* stream);

/* ---- direct KV snapshots (AMFK blobs through pinned host staging) ----------
 * The AMFK blob: a 56-byte little-endian header
 *   u32 magic 0x414D464B ("AMFK"), version 1, n_layers, n_tokens, n_kv_heads,
 *   head_dim, dtype (AMF_DTYPE_* numbering; 3 = fp8), reserved 0,
 *   u64 total_kv_bytes, model_hash, prefix_hash (= amf_hash_tokens(tokens)),
 * then one 32-byte entry per layer, u64 k_offset, k_bytes, v_offset, v_bytes
 * (offsets from the start of the payload), then the payload: K0 V0 K1 V1 ...
 * A layer without KV (recurrent/SSM: a zero K or V address) is recorded as
 * {total, 0, total, 0} and skipped on restore.
 * (Layout of core/amf_direct_kv.h:35-72; the files of AmfKvManager,
 * korith_vllm_ext/amf_kv_manager.py:44-64, 327-338, are the same format.)
 *
 * A context owns a pinned host staging buffer (hipHostMalloc) that holds the
 * last saved blob or the blob being restored, and grows by 10% headroom when a
 * larger one is needed (core/amf_direct_kv.cu:70-93), plus a copy stream of
 * default priority created on first use on the then-current device.  A
 * context is not thread-safe; use one per thread or serialise calls.
 *
 * Save and restore are stream-ordered on `stream` (NULL = the null stream):
 * copies start after the work queued there before the call, and a restore's
 * data is in place for work queued there after it.  Save returns once the
 * blob is complete in host memory.  Restore returns without a host wait; the
 * staging buffer stays in use until its copies end, and the context waits
 * for them before it next hands the buffer out or writes into it.
 *
 * Validation is complete before the first copy: a blob that is too short,
 * has the wrong magic or version, a truncated layer table or a layer entry
 * outside the payload returns AMF_ERR_FORMAT; a layer count or a layer's
 * byte size that differs from the caller's returns AMF_ERR_MISMATCH; nothing
 * is written to the device in either case. */
typedef struct AmfDirectKvCtx AmfDirectKvCtx;

/* New context; pinned staging of max_kv_bytes (none when 0: no HIP call is
 * made until the first save/restore).  NULL on failure (amf_last_error()).
 * Replaces amf_direct_kv_init (core/amf_direct_kv.h:80-84, .cu:98-125). */
AmfDirectKvCtx* amf_direct_kv_init(uint64_t max_kv_bytes);

/* Frees the context after its outstanding copies end; NULL is ignored.
 * Replaces amf_direct_kv_free (core/amf_direct_kv.h:86-87, .cu:127-136). */
void amf_direct_kv_free(AmfDirectKvCtx* ctx);

/* 1 when data holds at least a header and starts with the AMFK magic, else 0.
 * Replaces amf_direct_kv_is_direct_format (core/amf_direct_kv.h:122-124,
 * .cu:138-144). */
int amf_direct_kv_is_direct_format(const uint8_t* data, uint64_t size);

/* The context's pinned staging buffer, grown to at least `bytes`, in
 * *buf_out: read a snapshot file straight into it, then pass it to a restore
 * (the role of AmfStore::load_kv_into in core/amf_direct_kv.cu:323-327). */
int amf_direct_kv_staging(AmfDirectKvCtx* ctx, uint64_t bytes, uint8_t** buf_out);

/* Snapshot n_layers layers of contiguous KV: layer i's K is k_bytes[i] bytes
 * at device address k_ptrs[i], V likewise (host arrays).  Writes header,
 * layer table and payload into the staging buffer and returns it in
 * *blob_out / *blob_bytes_out (valid until the next call on ctx).  dtype is
 * the header tag; n_kv_heads and head_dim are recorded as given.
 * Replaces amf_direct_kv_save (core/amf_direct_kv.h:89-104, .cu:158-298)
 * without the llama.cpp context and store admission: the caller hands the
 * tensors and stores the blob. */
int amf_direct_kv_save(AmfDirectKvCtx* ctx, const uint64_t* k_ptrs, const uint64_t* k_bytes,
                       const uint64_t* v_ptrs, const uint64_t* v_bytes, uint32_t n_layers,
                       uint32_t n_kv_heads, uint32_t head_dim, uint32_t dtype,
                       uint64_t model_hash, const int32_t* tokens, int64_t n_tokens,
                       const uint8_t** blob_out, uint64_t* blob_bytes_out, void* stream);

/* Validate a blob against n_layers layers of contiguous KV (addresses and
 * sizes as in amf_direct_kv_save) and copy every layer's K and V into them;
 * *n_tokens_out receives the header's token count.  A blob outside the
 * staging buffer is first copied into it.
 * Replaces amf_direct_kv_restore (core/amf_direct_kv.h:106-120,
 * .cu:302-462) without the llama.cpp cell bookkeeping (the caller marks its
 * first n_tokens cells used). */
int amf_direct_kv_restore(AmfDirectKvCtx* ctx, const uint8_t* blob, uint64_t blob_bytes,
                          const uint64_t* k_ptrs, const uint64_t* k_bytes,
                          const uint64_t* v_ptrs, const uint64_t* v_bytes, uint32_t n_layers,
                          uint32_t* n_tokens_out, void* stream);

/* Paged forms, for vLLM's [.., num_blocks, block_size, H, D] caches: the
 * payload of layer i is the n_pages pages block_ids[0..n_pages) of its K
 * plane then of its V plane.  cache_planes: host array of 2 * n_layers plane
 * base addresses (K0, V0, K1, V1, ...; a layer whose two entries are 0 has no
 * KV); page p of a plane is at plane + p * cache_page_stride; block_ids:
 * device int32 (NULL = pages 0..n_pages-1).  Pages move through
 * dev_staging, a caller-owned device buffer of staging_bytes (at least two
 * pages) used as two slots: while one slot's pages are copied between host
 * and device on the context's copy stream, the other's are gathered from or
 * scattered into the cache on `stream`.  Out-of-range block ids are skipped
 * and flagged in err_flag as in amf_kv_scatter_pages.  With n_pages = 0 a
 * restore validates the header and layer count only and copies nothing
 * (AmfKvManager with an empty block table).
 * Replace the gather + D2H of amf_kv_manager.py:298-368 and the H2D +
 * scatter of amf_kv_manager.py:488-523, with the header of save_kv_state
 * (:327-348; n_kv_heads as the caller gives it). */
int amf_direct_kv_save_pages(AmfDirectKvCtx* ctx, const uint64_t* cache_planes,
                             int64_t cache_page_stride, const int32_t* block_ids,
                             int64_t pool_pages, int64_t n_pages, int64_t page_bytes,
                             uint32_t n_layers, uint32_t n_kv_heads, uint32_t head_dim,
                             uint32_t dtype, uint64_t model_hash, const int32_t* tokens,
                             int64_t n_tokens, void* dev_staging, int64_t staging_bytes,
                             const uint8_t** blob_out, uint64_t* blob_bytes_out,
                             int32_t* err_flag, void* stream);

int amf_direct_kv_restore_pages(AmfDirectKvCtx* ctx, const uint8_t* blob, uint64_t blob_bytes,
                                const uint64_t* cache_planes, int64_t cache_page_stride,
                                const int32_t* block_ids, int64_t pool_pages, int64_t n_pages,
                                int64_t page_bytes, uint32_t n_layers, void* dev_staging,
                                int64_t staging_bytes, uint32_t* n_tokens_out,
                                int32_t* err_flag, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AMF_HIP_H */
