// amf_direct_kv.hip - AMFK KV snapshots through pinned host staging.
//
// Host side of core/amf_direct_kv.{h,cu} (save: header + layer table + D2H of
// every layer's K and V into one pinned blob; restore: validate the blob,
// then H2D of every layer) over caller-given device tensors instead of a
// llama.cpp context, plus a paged form for vLLM caches that streams pages
// through a two-slot device staging ring: one slot crosses PCIe on the
// context's copy stream while the other is gathered from / scattered into the
// cache on the caller's stream.
#include <string.h>

#include <algorithm>
#include <vector>

#include "amf_internal.h"
#include "amf_kernel_util.h"

// ---- blob format (core/amf_direct_kv.h:35-72) ---------------------------------

namespace {

constexpr uint32_t kAmfkMagic = 0x414D464Bu;  // "AMFK" as a little-endian u32
constexpr uint32_t kAmfkVersion = 1u;
constexpr uint32_t kDtypeTagMax = 3u;  // f16, f32, bf16, f8

struct AmfkHeader {
  uint32_t magic, version, n_layers, n_tokens, n_kv_heads, head_dim, dtype, reserved;
  uint64_t total_kv_bytes, model_hash, prefix_hash;
};
static_assert(sizeof(AmfkHeader) == 56, "AMFK header is 56 bytes");

struct AmfkLayer {
  uint64_t k_offset, k_bytes, v_offset, v_bytes;
};
static_assert(sizeof(AmfkLayer) == 32, "AMFK layer entry is 32 bytes");

constexpr uint64_t kHeaderBytes = sizeof(AmfkHeader);
constexpr uint64_t kLayerBytes = sizeof(AmfkLayer);

}  // namespace

struct AmfDirectKvCtx {
  uint8_t* pinned = nullptr;
  uint64_t pinned_size = 0;
  int device = -1;
  hipStream_t copy = nullptr;
  hipEvent_t start = nullptr;    // the caller's stream at call entry
  hipEvent_t ready[2] = {};      // slot filled (H2D landed / pages gathered)
  hipEvent_t done[2] = {};       // slot's last reader finished
  bool slot_used[2] = {false, false};
  hipEvent_t pinned_busy = nullptr;  // last copy that reads or writes `pinned`
  bool pinned_pending = false;
};

namespace {

using amf::fail;
using amf::ok;

int hip_fail(const char* who, const char* what, hipError_t e) {
  return fail(AMF_ERR_RUNTIME, "%s: %s failed: %s", who, what, hipGetErrorString(e));
}

#define AMF_HIP_TRY(who, expr)                         \
  do {                                                 \
    hipError_t _e = (expr);                            \
    if (_e != hipSuccess) return hip_fail(who, #expr, _e); \
  } while (0)

// Waits (host) for the last copy that touches the staging buffer.
int wait_pinned(const char* who, AmfDirectKvCtx* c) {
  if (c->pinned_pending) {
    AMF_HIP_TRY(who, hipEventSynchronize(c->pinned_busy));
    c->pinned_pending = false;
  }
  return AMF_OK;
}

// Grows the staging buffer to hold `needed` bytes, 10% over (the growth rule
// of core/amf_direct_kv.cu:70-93).  Contents are not preserved.
int ensure_pinned(const char* who, AmfDirectKvCtx* c, uint64_t needed) {
  if (needed <= c->pinned_size) return AMF_OK;
  int rc = wait_pinned(who, c);
  if (rc) return rc;
  if (c->pinned) {
    AMF_HIP_TRY(who, hipHostFree(c->pinned));
    c->pinned = nullptr;
    c->pinned_size = 0;
  }
  const uint64_t alloc = needed + needed / 10;
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, alloc, hipHostMallocDefault);
  if (e != hipSuccess)
    return fail(AMF_ERR_RUNTIME, "%s: pinned allocation of %llu bytes failed: %s", who,
                (unsigned long long)alloc, hipGetErrorString(e));
  c->pinned = static_cast<uint8_t*>(p);
  c->pinned_size = alloc;
  return AMF_OK;
}

// Copy stream and events, created on the current device at first use.
int ensure_runtime(const char* who, AmfDirectKvCtx* c) {
  int dev = -1;
  AMF_HIP_TRY(who, hipGetDevice(&dev));
  if (c->copy) {
    if (dev != c->device)
      return fail(AMF_ERR_UNSUPPORTED, "%s: context was bound to device %d, current is %d", who,
                  c->device, dev);
    return AMF_OK;
  }
  AMF_HIP_TRY(who, hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking));
  c->device = dev;
  AMF_HIP_TRY(who, hipEventCreateWithFlags(&c->start, hipEventDisableTiming));
  AMF_HIP_TRY(who, hipEventCreateWithFlags(&c->pinned_busy, hipEventDisableTiming));
  for (int s = 0; s < 2; ++s) {
    AMF_HIP_TRY(who, hipEventCreateWithFlags(&c->ready[s], hipEventDisableTiming));
    AMF_HIP_TRY(who, hipEventCreateWithFlags(&c->done[s], hipEventDisableTiming));
  }
  return AMF_OK;
}

bool within_pinned(const AmfDirectKvCtx* c, const uint8_t* p, uint64_t n) {
  if (!c->pinned || p < c->pinned) return false;
  const uint64_t off = (uint64_t)(p - c->pinned);
  return off <= c->pinned_size && n <= c->pinned_size - off;
}

// Header + layer table checks shared by both restores (the checks of
// core/amf_direct_kv.cu:331-369, run before any copy).
int parse_blob(const char* who, const uint8_t* blob, uint64_t blob_bytes, uint32_t n_layers,
               AmfkHeader* hdr, std::vector<AmfkLayer>* table) {
  if (blob_bytes < kHeaderBytes)
    return fail(AMF_ERR_FORMAT, "%s: blob too small (%llu bytes)", who,
                (unsigned long long)blob_bytes);
  memcpy(hdr, blob, sizeof(*hdr));
  if (hdr->magic != kAmfkMagic)
    return fail(AMF_ERR_FORMAT, "%s: not an AMFK snapshot (magic=0x%08X)", who, hdr->magic);
  if (hdr->version != kAmfkVersion)
    return fail(AMF_ERR_FORMAT, "%s: version mismatch (got=%u, want=%u)", who, hdr->version,
                kAmfkVersion);
  if (hdr->n_layers != n_layers)
    return fail(AMF_ERR_MISMATCH, "%s: layer count mismatch (snapshot=%u, ctx=%u)", who,
                hdr->n_layers, n_layers);
  const uint64_t tbl_end = kHeaderBytes + (uint64_t)n_layers * kLayerBytes;
  if (blob_bytes < tbl_end)
    return fail(AMF_ERR_FORMAT, "%s: blob truncated (layer table missing)", who);
  table->resize(n_layers);
  if (n_layers) memcpy(table->data(), blob + kHeaderBytes, (size_t)n_layers * kLayerBytes);
  return AMF_OK;
}

// An entry's byte range must lie inside the payload (the reference trusts it).
int check_range(const char* who, uint32_t layer, const char* kv, uint64_t off, uint64_t bytes,
                uint64_t payload) {
  if (off > payload || bytes > payload - off)
    return fail(AMF_ERR_FORMAT, "%s: layer %u %s bytes [%llu, +%llu) outside the %llu-byte payload",
                who, layer, kv, (unsigned long long)off, (unsigned long long)bytes,
                (unsigned long long)payload);
  return AMF_OK;
}

void write_header(uint8_t* dst, uint32_t n_layers, uint64_t n_tokens, uint32_t n_kv_heads,
                  uint32_t head_dim, uint32_t dtype, uint64_t total, uint64_t model_hash,
                  uint64_t prefix_hash, const std::vector<AmfkLayer>& table) {
  AmfkHeader h{};
  h.magic = kAmfkMagic;
  h.version = kAmfkVersion;
  h.n_layers = n_layers;
  h.n_tokens = (uint32_t)n_tokens;
  h.n_kv_heads = n_kv_heads;
  h.head_dim = head_dim;
  h.dtype = dtype;
  h.reserved = 0;
  h.total_kv_bytes = total;
  h.model_hash = model_hash;
  h.prefix_hash = prefix_hash;
  memcpy(dst, &h, sizeof(h));
  if (n_layers) memcpy(dst + kHeaderBytes, table.data(), (size_t)n_layers * kLayerBytes);
}

int check_save_common(const char* who, AmfDirectKvCtx* c, uint32_t n_layers, uint32_t dtype,
                      const int32_t* tokens, int64_t n_tokens, const uint8_t** blob_out,
                      uint64_t* blob_bytes_out) {
  if (!c) return fail(AMF_ERR_INVALID_ARG, "%s: null context", who);
  if (!blob_out || !blob_bytes_out) return fail(AMF_ERR_INVALID_ARG, "%s: null blob outputs", who);
  if (n_layers == 0) return fail(AMF_ERR_INVALID_ARG, "%s: no attention layers", who);
  if (dtype > kDtypeTagMax) return fail(AMF_ERR_INVALID_ARG, "%s: dtype tag %u", who, dtype);
  if (n_tokens < 0 || n_tokens > (int64_t)UINT32_MAX || (n_tokens > 0 && !tokens))
    return fail(AMF_ERR_INVALID_ARG, "%s: bad tokens (n=%lld)", who, (long long)n_tokens);
  return AMF_OK;
}

// ---- paged staging copies -------------------------------------------------------
//
// One launch moves up to kSegMax segments (a run of consecutive block-table
// positions of one cache plane) between the cache and one staging slot.  The
// segment list travels in the kernel arguments, so no device table is built
// per chunk.  Workgroup (x, seg) moves page x of segment seg: 256 lanes of
// 16-byte vectors, four in flight, as page_copy_kernel.

constexpr int kSegMax = 64;
constexpr int kSegThreads = 256;
constexpr int kSegUnroll = 4;

struct SegBatch {
  uint64_t cache[kSegMax];  // plane base address
  uint64_t dense[kSegMax];  // staging address of the segment's first page
  int32_t j0[kSegMax];      // block-table position of its first page
  int32_t count[kSegMax];   // pages
};

template <bool kToCache>
__global__ __launch_bounds__(kSegThreads) void seg_copy_kernel(
    const SegBatch b, int64_t cache_stride, const int32_t* __restrict__ ids, int64_t pool,
    int64_t page_bytes, int32_t* err_flag) {
  const int seg = blockIdx.y;
  const int x = blockIdx.x;
  if (x >= b.count[seg]) return;
  const int64_t j = (int64_t)b.j0[seg] + x;
  const int64_t bid = ids ? (int64_t)ids[j] : j;
  if (bid < 0 || bid >= pool) {
    if (threadIdx.x == 0 && err_flag) atomicOr(err_flag, AMF_ERRFLAG_BLOCK_RANGE);
    return;
  }
  using amf::u32x4;
  u32x4* cp = reinterpret_cast<u32x4*>(b.cache[seg] + (uint64_t)(bid * cache_stride));
  u32x4* dp = reinterpret_cast<u32x4*>(b.dense[seg] + (uint64_t)((int64_t)x * page_bytes));
  const u32x4* s = kToCache ? dp : cp;
  u32x4* d = kToCache ? cp : dp;
  const int64_t n16 = page_bytes / 16;
  for (int64_t base = threadIdx.x; base < n16; base += kSegThreads * kSegUnroll) {
    u32x4 v[kSegUnroll];
#pragma unroll
    for (int u = 0; u < kSegUnroll; ++u) {
      const int64_t k = base + (int64_t)u * kSegThreads;
      if (k < n16) v[u] = amf::ld_stream(s + k);
    }
#pragma unroll
    for (int u = 0; u < kSegUnroll; ++u) {
      const int64_t k = base + (int64_t)u * kSegThreads;
      if (k < n16) amf::st_stream(v[u], d + k);
    }
  }
}

// A run of pages of one plane: block-table positions [j0, j0 + count), whose
// bytes sit at payload offset `host_off` in the blob.
struct PlaneRun {
  uint64_t plane;
  uint64_t host_off;
};

struct PagedArgs {
  const uint64_t* planes;
  int64_t stride;
  const int32_t* ids;
  int64_t pool;
  int64_t n_pages;
  int64_t page_bytes;
  uint8_t* staging;
  int64_t staging_bytes;
  int32_t* err_flag;
  hipStream_t stream;
};

int check_paged(const char* who, const PagedArgs& a, uint32_t n_layers) {
  if (!a.planes) return fail(AMF_ERR_INVALID_ARG, "%s: null cache_planes", who);
  if (n_layers > 32767) return fail(AMF_ERR_INVALID_ARG, "%s: %u layers", who, n_layers);
  if (a.page_bytes <= 0 || !amf::aligned16(a.page_bytes) || !amf::aligned16(a.stride) ||
      a.stride < a.page_bytes)
    return fail(AMF_ERR_INVALID_ARG,
                "%s: page_bytes=%lld and page stride %lld must be positive multiples of 16 with "
                "stride >= page_bytes",
                who, (long long)a.page_bytes, (long long)a.stride);
  if (a.pool <= 0 || a.n_pages < 0 || a.n_pages > 0x7FFFFFFF)
    return fail(AMF_ERR_INVALID_ARG, "%s: bad pool_pages=%lld / n_pages=%lld", who,
                (long long)a.pool, (long long)a.n_pages);
  if (!a.ids && a.n_pages > a.pool)
    return fail(AMF_ERR_INVALID_ARG, "%s: n_pages %lld > pool %lld with the identity map", who,
                (long long)a.n_pages, (long long)a.pool);
  for (uint32_t l = 0; l < n_layers; ++l)
    if ((a.planes[2 * l] == 0) != (a.planes[2 * l + 1] == 0))
      return fail(AMF_ERR_INVALID_ARG, "%s: layer %u has only one of its K/V planes", who, l);
  if (a.n_pages > 0) {
    if (!a.staging || ((uintptr_t)a.staging & 15))
      return fail(AMF_ERR_WORKSPACE, "%s: staging buffer missing or not 16-byte aligned", who);
    if (a.staging_bytes / 2 < a.page_bytes)
      return fail(AMF_ERR_WORKSPACE, "%s: staging of %lld bytes holds fewer than two %lld-byte pages",
                  who, (long long)a.staging_bytes, (long long)a.page_bytes);
  }
  return AMF_OK;
}

// Walks the planes' pages in chunks of one staging slot and issues, per
// chunk, the host<->slot copies on the copy stream and the slot<->cache launch
// on the caller's stream, ordered through the slot events.
class SlotPipeline {
 public:
  SlotPipeline(const char* who, AmfDirectKvCtx* c, const PagedArgs& a, bool to_cache,
               uint8_t* host_payload)
      : who_(who), c_(c), a_(a), to_cache_(to_cache), host_(host_payload) {
    slot_pages_ = (a.staging_bytes / 2) / a.page_bytes;
    slot_stride_ = slot_pages_ * a.page_bytes;
    if (slot_pages_ > 0x7FFFFFFF) slot_pages_ = 0x7FFFFFFF;
  }

  int add(const PlaneRun& run) {
    int64_t j = 0;
    while (j < a_.n_pages) {
      if (nseg_ == kSegMax || used_ == slot_pages_) {
        int rc = flush();
        if (rc) return rc;
      }
      const int64_t n = std::min<int64_t>(a_.n_pages - j, slot_pages_ - used_);
      b_.cache[nseg_] = run.plane;
      b_.dense[nseg_] = (uint64_t)used_ * a_.page_bytes;  // slot-relative until flush
      b_.j0[nseg_] = (int32_t)j;
      b_.count[nseg_] = (int32_t)n;
      host_off_[nseg_] = run.host_off + (uint64_t)j * a_.page_bytes;
      ++nseg_;
      used_ += n;
      j += n;
    }
    return AMF_OK;
  }

  int flush() {
    if (nseg_ == 0) return AMF_OK;
    const int s = chunk_ & 1;
    uint8_t* slot = a_.staging + s * slot_stride_;
    int max_count = 0;
    for (int i = 0; i < nseg_; ++i) {
      b_.dense[i] += (uint64_t)slot;
      max_count = std::max(max_count, b_.count[i]);
    }
    for (int i = nseg_; i < kSegMax; ++i) b_.count[i] = 0;
    hipStream_t kernel_stream = a_.stream;
    if (to_cache_) {
      if (c_->slot_used[s]) AMF_HIP_TRY(who_, hipStreamWaitEvent(c_->copy, c_->done[s], 0));
      int rc = copies(s, hipMemcpyHostToDevice);
      if (rc) return rc;
      AMF_HIP_TRY(who_, hipEventRecord(c_->ready[s], c_->copy));
      AMF_HIP_TRY(who_, hipStreamWaitEvent(kernel_stream, c_->ready[s], 0));
      int lr = launch(max_count, kernel_stream);
      if (lr) return lr;
      AMF_HIP_TRY(who_, hipEventRecord(c_->done[s], kernel_stream));
    } else {
      if (c_->slot_used[s]) AMF_HIP_TRY(who_, hipStreamWaitEvent(kernel_stream, c_->done[s], 0));
      int lr = launch(max_count, kernel_stream);
      if (lr) return lr;
      AMF_HIP_TRY(who_, hipEventRecord(c_->ready[s], kernel_stream));
      AMF_HIP_TRY(who_, hipStreamWaitEvent(c_->copy, c_->ready[s], 0));
      int rc = copies(s, hipMemcpyDeviceToHost);
      if (rc) return rc;
      AMF_HIP_TRY(who_, hipEventRecord(c_->done[s], c_->copy));
    }
    c_->slot_used[s] = true;
    ++chunk_;
    nseg_ = 0;
    used_ = 0;
    return AMF_OK;
  }

 private:
  // One copy per run of segments that are adjacent in both the blob and the
  // slot (consecutive planes of the payload, normally a whole chunk).
  int copies(int s, hipMemcpyKind kind) {
    int i = 0;
    while (i < nseg_) {
      uint64_t dev = b_.dense[i];
      uint64_t host = host_off_[i];
      uint64_t bytes = (uint64_t)b_.count[i] * a_.page_bytes;
      int k = i + 1;
      while (k < nseg_ && b_.dense[k] == dev + bytes && host_off_[k] == host + bytes) {
        bytes += (uint64_t)b_.count[k] * a_.page_bytes;
        ++k;
      }
      void* hp = host_ + host;
      void* dp = reinterpret_cast<void*>(dev);
      if (kind == hipMemcpyHostToDevice)
        AMF_HIP_TRY(who_, hipMemcpyAsync(dp, hp, bytes, kind, c_->copy));
      else
        AMF_HIP_TRY(who_, hipMemcpyAsync(hp, dp, bytes, kind, c_->copy));
      i = k;
    }
    (void)s;
    return AMF_OK;
  }

  int launch(int max_count, hipStream_t st) {
    dim3 grid((unsigned)max_count, (unsigned)nseg_);
    if (to_cache_)
      seg_copy_kernel<true><<<grid, kSegThreads, 0, st>>>(b_, a_.stride, a_.ids, a_.pool,
                                                          a_.page_bytes, a_.err_flag);
    else
      seg_copy_kernel<false><<<grid, kSegThreads, 0, st>>>(b_, a_.stride, a_.ids, a_.pool,
                                                           a_.page_bytes, a_.err_flag);
    return amf::check_launch(who_);
  }

  const char* who_;
  AmfDirectKvCtx* c_;
  PagedArgs a_;
  bool to_cache_;
  uint8_t* host_;
  int64_t slot_pages_ = 0;
  int64_t slot_stride_ = 0;
  SegBatch b_{};
  uint64_t host_off_[kSegMax] = {};
  int nseg_ = 0;
  int64_t used_ = 0;
  int64_t chunk_ = 0;
};

}  // namespace

// ---- C ABI ------------------------------------------------------------------------

extern "C" AmfDirectKvCtx* amf_direct_kv_init(uint64_t max_kv_bytes) {
  auto* c = new AmfDirectKvCtx{};
  if (max_kv_bytes > 0 && ensure_pinned("amf_direct_kv_init", c, max_kv_bytes) != AMF_OK) {
    delete c;
    return nullptr;
  }
  ok();
  return c;
}

extern "C" void amf_direct_kv_free(AmfDirectKvCtx* c) {
  if (!c) return;
  if (c->pinned_pending) (void)hipEventSynchronize(c->pinned_busy);
  if (c->copy) (void)hipStreamSynchronize(c->copy);
  for (int s = 0; s < 2; ++s) {
    if (c->slot_used[s]) (void)hipEventSynchronize(c->done[s]);
    if (c->ready[s]) (void)hipEventDestroy(c->ready[s]);
    if (c->done[s]) (void)hipEventDestroy(c->done[s]);
  }
  if (c->start) (void)hipEventDestroy(c->start);
  if (c->pinned_busy) (void)hipEventDestroy(c->pinned_busy);
  if (c->copy) (void)hipStreamDestroy(c->copy);
  if (c->pinned) (void)hipHostFree(c->pinned);
  delete c;
}

extern "C" int amf_direct_kv_is_direct_format(const uint8_t* data, uint64_t size) {
  if (!data || size < kHeaderBytes) return 0;
  uint32_t magic;
  memcpy(&magic, data, sizeof(magic));
  return magic == kAmfkMagic ? 1 : 0;
}

extern "C" int amf_direct_kv_staging(AmfDirectKvCtx* c, uint64_t bytes, uint8_t** buf_out) {
  const char* who = "amf_direct_kv_staging";
  if (!c || !buf_out) return fail(AMF_ERR_INVALID_ARG, "%s: null argument", who);
  int rc = wait_pinned(who, c);
  if (!rc) rc = ensure_pinned(who, c, bytes ? bytes : 1);
  if (rc) return rc;
  *buf_out = c->pinned;
  return ok();
}

extern "C" int amf_direct_kv_save(AmfDirectKvCtx* c, const uint64_t* k_ptrs,
                                  const uint64_t* k_bytes, const uint64_t* v_ptrs,
                                  const uint64_t* v_bytes, uint32_t n_layers,
                                  uint32_t n_kv_heads, uint32_t head_dim, uint32_t dtype,
                                  uint64_t model_hash, const int32_t* tokens, int64_t n_tokens,
                                  const uint8_t** blob_out, uint64_t* blob_bytes_out,
                                  void* stream) {
  const char* who = "amf_direct_kv_save";
  int rc = check_save_common(who, c, n_layers, dtype, tokens, n_tokens, blob_out, blob_bytes_out);
  if (rc) return rc;
  if (!k_ptrs || !k_bytes || !v_ptrs || !v_bytes)
    return fail(AMF_ERR_INVALID_ARG, "%s: null layer arrays", who);
  // Layer table: K then V of each layer back to back; a layer without KV
  // tensors is {total, 0, total, 0} (core/amf_direct_kv.cu:180-199).
  std::vector<AmfkLayer> table(n_layers);
  uint64_t total = 0;
  for (uint32_t l = 0; l < n_layers; ++l) {
    if (!k_ptrs[l] || !v_ptrs[l]) {
      table[l] = {total, 0, total, 0};
      continue;
    }
    table[l].k_offset = total;
    table[l].k_bytes = k_bytes[l];
    total += k_bytes[l];
    table[l].v_offset = total;
    table[l].v_bytes = v_bytes[l];
    total += v_bytes[l];
  }
  const uint64_t tbl_end = kHeaderBytes + (uint64_t)n_layers * kLayerBytes;
  if ((rc = wait_pinned(who, c)) || (rc = ensure_pinned(who, c, tbl_end + total)) ||
      (rc = ensure_runtime(who, c)))
    return rc;
  write_header(c->pinned, n_layers, (uint64_t)n_tokens, n_kv_heads, head_dim, dtype, total,
               model_hash, amf_hash_tokens(tokens, n_tokens), table);
  hipStream_t st = amf::as_stream(stream);
  uint8_t* payload = c->pinned + tbl_end;
  for (uint32_t l = 0; l < n_layers; ++l) {
    if (!k_ptrs[l] || !v_ptrs[l]) continue;
    const AmfkLayer& li = table[l];
    if (li.k_bytes)
      AMF_HIP_TRY(who, hipMemcpyAsync(payload + li.k_offset, (const void*)k_ptrs[l], li.k_bytes,
                                      hipMemcpyDeviceToHost, st));
    if (li.v_bytes)
      AMF_HIP_TRY(who, hipMemcpyAsync(payload + li.v_offset, (const void*)v_ptrs[l], li.v_bytes,
                                      hipMemcpyDeviceToHost, st));
  }
  AMF_HIP_TRY(who, hipEventRecord(c->pinned_busy, st));
  AMF_HIP_TRY(who, hipEventSynchronize(c->pinned_busy));
  *blob_out = c->pinned;
  *blob_bytes_out = tbl_end + total;
  return ok();
}

extern "C" int amf_direct_kv_restore(AmfDirectKvCtx* c, const uint8_t* blob, uint64_t blob_bytes,
                                     const uint64_t* k_ptrs, const uint64_t* k_bytes,
                                     const uint64_t* v_ptrs, const uint64_t* v_bytes,
                                     uint32_t n_layers, uint32_t* n_tokens_out, void* stream) {
  const char* who = "amf_direct_kv_restore";
  if (!c || !blob) return fail(AMF_ERR_INVALID_ARG, "%s: null context or blob", who);
  if (n_layers && (!k_ptrs || !k_bytes || !v_ptrs || !v_bytes))
    return fail(AMF_ERR_INVALID_ARG, "%s: null layer arrays", who);
  AmfkHeader hdr;
  std::vector<AmfkLayer> table;
  int rc = parse_blob(who, blob, blob_bytes, n_layers, &hdr, &table);
  if (rc) return rc;
  const uint64_t tbl_end = kHeaderBytes + (uint64_t)n_layers * kLayerBytes;
  const uint64_t payload_bytes = blob_bytes - tbl_end;
  for (uint32_t l = 0; l < n_layers; ++l) {
    if (!k_ptrs[l] || !v_ptrs[l]) continue;  // no KV in this layer of the caller's model
    const AmfkLayer& li = table[l];
    if (li.k_bytes != k_bytes[l] || li.v_bytes != v_bytes[l])
      return fail(AMF_ERR_MISMATCH,
                  "%s: layer %u size mismatch (K snapshot=%llu ctx=%llu; V snapshot=%llu "
                  "ctx=%llu)",
                  who, l, (unsigned long long)li.k_bytes, (unsigned long long)k_bytes[l],
                  (unsigned long long)li.v_bytes, (unsigned long long)v_bytes[l]);
    if ((rc = check_range(who, l, "K", li.k_offset, li.k_bytes, payload_bytes)) ||
        (rc = check_range(who, l, "V", li.v_offset, li.v_bytes, payload_bytes)))
      return rc;
  }
  if ((rc = ensure_runtime(who, c))) return rc;
  const uint8_t* src = blob;
  if (!within_pinned(c, blob, blob_bytes)) {
    if ((rc = wait_pinned(who, c)) || (rc = ensure_pinned(who, c, blob_bytes))) return rc;
    memcpy(c->pinned, blob, blob_bytes);
    src = c->pinned;
  }
  hipStream_t st = amf::as_stream(stream);
  const uint8_t* payload = src + tbl_end;
  for (uint32_t l = 0; l < n_layers; ++l) {
    if (!k_ptrs[l] || !v_ptrs[l]) continue;
    const AmfkLayer& li = table[l];
    if (li.k_bytes)
      AMF_HIP_TRY(who, hipMemcpyAsync((void*)k_ptrs[l], payload + li.k_offset, li.k_bytes,
                                      hipMemcpyHostToDevice, st));
    if (li.v_bytes)
      AMF_HIP_TRY(who, hipMemcpyAsync((void*)v_ptrs[l], payload + li.v_offset, li.v_bytes,
                                      hipMemcpyHostToDevice, st));
  }
  AMF_HIP_TRY(who, hipEventRecord(c->pinned_busy, st));
  c->pinned_pending = true;
  if (n_tokens_out) *n_tokens_out = hdr.n_tokens;
  return ok();
}

extern "C" int amf_direct_kv_save_pages(AmfDirectKvCtx* c, const uint64_t* cache_planes,
                                        int64_t cache_page_stride, const int32_t* block_ids,
                                        int64_t pool_pages, int64_t n_pages, int64_t page_bytes,
                                        uint32_t n_layers, uint32_t n_kv_heads, uint32_t head_dim,
                                        uint32_t dtype, uint64_t model_hash,
                                        const int32_t* tokens, int64_t n_tokens,
                                        void* dev_staging, int64_t staging_bytes,
                                        const uint8_t** blob_out, uint64_t* blob_bytes_out,
                                        int32_t* err_flag, void* stream) {
  const char* who = "amf_direct_kv_save_pages";
  int rc = check_save_common(who, c, n_layers, dtype, tokens, n_tokens, blob_out, blob_bytes_out);
  if (rc) return rc;
  PagedArgs a{cache_planes, cache_page_stride, block_ids, pool_pages, n_pages, page_bytes,
              static_cast<uint8_t*>(dev_staging), staging_bytes, err_flag,
              amf::as_stream(stream)};
  if ((rc = check_paged(who, a, n_layers))) return rc;
  const uint64_t plane_bytes = (uint64_t)n_pages * (uint64_t)page_bytes;
  std::vector<AmfkLayer> table(n_layers);
  uint64_t total = 0;
  for (uint32_t l = 0; l < n_layers; ++l) {
    if (!cache_planes[2 * l]) {
      table[l] = {total, 0, total, 0};
      continue;
    }
    table[l] = {total, plane_bytes, total + plane_bytes, plane_bytes};
    total += 2 * plane_bytes;
  }
  const uint64_t tbl_end = kHeaderBytes + (uint64_t)n_layers * kLayerBytes;
  if ((rc = wait_pinned(who, c)) || (rc = ensure_pinned(who, c, tbl_end + total)) ||
      (rc = ensure_runtime(who, c)))
    return rc;
  write_header(c->pinned, n_layers, (uint64_t)n_tokens, n_kv_heads, head_dim, dtype, total,
               model_hash, amf_hash_tokens(tokens, n_tokens), table);
  if (n_pages > 0) {
    SlotPipeline pipe(who, c, a, /*to_cache=*/false, c->pinned + tbl_end);
    for (uint32_t l = 0; l < n_layers; ++l) {
      if (!cache_planes[2 * l]) continue;
      if ((rc = pipe.add({cache_planes[2 * l], table[l].k_offset})) ||
          (rc = pipe.add({cache_planes[2 * l + 1], table[l].v_offset})))
        return rc;
    }
    if ((rc = pipe.flush())) return rc;
  }
  AMF_HIP_TRY(who, hipEventRecord(c->pinned_busy, c->copy));
  AMF_HIP_TRY(who, hipEventSynchronize(c->pinned_busy));
  *blob_out = c->pinned;
  *blob_bytes_out = tbl_end + total;
  return ok();
}

extern "C" int amf_direct_kv_restore_pages(AmfDirectKvCtx* c, const uint8_t* blob,
                                           uint64_t blob_bytes, const uint64_t* cache_planes,
                                           int64_t cache_page_stride, const int32_t* block_ids,
                                           int64_t pool_pages, int64_t n_pages,
                                           int64_t page_bytes, uint32_t n_layers,
                                           void* dev_staging, int64_t staging_bytes,
                                           uint32_t* n_tokens_out, int32_t* err_flag,
                                           void* stream) {
  const char* who = "amf_direct_kv_restore_pages";
  if (!c || !blob) return fail(AMF_ERR_INVALID_ARG, "%s: null context or blob", who);
  PagedArgs a{cache_planes, cache_page_stride, block_ids, pool_pages, n_pages, page_bytes,
              static_cast<uint8_t*>(dev_staging), staging_bytes, err_flag,
              amf::as_stream(stream)};
  int rc = check_paged(who, a, n_layers);
  if (rc) return rc;
  AmfkHeader hdr;
  std::vector<AmfkLayer> table;
  if ((rc = parse_blob(who, blob, blob_bytes, n_layers, &hdr, &table))) return rc;
  if (n_tokens_out) *n_tokens_out = hdr.n_tokens;
  if (n_pages == 0) return ok();  // nothing to place (an empty block table)
  const uint64_t tbl_end = kHeaderBytes + (uint64_t)n_layers * kLayerBytes;
  const uint64_t payload_bytes = blob_bytes - tbl_end;
  const uint64_t want = (uint64_t)n_pages * (uint64_t)page_bytes;
  for (uint32_t l = 0; l < n_layers; ++l) {
    const AmfkLayer& li = table[l];
    if (!cache_planes[2 * l] || (li.k_bytes == 0 && li.v_bytes == 0)) continue;
    if (li.k_bytes != want || li.v_bytes != want)
      return fail(AMF_ERR_MISMATCH,
                  "%s: layer %u holds K %llu / V %llu bytes, the cache needs %llu for %lld pages",
                  who, l, (unsigned long long)li.k_bytes, (unsigned long long)li.v_bytes,
                  (unsigned long long)want, (long long)n_pages);
    if ((rc = check_range(who, l, "K", li.k_offset, li.k_bytes, payload_bytes)) ||
        (rc = check_range(who, l, "V", li.v_offset, li.v_bytes, payload_bytes)))
      return rc;
  }
  if ((rc = ensure_runtime(who, c))) return rc;
  const uint8_t* src = blob;
  if (!within_pinned(c, blob, blob_bytes)) {
    if ((rc = wait_pinned(who, c)) || (rc = ensure_pinned(who, c, blob_bytes))) return rc;
    memcpy(c->pinned, blob, blob_bytes);
    src = c->pinned;
  }
  // Copies into the staging slots start after the caller's queued work (the
  // slots may still be read by it).
  AMF_HIP_TRY(who, hipEventRecord(c->start, a.stream));
  AMF_HIP_TRY(who, hipStreamWaitEvent(c->copy, c->start, 0));
  SlotPipeline pipe(who, c, a, /*to_cache=*/true, const_cast<uint8_t*>(src) + tbl_end);
  for (uint32_t l = 0; l < n_layers; ++l) {
    const AmfkLayer& li = table[l];
    if (!cache_planes[2 * l] || (li.k_bytes == 0 && li.v_bytes == 0)) continue;
    if ((rc = pipe.add({cache_planes[2 * l], li.k_offset})) ||
        (rc = pipe.add({cache_planes[2 * l + 1], li.v_offset})))
      return rc;
  }
  if ((rc = pipe.flush())) return rc;
  AMF_HIP_TRY(who, hipEventRecord(c->pinned_busy, c->copy));
  c->pinned_pending = true;
  return ok();
}
