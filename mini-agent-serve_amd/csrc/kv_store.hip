// kv_store.hip - append one step's k/v rows into the paged KV cache.
//
// Semantics (miniagentserve/models/devstral2/devstral2.py:170-173 with kv_indptr from :289,
// flashinfer.page.append_paged_kv_cache; cache layout from miniagentserve/engine/model_runner.py:83-85):
//   block-table form: b = batch_indices[t], p = positions[t],
//                     page = kv_indices[kv_indptr[b] + p / page_size], entry = p % page_size
//   slot form:        slot = slot_mapping[t] (negative = padding, skipped),
//                     page = slot / page_size, entry = slot % page_size
//   k_cache[page, entry, h, :] = key[t, h, :];  v_cache[page, entry, h, :] = value[t, h, :]
//
// A bit copy: one wavefront per (token, tensor), its destination resolved once per wavefront from
// wave-uniform (scalar-cache) index loads issued after the row's loads, so both latencies overlap;
// each lane moves 16-byte vectors, all loads issued before the stores.
// Duplicate destinations (padding rows aimed at the model runner's sink block) are plain racing
// stores of whole rows: one writer wins.
#include "device.h"

namespace mas {
namespace {

// One wavefront per workgroup and per (token, tensor): measured best on MI355X at every size, from
// the 64-token decode (2.17 us) to 16384 prefill tokens (ahead of 128/256/512-thread workgroups and
// of one wavefront moving both of a token's rows).
constexpr int kBlock = 64;
constexpr int kSplit = 2;  // wavefronts per token: one for k, one for v
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kUnroll = 2;

struct KvArgs {
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t page_stride, entry_stride, head_stride, num_pages, page_size;
  const uint16_t* key;
  int64_t key_stride, key_head_stride;
  const uint16_t* value;
  int64_t value_stride, value_head_stride;
  // block-table form
  const int32_t* batch_indices;
  const int32_t* positions;
  const int32_t* kv_indices;
  int64_t num_indices;
  const int32_t* kv_indptr;
  int64_t batch;
  // slot form
  const int64_t* slots;
  int64_t rows;
  int vec_per_head;  // head_dim / 8
  int vec_per_row;   // num_heads * head_dim / 8
  uint32_t* err;
};

// Resolves token t's (page, entry). Returns false when the token is skipped.
template <bool kSlotForm>
__device__ __forceinline__ bool resolve(const KvArgs& a, int64_t t, int64_t* page, int64_t* entry) {
  if constexpr (kSlotForm) {
    const int64_t slot = a.slots[t];
    if (slot < 0) return false;
    const int64_t pg = slot / a.page_size;
    if (pg >= a.num_pages) {
      report(a.err, MAS_ERRBIT_SLOT);
      return false;
    }
    *page = pg;
    *entry = slot - pg * a.page_size;
    return true;
  } else {
    // Both per-token indices are loaded before either is checked, so the two loads overlap.
    const int64_t b = a.batch_indices[t];
    const int64_t p = a.positions[t];
    const bool b_ok = b >= 0 && b < a.batch;
    if (!b_ok || p < 0) {
      report(a.err, b_ok ? MAS_ERRBIT_POSITION : MAS_ERRBIT_BATCH);
      return false;
    }
    const int64_t first = a.kv_indptr[b];
    const int64_t end = a.kv_indptr[b + 1];
    const int64_t idx = first + p / a.page_size;
    if (idx < 0 || idx >= a.num_indices || idx >= end) {
      report(a.err, MAS_ERRBIT_PAGE);
      return false;
    }
    const int64_t pg = a.kv_indices[idx];
    if (pg < 0 || pg >= a.num_pages) {
      report(a.err, MAS_ERRBIT_PAGE);
      return false;
    }
    *page = pg;
    *entry = p % a.page_size;
    return true;
  }
}

// Element offset of 16-byte vector v of a token's row, for a row made of heads of vec_per_head
// vectors placed head_stride elements apart.
__device__ __forceinline__ int64_t vec_offset(int v, int vec_per_head, int64_t head_stride, bool contiguous) {
  if (contiguous) return 8 * static_cast<int64_t>(v);
  const int h = v / vec_per_head;
  return h * head_stride + 8 * (v - h * vec_per_head);
}

// The source rows are loaded before the destination is resolved: the k/v loads do not depend on
// it, so the index loads (scalar cache) and the data loads are in flight together.
// kSplit: 1 = one wavefront moves a token's k and v rows; 2 = one wavefront per (token, tensor).
template <bool kSlotForm, bool kContig, int kSplit>
__global__ __launch_bounds__(kBlock) void kv_store(KvArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t w = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_id_uniform();
  const int64_t t = w / kSplit;
  if (t >= a.rows) return;
  const int half = static_cast<int>(w - t * kSplit);  // kSplit == 2: 0 moves k, 1 moves v
  const uint16_t* ksrc = a.key + t * a.key_stride;
  const uint16_t* vsrc = a.value + t * a.value_stride;
  const int nv = a.vec_per_row;
  const int chunks = (nv + kWave * kUnroll - 1) / (kWave * kUnroll);
  int64_t dst_row = 0;
  for (int c = 0; c < chunks; ++c) {
    u32x4 kv[kUnroll], vv[kUnroll];
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {
      const int v = c * kWave * kUnroll + j * kWave + lane;
      const int vl = v < nv ? v : nv - 1;
      if constexpr (kSplit == 1) {
        kv[j] = load_stream(ksrc + vec_offset(vl, a.vec_per_head, a.key_head_stride, kContig));
        vv[j] = load_stream(vsrc + vec_offset(vl, a.vec_per_head, a.value_head_stride, kContig));
      } else {
        kv[j] = half == 0 ? load_stream(ksrc + vec_offset(vl, a.vec_per_head, a.key_head_stride, kContig))
                          : load_stream(vsrc + vec_offset(vl, a.vec_per_head, a.value_head_stride, kContig));
      }
    }
    load_fence();
    if (c == 0) {
      int64_t page = 0, entry = 0;
      if (!resolve<kSlotForm>(a, t, &page, &entry)) return;
      dst_row = page * a.page_stride + entry * a.entry_stride;
    }
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {
      const int v = c * kWave * kUnroll + j * kWave + lane;
      if (v < nv) {
        const int64_t off = dst_row + vec_offset(v, a.vec_per_head, a.head_stride, kContig);
        if constexpr (kSplit == 1) {
          store_stream(a.k_cache + off, kv[j]);
          store_stream(a.v_cache + off, vv[j]);
        } else {
          store_stream((half == 0 ? a.k_cache : a.v_cache) + off, kv[j]);
        }
      }
    }
  }
}

// Returns MAS_OK with *empty set when there is nothing to store.
int check_common(const KvArgs& a, int64_t num_heads, int64_t head_dim, bool* empty) {
  if (a.rows < 0 || num_heads < 0 || head_dim < 0 || a.num_pages < 0 || a.page_size <= 0) return MAS_ERR_INVALID_VALUE;
  if (head_dim % 8 != 0) return MAS_ERR_UNSUPPORTED;
  if (num_heads * head_dim / 8 > INT32_MAX) return MAS_ERR_UNSUPPORTED;
  *empty = a.rows == 0 || num_heads == 0 || head_dim == 0;
  if (*empty) return MAS_OK;
  if (a.k_cache == nullptr || a.v_cache == nullptr || a.key == nullptr || a.value == nullptr)
    return MAS_ERR_INVALID_VALUE;
  const bool ok = aligned16(a.k_cache) && aligned16(a.v_cache) && aligned16(a.key) && aligned16(a.value) &&
                  a.page_stride % 8 == 0 && a.entry_stride % 8 == 0 && a.head_stride % 8 == 0 &&
                  a.key_stride % 8 == 0 && a.key_head_stride % 8 == 0 && a.value_stride % 8 == 0 &&
                  a.value_head_stride % 8 == 0;
  return ok ? MAS_OK : MAS_ERR_MISALIGNED;
}

// Rows whose heads sit back to back in the source and in the cache entry (NHD caches fed by the
// q/k/v column views) are one contiguous run at both ends: no per-vector head arithmetic.
template <bool kSlotForm>
int launch(const KvArgs& a, hipStream_t s) {
  const int64_t head_dim = 8 * static_cast<int64_t>(a.vec_per_head);
  const bool contiguous = a.key_head_stride == head_dim && a.value_head_stride == head_dim && a.head_stride == head_dim;
  const int64_t blocks = cdiv(a.rows * kSplit, kWavesPerBlock);
  if (blocks > INT32_MAX) return MAS_ERR_UNSUPPORTED;
  if (contiguous)
    hipLaunchKernelGGL((kv_store<kSlotForm, true, kSplit>), dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, s,
                       a);
  else
    hipLaunchKernelGGL((kv_store<kSlotForm, false, kSplit>), dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, s,
                       a);
  return launch_status();
}

}  // namespace
}  // namespace mas

extern "C" int mas_append_paged_kv_cache_bf16(void* k_cache, void* v_cache, int64_t page_stride,
                                              int64_t entry_stride, int64_t head_stride, int64_t num_pages,
                                              int64_t page_size, const void* key, int64_t key_stride,
                                              int64_t key_head_stride, const void* value, int64_t value_stride,
                                              int64_t value_head_stride, const int32_t* batch_indices,
                                              const int32_t* positions, const int32_t* kv_indices,
                                              int64_t num_indices, const int32_t* kv_indptr, int64_t batch,
                                              int64_t rows, int64_t num_heads, int64_t head_dim, uint32_t* err,
                                              hipStream_t stream) {
  using namespace mas;
  KvArgs a{static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), page_stride, entry_stride,
           head_stride, num_pages, page_size, static_cast<const uint16_t*>(key), key_stride, key_head_stride,
           static_cast<const uint16_t*>(value), value_stride, value_head_stride, batch_indices, positions,
           kv_indices, num_indices, kv_indptr, batch, nullptr, rows, static_cast<int>(head_dim / 8),
           static_cast<int>(num_heads * head_dim / 8), err};
  bool empty = false;
  if (const int st = check_common(a, num_heads, head_dim, &empty); st != MAS_OK || empty) return st;
  if (batch_indices == nullptr || positions == nullptr || kv_indptr == nullptr || batch < 0 || num_indices < 0)
    return MAS_ERR_INVALID_VALUE;
  if (num_indices > 0 && kv_indices == nullptr) return MAS_ERR_INVALID_VALUE;
  return launch<false>(a, stream);
}

extern "C" int mas_store_kv_slots_bf16(void* k_cache, void* v_cache, int64_t page_stride, int64_t entry_stride,
                                       int64_t head_stride, int64_t num_pages, int64_t page_size, const void* key,
                                       int64_t key_stride, int64_t key_head_stride, const void* value,
                                       int64_t value_stride, int64_t value_head_stride, const int64_t* slot_mapping,
                                       int64_t rows, int64_t num_heads, int64_t head_dim, uint32_t* err,
                                       hipStream_t stream) {
  using namespace mas;
  KvArgs a{static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), page_stride, entry_stride,
           head_stride, num_pages, page_size, static_cast<const uint16_t*>(key), key_stride, key_head_stride,
           static_cast<const uint16_t*>(value), value_stride, value_head_stride, nullptr, nullptr, nullptr, 0, nullptr,
           0, slot_mapping, rows, static_cast<int>(head_dim / 8), static_cast<int>(num_heads * head_dim / 8), err};
  bool empty = false;
  if (const int st = check_common(a, num_heads, head_dim, &empty); st != MAS_OK || empty) return st;
  if (slot_mapping == nullptr) return MAS_ERR_INVALID_VALUE;
  return launch<true>(a, stream);
}
