// rope_append.hip - RoPE on q/k and the paged KV append of (rotated k, v) in one pass.
//
// The reference runs these back to back on the same token rows
// (miniagentserve/models/devstral2/devstral2.py:163-173): apply_rope_with_cos_sin_cache_inplace
// rotates the q and k column views of the qkv output in place, then append_paged_kv_cache copies
// the rotated k and the v rows into the cache pages. Fused, each k row is read once instead of
// twice and the step launches one kernel instead of two. The results are those of the two calls:
// q and k are rotated in place; k_cache / v_cache receive rotated k and v at
// page = kv_indices[kv_indptr[b] + pos / page_size], entry = pos % page_size. A position outside the
// table leaves that token's q/k unrotated (and the cache receives the unrotated k, as the separate
// calls would); a destination out of range skips the cache write only.
//
// Optional llama-4 query scaling (devstral2.py:175-179): with a q-scale table S (bf16, row k =
// bf16(1 + beta * log1p(k)), built by the caller with the reference's own torch expression), each q
// element becomes bf16(f32(bf16(rope(q))) * f32(S[pos / interval])) - the reference's two roundings,
// so q ends bit-identical to its query_states after line 179. A scale of exactly 1 (every position
// below the interval) leaves the rotated value unchanged and is skipped. A position past the
// scale table leaves q rotated but unscaled and is reported.
//
// Work item: one wavefront = one token x PASSES x (64 / LPH) heads of the list
// [q heads | k heads | v heads], LPH = head_dim / 16 lanes per head. The rotary dimension equals
// head_dim, so a lane's two 16-byte vectors (rotation pairs i and i + D/2, or 8 interleaved pairs)
// cover its part of the head completely and double as the cache row. Head loads are issued first;
// the position, the table row and the destination page (wave-uniform, scalar cache) follow.
#include "device.h"

namespace mas {
namespace {

// One wavefront per workgroup and one pass (64 / LPH heads) per wavefront: measured best on MI355X
// at decode (3.09 us for 64 tokens) and on par or better at prefill (2 and 3 passes, 128-512 threads).
constexpr int kBlock = 64;
constexpr int kWavesPerBlock = kBlock / kWave;

struct FusedArgs {
  uint16_t* q;
  int64_t q_stride, q_head_stride;
  uint16_t* k;
  int64_t k_stride, k_head_stride;
  const uint16_t* v;
  int64_t v_stride, v_head_stride;
  const int32_t* positions;
  const int32_t* batch_indices;
  const float* table;
  int64_t table_stride, table_rows;
  const uint16_t* q_scale;
  int64_t q_scale_rows, q_scale_interval;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t page_stride, entry_stride, head_stride, num_pages, page_size;
  const int32_t* kv_indices;
  int64_t num_indices;
  const int32_t* kv_indptr;
  int64_t batch;
  int64_t rows;
  int num_q_heads, num_kv_heads, groups_per_token;
  uint32_t* err;
};

// Errors set bits in *errbits, reported once at the end of the kernel: a global atomic on a path
// before the index loads would keep the compiler from reading them through the scalar cache (it
// would load them as vectors and wait for every load in flight, the head rows included).
__device__ __forceinline__ bool resolve_page(const FusedArgs& a, int64_t t, int64_t pos, int64_t* dst_row,
                                             uint32_t* errbits) {
  const int64_t b = a.batch_indices[t];
  const bool b_ok = b >= 0 && b < a.batch;
  if (!b_ok || pos < 0) {
    *errbits |= b_ok ? MAS_ERRBIT_POSITION : MAS_ERRBIT_BATCH;
    return false;
  }
  const int64_t end = a.kv_indptr[b + 1];
  const int64_t idx = static_cast<int64_t>(a.kv_indptr[b]) + pos / a.page_size;
  if (idx < 0 || idx >= a.num_indices || idx >= end) {
    *errbits |= MAS_ERRBIT_PAGE;
    return false;
  }
  const int64_t page = a.kv_indices[idx];
  if (page < 0 || page >= a.num_pages) {
    *errbits |= MAS_ERRBIT_PAGE;
    return false;
  }
  *dst_row = page * a.page_stride + (pos % a.page_size) * a.entry_stride;
  return true;
}

template <int LPH, bool kNeox, int PASSES>
__global__ __launch_bounds__(kBlock) void rope_append(FusedArgs a) {
  constexpr int kHeadsPerPass = kWave / LPH;
  constexpr int kHalf = LPH * 8;  // head_dim / 2
  const int lane = threadIdx.x & (kWave - 1);
  const int slot = lane / LPH;
  const int chunk = lane % LPH;
  // Workgroups go to the 8 XCDs round-robin by id; token t's wavefronts all run on XCD t % 8, so
  // its cos/sin row is fetched into one L2 (and tokens 8k apart, the same position in sequences of
  // a multiple of 8 tokens, share it).
  const int64_t xcd = blockIdx.x % kXcds;
  const int64_t work = static_cast<int64_t>(blockIdx.x / kXcds) * kWavesPerBlock + wave_id_uniform();
  const int64_t tx = work / a.groups_per_token;
  const int64_t t = tx * kXcds + xcd;
  if (t >= a.rows) return;
  const int group = static_cast<int>(work - tx * a.groups_per_token);
  const int hq = a.num_q_heads, hkv = a.num_kv_heads;
  const int total = hq + 2 * hkv;

  const int off_a = kNeox ? chunk * 8 : chunk * 16;
  const int off_b = kNeox ? kHalf + chunk * 8 : chunk * 16 + 8;

  const uint16_t* src[PASSES];
  u32x4 va[PASSES], vb[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    int h = (group * PASSES + p) * kHeadsPerPass + slot;
    h = h < total ? h : total - 1;
    src[p] = h < hq ? a.q + t * a.q_stride + h * a.q_head_stride
             : h < hq + hkv ? a.k + t * a.k_stride + (h - hq) * a.k_head_stride
                            : a.v + t * a.v_stride + (h - hq - hkv) * a.v_head_stride;
    va[p] = load_stream(src[p] + off_a);
    vb[p] = load_stream(src[p] + off_b);
  }
  load_fence();

  // Which parts of the head list this wavefront covers (uniform).
  const int first = group * PASSES * kHeadsPerPass;
  const int last = (first + PASSES * kHeadsPerPass < total ? first + PASSES * kHeadsPerPass : total) - 1;
  const bool rotates = first < hq + hkv;
  const bool appends = last >= hq;
  const int64_t pos = a.positions[t];
  bool rope_ok = rotates;
  uint32_t errbits = 0;  // reported at the end (see resolve_page)
  if (rotates && (pos < 0 || pos >= a.table_rows)) {
    if (group == 0) errbits |= MAS_ERRBIT_POSITION;
    rope_ok = false;
  }
  // The table row loads first (they need only the position), then the page lookup, whose scalar
  // loads are waited on one by one while the table rows are in flight; nothing reads the table
  // rows or the head rows until both are issued. The loads are unconditional (row 0 stands in for
  // a bad position and is never used; the host rejects an empty table), so no branch joins on them.
  const float* trow = a.table + (rope_ok ? pos : 0) * a.table_stride + chunk * 8;
  const f32x4 c0 = load_cached_f4(trow);
  const f32x4 c1 = load_cached_f4(trow + 4);
  const f32x4 s0 = load_cached_f4(trow + kHalf);
  const f32x4 s1 = load_cached_f4(trow + kHalf + 4);
  load_fence();
  int64_t dst_row = 0;
  const bool cache_ok = appends && resolve_page(a, t, pos, &dst_row, &errbits);
  load_fence();
  float cs[8], sn[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    cs[i] = c0[i];
    cs[4 + i] = c1[i];
    sn[i] = s0[i];
    sn[4 + i] = s1[i];
  }
  // After the table loads: the 2-byte scale entry is a vector load, and waiting for it waits for
  // every load issued before it, all of which the rotation needs anyway.
  float q_scale = 1.0f;
  if (a.q_scale != nullptr && rope_ok && first < hq) {
    const int64_t row = pos / a.q_scale_interval;
    if (row < a.q_scale_rows) {
      q_scale = bf16_lo(a.q_scale[row]);
    } else {
      errbits |= MAS_ERRBIT_POSITION;
    }
  }

#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int h = (group * PASSES + p) * kHeadsPerPass + slot;
    if (h >= total) continue;
    const bool is_v = h >= hq + hkv;
    const bool is_q = h < hq;
    u32x4 oa = va[p], ob = vb[p];
    if (!is_v && rope_ok) {
      float xa[8], xb[8], ya[8], yb[8];
      unpack8(va[p], xa);
      unpack8(vb[p], xb);
      if constexpr (kNeox) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          ya[i] = xa[i] * cs[i] - xb[i] * sn[i];
          yb[i] = xb[i] * cs[i] + xa[i] * sn[i];
        }
      } else {
        float x[16], y[16];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          x[i] = xa[i];
          x[8 + i] = xb[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          y[2 * i] = x[2 * i] * cs[i] - x[2 * i + 1] * sn[i];
          y[2 * i + 1] = x[2 * i + 1] * cs[i] + x[2 * i] * sn[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          ya[i] = y[i];
          yb[i] = y[8 + i];
        }
      }
      oa = pack8(ya);
      ob = pack8(yb);
      if (is_q && q_scale != 1.0f) {
        float za[8], zb[8];
        unpack8(oa, za);
        unpack8(ob, zb);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          za[i] *= q_scale;
          zb[i] *= q_scale;
        }
        oa = pack8(za);
        ob = pack8(zb);
      }
      uint16_t* dst = const_cast<uint16_t*>(src[p]);  // q or k rows, rotated in place
      store_stream(dst + off_a, oa);
      store_stream(dst + off_b, ob);
    }
    if (!is_q && cache_ok) {
      const int kvh = is_v ? h - hq - hkv : h - hq;
      uint16_t* dst = (is_v ? a.v_cache : a.k_cache) + dst_row + kvh * a.head_stride;
      store_stream(dst + off_a, oa);
      store_stream(dst + off_b, ob);
    }
  }
  if (errbits != 0 && lane == 0) report(a.err, errbits);
}

template <int LPH, bool kNeox, int PASSES>
int launch(FusedArgs a, hipStream_t s) {
  constexpr int kHeadsPerWave = (kWave / LPH) * PASSES;
  a.groups_per_token = static_cast<int>(cdiv(a.num_q_heads + 2 * a.num_kv_heads, kHeadsPerWave));
  const int64_t blocks = kXcds * cdiv(cdiv(a.rows, kXcds) * a.groups_per_token, kWavesPerBlock);
  if (blocks > INT32_MAX) return MAS_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((rope_append<LPH, kNeox, PASSES>), dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, s, a);
  return launch_status();
}

template <int LPH>
int dispatch(const FusedArgs& a, bool neox, hipStream_t s) {
  return neox ? launch<LPH, true, 1>(a, s) : launch<LPH, false, 1>(a, s);
}

}  // namespace
}  // namespace mas

extern "C" int mas_rope_append_paged_kv_cache_bf16(
    void* q, int64_t q_stride, int64_t q_head_stride, int64_t num_q_heads, void* k, int64_t k_stride,
    int64_t k_head_stride, const void* v, int64_t v_stride, int64_t v_head_stride, int64_t num_kv_heads,
    const int32_t* positions, const float* table, int64_t table_stride, int64_t table_rows, int64_t rows,
    int64_t head_dim, int is_neox, void* k_cache, void* v_cache, int64_t page_stride, int64_t entry_stride,
    int64_t head_stride, int64_t num_pages, int64_t page_size, const int32_t* batch_indices,
    const int32_t* kv_indices, int64_t num_indices, const int32_t* kv_indptr, int64_t batch,
    const void* q_scale_table, int64_t q_scale_rows, int64_t q_scale_interval, uint32_t* err, hipStream_t stream) {
  using namespace mas;
  if (rows < 0 || num_q_heads < 0 || num_kv_heads < 0 || head_dim <= 0 || table_rows < 0 || num_pages < 0 ||
      page_size <= 0 || batch < 0 || num_indices < 0)
    return MAS_ERR_INVALID_VALUE;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256 && head_dim != 512)
    return MAS_ERR_UNSUPPORTED;
  if (num_q_heads + 2 * num_kv_heads > INT32_MAX) return MAS_ERR_UNSUPPORTED;
  if (rows == 0 || num_q_heads + num_kv_heads == 0) return MAS_OK;
  if (table_rows == 0) return MAS_ERR_INVALID_VALUE;  // every token's row is loaded, even a bad position's
  if (positions == nullptr || table == nullptr || batch_indices == nullptr || kv_indptr == nullptr)
    return MAS_ERR_INVALID_VALUE;
  if ((num_q_heads > 0 && q == nullptr) || (num_kv_heads > 0 && (k == nullptr || v == nullptr || k_cache == nullptr ||
                                                                  v_cache == nullptr)))
    return MAS_ERR_INVALID_VALUE;
  if (num_indices > 0 && kv_indices == nullptr) return MAS_ERR_INVALID_VALUE;
  if (table_stride < head_dim && table_rows > 1) return MAS_ERR_INVALID_VALUE;
  if (q_scale_table != nullptr && (q_scale_rows < 1 || q_scale_interval < 1)) return MAS_ERR_INVALID_VALUE;
  const bool q_ok = num_q_heads == 0 || (aligned16(q) && q_stride % 8 == 0 && q_head_stride % 8 == 0);
  const bool kv_ok = num_kv_heads == 0 ||
                     (aligned16(k) && aligned16(v) && aligned16(k_cache) && aligned16(v_cache) && k_stride % 8 == 0 &&
                      k_head_stride % 8 == 0 && v_stride % 8 == 0 && v_head_stride % 8 == 0 &&
                      page_stride % 8 == 0 && entry_stride % 8 == 0 && head_stride % 8 == 0);
  if (!q_ok || !kv_ok || !aligned16(table) || table_stride % 4 != 0 ||
      (reinterpret_cast<uintptr_t>(q_scale_table) & 1u) != 0)
    return MAS_ERR_MISALIGNED;
  FusedArgs a{static_cast<uint16_t*>(q), q_stride, q_head_stride, static_cast<uint16_t*>(k), k_stride, k_head_stride,
              static_cast<const uint16_t*>(v), v_stride, v_head_stride, positions, batch_indices, table, table_stride,
              table_rows, static_cast<const uint16_t*>(q_scale_table), q_scale_rows, q_scale_interval, static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), page_stride, entry_stride,
              head_stride, num_pages, page_size, kv_indices, num_indices, kv_indptr, batch, rows,
              static_cast<int>(num_q_heads), static_cast<int>(num_kv_heads), 0, err};
  const bool neox = is_neox != 0;
  switch (head_dim) {
    case 32: return dispatch<2>(a, neox, stream);
    case 64: return dispatch<4>(a, neox, stream);
    case 128: return dispatch<8>(a, neox, stream);
    case 256: return dispatch<16>(a, neox, stream);
    case 512: return dispatch<32>(a, neox, stream);
    default: return MAS_ERR_UNSUPPORTED;
  }
}
