// attention.hip - paged decode attention over the NHD KV cache the store kernels write.
//
// Semantics: flashinfer.decode.trtllm_batch_decode_with_kv_cache as called at
// miniagentserve/models/devstral2/devstral2.py:184-196. For decode row b and query head h (kv head
// h / G, G = Hq / Hk), over the positions p < seq_lens[b], whose key and value rows sit at
// page = block_tables[b, p / page_size], entry = p % page_size (the layout written at :170-173):
//   s_p = bmm1_scale * (q[b, h] . k_p),   out[b, h] = bmm2_scale * sum_p softmax(s)_p * v_p,
// in fp32 from the bf16 inputs, rounded once to bf16.
//
// Split-KV in two kernels:
//  1. decode_attn_split - one wavefront per (kv head, split of split_len positions, row), kv heads
//     adjacent in the grid so that the 256-byte slices of each 2 KB position block are read close
//     together. The split is walked in steps of 32 positions with the next step's
//     key and value loads in flight: Q.K^T on MFMA (v_mfma_f32_16x16x32_bf16; the kv head's G
//     query heads are the rows of A, zero-padded to 16; 16 positions per tile are the
//     columns of B, read straight from the cache rows), an online softmax in the MFMA result
//     layout, then P.V on MFMA with P and the value rows passed through LDS (read back
//     transposed). The split's running (max, sum) and unnormalised O go to the caller's workspace.
//  2. decode_attn_combine - one wavefront per (query head, row) merges the splits and writes bf16.
// A row whose positions fit one split skips both steps' partials: the split kernel writes its output
// straight from the registers (as merging one split gives) and the combine kernel leaves it alone.
// Scores live in the log2 domain (bmm1_scale * log2 e folded in), so every exponential is one
// v_exp_f32. A position whose page id is out of range is skipped (MAS_ERRBIT_PAGE); seq_lens past
// the block table's reach is clamped to it (MAS_ERRBIT_POSITION); a row with no position gets zeros.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "device.h"

namespace mas {
namespace {

constexpr int kChunk = 256;          // positions per chunk
constexpr float kNegInf = -__builtin_huge_valf();

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_stride, q_head_stride;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int64_t page_stride, entry_stride, head_stride, num_pages;
  const int32_t* block_tables;
  int64_t bt_stride, max_blocks;
  const int32_t* seq_lens;
  int hq, hk, group, log2_page, max_splits;
  int split_len;     // longest split: 64, 128, or a multiple of the 256-position chunk
  int row_target;    // small grids: splits wanted per row (the GPU's SIMDs over rows x kv heads)
  float scale_log2;  // bmm1_scale * log2(e)
  float out_scale;   // bmm2_scale
  float* part_o;     // [batch][hq][max_splits][D]
  float* part_ml;    // [batch][hq][max_splits][2]: running max (log2 domain), sum
  void* out;                // bf16, or fp8 e4m3fn codes when out_fp8
  int64_t out_stride, out_head_stride;
  int out_fp8;              // out = e4m3fn(clamp(bf16(O) / quant scale, +-448)): the o_proj input quantize
  const float* quant_scale_dev;
  float quant_scale_host;
  uint32_t* err;
};


// seq_lens[b] clamped to [0, max_blocks * page_size].
__device__ __forceinline__ int kv_len(const DecodeArgs& a, int b) {
  const int64_t L = a.seq_lens[b];
  const int64_t cap = a.max_blocks << a.log2_page;
  return static_cast<int>(L < 0 ? 0 : (L > cap ? cap : L));
}

// The split length of a row of L positions, chosen from the row's own length: 256 positions, or,
// in small grids (4+ splits wanted per row), 128 or 64 when the row's share L / row_target is that
// short; at most split_len, and at least the fewest 64-position units that keep the row within the
// grid's max_splits. The grid is sized from the block table's reach, which can far exceed the rows
// (a graph captured for the longest context): a row then still gets splits as short as its own
// length calls for.
__device__ __forceinline__ int row_split_len(const DecodeArgs& a, int L) {
  // large grids: the host's split for rows of 4+ such splits, 256 positions for shorter rows
  int len = L >= 4 * a.split_len ? a.split_len : 256;
  if (a.row_target >= 4) len = L <= 64 * a.row_target ? 64 : (L <= 128 * a.row_target ? 128 : 256);
  len = min(len, a.split_len);
  if (L > len * a.max_splits) len = 64 * (((L + 63) / 64 + a.max_splits - 1) / a.max_splits);  // within the grid
  return len;
}

// The output element(s) of row b, query head h, starting at head-dim column `col`: bf16 y, or its
// fp8 quantize (the o_proj input quantize of devstral2.py:93-95,110-111) with out_fp8.
template <int N>
__device__ __forceinline__ void store_output(const DecodeArgs& a, int b, int h, int col, const float (&y)[N]) {
  const int64_t at = b * a.out_stride + h * a.out_head_stride + col;
  uint32_t w[(N + 1) / 2];  // bf16 pairs
  if constexpr (N == 1) {
    w[0] = pack_bf16x2(y[0], 0.f);
  } else {
#pragma unroll
    for (int e = 0; e < N / 2; ++e) w[e] = pack_bf16x2(y[2 * e], y[2 * e + 1]);
  }
  if (a.out_fp8) {
    const float qs = a.quant_scale_dev != nullptr ? *a.quant_scale_dev : a.quant_scale_host;
    const float rcp = 1.0f / qs;
    float qv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ee = e < N ? e : 0;
      const float v = (ee & 1) ? bf16_hi(w[ee / 2]) : bf16_lo(w[ee / 2]);
      qv[e] = div_by_scale(v, qs, rcp);
    }
    const uint32_t codes = fp8x4_saturate_encode(qv[0], qv[1], qv[2], qv[3]);
    uint8_t* dst = static_cast<uint8_t*>(a.out) + at;
    if constexpr (N == 1) {
      dst[0] = static_cast<uint8_t>(codes);
    } else if constexpr (N == 2) {
      *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(codes);
    } else {
      *reinterpret_cast<uint32_t*>(dst) = codes;
    }
  } else {
    uint16_t* dst = static_cast<uint16_t*>(a.out) + at;
    if constexpr (N == 1) {
      dst[0] = static_cast<uint16_t>(w[0]);
    } else if constexpr (N == 2) {
      *reinterpret_cast<uint32_t*>(dst) = w[0];
    } else {
      *reinterpret_cast<u32x2*>(dst) = u32x2{w[0], w[1]};
    }
  }
}

// Key loads go through the cache hierarchy: a wavefront's load instruction reads 64 bytes of each
// of 16 key rows, so the other half of each 128-byte line comes with the next instruction. Value
// loads read whole rows and bypass it (non-temporal).
__device__ __forceinline__ u32x4 attn_load_k(const uint16_t* p) { return load_cached(p); }
__device__ __forceinline__ u32x4 attn_load_v(const uint16_t* p) { return load_stream(p); }

// One wavefront per workgroup of the split kernel (kv heads of one position block in consecutive
// workgroups); LDS traffic is ordered within the wavefront only.
constexpr int kAttnWaves = 1;
// Wavefronts per SIMD the split kernel's registers are capped for (two load buffers of a step each).
constexpr int kAttnMinWaves = 2;

// Orders this wavefront's LDS writes before its later reads (and reads before later writes).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// One step: 32 positions - two MFMA tiles of keys, and the value rows in the 16-byte layout.
template <int D>
struct StepLoads {
  static constexpr int KS = D / 32;
  static constexpr int VPS = 32 / (64 / (D / 8));  // value rows per lane per step
  u32x4 k[2][KS];
  u32x4 v[VPS];
  bool kok[2];
  bool vok[VPS];
};

// Issues the key and value loads of the step at position ps. With kBig (pages of at least 256
// positions) the step lies in one page, whose id `page_u` the caller read as a scalar; otherwise
// page ids come from pg (the chunk's block-table entries in LDS, first = the chunk's first block
// index). Rows of masked positions (past `end`, or with a page id outside the cache) are loaded
// from row 0 of page 0 and flagged; `bad` collects out-of-range page ids of real positions.
template <int D, bool kBig>
__device__ __forceinline__ void issue_step(const DecodeArgs& a, StepLoads<D>& st, int ps, int end, int kvh,
                                           const int32_t* pg, int first, int32_t page_u, int n, int r, int pv_d,
                                           int pv_grp, bool& bad) {
  constexpr int PPW = 64 / (D / 8);
  const int mask = (1 << a.log2_page) - 1;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int p = ps + 16 * t + n;
    const bool valid = p < end;
    const int pc = valid ? p : end - 1;
    const int32_t page = kBig ? page_u : pg[(pc >> a.log2_page) - first];
    const bool ok = page >= 0 && page < a.num_pages;
    bad |= valid && !ok;
    st.kok[t] = valid && ok;
    if constexpr (kBig) {
      // the page's base is wave-uniform; the in-page byte offset fits 32 bits (checked at launch)
      const char* base = reinterpret_cast<const char*>(a.k_cache + (ok ? static_cast<int64_t>(page) : 0) * a.page_stride +
                                                       kvh * a.head_stride);
      const uint32_t off = 2u * (static_cast<uint32_t>(pc & mask) * static_cast<uint32_t>(a.entry_stride) + 8u * r);
#pragma unroll
      for (int ks = 0; ks < StepLoads<D>::KS; ++ks)
        st.k[t][ks] = attn_load_k(reinterpret_cast<const uint16_t*>(base + (off + 64u * ks)));
    } else {
      const int64_t row = (ok ? static_cast<int64_t>(page) : 0) * a.page_stride +
                          static_cast<int64_t>(pc & mask) * a.entry_stride + kvh * a.head_stride;
#pragma unroll
      for (int ks = 0; ks < StepLoads<D>::KS; ++ks) st.k[t][ks] = attn_load_k(a.k_cache + row + 32 * ks + 8 * r);
    }
  }
#pragma unroll
  for (int u = 0; u < StepLoads<D>::VPS; ++u) {
    const int p = ps + PPW * u + pv_grp;
    const bool valid = p < end;
    const int pc = valid ? p : end - 1;
    const int32_t page = kBig ? page_u : pg[(pc >> a.log2_page) - first];
    const bool ok = page >= 0 && page < a.num_pages;
    st.vok[u] = valid && ok;
    if constexpr (kBig) {
      const char* base = reinterpret_cast<const char*>(a.v_cache + (ok ? static_cast<int64_t>(page) : 0) * a.page_stride +
                                                       kvh * a.head_stride);
      const uint32_t off = 2u * (static_cast<uint32_t>(pc & mask) * static_cast<uint32_t>(a.entry_stride) + 8u * pv_d);
      st.v[u] = attn_load_v(reinterpret_cast<const uint16_t*>(base + off));
    } else {
      const int64_t row = (ok ? static_cast<int64_t>(page) : 0) * a.page_stride +
                          static_cast<int64_t>(pc & mask) * a.entry_stride + kvh * a.head_stride;
      st.v[u] = attn_load_v(a.v_cache + row + 8 * pv_d);
    }
  }
}

// One wavefront per (kv head, split, row); a split is split_len positions (whole chunks of 256, or
// 64 / 128 for small grids),
// walked in steps of 32 with the next step's loads in flight (head_dim <= 128). Per step:
// Q.K^T on MFMA -> online softmax (the running max, sum and O rescale live in the MFMA result
// layout: lane (n, r) holds heads 4r..4r+3) -> P and the value rows through LDS, where they are
// read back transposed as MFMA operands -> P.V on MFMA (16x16x32: the 32 positions of the step are
// the reduction). P enters as two bf16 terms, hi = bf16(P) and lo = bf16(P - hi), two MFMAs per
// tile, so it keeps ~16 significant bits (one bf16 term alone rounds it to 8). O stays in
// 4 * D / 16 accumulator registers whatever the group size.
template <int GP, int D, bool kBig>
__global__ __launch_bounds__(64 * kAttnWaves, D <= 128 ? kAttnMinWaves : 1) void decode_attn_split(DecodeArgs a) {
  constexpr int KS = D / 32;
  constexpr int DT = D / 16;               // MFMA tiles over the head dim for P.V
  constexpr int LPP = D / 8;               // value-row layout: lanes per row
  constexpr int PPW = 64 / LPP;            // value-row layout: rows per wavefront load
  constexpr int kStep = 32;
  constexpr int VPS = kStep / PPW;
  constexpr int RG = GP / 4;
  constexpr bool kPrefetch = D <= 128;
  constexpr int VROW = D + 16;             // bf16 per LDS value row: the 4 rows of a transposing read
                                           // start 8 banks apart
  constexpr int PROW = kStep + 8;          // bf16 per LDS P row: 16-byte aligned, conflict-free reads
  constexpr int kChunkPages = 257;         // block-table entries one 256-position chunk can touch
  __shared__ __align__(16) uint16_t v_lds_all[kAttnWaves][kStep * VROW];
  __shared__ __align__(16) uint16_t p_lds_all[kAttnWaves][2][16 * PROW];  // P as hi and lo bf16 terms
  __shared__ int32_t pg_lds_all[kAttnWaves][kChunkPages];

  const int lane = threadIdx.x & 63;
  const int wave = wave_id_uniform();
  const int kvh = blockIdx.x * kAttnWaves + wave;  // kv heads adjacent: one 2 KB position block
  const int split = blockIdx.y, b = blockIdx.z;
  if (kvh >= a.hk) return;
  uint16_t* v_lds = v_lds_all[wave];
  uint16_t(*p_lds)[16 * PROW] = p_lds_all[wave];
  int32_t* pg_lds = pg_lds_all[wave];
  const int L = kv_len(a, b);
  const int split_len = row_split_len(a, L);
  const int start = split * split_len;
  if (start >= L) return;
  const int end = min(start + split_len, L);
  const int G = a.group;
  const int n = lane & 15, r = lane >> 4;
  const int pv_d = lane % LPP, pv_grp = lane / LPP;

  bf16x8 qa[KS];
  {
    const int g = n < G ? n : 0;
    const uint16_t* qrow = a.q + b * a.q_stride + static_cast<int64_t>(kvh * G + g) * a.q_head_stride + 8 * r;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 v = load_cached(qrow + 32 * ks);
      if (n >= G) v = u32x4{0u, 0u, 0u, 0u};
      qa[ks] = __builtin_bit_cast(bf16x8, v);
    }
  }

  // The block-table entries of the chunk starting at cs, into LDS (clamped to the table).
  const int32_t* bt = a.block_tables + b * a.bt_stride;
  auto load_pages = [&](int cs) {
    const int first = cs >> a.log2_page;
    const int last = min((cs + kChunk - 1) >> a.log2_page, static_cast<int>(a.max_blocks) - 1);
    for (int i = lane; i <= last - first; i += 64) pg_lds[i] = bt[first + i];
    wave_lds_sync();
    return first;
  };

  float m_run[4], l_run[4];
  f32x4 acc[DT];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = kNegInf;
    l_run[i] = 0.f;
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nsteps = (end - start + kStep - 1) / kStep;
  int first = kBig ? 0 : load_pages(start);

  // One step over the loads of `c`: scores, online softmax, P.V.
  auto compute = [&](const StepLoads<D>& c) {
    // ---- scores (lane: heads 4r+i at positions ps + 16 t + n)
    f32x4 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4 acc_s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        acc_s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[ks], __builtin_bit_cast(bf16x8, c.k[t][ks]), acc_s, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) s[t][j] = c.kok[t] ? acc_s[j] * a.scale_log2 : kNegInf;
    }

    // ---- online softmax; O (same layout) rescaled by alpha
    wave_lds_sync();  // the previous step's LDS reads are done
    float alpha[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float mx = row_max16(fmaxf(s[0][j], s[1][j]));
      const float m_new = fmaxf(m_run[j], mx);
      const float m_use = m_new == kNegInf ? 0.f : m_new;
      alpha[j] = __builtin_amdgcn_exp2f(m_run[j] - m_use);
      s[0][j] = __builtin_amdgcn_exp2f(s[0][j] - m_use);
      s[1][j] = __builtin_amdgcn_exp2f(s[1][j] - m_use);
      l_run[j] = l_run[j] * alpha[j] + row_sum16(s[0][j] + s[1][j]);
      m_run[j] = m_new;
    }
    // O is rescaled only when some row's max moved (alpha == 1 leaves it unchanged anyway)
    if (__builtin_amdgcn_ballot_w64(alpha[0] != 1.f || alpha[1] != 1.f || alpha[2] != 1.f || alpha[3] != 1.f)) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt][j] *= alpha[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (r < RG) {
        const uint32_t hi = pack_bf16x2(s[0][j], s[1][j]);
        const uint32_t lo = pack_bf16x2(s[0][j] - bf16_lo(hi), s[1][j] - bf16_hi(hi));
        uint16_t* row_hi = p_lds[0] + (4 * r + j) * PROW;
        uint16_t* row_lo = p_lds[1] + (4 * r + j) * PROW;
        row_hi[n] = static_cast<uint16_t>(hi);
        row_hi[16 + n] = static_cast<uint16_t>(hi >> 16);
        row_lo[n] = static_cast<uint16_t>(lo);
        row_lo[16 + n] = static_cast<uint16_t>(lo >> 16);
      }
    }
    // value rows into LDS (masked rows zeroed)
#pragma unroll
    for (int u = 0; u < VPS; ++u) {
      const u32x4 v = c.vok[u] ? c.v[u] : u32x4{0u, 0u, 0u, 0u};
      uint16_t* dst = v_lds + (PPW * u + pv_grp) * VROW + 8 * pv_d;
      *reinterpret_cast<u32x2*>(dst) = u32x2{v[0], v[1]};
      *reinterpret_cast<u32x2*>(dst + 4) = u32x2{v[2], v[3]};
    }
    wave_lds_sync();

    // ---- P.V: A = P[head][32 positions], B = V[32 positions][16 of the head dim], per dim tile
    const bf16x8 pa_hi = *reinterpret_cast<const bf16x8*>(p_lds[0] + n * PROW + 8 * r);
    const bf16x8 pa_lo = *reinterpret_cast<const bf16x8*>(p_lds[1] + n * PROW + 8 * r);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      // lane (n, r): positions 8r .. 8r + 7 of head-dim column 16 dt + n, as P's operand holds them
      const i16x4 lo = read_column4(v_lds, VROW, 8 * r, 16 * dt, n);
      const i16x4 hi = read_column4(v_lds, VROW, 8 * r + 4, 16 * dt, n);
      const bf16x8 vb = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa_lo, vb, acc[dt], 0, 0, 0);
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa_hi, vb, acc[dt], 0, 0, 0);
    }
  };
  // Issues step j's loads. Small pages: the chunk's block-table entries go to LDS when step j opens
  // a chunk. Big pages: the step's page id is one scalar load, so no wait on the vector loads in
  // flight is needed to find it.
  bool bad = false;
  auto issue = [&](StepLoads<D>& dst, int j) {
    const int ps = start + j * kStep;
    if constexpr (kBig) {
      issue_step<D, true>(a, dst, ps, end, kvh, nullptr, 0, bt[ps >> a.log2_page], n, r, pv_d, pv_grp, bad);
    } else {
      if (j > 0 && (j & 7) == 0) first = load_pages(ps);
      issue_step<D, false>(a, dst, ps, end, kvh, pg_lds, first, 0, n, r, pv_d, pv_grp, bad);
    }
  };

  if constexpr (kPrefetch) {
    // Two load buffers used in turn (no copy between them) and no branch around a load inside the
    // loop, so computing a step waits only for its own loads while the next step's are in flight.
    StepLoads<D> ld0, ld1;
    issue(ld0, 0);
    int i = 0;
    for (; i + 2 < nsteps; i += 2) {
      issue(ld1, i + 1);
      compute(ld0);
      issue(ld0, i + 2);
      compute(ld1);
    }
    if (i + 1 < nsteps) {
      issue(ld1, i + 1);
      compute(ld0);
      compute(ld1);
    } else {
      compute(ld0);
    }
  } else {
    StepLoads<D> cur;
    for (int i = 0; i < nsteps; ++i) {
      issue(cur, i);
      compute(cur);
    }
  }
  if (__builtin_amdgcn_ballot_w64(bad) != 0 && lane == 0) report(a.err, MAS_ERRBIT_PAGE);

  if (L <= split_len) {
    // The row's only split: its output is O / l * bmm2_scale, what merging one split gives.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int g = 4 * r + j;
      if (g < G) {
        const float sc = l_run[j] > 0.f ? a.out_scale / l_run[j] : 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const float y[1] = {acc[dt][j] * sc};
          store_output<1>(a, b, kvh * G + g, 16 * dt + n, y);
        }
      }
    }
    return;
  }

  // ---- partials. Lane (n, r) holds O[head 4r+j][16 dt + n]: the rows go through LDS (the value
  // buffer, free after the last step) so that each lane stores 16-byte pieces of whole head rows,
  // a few wide stores per wavefront in place of 4 * DT scattered 4-byte ones.
  constexpr int OROW = D + 4;  // floats per LDS row: the 4 lane groups' rows start 16 banks apart
  static_assert(16 * OROW * 4 <= kStep * VROW * 2, "partial rows fit the value buffer");
  float* o_lds = reinterpret_cast<float*>(v_lds);
  wave_lds_sync();  // the last step's value reads are done
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o_lds[(4 * r + j) * OROW + 16 * dt + n] = acc[dt][j];
  wave_lds_sync();
  const int64_t base = (static_cast<int64_t>(b) * a.hq + kvh * G) * a.max_splits + split;
  constexpr int kVecs = D / 4;  // 16-byte pieces per head row
#pragma unroll
  for (int u = 0; u < GP * kVecs / 64; ++u) {
    const int idx = 64 * u + lane;
    const int g = idx / kVecs, c = idx % kVecs;
    if (g < G) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(o_lds + g * OROW + 4 * c);
      // non-temporal: the rows are read once, by the merge, and plain stores in the middle of the
      // key/value stream cost 1.7-2% of the call on MI355X (64 rows up to 8192 positions)
      __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(a.part_o + (base + static_cast<int64_t>(g) * a.max_splits) * D +
                                                              4 * c));
    }
  }
  // (max, sum) of head 4r + n from the lanes n < 4 (every lane of a 16-lane group holds its 4 heads')
  const int jn = n & 3;
  const float m_sel = jn == 0 ? m_run[0] : jn == 1 ? m_run[1] : jn == 2 ? m_run[2] : m_run[3];
  const float l_sel = jn == 0 ? l_run[0] : jn == 1 ? l_run[1] : jn == 2 ? l_run[2] : l_run[3];
  if (n < 4 && 4 * r + n < G)
    *reinterpret_cast<f32x2*>(a.part_ml + (base + static_cast<int64_t>(4 * r + n) * a.max_splits) * 2) =
        f32x2{m_sel, l_sel};
}

// Max over the 64 lanes of a wavefront.
__device__ __forceinline__ float wave_max(float v) {
  v = row_max16(v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// One wavefront per (query head, row): lane s reads split s's (max, sum) (64 splits per pass), the
// weights are broadcast with readlane, and each lane accumulates D / 64 head-dim elements.
template <int D>
__global__ __launch_bounds__(64) void decode_attn_combine(DecodeArgs a) {
  constexpr int DPL = D / 64;  // head-dim elements per lane
  const int lane = threadIdx.x;
  const int h = blockIdx.x, b = blockIdx.y;
  const int64_t raw = a.seq_lens[b];
  const int64_t cap = a.max_blocks << a.log2_page;
  // reported at the end: a global atomic here would turn the loads below into waits on every load
  const bool len_bad = raw < 0 || raw > cap;
  const int L = static_cast<int>(raw < 0 ? 0 : (raw > cap ? cap : raw));
  const int split_len = row_split_len(a, L);
  const int nsplit = (L + split_len - 1) / split_len;
  if (nsplit == 1) {  // the split kernel wrote this row's output
    if (len_bad && h == 0 && lane == 0) report(a.err, MAS_ERRBIT_POSITION);
    return;
  }
  const int64_t base = (static_cast<int64_t>(b) * a.hq + h) * a.max_splits;
  float acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) acc[e] = 0.f;
  float lsum = 0.f;
  constexpr int kOneRound = 32;
  if (nsplit <= kOneRound) {
    // Every load in one round trip: lane s reads split s's (max, sum), and all splits' partial O
    // rows are loaded (indices past the last split clamped to it, weighted 0) before the max is
    // known. Same weights and summation order as the general path below.
    const int sl = lane < nsplit ? lane : (nsplit > 0 ? nsplit - 1 : 0);
    const f32x2 ml = *reinterpret_cast<const f32x2*>(a.part_ml + (base + sl) * 2);
    const float* po = a.part_o + base * D + DPL * lane;
    float v[kOneRound][DPL];
#pragma unroll
    for (int u = 0; u < kOneRound; ++u) {
      const int su = u < nsplit ? u : sl;
#pragma unroll
      for (int e = 0; e < DPL; ++e) v[u][e] = po[su * D + e];
    }
    const float m_lane = lane < nsplit ? ml[0] : kNegInf;
    const float mx = wave_max(m_lane);
    if (mx != kNegInf) {
      const float wgt = lane < nsplit ? __builtin_amdgcn_exp2f(m_lane - mx) : 0.f;
      lsum = wgt * ml[1];
#pragma unroll
      for (int u = 0; u < kOneRound; ++u) {
        if (u < nsplit) {
          const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wgt), u));
#pragma unroll
          for (int e = 0; e < DPL; ++e) acc[e] = __builtin_fmaf(wj, v[u][e], acc[e]);
        }
      }
    }
  } else {
    float mx = kNegInf;
    for (int s = lane; s < nsplit; s += 64) mx = fmaxf(mx, a.part_ml[(base + s) * 2]);
    mx = wave_max(mx);
    if (mx != kNegInf) {
      for (int s0 = 0; s0 < nsplit; s0 += 64) {
        float wgt = 0.f;
        if (s0 + lane < nsplit) {
          const f32x2 ml = *reinterpret_cast<const f32x2*>(a.part_ml + (base + s0 + lane) * 2);
          wgt = __builtin_amdgcn_exp2f(ml[0] - mx);
          lsum = __builtin_fmaf(wgt, ml[1], lsum);
        }
        const int cnt = min(64, nsplit - s0);
        const float* po = a.part_o + (base + s0) * D + DPL * lane;
        // eight splits' partials loaded before any is used, so their loads are in flight together
        constexpr int kU = 8;
        int j = 0;
        for (; j + kU <= cnt; j += kU) {
          float v[kU][DPL];
#pragma unroll
          for (int u = 0; u < kU; ++u)
#pragma unroll
            for (int e = 0; e < DPL; ++e) v[u][e] = po[(j + u) * D + e];
#pragma unroll
          for (int u = 0; u < kU; ++u) {
            const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wgt), j + u));
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[e] = __builtin_fmaf(wj, v[u][e], acc[e]);
          }
        }
        for (; j < cnt; ++j) {
          const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wgt), j));
#pragma unroll
          for (int e = 0; e < DPL; ++e) acc[e] = __builtin_fmaf(wj, po[j * D + e], acc[e]);
        }
      }
    }
  }
  if (len_bad && h == 0 && lane == 0) report(a.err, MAS_ERRBIT_POSITION);
  const float denom = wave_sum(lsum);
  const float scale = denom > 0.f ? a.out_scale / denom : 0.f;
  float y[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) y[e] = acc[e] * scale;
  store_output<DPL>(a, b, h, DPL * lane, y);
}

template <int GP, int D>
int launch(const DecodeArgs& a, int64_t batch, int64_t hk, hipStream_t s) {
  const dim3 grid(static_cast<uint32_t>(cdiv(hk, kAttnWaves)), static_cast<uint32_t>(a.max_splits),
                  static_cast<uint32_t>(batch));
  // Pages of at least one chunk: every 32-position step lies in one page, addressed from its base
  // with 32-bit byte offsets (the largest in-page offset is checked here).
  const int64_t page_size = int64_t{1} << a.log2_page;
  const int64_t in_page = 2 * ((page_size - 1) * a.entry_stride + D);
  if (page_size >= kChunk && in_page <= INT32_MAX)
    hipLaunchKernelGGL((decode_attn_split<GP, D, true>), grid, dim3(64 * kAttnWaves), 0, s, a);
  else
    hipLaunchKernelGGL((decode_attn_split<GP, D, false>), grid, dim3(64 * kAttnWaves), 0, s, a);
  if (const int st = launch_status(); st != MAS_OK) return st;
  hipLaunchKernelGGL((decode_attn_combine<D>), dim3(static_cast<uint32_t>(a.hq), static_cast<uint32_t>(batch)),
                     dim3(64), 0, s, a);
  return launch_status();
}

template <int D>
int dispatch_group(const DecodeArgs& a, int64_t batch, int64_t hk, hipStream_t s) {
  if (a.group <= 4) return launch<4, D>(a, batch, hk, s);
  if (a.group <= 8) return launch<8, D>(a, batch, hk, s);
  if (a.group <= 12) return launch<12, D>(a, batch, hk, s);
  return launch<16, D>(a, batch, hk, s);
}

}  // namespace
}  // namespace mas

namespace mas {
namespace {
// Workspace bytes of the partials: (max, sum) and an unnormalised O row per (row, query head, split).
int64_t decode_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t splits) {
  return batch * num_q_heads * (splits > 0 ? splits : 1) * (head_dim + 2) * 4;
}
}  // namespace
}  // namespace mas

extern "C" int64_t mas_paged_decode_attention_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t head_dim,
                                                               int64_t max_blocks, int64_t page_size,
                                                               int64_t chunks_per_split) {
  using namespace mas;
  if (batch < 0 || num_q_heads < 0 || head_dim <= 0 || max_blocks < 0 || page_size <= 0 || chunks_per_split < 1)
    return -1;
  const int64_t chunks = cdiv(max_blocks * page_size, kChunk);
  return decode_workspace_bytes(batch, num_q_heads, head_dim, cdiv(chunks, chunks_per_split));
}

namespace mas {
namespace {

// Returned by decode_attention when even one split per row does not fit the workspace.
constexpr int kWorkspaceTooSmall = -1000;

int decode_attention(void* out, int64_t out_stride, int64_t out_head_stride, const void* q, int64_t q_stride,
                     int64_t q_head_stride, const void* k_cache, const void* v_cache, int64_t page_stride,
                     int64_t entry_stride, int64_t head_stride, int64_t num_pages, int64_t page_size,
                     const int32_t* block_tables, int64_t block_table_stride, int64_t max_blocks,
                     const int32_t* seq_lens, int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                     int64_t head_dim, float bmm1_scale, float bmm2_scale, int out_fp8, const float* out_scale_dev,
                     float out_scale_host, void* workspace, int64_t workspace_bytes, uint32_t* err,
                     hipStream_t stream) {
  if (batch < 0 || num_q_heads < 0 || num_kv_heads < 0 || num_pages < 0 || page_size <= 0 || max_blocks < 0 ||
      workspace_bytes < 0)
    return MAS_ERR_INVALID_VALUE;
  if (batch == 0 || num_q_heads == 0) return MAS_OK;
  if (num_kv_heads == 0 || num_q_heads % num_kv_heads != 0) return MAS_ERR_INVALID_VALUE;
  const int64_t group = num_q_heads / num_kv_heads;
  if (group > 16 || (head_dim != 64 && head_dim != 128 && head_dim != 256)) return MAS_ERR_UNSUPPORTED;
  if ((page_size & (page_size - 1)) != 0) return MAS_ERR_UNSUPPORTED;
  const int64_t cap = max_blocks * page_size;
  if (cap > (int64_t{1} << 30) || batch > 65535 || num_kv_heads > 65535 || num_q_heads > 65535)
    return MAS_ERR_UNSUPPORTED;
  if (out == nullptr || q == nullptr || seq_lens == nullptr || (cap > 0 && (k_cache == nullptr || v_cache == nullptr ||
                                                                            block_tables == nullptr || num_pages == 0)))
    return MAS_ERR_INVALID_VALUE;
  if (out_fp8 && out_scale_dev == nullptr && !(out_scale_host > 0.f)) return MAS_ERR_INVALID_VALUE;
  const bool aligned = aligned16(q) && aligned16(out) && q_stride % 8 == 0 && q_head_stride % 8 == 0 &&
                       out_stride % 8 == 0 && out_head_stride % 8 == 0 &&
                       (cap == 0 || (aligned16(k_cache) && aligned16(v_cache) && page_stride % 8 == 0 &&
                                     entry_stride % 8 == 0 && head_stride % 8 == 0)) &&
                       (reinterpret_cast<uintptr_t>(workspace) & 15u) == 0;
  if (!aligned) return MAS_ERR_MISALIGNED;

  // The smallest split (most parallelism) whose partials fit the workspace, with at most
  // kMaxSplitItems (row, kv head, split) work items and kMaxRowSplits splits per row: past those,
  // more splits only add per-split overhead, partials and combine passes (64 rows x 8 kv heads x
  // 128 splits of 256 positions: 804 us per call, with 4 chunks per split 738 us; 8 rows x 8 kv
  // heads x 128 splits: 124 us, with 2 chunks per split 117 us).
  const int64_t chunks = cdiv(cap, kChunk);
  constexpr int64_t kMaxSplitItems = 16384, kMaxRowSplits = 64;
  int64_t per_split = 1;
  while (per_split < chunks &&
         (mas_paged_decode_attention_workspace_bytes(batch, num_q_heads, head_dim, max_blocks, page_size, per_split) >
              workspace_bytes ||
          cdiv(chunks, per_split) > kMaxRowSplits || batch * num_kv_heads * cdiv(chunks, per_split) > kMaxSplitItems))
    per_split *= 2;
  if (per_split > chunks) per_split = chunks > 0 ? chunks : 1;
  if (workspace == nullptr) return MAS_ERR_INVALID_VALUE;
  if (mas_paged_decode_attention_workspace_bytes(batch, num_q_heads, head_dim, max_blocks, page_size, per_split) >
      workspace_bytes)
    return kWorkspaceTooSmall;
  int64_t split_len = per_split * kChunk;
  // Small grids: splits of 128 or 64 positions while the grid holds fewer work items than the GPU
  // has SIMDs, at most 128 splits per row and within the workspace. A split of 256 positions is 8
  // dependent steps; with few wavefronts those steps' latencies, not bandwidth, set the time (on
  // MI355X: 16 rows of up to 512 positions 15.8 -> 10.1 us, one row of up to 4096 14.8 -> 9.6 us;
  // at one item per SIMD and more, shorter splits lost: 64 rows of up to 512, 22.0 -> 23.5 us).
  if (per_split == 1 && cap > 0) {
    int cus = 0;
    if (const int st = device_cu_count(&cus); st != MAS_OK) return st;
    const int64_t simds = static_cast<int64_t>(cus) * 4;
    while (split_len > 64 && batch * num_kv_heads * cdiv(cap, split_len) < simds &&
           cdiv(cap, split_len / 2) <= 2 * kMaxRowSplits &&
           decode_workspace_bytes(batch, num_q_heads, head_dim, cdiv(cap, split_len / 2)) <= workspace_bytes)
      split_len /= 2;
  }
  const int64_t splits = cap > 0 ? cdiv(cap, split_len) : 1;

  int log2_page = 0;
  while ((int64_t{1} << log2_page) < page_size) ++log2_page;
  DecodeArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_stride = q_stride;
  a.q_head_stride = q_head_stride;
  a.k_cache = static_cast<const uint16_t*>(k_cache);
  a.v_cache = static_cast<const uint16_t*>(v_cache);
  a.page_stride = page_stride;
  a.entry_stride = entry_stride;
  a.head_stride = head_stride;
  a.num_pages = num_pages;
  a.block_tables = block_tables;
  a.bt_stride = block_table_stride;
  a.max_blocks = max_blocks;
  a.seq_lens = seq_lens;
  a.hq = static_cast<int>(num_q_heads);
  a.hk = static_cast<int>(num_kv_heads);
  a.group = static_cast<int>(group);
  a.log2_page = log2_page;
  a.split_len = static_cast<int>(split_len);
  {
    int cus = 0;
    if (const int st = device_cu_count(&cus); st != MAS_OK) return st;
    a.row_target = static_cast<int>(std::max<int64_t>(1, static_cast<int64_t>(cus) * 4 / std::max<int64_t>(1, batch * num_kv_heads)));
  }
  a.max_splits = static_cast<int>(splits);
  a.scale_log2 = bmm1_scale * 1.4426950408889634f;
  a.out_scale = bmm2_scale;
  a.part_o = static_cast<float*>(workspace);
  a.part_ml = a.part_o + batch * num_q_heads * splits * head_dim;
  a.out = out;
  a.out_stride = out_stride;
  a.out_head_stride = out_head_stride;
  a.out_fp8 = out_fp8 != 0;
  a.quant_scale_dev = out_scale_dev;
  a.quant_scale_host = out_scale_host;
  a.err = err;
  switch (head_dim) {
    case 64: return dispatch_group<64>(a, batch, num_kv_heads, stream);
    case 128: return dispatch_group<128>(a, batch, num_kv_heads, stream);
    default: return dispatch_group<256>(a, batch, num_kv_heads, stream);
  }
}

// Scratch of the no-allocation entry point: the split partials in the library's own device memory,
// one copy per GPU the library runs on, kept until the process ends. Host code uses the address
// hipGetSymbolAddress returns for the current device (the array's name is a host-side stand-in).
constexpr int64_t kScratchBytes = MAS_DECODE_ATTENTION_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

// The scratch array's address on the stream's device, looked up once per device with that device
// current (and the caller's current device restored). The lookup may load the code object that
// holds the array, so it is not made while `stream` is being captured into a graph: such a first
// call returns MAS_ERR_NOT_READY, and one call outside capture on the device sets it up.
int scratch_address(hipStream_t stream, void** ptr) {
  int dev = 0;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess) return MAS_ERR_DEVICE;
  if (dev < 0 || dev >= kMaxDevices) return MAS_ERR_UNSUPPORTED;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capture) != hipSuccess) return MAS_ERR_DEVICE;
    if (capture != hipStreamCaptureStatusNone) return MAS_ERR_NOT_READY;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      int current = 0;
      if (hipGetDevice(&current) != hipSuccess) return MAS_ERR_DEVICE;
      if (current != dev && hipSetDevice(dev) != hipSuccess) return MAS_ERR_DEVICE;
      const hipError_t st = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (current != dev && hipSetDevice(current) != hipSuccess) return MAS_ERR_DEVICE;
      if (st != hipSuccess || p == nullptr) return MAS_ERR_DEVICE;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return MAS_OK;
}

}  // namespace
}  // namespace mas

extern "C" int mas_paged_decode_attention_bf16(void* out, int64_t out_stride, int64_t out_head_stride, const void* q,
                                               int64_t q_stride, int64_t q_head_stride, const void* k_cache,
                                               const void* v_cache, int64_t page_stride, int64_t entry_stride,
                                               int64_t head_stride, int64_t num_pages, int64_t page_size,
                                               const int32_t* block_tables, int64_t block_table_stride,
                                               int64_t max_blocks, const int32_t* seq_lens, int64_t batch,
                                               int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                               float bmm1_scale, float bmm2_scale, int out_fp8,
                                               const float* out_scale_dev, float out_scale_host, void* workspace,
                                               int64_t workspace_bytes, uint32_t* err, hipStream_t stream) {
  const int st = mas::decode_attention(out, out_stride, out_head_stride, q, q_stride, q_head_stride, k_cache, v_cache,
                                       page_stride, entry_stride, head_stride, num_pages, page_size, block_tables,
                                       block_table_stride, max_blocks, seq_lens, batch, num_q_heads, num_kv_heads,
                                       head_dim, bmm1_scale, bmm2_scale, out_fp8, out_scale_dev, out_scale_host,
                                       workspace, workspace_bytes, err, stream);
  return st == mas::kWorkspaceTooSmall ? MAS_ERR_INVALID_VALUE : st;
}

extern "C" int mas_paged_decode_attention_bf16_noalloc(
    void* out, int64_t out_stride, int64_t out_head_stride, const void* q, int64_t q_stride, int64_t q_head_stride,
    const void* k_cache, const void* v_cache, int64_t page_stride, int64_t entry_stride, int64_t head_stride,
    int64_t num_pages, int64_t page_size, const int32_t* block_tables, int64_t block_table_stride,
    int64_t max_blocks, const int32_t* seq_lens, int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
    int64_t head_dim, float bmm1_scale, float bmm2_scale, int out_fp8, const float* out_scale_dev,
    float out_scale_host, uint32_t* err, hipStream_t stream) {
  void* ws = nullptr;
  if (const int st = mas::scratch_address(stream, &ws); st != MAS_OK) return st;
  const int st = mas::decode_attention(out, out_stride, out_head_stride, q, q_stride, q_head_stride, k_cache, v_cache,
                                       page_stride, entry_stride, head_stride, num_pages, page_size, block_tables,
                                       block_table_stride, max_blocks, seq_lens, batch, num_q_heads, num_kv_heads,
                                       head_dim, bmm1_scale, bmm2_scale, out_fp8, out_scale_dev, out_scale_host, ws,
                                       mas::kScratchBytes, err, stream);
  return st == mas::kWorkspaceTooSmall ? MAS_ERR_SCRATCH : st;
}
