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
//  1. decode_attn_split - one wavefront per (split of chunks_per_split * 256 positions, kv head,
//     row). Per 256-position chunk: Q.K^T on MFMA (v_mfma_f32_16x16x32_bf16: the kv head's G
//     query heads are the rows of A, zero-padded to 16; a tile of 16 positions is the columns of B,
//     each lane reading a 16-byte slice of one key row straight from the cache), then the exact
//     max / exp / sum over the chunk in registers with DPP row reductions, merged into the split's
//     running (max, sum), then P.V on the vector ALUs with each lane reading 16-byte slices of value
//     rows (D / 8 lanes per position). The split writes its (max, sum) and unnormalised O to the
//     caller's workspace.
//  2. decode_attn_combine - one wavefront per (query head, row) merges the splits and writes bf16.
// Scores live in the log2 domain (bmm1_scale * log2 e folded in), so every exponential is one
// v_exp_f32. A position whose page id is out of range is skipped (MAS_ERRBIT_PAGE); seq_lens past
// the block table's reach is clamped to it (MAS_ERRBIT_POSITION); a row with no position gets zeros.
#include "device.h"

namespace mas {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kChunk = 256;          // positions per chunk
constexpr int kTiles = kChunk / 16;  // MFMA tiles of 16 positions per chunk
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
  int hq, group, log2_page, chunks_per_split, max_splits;
  float scale_log2;  // bmm1_scale * log2(e)
  float out_scale;   // bmm2_scale
  float* part_o;     // [batch][hq][max_splits][D]
  float* part_ml;    // [batch][hq][max_splits][2]: running max (log2 domain), sum
  uint16_t* out;
  int64_t out_stride, out_head_stride;
  uint32_t* err;
};

__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp_move<0xb1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_move<0x4e>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_move<0x141>(v));  // row_half_mirror
  return fmaxf(v, dpp_move<0x140>(v));  // row_mirror
}

__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_move<0xb1>(v);
  v += dpp_move<0x4e>(v);
  v += dpp_move<0x141>(v);
  return v + dpp_move<0x140>(v);
}

// seq_lens[b] clamped to [0, max_blocks * page_size].
__device__ __forceinline__ int kv_len(const DecodeArgs& a, int b) {
  const int64_t L = a.seq_lens[b];
  const int64_t cap = a.max_blocks << a.log2_page;
  return static_cast<int>(L < 0 ? 0 : (L > cap ? cap : L));
}

// Element offset of position p's row for kv head kvh; page 0 (in bounds) when the page id is not.
__device__ __forceinline__ int64_t kv_row(const DecodeArgs& a, int b, int kvh, int p, bool* ok) {
  const int32_t page = a.block_tables[b * a.bt_stride + (p >> a.log2_page)];
  *ok = page >= 0 && page < a.num_pages;
  return (*ok ? static_cast<int64_t>(page) : 0) * a.page_stride +
         static_cast<int64_t>(p & ((1 << a.log2_page) - 1)) * a.entry_stride + kvh * a.head_stride;
}

template <int GP, int D>
__global__ __launch_bounds__(64) void decode_attn_split(DecodeArgs a) {
  constexpr int KS = D / 32;     // MFMA k-steps per tile
  constexpr int LPP = D / 8;     // P.V layout: lanes per position
  constexpr int PPW = 64 / LPP;  // P.V layout: positions per wavefront step
  constexpr int RG = GP / 4;     // MFMA result rows of 4 heads that hold query heads
  constexpr int U = 32 / PPW;    // P.V: positions per lane per load group (32 per wavefront)
  constexpr int TG = KS <= 4 ? 4 : 2;  // pass 1: tiles per load group (KS * TG 16-byte loads in flight)
  __shared__ __align__(16) float p_lds[kChunk * GP];  // softmax numerators, [position][head]
  __shared__ int64_t row_lds[kChunk];                 // each chunk position's row offset, -1 if masked
  __shared__ float alpha_lds[GP];                     // rescale of the running O for this chunk

  const int lane = threadIdx.x;
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int L = kv_len(a, b);
  const int start = split * a.chunks_per_split * kChunk;
  if (start >= L) return;
  const int end = min(start + a.chunks_per_split * kChunk, L);
  const int G = a.group;
  const int n = lane & 15, r = lane >> 4;

  // A operand: query head (lane & 15) of this kv head's group, k = 32 * ks + 8 * (lane >> 4) + 0..7.
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

  float m_run[4], l_run[4];  // score layout: head 4 * r + i
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = kNegInf;
    l_run[i] = 0.f;
  }
  float o[GP][8];  // P.V layout: head g, head-dim 8 * (lane % LPP) + e
#pragma unroll
  for (int g = 0; g < GP; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
  const int pv_d = lane % LPP, pv_grp = lane / LPP;

  for (int cstart = start; cstart < end; cstart += kChunk) {
    __syncthreads();  // the previous chunk's P.V reads are done before the LDS is rewritten

    // ---- pass 1: scores, TG tiles of 16 positions per load group; lane holds heads 4r+i at
    // position cstart + 16 t + n (the MFMA result layout).
    f32x4 s[kTiles];
#pragma unroll
    for (int t0 = 0; t0 < kTiles; t0 += TG) {
      int64_t rows[TG];
      bool oks[TG];
#pragma unroll
      for (int j = 0; j < TG; ++j) {
        const int p = cstart + 16 * (t0 + j) + n;
        const bool valid = p < end;
        bool ok;
        rows[j] = kv_row(a, b, kvh, valid ? p : end - 1, &ok);
        if (valid && !ok && r == 0) report(a.err, MAS_ERRBIT_PAGE);
        oks[j] = valid && ok;
      }
      u32x4 kb[TG][KS];
#pragma unroll
      for (int j = 0; j < TG; ++j)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kb[j][ks] = load_stream(a.k_cache + rows[j] + 32 * ks + 8 * r);
      load_fence();
#pragma unroll
      for (int j = 0; j < TG; ++j) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[ks], __builtin_bit_cast(bf16x8, kb[j][ks]), acc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) s[t0 + j][i] = oks[j] ? acc[i] * a.scale_log2 : kNegInf;
        if (r == 0) row_lds[16 * (t0 + j) + n] = oks[j] ? rows[j] : -1;
      }
    }

    // ---- softmax over the chunk, merged into the split's running max and sum
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float mx = kNegInf;
#pragma unroll
      for (int t = 0; t < kTiles; ++t) mx = fmaxf(mx, s[t][i]);
      mx = row_max16(mx);
      const float m_new = fmaxf(m_run[i], mx);
      const float m_use = m_new == kNegInf ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run[i] - m_use);
      float sum = 0.f;
#pragma unroll
      for (int t = 0; t < kTiles; ++t) {
        s[t][i] = __builtin_amdgcn_exp2f(s[t][i] - m_use);
        sum += s[t][i];
      }
      l_run[i] = l_run[i] * alpha + row_sum16(sum);
      m_run[i] = m_new;
      if (n == 0 && r < RG) alpha_lds[4 * r + i] = alpha;
    }
    if (r < RG) {
#pragma unroll
      for (int t = 0; t < kTiles; ++t) *reinterpret_cast<f32x4*>(&p_lds[(16 * t + n) * GP + 4 * r]) = s[t];
    }
    __syncthreads();

    // ---- pass 2: P.V; masked positions have P = 0 and their (in-bounds) value row zeroed
#pragma unroll
    for (int g = 0; g < GP; ++g) {
      const float al = alpha_lds[g];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] *= al;
    }
    const int npos = min(kChunk, end - cstart);
    for (int j0 = 0; j0 < npos; j0 += 32) {
      int64_t vrow[U];
#pragma unroll
      for (int u = 0; u < U; ++u) vrow[u] = row_lds[j0 + PPW * u + pv_grp];
      u32x4 vv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) vv[u] = load_stream(a.v_cache + (vrow[u] >= 0 ? vrow[u] : 0) + 8 * pv_d);
      load_fence();
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int pl = j0 + PPW * u + pv_grp;
        if (vrow[u] < 0) vv[u] = u32x4{0u, 0u, 0u, 0u};
        float vf[8];
        unpack8(vv[u], vf);
        const float* prow = &p_lds[pl * GP];
#pragma unroll
        for (int g = 0; g < GP; ++g) {
          const float pg = prow[g];
#pragma unroll
          for (int e = 0; e < 8; ++e) o[g][e] = __builtin_fmaf(pg, vf[e], o[g][e]);
        }
      }
    }
  }

  // ---- sum O over the PPW position groups, then write the split's partials
#pragma unroll
  for (int off = LPP; off < 64; off <<= 1)
#pragma unroll
    for (int g = 0; g < GP; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] += __shfl_xor(o[g][e], off);
  const int64_t base = (static_cast<int64_t>(b) * a.hq + kvh * G) * a.max_splits + split;
  if (lane < LPP) {
#pragma unroll
    for (int g = 0; g < GP; ++g) {
      if (g < G) {
        float* dst = a.part_o + (base + static_cast<int64_t>(g) * a.max_splits) * D + 8 * lane;
        *reinterpret_cast<f32x4*>(dst) = f32x4{o[g][0], o[g][1], o[g][2], o[g][3]};
        *reinterpret_cast<f32x4*>(dst + 4) = f32x4{o[g][4], o[g][5], o[g][6], o[g][7]};
      }
    }
  }
  if (n == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int g = 4 * r + i;
      if (g < G) {
        *reinterpret_cast<f32x2*>(a.part_ml + (base + static_cast<int64_t>(g) * a.max_splits) * 2) =
            f32x2{m_run[i], l_run[i]};
      }
    }
  }
}

template <int D>
__global__ __launch_bounds__(64) void decode_attn_combine(DecodeArgs a) {
  constexpr int DPL = D / 64;  // head-dim elements per lane
  const int lane = threadIdx.x;
  const int h = blockIdx.x, b = blockIdx.y;
  const int64_t raw = a.seq_lens[b];
  if (h == 0 && lane == 0 && (raw < 0 || raw > (a.max_blocks << a.log2_page))) report(a.err, MAS_ERRBIT_POSITION);
  const int L = kv_len(a, b);
  const int split_len = a.chunks_per_split * kChunk;
  const int nsplit = (L + split_len - 1) / split_len;
  const int64_t base = (static_cast<int64_t>(b) * a.hq + h) * a.max_splits;
  float mx = kNegInf;
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, a.part_ml[(base + s) * 2]);
  float acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) acc[e] = 0.f;
  float denom = 0.f;
  if (mx != kNegInf) {
    for (int s = 0; s < nsplit; ++s) {
      const f32x2 ml = *reinterpret_cast<const f32x2*>(a.part_ml + (base + s) * 2);
      const float w = __builtin_amdgcn_exp2f(ml[0] - mx);
      denom += w * ml[1];
      const float* po = a.part_o + (base + s) * D + DPL * lane;
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[e] = __builtin_fmaf(w, po[e], acc[e]);
    }
  }
  const float scale = denom > 0.f ? a.out_scale / denom : 0.f;
  uint16_t* dst = a.out + b * a.out_stride + h * a.out_head_stride + DPL * lane;
  if constexpr (DPL == 1) {
    dst[0] = static_cast<uint16_t>(pack_bf16x2(acc[0] * scale, 0.f));
  } else if constexpr (DPL == 2) {
    *reinterpret_cast<uint32_t*>(dst) = pack_bf16x2(acc[0] * scale, acc[1] * scale);
  } else {
    *reinterpret_cast<u32x2*>(dst) =
        u32x2{pack_bf16x2(acc[0] * scale, acc[1] * scale), pack_bf16x2(acc[2] * scale, acc[3] * scale)};
  }
}

template <int GP, int D>
int launch(const DecodeArgs& a, int64_t batch, int64_t hk, hipStream_t s) {
  hipLaunchKernelGGL((decode_attn_split<GP, D>),
                     dim3(static_cast<uint32_t>(a.max_splits), static_cast<uint32_t>(hk), static_cast<uint32_t>(batch)),
                     dim3(64), 0, s, a);
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

extern "C" int64_t mas_paged_decode_attention_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t head_dim,
                                                               int64_t max_blocks, int64_t page_size,
                                                               int64_t chunks_per_split) {
  using namespace mas;
  if (batch < 0 || num_q_heads < 0 || head_dim <= 0 || max_blocks < 0 || page_size <= 0 || chunks_per_split < 1)
    return -1;
  const int64_t chunks = cdiv(max_blocks * page_size, kChunk);
  const int64_t splits = cdiv(chunks, chunks_per_split);
  return batch * num_q_heads * (splits > 0 ? splits : 1) * (head_dim + 2) * 4;
}

extern "C" int mas_paged_decode_attention_bf16(void* out, int64_t out_stride, int64_t out_head_stride, const void* q,
                                               int64_t q_stride, int64_t q_head_stride, const void* k_cache,
                                               const void* v_cache, int64_t page_stride, int64_t entry_stride,
                                               int64_t head_stride, int64_t num_pages, int64_t page_size,
                                               const int32_t* block_tables, int64_t block_table_stride,
                                               int64_t max_blocks, const int32_t* seq_lens, int64_t batch,
                                               int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                               float bmm1_scale, float bmm2_scale, void* workspace,
                                               int64_t workspace_bytes, uint32_t* err, hipStream_t stream) {
  using namespace mas;
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
  const bool aligned = aligned16(q) && aligned16(out) && q_stride % 8 == 0 && q_head_stride % 8 == 0 &&
                       out_stride % 8 == 0 && out_head_stride % 8 == 0 &&
                       (cap == 0 || (aligned16(k_cache) && aligned16(v_cache) && page_stride % 8 == 0 &&
                                     entry_stride % 8 == 0 && head_stride % 8 == 0)) &&
                       (reinterpret_cast<uintptr_t>(workspace) & 15u) == 0;
  if (!aligned) return MAS_ERR_MISALIGNED;

  // The smallest split (most parallelism) whose partials fit the workspace.
  const int64_t chunks = cdiv(cap, kChunk);
  int64_t per_split = 1;
  while (per_split < chunks &&
         mas_paged_decode_attention_workspace_bytes(batch, num_q_heads, head_dim, max_blocks, page_size, per_split) >
             workspace_bytes)
    per_split *= 2;
  if (per_split > chunks) per_split = chunks > 0 ? chunks : 1;
  if (mas_paged_decode_attention_workspace_bytes(batch, num_q_heads, head_dim, max_blocks, page_size, per_split) >
          workspace_bytes ||
      workspace == nullptr)
    return MAS_ERR_INVALID_VALUE;
  const int64_t splits = chunks > 0 ? cdiv(chunks, per_split) : 1;

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
  a.group = static_cast<int>(group);
  a.log2_page = log2_page;
  a.chunks_per_split = static_cast<int>(per_split);
  a.max_splits = static_cast<int>(splits);
  a.scale_log2 = bmm1_scale * 1.4426950408889634f;
  a.out_scale = bmm2_scale;
  a.part_o = static_cast<float*>(workspace);
  a.part_ml = a.part_o + batch * num_q_heads * splits * head_dim;
  a.out = static_cast<uint16_t*>(out);
  a.out_stride = out_stride;
  a.out_head_stride = out_head_stride;
  a.err = err;
  switch (head_dim) {
    case 64: return dispatch_group<64>(a, batch, num_kv_heads, stream);
    case 128: return dispatch_group<128>(a, batch, num_kv_heads, stream);
    default: return dispatch_group<256>(a, batch, num_kv_heads, stream);
  }
}
