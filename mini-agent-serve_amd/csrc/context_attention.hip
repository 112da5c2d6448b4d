// context_attention.hip - causal paged attention of prompt rows over the KV cache.
//
// Semantics: flashinfer.prefill.trtllm_batch_context_with_kv_cache as called at
// miniagentserve/models/devstral2/devstral2.py:198-213. Prompt row j owns query tokens
// [cu_seqlens_q[j], cu_seqlens_q[j + 1]) (q_len of them) and seq_lens[j] cached + new positions
// (kv_len); query token i sits at position kv_len - q_len + i and attends to the positions
// 0..that, whose key / value rows are at page = block_tables[j, p / page_size],
// entry = p % page_size. For query head h (kv head h / G):
//   out[t, h] = bmm2_scale * sum_p softmax_p(bmm1_scale * q[t, h] . k_p) * v_p,
// fp32 accumulation, P rounded to bf16 for the P.V product (as flash-attention kernels do), the
// output rounded once to bf16.
//
// One workgroup of four (or, for groups of 8+ query heads, eight) wavefronts per (kv head, head
// group, token tile, prompt row). Each wavefront owns 32 query rows: 32 consecutive tokens of one
// query head; the wavefronts cover up to four heads of the kv head's group and one or more
// 32-token tiles of them (more tokens of fewer heads for groups of 1 or 2), so every 64-position
// key / value tile they stage in LDS serves 128 (256) query rows. Per tile:
//   S^T = K Q^T on MFMA (v_mfma_f32_32x32x16_bf16; A = 32 key rows read from LDS, B = the
//   wavefront's 32 query rows, held in registers), causal mask, online softmax per query row, then
//   O^T += V^T P^T on MFMA, where P^T is packed to bf16 straight from the S^T accumulators and V^T
//   is read from the row-major value tile with gfx950's transposing LDS read (ds_read_b64_tr_b16:
//   in each group of 16 lanes, lane 4a + b receives element b of the 4-element rows that lanes
//   a, a + 4, a + 8, a + 12 point at), two per operand, in the position order the packing implies.
// Tiles are software-pipelined over two LDS buffers: while tile i is in the softmax, tile i + 1's
// score MFMAs run and tile i + 2's key and value loads are in flight.
#include <algorithm>

#include "device.h"

namespace mas {
namespace {

constexpr int kTileP = 64;        // key positions per tile
constexpr int kRowsPerWave = 32;  // query rows (tokens of one head) per wavefront
constexpr int kMaxCtxSplits = 32;  // split-KV: key-range splits per token tile, at most
constexpr float kNegInf = -__builtin_huge_valf();

struct ContextArgs {
  const uint16_t* q;
  int64_t q_stride, q_head_stride;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int64_t page_stride, entry_stride, head_stride, num_pages;
  const int32_t* block_tables;
  int64_t bt_stride, max_blocks;
  const int32_t* seq_lens;
  const int32_t* cu_seqlens_q;
  int hq, hk, group, heads_per_wg, log2_page;
  // Split-KV (kv_splits > 1, for grids of fewer workgroups than CUs): split s of a token tile walks
  // key tiles [s * t, (s + 1) * t), t = split_tiles(its key tiles, kv_splits) (the last split: to
  // the end), and writes its (max, sum, unnormalised O) per (token, head) to part_ml / part_o,
  // indexed by (row * row_tokens + token, head, split); context_combine merges them. Token tiles
  // reaching fewer than split_from key tiles are not split: split 0 computes them whole and writes
  // their output.
  int kv_splits, row_tokens, split_from;
  float* part_o;
  float* part_ml;
  float scale_log2;
  float out_scale;
  void* out;                // bf16, or fp8 e4m3fn codes when out_fp8
  int64_t out_stride, out_head_stride;
  int out_fp8;              // out = e4m3fn(clamp(bf16(O) / quant scale, +-448)): the o_proj input quantize
  const float* quant_scale_dev;
  float quant_scale_host;
  uint32_t* err;
};

// Wavefronts per workgroup (kWaves, 4 or 8): each stages its share of every key / value tile, and
// all of them read it. The register allocation is capped for two wavefronts per SIMD (8 / kWaves
// workgroups per CU, at most 256 VGPRs per lane). Eight wavefronts (two 32-token tiles of the same
// heads per workgroup: half the staging per flop) measured ~2% faster with 12 query heads per kv
// head (123B, 4 x 4096 tokens) and ~4% slower with 4 (24B, 4 x 2048: the grid halves), in
// alternating runs on one box; the launch picks 8 when a kv head has at least 8 query heads.

typedef float f32x16 __attribute__((ext_vector_type(16)));

// v_mfma_f32_32x32x16_bf16 (checked on MI355X): lane l, element e of A holds A[l % 32][8 (l / 32) + e],
// of B holds B[8 (l / 32) + e][l % 32]; element j of the result holds D[8 (j / 4) + 4 (l / 32) + j % 4][l % 32].
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// How a tile's key / value rows find their pages (the block-table reads of a tile):
//   kPagesTile  - pages of at least a tile: the tile lies in one page, one scalar read per tile;
//   kPagesStep1 - pages of at least a thread-row step (kPosStep positions): each step of a tile lies
//                 in one page, one scalar read per step, each lane adding its fixed row offset;
//   kPagesStep  - pages of at least half of a thread-row step: the rows of step u lie in one or two
//                 pages, read with scalar loads, each lane picking its own;
//   kPagesLane  - smaller pages: each lane reads the page of each of its rows (vector loads).
// Vector loads of block-table entries make the compiler wait for them, and such waits cover every
// vector load issued before them, the next tiles' key / value loads included: they stall the
// software pipeline, which the scalar reads do not.
constexpr int kPagesLane = 0, kPagesStep = 1, kPagesTile = 2, kPagesStep1 = 3;

// Key tiles per split of a token tile that reaches `ntiles` key tiles: its kv_splits splits share
// them evenly, at least 4 each (fewer splits then hold them all). From the tile's own reach, not
// the block table's, so that a table much wider than the rows (a graph captured for the longest
// context) still spreads each row over all the splits.
__device__ __forceinline__ int split_tiles(int ntiles, int kv_splits) {
  return max(4, (ntiles + kv_splits - 1) / kv_splits);
}

// kSplit: a split-KV launch (a separate instance, so that the one-kernel instances keep their code).
template <int D, int kPages, int kWaves, bool kSplit>
__global__ __launch_bounds__(64 * kWaves, 8 / kWaves) void context_attn(ContextArgs a) {
  constexpr int kCtxWaves = kWaves;
  constexpr int kCtxThreads = 64 * kWaves;
  constexpr int KS = D / 16;            // MFMA k-steps over the head dim (S^T)
  constexpr int DB = D / 32;            // 32-dim blocks of O^T
  constexpr int KROW = D + 8;           // bf16 per LDS key row (+16 B: conflict-free A reads)
  constexpr int VROW = D + 16;          // bf16 per LDS value row (+32 B: conflict-free column reads)
  constexpr int CPR = D / 8;            // 16-byte chunks per key / value row
  constexpr int LOADS = kTileP * CPR / kCtxThreads;  // 16-byte chunks per thread per tile, each of K and V
  // Two tile buffers: with the software pipeline, the next tile's keys are read while this tile's
  // values are.
  constexpr int kBufs = 2;
  __shared__ __align__(16) uint16_t k_lds_all[kBufs][kTileP * KROW];
  __shared__ __align__(16) uint16_t v_lds_all[kBufs][kTileP * VROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id_uniform();
  const int n = lane & 31, hf = lane >> 5;  // this lane's query row (token) and lane half
  const int hgroups = (a.group + a.heads_per_wg - 1) / a.heads_per_wg;
  const int kvh = blockIdx.x / hgroups, hg = blockIdx.x - kvh * hgroups;
  const int row = kSplit ? blockIdx.z / a.kv_splits : blockIdx.z;
  const int split = kSplit ? blockIdx.z - row * a.kv_splits : 0;
  const int q0 = a.cu_seqlens_q[row], q_len = a.cu_seqlens_q[row + 1] - q0;
  const int tokens_per_wg = kRowsPerWave * (kCtxWaves / a.heads_per_wg);
  // Token tiles in reverse launch order: the last tiles reach the most positions, so they start first.
  const int tile_idx = static_cast<int>(gridDim.y - 1 - blockIdx.y);
  const int tile_tok = tile_idx * tokens_per_wg;
  if (tile_tok >= q_len) return;  // uniform over the workgroup
  // kv_len clamped to the block table's reach; a kv_len below q_len leaves the first tokens with
  // negative positions: they see no key and get zeros.
  const int64_t cap = a.max_blocks << a.log2_page;
  const int64_t raw_len = a.seq_lens[row];
  // Error bits are reported at the end: a global atomic before the tile loop would keep the
  // compiler from reading the block table through the scalar cache.
  // also flagged: a row with more query tokens than the grid covers (max_q_len too small); the
  // tokens past the grid are left unwritten
  const bool len_bad = raw_len < q_len || raw_len > cap || q_len > static_cast<int>(gridDim.y) * tokens_per_wg;
  const int kv_len = static_cast<int>(raw_len < 0 ? 0 : (raw_len > cap ? cap : raw_len));
  const int shift = kv_len - q_len;  // position of query token i = shift + i

  // This wavefront's head and tokens.
  const int hsub = wave % a.heads_per_wg;
  const int g = hg * a.heads_per_wg + hsub;
  const bool head_ok = g < a.group;
  const int h = kvh * a.group + (head_ok ? g : 0);
  const int tok = tile_tok + kRowsPerWave * (wave / a.heads_per_wg);  // first of 32 tokens
  const bool wave_live = head_ok && tok < q_len;

  // B operands of S^T = K Q^T: token tok + n, head-dim 16 ks + 8 hf + 0..7 (zero past q_len).
  bf16x8 qb[KS];
  {
    const int t = tok + n;
    const bool ok = wave_live && t < q_len;
    const uint16_t* src = a.q + static_cast<int64_t>(q0 + (ok ? t : 0)) * a.q_stride + h * a.q_head_stride + 8 * hf;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 v = load_cached(src + 16 * ks);
      if (!ok) v = u32x4{0u, 0u, 0u, 0u};
      qb[ks] = __builtin_bit_cast(bf16x8, v);
    }
  }

  // Causal reach of the workgroup: positions 0 .. shift + last token.
  const int last_tok = min(tile_tok + tokens_per_wg, q_len) - 1;
  const int reach = shift + last_tok + 1;  // <= kv_len
  const int ntiles = reach > 0 ? (reach + kTileP - 1) / kTileP : 0;
  // This workgroup's key tiles: all of them, or its split's share.
  const bool split_tile = kSplit && ntiles >= a.split_from;
  const int per_split = split_tile ? split_tiles(ntiles, a.kv_splits) : ntiles;
  const int it_begin = kSplit ? split * per_split : 0;
  const int it_end = !split_tile || split == a.kv_splits - 1 ? ntiles : min(ntiles, it_begin + per_split);
  // an empty split (uniform), which the merge skips; split 0 of a tile that is not split goes on,
  // to write its output (zeros for a tile that reaches no key)
  if (kSplit && it_begin >= it_end && (split_tile || split > 0)) {
    if (len_bad && tid == 0 && blockIdx.x == 0 && tile_idx == 0 && split == 0) report(a.err, MAS_ERRBIT_POSITION);
    return;
  }

  float m_run = kNegInf, l_run = 0.f;  // token n's running max (raw score units) and sum
  f32x16 acc[DB];                      // O^T: element j of block db holds O[token n][32 db + 8 (j/4) + 4 hf + j%4]
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};

  const int32_t* bt = a.block_tables + row * a.bt_stride;
  const int pmask = (1 << a.log2_page) - 1;
  // Thread's chunks of a tile: chunk c = tid + T u (T threads) -> position tid / CPR + (T / CPR) u, head-dim
  // chunk tid % CPR (the same for every u). Rows past kv_len or on a page id outside the cache load
  // row 0 of page 0 and are zeroed when stored; the flags are kept so that the loads themselves are
  // not waited on here. With pages of at least a tile, a tile lies in one page: one (wave-uniform)
  // block-table read per tile and precomputed per-thread offsets.
  constexpr int kPosStep = kCtxThreads / CPR;
  const int dcol = tid % CPR, prow = tid / CPR;
  const int64_t lane_off = static_cast<int64_t>(prow) * a.entry_stride + kvh * a.head_stride + 8 * dcol;
  struct TileRegs {
    u32x4 k[LOADS], v[LOADS];
    bool lok[LOADS];
    bool full;  // every chunk of the tile valid: stores need no zeroing
  };
  bool page_bad = false;  // a real position's page id outside the cache (reported once, at the end)
  const int last_page = kv_len > 0 ? (kv_len - 1) >> a.log2_page : 0;  // the sequence's last block-table entry
  auto issue_tile = [&](TileRegs& tr, int base) {
    if constexpr (kPages == kPagesTile) {
      const int32_t page = bt[base >> a.log2_page];
      const bool ok = page >= 0 && page < a.num_pages;
      page_bad |= !ok;
      const int64_t tile_off = (ok ? static_cast<int64_t>(page) : 0) * a.page_stride +
                               static_cast<int64_t>(base & pmask) * a.entry_stride;
      tr.full = ok && base + kTileP <= kv_len;
#pragma unroll
      for (int u = 0; u < LOADS; ++u) {
        const int64_t off = tile_off + lane_off + static_cast<int64_t>(kPosStep * u) * a.entry_stride;
        tr.k[u] = load_cached(a.k_cache + off);
        tr.v[u] = load_cached(a.v_cache + off);
        tr.lok[u] = ok && base + prow + kPosStep * u < kv_len;
      }
    } else if constexpr (kPages == kPagesStep1) {
      // Step u starts at a multiple of kPosStep <= page size, so its rows lie in one page at entries
      // (gp & pmask) + prow: a wave-uniform base per step plus the lane's fixed offset. Rows past
      // kv_len are read from inside that page (the sequence's last page for steps past its end) and
      // zeroed when staged.
      bool all_ok = true;
#pragma unroll
      for (int u = 0; u < LOADS; ++u) {
        const int gp = base + kPosStep * u;  // the step's first position (wave-uniform)
        const int32_t page = bt[min(gp >> a.log2_page, last_page)];
        const bool ok = page >= 0 && page < a.num_pages;
        page_bad |= !ok && gp < kv_len;
        all_ok = all_ok && ok;
        const int64_t off = (ok ? static_cast<int64_t>(page) : 0) * a.page_stride +
                            static_cast<int64_t>(gp & pmask) * a.entry_stride + lane_off;
        tr.k[u] = load_cached(a.k_cache + off);
        tr.v[u] = load_cached(a.v_cache + off);
        tr.lok[u] = ok && gp + prow < kv_len;
      }
      tr.full = all_ok && base + kTileP <= kv_len;
    } else if constexpr (kPages == kPagesStep) {
      const int sub = prow >> a.log2_page;  // 0 or 1: which of the step's pages holds this lane's row
      if (base + kTileP <= kv_len) {
        // A full tile: every row is real, so the lane's row offset in its page is fixed (the step
        // starts a page when it spans two) and only the page bases change.
        bool all_ok = true;
#pragma unroll
        for (int u = 0; u < LOADS; ++u) {
          const int gp = base + kPosStep * u;  // the step's first position (wave-uniform)
          const int i0 = gp >> a.log2_page;
          const int32_t page0 = bt[i0];
          const int32_t page1 = bt[min(i0 + 1, last_page)];
          const bool ok0 = page0 >= 0 && page0 < a.num_pages, ok1 = page1 >= 0 && page1 < a.num_pages;
          const int32_t page = sub ? page1 : page0;
          const bool ok = sub ? ok1 : ok0;
          all_ok = all_ok && ok0 && (kPosStep <= (1 << a.log2_page) || ok1);
          page_bad |= !ok;
          const int64_t off = (ok ? static_cast<int64_t>(page) : 0) * a.page_stride +
                              static_cast<int64_t>((gp + prow) & pmask) * a.entry_stride + kvh * a.head_stride +
                              8 * dcol;
          tr.k[u] = load_cached(a.k_cache + off);
          tr.v[u] = load_cached(a.v_cache + off);
          tr.lok[u] = ok;
        }
        tr.full = all_ok;
      } else {
        tr.full = false;
#pragma unroll
        for (int u = 0; u < LOADS; ++u) {
          const int gp = base + kPosStep * u;
          const int i0 = min(gp >> a.log2_page, last_page);
          const int32_t page0 = bt[i0];
          const int32_t page1 = bt[min(i0 + 1, last_page)];
          const int32_t page = sub ? page1 : page0;
          const int p = gp + prow;
          const int pc = p < kv_len ? p : kv_len - 1;
          const bool ok = page >= 0 && page < a.num_pages;
          page_bad |= !ok && p < kv_len;
          const int64_t off = (ok ? static_cast<int64_t>(page) : 0) * a.page_stride +
                              static_cast<int64_t>(pc & pmask) * a.entry_stride + kvh * a.head_stride + 8 * dcol;
          tr.k[u] = load_cached(a.k_cache + off);
          tr.v[u] = load_cached(a.v_cache + off);
          tr.lok[u] = ok && p < kv_len;
        }
      }
    } else {
      tr.full = false;
#pragma unroll
      for (int u = 0; u < LOADS; ++u) {
        const int p = base + prow + kPosStep * u;
        const int pc = p < kv_len ? p : kv_len - 1;
        const int32_t page = bt[pc >> a.log2_page];
        const bool ok = page >= 0 && page < a.num_pages;
        page_bad |= !ok && p < kv_len;
        const int64_t off = (ok ? static_cast<int64_t>(page) : 0) * a.page_stride +
                            static_cast<int64_t>(pc & pmask) * a.entry_stride + kvh * a.head_stride + 8 * dcol;
        tr.k[u] = load_cached(a.k_cache + off);
        tr.v[u] = load_cached(a.v_cache + off);
        tr.lok[u] = ok && p < kv_len;
      }
    }
  };
  // The tile in `tr` into LDS buffer `buf` (rows past kv_len or on a bad page zeroed).
  auto stage = [&](const TileRegs& tr, int buf) {
    uint16_t* k_lds = k_lds_all[buf];
    uint16_t* v_lds = v_lds_all[buf];
    if (tr.full) {
#pragma unroll
      for (int u = 0; u < LOADS; ++u) {
        const int p = prow + kPosStep * u;
        *reinterpret_cast<u32x4*>(k_lds + p * KROW + 8 * dcol) = tr.k[u];
        *reinterpret_cast<u32x4*>(v_lds + p * VROW + 8 * dcol) = tr.v[u];
      }
    } else {
#pragma unroll
      for (int u = 0; u < LOADS; ++u) {
        const int p = prow + kPosStep * u;
        const u32x4 kv = tr.lok[u] ? tr.k[u] : u32x4{0u, 0u, 0u, 0u};
        const u32x4 vv = tr.lok[u] ? tr.v[u] : u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(k_lds + p * KROW + 8 * dcol) = kv;
        *reinterpret_cast<u32x4*>(v_lds + p * VROW + 8 * dcol) = vv;
      }
    }
  };

  // Transposing-read coordinates of this lane's 16-lane group: head-dim column offset and row half.
  const int grp_col = 16 * ((lane >> 4) & 1), k16 = lane & 15;
  const float c = a.scale_log2;
  // ---- S^T = K Q^T: element j of s[pb] holds S[token n][position base + 32 pb + 8 (j/4) + 4 hf + j%4]
  auto scores = [&](int buf, f32x16 (&s)[2]) {
    const uint16_t* k_lds = k_lds_all[buf];
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      s[pb] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 ka = *reinterpret_cast<const bf16x8*>(k_lds + (32 * pb + n) * KROW + 16 * ks + 8 * hf);
        s[pb] = mfma32(ka, qb[ks], s[pb]);
      }
    }
  };
  // ---- causal mask, only on tiles that cross the diagonal of the wavefront's first row or the end
  // of the sequence (a wavefront-uniform branch)
  auto mask = [&](f32x16 (&s)[2], int base) {
    if (base + kTileP - 1 > shift + tok || base + kTileP > kv_len) {
      const int qpos = shift + tok + n;  // this lane's query row position
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int kp = base + 32 * pb + 8 * (j >> 2) + 4 * hf + (j & 3);
          if (kp > qpos || kp >= kv_len) s[pb][j] = kNegInf;
        }
    }
  };
  // ---- online softmax per query row; scores stay in raw units, the scale enters the exponent
  // through one fma: p = 2^(s c - m c). P^T is packed to bf16 as the B operands of O^T += V^T P^T:
  // k-step kk = positions 16 kk .. 16 kk + 15, lane half hf holding 16 kk + 4 hf + e (e < 4) and
  // 16 kk + 8 + 4 hf + e - 4 (e >= 4), i.e. elements 8 (kk % 2) .. + 7 of s[kk / 2]. Returns the
  // factor O must be rescaled by.
  auto softmax = [&](f32x16 (&s)[2], bf16x8 (&pbo)[4]) {
    float mx = kNegInf;
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[pb][j]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == kNegInf ? 0.f : m_new;
    const float mc = m_use * c;
    const float alpha = __builtin_amdgcn_exp2f(__builtin_fmaf(m_run, c, -mc));
    float sum = 0.f;
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        s[pb][j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[pb][j], c, -mc));
        sum += s[pb][j];
      }
    sum += __shfl_xor(sum, 32);
    l_run = l_run * alpha + sum;
    m_run = m_new;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int o = 8 * (kk & 1);
      const f32x16& sv = s[kk >> 1];
      const u32x4 packed = {pack_bf16x2(sv[o], sv[o + 1]), pack_bf16x2(sv[o + 2], sv[o + 3]),
                            pack_bf16x2(sv[o + 4], sv[o + 5]), pack_bf16x2(sv[o + 6], sv[o + 7])};
      pbo[kk] = __builtin_bit_cast(bf16x8, packed);
    }
    return alpha;
  };
  // O rescale, skipped when no row's max moved
  auto rescale = [&](float alpha) {
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[db] *= alpha;
    }
  };
  // ---- O^T += V^T P^T: A = V^T[32 dims][16 positions], read transposed from the row-major value
  // tile in the position order of pbo
  auto pv = [&](int buf, const bf16x8 (&pbo)[4]) {
    const uint16_t* v_lds = v_lds_all[buf];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const i16x4 lo = read_column4(v_lds, VROW, 16 * kk + 4 * hf, 32 * db + grp_col, k16);
        const i16x4 hi = read_column4(v_lds, VROW, 16 * kk + 8 + 4 * hf, 32 * db + grp_col, k16);
        const bf16x8 va = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        acc[db] = mfma32(va, pbo[kk], acc[db]);
      }
    }
  };

  TileRegs tr;
  // Software pipeline over tiles: tile it + 1's scores (MFMA, keys from the other LDS buffer) are
  // computed in the same block as tile it's softmax (VALU), so the two overlap; then tile it's P.V.
  // Buffer it & 1 holds tile it, buffer (it + 1) & 1 tile it + 1 (staged after the barrier that
  // ends every read of tile it - 1, which used that buffer).
  f32x16 s_a[2], s_b[2];
  if (it_begin < it_end) {
    issue_tile(tr, it_begin * kTileP);
    stage(tr, it_begin & 1);
    __syncthreads();
    if (it_begin + 1 < it_end) issue_tile(tr, (it_begin + 1) * kTileP);
    if (wave_live) scores(it_begin & 1, s_a);
  }
  // One tile; `cur` holds its scores, `nxt` receives the next tile's. Called with the two score
  // arrays in turn (no copy between them).
  auto step = [&](int it, f32x16 (&cur)[2], f32x16 (&nxt)[2]) {
    const int buf = it & 1;
    __syncthreads();  // tile it - 1's reads (of buffer buf ^ 1) are done
    if (it + 1 < it_end) stage(tr, buf ^ 1);
    __syncthreads();
    if (it + 2 < it_end) issue_tile(tr, (it + 2) * kTileP);
    if (wave_live) {
      mask(cur, it * kTileP);
      bf16x8 pbo[4];
      scores(buf ^ 1, nxt);  // the next tile's (stale buffer contents after the last tile: unused)
      const float alpha = softmax(cur, pbo);
      rescale(alpha);
      pv(buf, pbo);
    }
  };
  int it = it_begin;
  for (; it + 1 < it_end; it += 2) {
    step(it, s_a, s_b);
    step(it + 1, s_b, s_a);
  }
  if (it < it_end) step(it, s_a, s_b);
  if (__builtin_amdgcn_ballot_w64(page_bad) != 0 && lane == 0) report(a.err, MAS_ERRBIT_PAGE);
  // reported by the workgroup of token tile 0, which every row with a query token has
  if (len_bad && tid == 0 && blockIdx.x == 0 && tile_idx == 0) report(a.err, MAS_ERRBIT_POSITION);

  if (!wave_live) return;
  const int t = tok + n;
  if (t >= q_len) return;
  if (split_tile) {
    // ---- this split's partial: O row (lane half hf holds columns 32 db + 8 q + 4 hf .. + 3) and
    // (max, sum), both halves holding the same (max, sum)
    const int64_t pi = ((static_cast<int64_t>(row) * a.row_tokens + t) * a.hq + h) * a.kv_splits + split;
    float* po = a.part_o + pi * D + 4 * hf;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x16& o = acc[db];
        *reinterpret_cast<f32x4*>(po + 32 * db + 8 * q) = f32x4{o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
      }
    if (hf == 0) *reinterpret_cast<f32x2*>(a.part_ml + pi * 2) = f32x2{m_run, l_run};
    return;
  }
  // ---- out[token][h][32 db + 8 q + 4 hf + i] = O / l * bmm2_scale (bf16), or its fp8 quantize
  const float qs = a.out_fp8 ? (a.quant_scale_dev != nullptr ? *a.quant_scale_dev : a.quant_scale_host) : 1.f;
  const float rcp = 1.0f / qs;
  const float sc = l_run > 0.f ? a.out_scale / l_run : 0.f;
  const int64_t at = static_cast<int64_t>(q0 + t) * a.out_stride + h * a.out_head_stride + 4 * hf;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x16& o = acc[db];
      const uint32_t y0 = pack_bf16x2(o[4 * q] * sc, o[4 * q + 1] * sc);
      const uint32_t y1 = pack_bf16x2(o[4 * q + 2] * sc, o[4 * q + 3] * sc);
      const int64_t e = at + 32 * db + 8 * q;
      if (a.out_fp8) {
        // the quantize the reference applies to the bf16 attention output (devstral2.py:93-95,110-111)
        *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.out) + e) =
            fp8x4_saturate_encode(div_by_scale(bf16_lo(y0), qs, rcp), div_by_scale(bf16_hi(y0), qs, rcp),
                                  div_by_scale(bf16_lo(y1), qs, rcp), div_by_scale(bf16_hi(y1), qs, rcp));
      } else {
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.out) + e) = u32x2{y0, y1};
      }
    }
  }
}

// One wavefront per (row, token, query head) of a split-KV launch: merges the token's non-empty
// splits with weights 2^(c (m_s - max m)) (c = bmm1_scale * log2 e, maxima in raw score units as
// the split kernel keeps them) and writes O / l * bmm2_scale as bf16, or its fp8 quantize. Every
// load is issued in one round trip: lane s reads split s's (max, sum) and 16 (32 past 16 splits)
// partial O rows are loaded (indices past the last split clamped to it, weighted 0) before the
// max is known. A token that sees no position (all maxima -inf) gets zeros.
template <int D>
__global__ __launch_bounds__(64) void context_combine(ContextArgs a, int tokens_per_wg) {
  constexpr int DPL = D / 64;  // head-dim elements per lane
  const int lane = threadIdx.x;
  const int id = static_cast<int>(blockIdx.x);  // < rows * row_tokens * hq <= 2^31 - 1 (host-checked)
  const int rt = id / a.hq, h = id - rt * a.hq;
  const int row = rt / a.row_tokens, t = rt - row * a.row_tokens;
  const int q0 = a.cu_seqlens_q[row], q_len = a.cu_seqlens_q[row + 1] - q0;
  if (t >= q_len) return;
  // the token tile's key tiles, as the split kernel counts them
  const int64_t cap = a.max_blocks << a.log2_page;
  const int64_t raw_len = a.seq_lens[row];
  const int kv_len = static_cast<int>(raw_len < 0 ? 0 : (raw_len > cap ? cap : raw_len));
  const int tile_tok = t / tokens_per_wg * tokens_per_wg;
  const int reach = kv_len - q_len + min(tile_tok + tokens_per_wg, q_len);
  const int ntiles = reach > 0 ? (reach + kTileP - 1) / kTileP : 0;
  if (ntiles < a.split_from) return;  // not split: the split kernel wrote this token's output
  const int per_split = split_tiles(ntiles, a.kv_splits);
  const int nsplit = min(a.kv_splits, (ntiles + per_split - 1) / per_split);  // <= kMaxCtxSplits
  const int64_t base = ((static_cast<int64_t>(row) * a.row_tokens + t) * a.hq + h) * a.kv_splits;
  float acc[DPL], l = 0.f;
#pragma unroll
  for (int e = 0; e < DPL; ++e) acc[e] = 0.f;
  if (nsplit > 0) {
    const int sl = lane < nsplit ? lane : nsplit - 1;
    const f32x2 ml = *reinterpret_cast<const f32x2*>(a.part_ml + (base + sl) * 2);
    const float* po = a.part_o + base * D + DPL * lane;
    // slots in two halves of 16; the second only when there are more than 16 splits
    float v[kMaxCtxSplits][DPL];
    auto load_half = [&](int u0) {
#pragma unroll
      for (int u = u0; u < u0 + 16; ++u) {
        const float* src = po + min(u, nsplit - 1) * D;
        if constexpr (DPL == 2) {
          const f32x2 x = *reinterpret_cast<const f32x2*>(src);
          v[u][0] = x[0];
          v[u][1] = x[1];
        } else {
          v[u][0] = src[0];
        }
      }
    };
    load_half(0);
    if (nsplit > 16) load_half(16);
    // max and sum over lanes 0..31 (the splits): two 16-lane rows, read out and combined
    const float m_lane = lane < nsplit ? ml[0] : kNegInf;
    const float mr = row_max16(m_lane);
    const float mx = fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mr), 0)),
                           __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mr), 16)));
    if (mx != kNegInf) {
      const float c = a.scale_log2;
      const float wgt = lane < nsplit ? __builtin_amdgcn_exp2f(__builtin_fmaf(m_lane, c, -mx * c)) : 0.f;
      const float lr = row_sum16(wgt * ml[1]);
      l = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lr), 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lr), 16));
      // every loaded slot, in order: the weight is 0 past the last split (its value a finite copy)
      auto add_half = [&](int u0) {
#pragma unroll
        for (int u = u0; u < u0 + 16; ++u) {
          const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wgt), u));
#pragma unroll
          for (int e = 0; e < DPL; ++e) acc[e] = __builtin_fmaf(wj, v[u][e], acc[e]);
        }
      };
      add_half(0);
      if (nsplit > 16) add_half(16);
    }
  }
  const float sc = l > 0.f ? a.out_scale / l : 0.f;
  const int64_t at = static_cast<int64_t>(q0 + t) * a.out_stride + h * a.out_head_stride + DPL * lane;
  uint32_t y[(DPL + 1) / 2];
  if constexpr (DPL == 1) {
    y[0] = pack_bf16x2(acc[0] * sc, 0.f);
  } else {
#pragma unroll
    for (int e = 0; e < DPL / 2; ++e) y[e] = pack_bf16x2(acc[2 * e] * sc, acc[2 * e + 1] * sc);
  }
  if (a.out_fp8) {
    // the quantize the reference applies to the bf16 attention output (devstral2.py:93-95,110-111)
    const float qs = a.quant_scale_dev != nullptr ? *a.quant_scale_dev : a.quant_scale_host;
    const float rcp = 1.0f / qs;
    float qv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ee = e < DPL ? e : 0;
      qv[e] = div_by_scale((ee & 1) ? bf16_hi(y[ee / 2]) : bf16_lo(y[ee / 2]), qs, rcp);
    }
    const uint32_t codes = fp8x4_saturate_encode(qv[0], qv[1], qv[2], qv[3]);
    uint8_t* dst = static_cast<uint8_t*>(a.out) + at;
    if constexpr (DPL == 1) {
      dst[0] = static_cast<uint8_t>(codes);
    } else {
      *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(codes);
    }
  } else {
    uint16_t* dst = static_cast<uint16_t*>(a.out) + at;
    if constexpr (DPL == 1) {
      dst[0] = static_cast<uint16_t>(y[0]);
    } else {
      *reinterpret_cast<uint32_t*>(dst) = y[0];
    }
  }
}

template <int D, int kWaves, bool kSplit>
void launch_context_mode(int mode, dim3 grid, dim3 block, hipStream_t stream, const ContextArgs& a) {
  if (mode == kPagesTile) hipLaunchKernelGGL((context_attn<D, kPagesTile, kWaves, kSplit>), grid, block, 0, stream, a);
  else if (mode == kPagesStep1)
    hipLaunchKernelGGL((context_attn<D, kPagesStep1, kWaves, kSplit>), grid, block, 0, stream, a);
  else if (mode == kPagesStep)
    hipLaunchKernelGGL((context_attn<D, kPagesStep, kWaves, kSplit>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((context_attn<D, kPagesLane, kWaves, kSplit>), grid, block, 0, stream, a);
}

// Workgroup shape for a query-head group: heads per workgroup, wavefronts, and query tokens per
// token tile (32 per wavefront, the wavefronts split between the heads).
struct ContextLaunch {
  int heads_per_wg, waves;
  int64_t tokens_per_wg;
};

ContextLaunch context_launch(int64_t group) {
  const int heads_per_wg = group >= 4 ? 4 : (group == 2 ? 2 : 1);
  const int waves = group >= 8 ? 8 : 4;
  return {heads_per_wg, waves, kRowsPerWave * (waves / heads_per_wg)};
}

// Bytes of split-KV partials: (max, sum) and an unnormalised fp32 O row per (row, token slot of
// the grid, query head, split).
int64_t context_partial_bytes(int64_t rows, int64_t row_tokens, int64_t num_q_heads, int64_t head_dim,
                              int64_t splits) {
  return rows * row_tokens * num_q_heads * splits * (head_dim + 2) * 4;
}

template <bool kSplit>
void launch_context(int64_t head_dim, int waves, int mode, dim3 grid, dim3 block, hipStream_t stream,
                    const ContextArgs& a) {
  if (head_dim == 64) {
    if (waves == 8) launch_context_mode<64, 8, kSplit>(mode, grid, block, stream, a);
    else launch_context_mode<64, 4, kSplit>(mode, grid, block, stream, a);
  } else {
    if (waves == 8) launch_context_mode<128, 8, kSplit>(mode, grid, block, stream, a);
    else launch_context_mode<128, 4, kSplit>(mode, grid, block, stream, a);
  }
}

}  // namespace
}  // namespace mas

extern "C" int mas_paged_context_attention_bf16(void* out, int64_t out_stride, int64_t out_head_stride, const void* q,
                                                int64_t q_stride, int64_t q_head_stride, const void* k_cache,
                                                const void* v_cache, int64_t page_stride, int64_t entry_stride,
                                                int64_t head_stride, int64_t num_pages, int64_t page_size,
                                                const int32_t* block_tables, int64_t block_table_stride,
                                                int64_t max_blocks, const int32_t* seq_lens,
                                                const int32_t* cu_seqlens_q, int64_t num_rows, int64_t max_q_len,
                                                int64_t max_kv_len, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                                float bmm1_scale, float bmm2_scale, int out_fp8,
                                                const float* out_scale_dev, float out_scale_host, void* workspace,
                                                int64_t workspace_bytes, uint32_t* err, hipStream_t stream) {
  using namespace mas;
  if (num_rows < 0 || max_q_len < 0 || num_q_heads < 0 || num_kv_heads < 0 || num_pages < 0 || page_size <= 0 ||
      max_blocks < 0 || workspace_bytes < 0)
    return MAS_ERR_INVALID_VALUE;
  if (num_rows == 0 || max_q_len == 0 || num_q_heads == 0) return MAS_OK;
  if (num_kv_heads == 0 || num_q_heads % num_kv_heads != 0) return MAS_ERR_INVALID_VALUE;
  if (!(bmm1_scale > 0.f)) return MAS_ERR_INVALID_VALUE;  // the row max is taken over unscaled scores
  if (out_fp8 && out_scale_dev == nullptr && !(out_scale_host > 0.f)) return MAS_ERR_INVALID_VALUE;
  if ((head_dim != 64 && head_dim != 128) || (page_size & (page_size - 1)) != 0) return MAS_ERR_UNSUPPORTED;
  const int64_t cap = max_blocks * page_size;
  if (cap > (int64_t{1} << 30) || num_rows > 65535 || num_q_heads > 65535) return MAS_ERR_UNSUPPORTED;
  if (out == nullptr || q == nullptr || seq_lens == nullptr || cu_seqlens_q == nullptr || k_cache == nullptr ||
      v_cache == nullptr || block_tables == nullptr || num_pages == 0 || cap == 0)
    return MAS_ERR_INVALID_VALUE;
  const bool aligned = aligned16(q) && aligned16(out) && aligned16(k_cache) && aligned16(v_cache) &&
                       q_stride % 8 == 0 && q_head_stride % 8 == 0 && out_stride % 8 == 0 &&
                       out_head_stride % 8 == 0 && page_stride % 8 == 0 && entry_stride % 8 == 0 &&
                       head_stride % 8 == 0;
  if (!aligned) return MAS_ERR_MISALIGNED;
  const int64_t group = num_q_heads / num_kv_heads;
  const ContextLaunch shape = context_launch(group);
  const int heads_per_wg = shape.heads_per_wg, waves = shape.waves;
  const int64_t tokens_per_wg = shape.tokens_per_wg;
  const int64_t hgroups = cdiv(group, heads_per_wg);
  const int64_t gx = num_kv_heads * hgroups, gy = cdiv(max_q_len, tokens_per_wg);
  if (gx > INT32_MAX || gy > 65535) return MAS_ERR_UNSUPPORTED;

  // Split-KV for grids of fewer workgroups than CUs (few new tokens after a long cached prefix):
  // each token tile's key range is split over up to kMaxCtxSplits workgroups of at least 4 key
  // tiles each, when the workspace holds the partials (workspace_bytes 0: no split). Each token
  // tile divides its own key tiles among the splits (split_tiles); max_kv_len (if positive, else
  // the block table's reach) only sizes the estimate that picks the split count. The split count
  // minimises an estimate in microseconds fitted on MI355X: (tiles per split + 4.8, a workgroup's
  // fixed cost) x 1.8 us with at most one workgroup per CU, else x 2.1 us per round of resident
  // workgroups, plus, when split, the merge (a launch, then its bytes at 5 TB/s or 0.6 ns per
  // (token, head), whichever is longer); a split must beat the one-kernel estimate by 20%. Whole
  // rounds matter: one row of 256 new tokens after 2048 (64 workgroups) took 39 us in 8 splits
  // (512 workgroups, one round of two per CU) and 49 us in 9. The merge's per-(token, head) cost
  // decides for many short rows: 24 rows of 32 new tokens after 512 took 26.6 us unsplit and
  // 44.9 in 2 splits. A grid with a workgroup on every CU gains nothing (4 rows of 256 after
  // 8192: 256 workgroups, 237 us either way) and is not split.
  const int64_t row_tokens = gy * tokens_per_wg;
  auto partial_bytes = [&](int64_t splits) {
    return context_partial_bytes(num_rows, row_tokens, num_q_heads, head_dim, splits);
  };
  int64_t kv_splits = 1, split_from = INT32_MAX;
  const int64_t base_wgs = gx * gy * num_rows;
  if (workspace != nullptr && workspace_bytes > 0 && (reinterpret_cast<uintptr_t>(workspace) & 15u) == 0) {
    int cus = 0;
    if (const int st = device_cu_count(&cus); st != MAS_OK) return st;
    const int64_t resident = static_cast<int64_t>(cus) * (8 / waves);
    const int64_t max_tiles = cdiv(cap, kTileP);
    const int64_t hint_tiles = max_kv_len > 0 ? std::min(max_tiles, cdiv(max_kv_len, kTileP)) : max_tiles;
    if (base_wgs < cus && num_rows * row_tokens * num_q_heads <= INT32_MAX) {
      const double merges = static_cast<double>(num_rows * row_tokens * num_q_heads);
      auto cost = [&](int64_t k, int64_t tiles) {  // microseconds
        const int64_t wgs = base_wgs * k;
        const double per_wg = static_cast<double>(tiles) + 4.8;
        double t = wgs <= cus ? per_wg * 1.8 : static_cast<double>(cdiv(wgs, resident)) * per_wg * 2.1;
        if (k > 1) t += 2.0 + std::max(static_cast<double>(partial_bytes(k)) / 5.0e6, merges * 6.0e-4);
        return t;
      };
      // The best split count for token tiles that all reach `reach` key tiles (1: no split).
      // at most two rounds of resident workgroups: a split grid whose rows turn out shorter than
      // the hint (tiles below split_from are not split) pays for its empty workgroups
      const int64_t grid_most = std::max<int64_t>(1, 2 * resident / base_wgs);
      auto best_splits = [&](int64_t reach) {
        const int64_t most = std::min<int64_t>({kMaxCtxSplits, reach / 4, 65535 / num_rows, grid_most});
        double best = 0.8 * cost(1, reach);
        int64_t k_best = 1;
        for (int64_t k = 2; k <= most; ++k) {
          const int64_t tiles = cdiv(reach, k);
          if (cdiv(reach, tiles) != k) continue;  // the same split as a smaller count
          if (partial_bytes(k) > workspace_bytes) break;
          if (const double c = cost(k, tiles); c < best) {
            best = c;
            k_best = k;
          }
        }
        return k_best;
      };
      kv_splits = best_splits(hint_tiles);
      if (kv_splits > 1) {
        // The shortest reach (in powers of two) worth splitting: tiles of rows shorter than the
        // hint (a graph's table far wider than its rows) are computed whole when splitting them
        // would cost more than it saves.
        split_from = hint_tiles;
        for (int64_t reach = 4; reach < hint_tiles; reach *= 2)
          if (best_splits(reach) > 1) {
            split_from = reach;
            break;
          }
      }
    }
  }
  int log2_page = 0;
  while ((int64_t{1} << log2_page) < page_size) ++log2_page;
  ContextArgs a{};
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
  a.cu_seqlens_q = cu_seqlens_q;
  a.hq = static_cast<int>(num_q_heads);
  a.hk = static_cast<int>(num_kv_heads);
  a.group = static_cast<int>(group);
  a.heads_per_wg = heads_per_wg;
  a.log2_page = log2_page;
  a.scale_log2 = bmm1_scale * 1.4426950408889634f;
  a.out_scale = bmm2_scale;
  a.out = out;
  a.out_stride = out_stride;
  a.out_head_stride = out_head_stride;
  a.out_fp8 = out_fp8 != 0;
  a.quant_scale_dev = out_scale_dev;
  a.quant_scale_host = out_scale_host;
  a.err = err;
  a.kv_splits = static_cast<int>(kv_splits);
  a.row_tokens = static_cast<int>(row_tokens);
  a.split_from = static_cast<int>(split_from);
  a.part_o = static_cast<float*>(workspace);
  a.part_ml = kv_splits > 1 ? a.part_o + num_rows * row_tokens * num_q_heads * kv_splits * head_dim : nullptr;
  const dim3 grid(static_cast<uint32_t>(gx), static_cast<uint32_t>(gy), static_cast<uint32_t>(num_rows * kv_splits));
  // Page mode: a tile within one page, a thread-row step within one or two pages, or per lane.
  const int64_t pos_step = 64 * waves / (head_dim / 8);
  const int mode = page_size >= kTileP     ? kPagesTile
                   : page_size >= pos_step ? kPagesStep1
                   : 2 * page_size >= pos_step ? kPagesStep
                                               : kPagesLane;
  const dim3 block(static_cast<uint32_t>(64 * waves));
  if (kv_splits > 1) launch_context<true>(head_dim, waves, mode, grid, block, stream, a);
  else launch_context<false>(head_dim, waves, mode, grid, block, stream, a);
  if (const int st = launch_status(); st != MAS_OK || kv_splits == 1) return st;
  const int64_t merges = num_rows * row_tokens * num_q_heads;  // <= INT32_MAX when split
  if (head_dim == 64)
    hipLaunchKernelGGL(context_combine<64>, dim3(static_cast<uint32_t>(merges)), dim3(64), 0, stream, a,
                       static_cast<int>(tokens_per_wg));
  else
    hipLaunchKernelGGL(context_combine<128>, dim3(static_cast<uint32_t>(merges)), dim3(64), 0, stream, a,
                       static_cast<int>(tokens_per_wg));
  return launch_status();
}

extern "C" int64_t mas_paged_context_attention_workspace_bytes(int64_t num_rows, int64_t max_q_len,
                                                                int64_t num_q_heads, int64_t num_kv_heads,
                                                                int64_t head_dim) {
  using namespace mas;
  if (num_rows < 0 || max_q_len < 0 || num_q_heads < 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      (head_dim != 64 && head_dim != 128))
    return -1;
  const int64_t tokens = context_launch(num_q_heads / num_kv_heads).tokens_per_wg;
  return context_partial_bytes(num_rows, cdiv(max_q_len, tokens) * tokens, num_q_heads, head_dim, kMaxCtxSplits);
}
