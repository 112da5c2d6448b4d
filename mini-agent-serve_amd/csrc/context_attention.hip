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
//   wavefront's 32 query rows, held in registers), causal mask, online softmax per query row (its
//   running max moved only by rises of more than 2^8 in p, so O is seldom rescaled), then
//   O^T += V^T P^T on MFMA, where P^T is packed to bf16 straight from the S^T accumulators and V^T
//   is read from the row-major value tile with gfx950's transposing LDS read (ds_read_b64_tr_b16:
//   in each group of 16 lanes, lane 4a + b receives element b of the 4-element rows that lanes
//   a, a + 4, a + 8, a + 12 point at), two per operand, in the position order the packing implies.
// Tiles are software-pipelined over two LDS buffers each of keys and values: while tile i is in the
// softmax, tile i + 1's score MFMAs run. With pages of at least a tile, the tiles go to LDS by DMA,
// keys a tile ahead of values (tile i + 2's keys and tile i + 1's values in flight), one barrier
// per tile; smaller pages stage tile i + 2 through registers, two barriers per tile.
#include <algorithm>

#include "device.h"

namespace mas {
namespace {

constexpr int kTileP = 64;        // key positions per tile
constexpr int kRowsPerWave = 32;  // query rows (tokens of one head) per wavefront
constexpr int kMaxCtxSplits = 32;  // split-KV: key-range splits per token tile, at most
constexpr float kNegInf = -__builtin_huge_valf();
// The online softmax's lazy reference point: p = 2^(s c - m c) stays below 2^kLazyLog2.
constexpr float kLazyLog2 = 8.f;

typedef int i32x4 __attribute__((ext_vector_type(4)));

// How a launch maps workgroups to work:
//   kWorkGrid  - one workgroup per (kv head block, token tile, row) of the host's grid;
//   kWorkSplit - the same grid with each row's token tiles split over kv_splits key ranges (the
//                split count picked on the host, from the grid's size);
//   kWorkPlan  - one workgroup per item of a plan that context_plan wrote from the real lengths on
//                the device (a graph captured with padded rows and token counts: the host only knows
//                bounds, so the split decision waits for the lengths);
//   kWorkSelfPlan - the same plan, laid out by each workgroup itself from the rows' lengths (at most
//                64 rows: one per lane), with no planner launch; the workgroups write the split
//                units the merge reads.
constexpr int kWorkGrid = 0, kWorkSplit = 1, kWorkPlan = 2, kWorkSelfPlan = 3;
constexpr int kSelfPlanMaxRows = 64;

// The planner: one workgroup; rows and (row, token tile) units it handles, at most.
constexpr int kPlanThreads = 256;
constexpr int kPlanMaxRows = 512;
constexpr int kPlanMaxUnits = 2048;
constexpr int kPlanMaxTokens = 1024;  // planned launches: the grid's token tiles cover at most this many tokens
// Planned launches: at least this many rows. The runner's graph steps have 17 prompt rows, nearly
// all padding; a grid of a few rows that fills the GPU is more likely full than padded (4 rows of
// 256 new tokens after 8192: planning it cost 5-14 us of 231).
constexpr int kPlanMinRows = 8;

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
  // The grid launch's order: (head block, row, token tile) with token tiles slowest when set, else
  // (head block, token tile, row) with rows slowest.
  int tile_major;
  float* part_o;
  float* part_ml;
  // Planned launches (kWorkPlan): the plan's counts (items, split units, splits), its items (two
  // i32x4 each: {q0, q_len, kv_len, row | split << 16 | splits << 24}, {tile | head block << 16,
  // first key tile, end key tile, partial slot or -1}) and its split units ({q0, q_len, kv_len, row},
  // {first token, splits used, splits, first partial slot}). Partials of slot s: (token of the
  // tile, head of the block, split) entries at ((s * tokens + token) * heads + head) * splits + split.
  // A self-planned launch (kWorkSelfPlan) writes plan_hdr[1] and the split units itself.
  int* plan_hdr;
  const i32x4* plan_items;
  i32x4* plan_units;
  int plan_rows, plan_gy;  // the rows and token tiles per row of the unsplit grid
  // kWorkSelfPlan: what the plan's estimate needs (CUs, resident workgroups, the grid's workgroups,
  // the partial entries the workspace holds) and the block table's reach
  int plan_cus, plan_resident;
  int plan_lt, plan_hb;  // log2 of the tokens per token tile, head blocks per (row, token tile)
  int64_t plan_item_cap, plan_entry_cap, plan_cap;
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

// A raw buffer resource: no stride, `bytes` records (a load at a byte offset past them returns
// zeros), dword 3 = 0x00020000 (the 32-bit data format that untyped buffer loads take on gfx9).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const uint16_t* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, bytes, 0x00020000);
}
// LDS DMA: lane i of the wavefront writes the 16 bytes at byte offset voffset of resource r to LDS
// address dst + 16 i (dst wavefront-uniform); zeros for an offset past the resource's records.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint16_t* dst, int voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(dst), 16, voffset, 0, 0, 0);
}
// s_waitcnt vmcnt(0) (expcnt and lgkmcnt fields at their maxima: not waited on)
constexpr int kWaitVmcnt0 = 0x0f70;

// How a tile's key / value rows find their pages (the block-table reads of a tile):
//   kPagesTile  - pages of at least a tile: the tile lies in one page, one scalar read per tile;
//   kPagesMulti8 / 16 / 32 - pages of 8, 16 or 32 slots (LDS DMA, as kPagesTile): the tile's pages
//                 are dealt out to the wavefronts, each page loaded under a buffer resource of its own;
//   kPagesLane  - pages of 1-4 slots, and layouts whose in-page byte offsets do not fit the DMA
//                 modes' 31 bits: each lane reads the page of each of its rows (vector loads) into
//                 registers, staged into LDS a tile ahead (two barriers per tile).
// Vector loads of block-table entries make the compiler wait for them, and such waits cover every
// vector load issued before them, the next tiles' key / value loads included: the DMA modes read
// them as scalars. (Modes for pages of at least a thread-row step, staged through registers with
// scalar page reads, served pages of 8-32 slots before the DMA modes.)
constexpr int kPagesLane = 0, kPagesTile = 2;
// kPagesMulti8 + i: pages of 8 << i slots (i < 3)
constexpr int kPagesMulti8 = 4, kPagesMulti16 = 5, kPagesMulti32 = 6;

// Key tiles per split of a token tile that reaches `ntiles` key tiles: its kv_splits splits share
// them evenly, at least 4 each (fewer splits then hold them all). From the tile's own reach, not
// the block table's, so that a table much wider than the rows (a graph captured for the longest
// context) still spreads each row over all the splits.
__host__ __device__ __forceinline__ int split_tiles(int ntiles, int kv_splits) {
  return max(4, (ntiles + kv_splits - 1) / kv_splits);
}

// The split count's estimate, in microseconds fitted on MI355X, for a grid of `base` workgroups
// whose token tiles each reach `tiles` key tiles, split k ways: (tiles per split + 4.8, a
// workgroup's fixed cost) x 1.8 us with at most one workgroup per CU, else x 2.1 us per round of
// resident workgroups, plus, when split, the merge (a launch, then its bytes at 5 TB/s or 0.6 ns
// per (token, head), whichever is longer). The host evaluates it for its grid, the planner for the
// real lengths.
struct SplitModel {
  int64_t base;               // workgroups of the unsplit grid
  int64_t cus, resident;      // CUs, and workgroups resident at once
  double merges;              // (token, head) pairs the merge visits
  int64_t partial_per_split;  // bytes of partials per split
  int64_t capacity;           // bytes of partials the workspace holds
  int64_t max_splits;         // splits the launch can express
};

__host__ __device__ inline double split_cost(const SplitModel& m, int64_t k, int64_t tiles) {
  const int64_t wgs = m.base * k;
  const double per_wg = static_cast<double>(tiles) + 4.8;
  double t = wgs <= m.cus ? per_wg * 1.8 : static_cast<double>((wgs + m.resident - 1) / m.resident) * per_wg * 2.1;
  if (k > 1) t += 2.0 + fmax(static_cast<double>(m.partial_per_split * k) / 5.0e6, m.merges * 6.0e-4);
  return t;
}

// The best split count for token tiles that all reach `reach` key tiles (1: no split): at most
// kMaxCtxSplits of at least 4 tiles, at most two rounds of resident workgroups (a split grid whose
// rows turn out shorter than the estimate assumed pays for its empty workgroups), partials within
// the workspace, and 20% better than one kernel.
__host__ __device__ inline int64_t best_splits(const SplitModel& m, int64_t reach) {
  const int64_t grid_most = m.base > 0 ? (2 * m.resident / m.base > 1 ? 2 * m.resident / m.base : 1) : 1;
  int64_t most = reach / 4;
  if (most > kMaxCtxSplits) most = kMaxCtxSplits;
  if (most > m.max_splits) most = m.max_splits;
  if (most > grid_most) most = grid_most;
  double best = 0.8 * split_cost(m, 1, reach);
  int64_t k_best = 1;
  for (int64_t k = 2; k <= most; ++k) {
    const int64_t tiles = (reach + k - 1) / k;
    if ((reach + tiles - 1) / tiles != k) continue;  // the same split as a smaller count
    if (m.partial_per_split * k > m.capacity) break;
    if (const double c = split_cost(m, k, tiles); c < best) {
      best = c;
      k_best = k;
    }
  }
  return k_best;
}

// The shortest reach (in powers of two from 4) worth splitting, for a split count picked at
// `hint` key tiles: token tiles reaching fewer (rows shorter than the hint, as under a graph's
// table far wider than its rows) are computed whole.
__host__ __device__ inline int64_t split_from_reach(const SplitModel& m, int64_t hint) {
  for (int64_t reach = 4; reach < hint; reach *= 2)
    if (best_splits(m, reach) > 1) return reach;
  return hint;
}

// The planner's estimate (SplitModel's terms, with the real lengths): split k ways, the longest
// unit is cut into ranges of per = max(4, ceil(longest / k)) key tiles and so is every unit longer
// than per; the rest stay whole. Its time is that of a workgroup of per tiles, (per + 4.8) x 1.8 us
// with at most one workgroup per CU, else x 2.1 us per round of resident workgroups, plus, split,
// 5 us (the merge's launch and the planner's item writes, 3 us more than an unsplit plan's on
// MI355X) and the merge: the partials' bytes at 5 TB/s or 0.9 ns per (token, head) pair of the
// split units, whichever is longer (the planned merge takes its pairs in turn on a fixed grid:
// 12,288 pairs in 9.6-11 us, against 0.6 ns per pair for the grid launch's merge, which has a
// wavefront per pair).
struct PlanModel {
  int units, head_blocks, longest;
  int cus, resident;
  int item_cap;           // workgroups of the main grid
  int64_t entry_cap;      // partial entries the workspace holds
  int entries_per_unit;   // partial entries of a split unit per split (head blocks x tokens x heads)
  float pair_us;          // merge microseconds per split unit (its (token, head) pairs)
  float entry_us;         // microseconds per partial entry moved at 5 TB/s
};

__device__ float plan_time(const PlanModel& m, int wgs, int per) {
  const float per_wg = static_cast<float>(per) + 4.8f;
  return wgs <= m.cus ? per_wg * 1.8f : static_cast<float>((wgs + m.resident - 1) / m.resident) * per_wg * 2.1f;
}

// Whether no split can pay for units reaching at most `longest` key tiles: the unsplit estimate,
// at most one workgroup per CU (else no split is weighed), against the least any split costs (a
// split length of 4 tiles in one round, plus the fixed 5 us).
__device__ bool plan_never_splits(int longest) {
  return 0.8f * ((static_cast<float>(longest) + 4.8f) * 1.8f) <= (4.f + 4.8f) * 1.8f + 5.0f;
}

// The split length for k splits, or 0 where k is not weighed (the same split as a smaller count,
// or more splits than kMaxCtxSplits).
__device__ int plan_per(const PlanModel& m, int k) {
  if (k > kMaxCtxSplits) return 0;
  const int tiles = (m.longest + k - 1) / k;
  if ((m.longest + tiles - 1) / tiles != k) return 0;
  return max(4, tiles);
}

// ---- planned launches planned in the kernels --------------------------------------------------
// With at most 64 rows (the runner's graph steps have 17), every workgroup of the attention kernel
// and of its merge lays the plan out itself from the rows' real lengths, one row per lane, instead
// of reading it from a planner launch: the same units, split count, items and partial slots as
// context_plan writes, so the same results, with one launch fewer.

// Key tiles that token tile t of a row reaches (shift = kv_len - q_len; tokens per tile 2^lt).
__device__ __forceinline__ int tile_key_tiles(int shift, int q_len, int lt, int t) {
  const int reach = shift + min((t + 1) << lt, q_len);
  return reach > 0 ? (reach + kTileP - 1) / kTileP : 0;
}

// A row as the plan sees it (this lane's row; lanes past the rows hold an empty one).
struct PlanRow {
  int q0, q_len, kv, tiles, shift;
  bool bad;  // a length error the plan reports (kv_len below q_len or past the table, or more tokens
             // than the grid's token tiles cover)
};

__device__ __forceinline__ PlanRow plan_row(const int32_t* cu_seqlens_q, const int32_t* seq_lens, int rows, int gy,
                                            int lt, int64_t cap, int lane) {
  PlanRow r{0, 0, 0, 0, 0, false};
  if (lane < rows) {
    const int q0 = cu_seqlens_q[lane];
    const int64_t q_len = static_cast<int64_t>(cu_seqlens_q[lane + 1]) - q0;
    const int64_t raw = seq_lens[lane];
    const int64_t covered = static_cast<int64_t>(gy) << lt;
    r.q0 = q0;
    r.q_len = q_len > 0 ? static_cast<int>(q_len) : 0;
    r.kv = static_cast<int>(raw < 0 ? 0 : (raw > cap ? cap : raw));
    if (q_len > 0) {
      r.tiles = static_cast<int>((min(q_len, covered) + (int64_t{1} << lt) - 1) >> lt);
      r.bad = raw < q_len || raw > cap || q_len > covered;
    }
    r.shift = r.kv - r.q_len;
  }
  return r;
}

// Token tiles of a row reaching more than p key tiles: its last ones (a tile's reach grows with it).
__device__ __forceinline__ int tiles_over(int shift, int q_len, int tiles, int lt, int p) {
  if (tiles == 0 || tile_key_tiles(shift, q_len, lt, tiles - 1) <= p) return 0;
  const int x = p * kTileP - shift;  // tile t < tiles - 1 qualifies when (t + 1) * 2^lt > x
  const int t0 = x < 0 ? 0 : x >> lt;
  return tiles - min(t0, tiles - 1);
}

// Integer quotients of small operands without the integer-division sequence: rb = rcp_small(b)
// (v_rcp_f32, within 1 ulp of 1 / b). For a numerator below 2^22 the fp32 quotient is within 3/4 of
// the real one, so one correction each way gives the exact integer result.
__device__ __forceinline__ float rcp_small(int b) { return __builtin_amdgcn_rcpf(static_cast<float>(b)); }

// floor(a / b) for 0 <= a < 2^22 and b >= 1.
__device__ __forceinline__ int floor_div_small(int a, int b, float rb) {
  int q = static_cast<int>(static_cast<float>(a) * rb);
  q -= q * b > a ? 1 : 0;
  q += (q + 1) * b <= a ? 1 : 0;
  return q;
}

// ceil(a / b) for 0 <= a, a + b <= 2^22 and b >= 1.
__device__ __forceinline__ int ceil_div_small(int a, int b, float rb) { return floor_div_small(a + b - 1, b, rb); }

__device__ __forceinline__ int lane_i(int x, int l) { return __builtin_amdgcn_readlane(x, l); }

// Minimum over the 64 lanes: DPP within rows of 16, then the four rows' minima.
__device__ __forceinline__ float wave_min_f(float v) {
  v = fminf(v, dpp_move<0xb1>(v));   // quad_perm [1,0,3,2]
  v = fminf(v, dpp_move<0x4e>(v));   // quad_perm [2,3,0,1]
  v = fminf(v, dpp_move<0x141>(v));  // row_half_mirror
  v = fminf(v, dpp_move<0x140>(v));  // row_mirror
  const auto rd = [&](int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); };
  return fminf(fminf(rd(0), rd(16)), fminf(rd(32), rd(48)));
}

// What the plan's two kernels need besides ContextArgs' fields.
struct PlanShape {
  int rows, gy, lt, head_blocks, heads_per_wg, hq, head_dim;  // token tiles of 2^lt tokens
};

// The plan's split decision, as context_plan makes it: the split count (1: none) and length, the
// rows with query tokens, and the unsplit plan's workgroups.
struct SelfPlan {
  int splits, per;
  uint64_t live;
  int grid_items;
};

// Every row-wise sum below is a scalar loop over the rows with query tokens (`live`, one to three in
// the runner's graph steps), reading each row's fields from its lane. context_plan checks after the
// split count that the plan's workgroups and partials fit; they always do: the estimate admits a
// count only if its bounds on both fit (at most (units + split units x (count - 1)) x head blocks
// workgroups, since no unit is cut into more ranges than the count, and exactly the partials).
__device__ SelfPlan self_plan(const PlanRow& r, const PlanShape& s, int cus, int resident, int64_t item_cap,
                              int64_t entry_cap, int lane) {
  const uint64_t live = __ballot(r.tiles > 0);
  SelfPlan pl{1, 0, live, s.rows * s.gy * s.head_blocks};
  int units = 0, longest = 0;
  for (uint64_t b = live; b != 0; b &= b - 1) {
    const int q = __builtin_ctzll(b), tiles = lane_i(r.tiles, q);
    units += tiles;
    longest = max(longest, tile_key_tiles(lane_i(r.shift, q), lane_i(r.q_len, q), s.lt, tiles - 1));
  }
  if (plan_never_splits(longest) || units == 0 || units * s.head_blocks >= cus) return pl;
  PlanModel m{};
  m.units = units;
  m.head_blocks = s.head_blocks;
  m.longest = longest;
  m.cus = cus;
  m.resident = resident;
  m.item_cap = static_cast<int>(item_cap);
  m.entry_cap = entry_cap;
  m.entries_per_unit = s.head_blocks * (s.heads_per_wg << s.lt);
  m.pair_us = static_cast<float>(1 << s.lt) * s.hq * 9.0e-4f;
  m.entry_us = (s.head_dim + 2) * 4.f / 5.0e6f;
  // the workgroup rounds of plan_time from a reciprocal of the resident count (every operand here
  // is below 2^22, host-checked)
  const float rres = rcp_small(resident);
  const auto time_of = [&](int wgs, int per) {
    const float per_wg = static_cast<float>(per) + 4.8f;
    return wgs <= cus ? per_wg * 1.8f : static_cast<float>(ceil_div_small(wgs, resident, rres)) * per_wg * 2.1f;
  };
  // lane l weighs l + 2 splits (plan_best_splits), counting the units longer than its split length;
  // its split length as plan_per gives it
  const int k = lane + 2;
  const int tiles_k = ceil_div_small(longest, k, rcp_small(k));
  const int per_k =
      k <= kMaxCtxSplits && ceil_div_small(longest, tiles_k, rcp_small(tiles_k)) == k ? max(4, tiles_k) : 0;
  float c = __builtin_huge_valf();
  if (per_k != 0 && per_k < longest) {
    int split = 0;
    for (uint64_t b = live; b != 0; b &= b - 1) {
      const int q = __builtin_ctzll(b);
      split += tiles_over(lane_i(r.shift, q), lane_i(r.q_len, q), lane_i(r.tiles, q), s.lt, per_k);
    }
    const int64_t wgs = static_cast<int64_t>(units + split * (k - 1)) * s.head_blocks;  // at most
    const int64_t entries = static_cast<int64_t>(split) * m.entries_per_unit * k;
    if (wgs <= m.item_cap && entries <= m.entry_cap)
      c = time_of(static_cast<int>(wgs), per_k) + 5.0f +
          fmaxf(static_cast<float>(entries) * m.entry_us, static_cast<float>(split) * m.pair_us);
  }
  const float low = wave_min_f(c);
  if (!(low < 0.8f * time_of(units * s.head_blocks, longest))) return pl;
  pl.splits = __builtin_ctzll(__ballot(c == low)) + 2;
  pl.per = max(4, ceil_div_small(longest, pl.splits, rcp_small(pl.splits)));
  return pl;
}

// Sum over the 64 lanes (|sum| < 2^31): DPP within rows of 16, then the four rows' sums.
__device__ __forceinline__ int wave_sum_i(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false);   // quad_perm [1,0,3,2]
  v += __builtin_amdgcn_update_dpp(0, v, 0x4e, 0xf, 0xf, false);   // quad_perm [2,3,0,1]
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false);  // row_half_mirror
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xf, 0xf, false);  // row_mirror
  return lane_i(v, 0) + lane_i(v, 16) + lane_i(v, 32) + lane_i(v, 48);
}

// A self-planned launch's workgroup (run by one wavefront): lays out the plan from the rows'
// lengths and finds workgroup `i`'s item in the layout of ContextArgs::plan_items. Items are in row
// order, a row's token tiles longest reach first, each tile's key ranges times the head blocks
// (head block fastest); a split plan's split units are a row's first tiles. An unsplit plan is the
// grid launch's work without its empty workgroups, in row order. Workgroup 0 also reports the rows' length errors
// and writes the split-unit count to plan_hdr[1]; the workgroup of each split unit's first range and
// head block writes the unit's plan_units entry: what context_plan writes for the merge. Returns
// false for a workgroup past the plan's items.
template <int D>
__device__ __forceinline__ bool self_plan_item(const ContextArgs& a, int lane, int i, i32x4& d0, i32x4& d1) {
  const int lt = a.plan_lt, hb = a.plan_hb;  // log2 tokens per tile, head blocks
  const float rhb = rcp_small(hb);
  const PlanShape shape{a.plan_rows, a.plan_gy, lt, hb, a.heads_per_wg, a.hq, D};
  const PlanRow r = plan_row(a.cu_seqlens_q, a.seq_lens, a.plan_rows, a.plan_gy, lt, a.plan_cap, lane);
  if (i == 0 && __ballot(r.bad) != 0 && lane == 0) report(a.err, MAS_ERRBIT_POSITION);
  // No plan has more items than every token tile cut into ranges of 4 key tiles (the shortest
  // split) per head block: workgroups past that bound leave before the plan is laid out. A row's
  // last tile reaches the most key tiles. Clamped to the grid (item_cap < 2^24, host-checked).
  int64_t cut = 0;
  if (r.tiles > 0)
    cut = static_cast<int64_t>(r.tiles) * max(1, (tile_key_tiles(r.shift, r.q_len, lt, r.tiles - 1) + 3) >> 2) * hb;
  const int bound = wave_sum_i(static_cast<int>(min(cut, a.plan_item_cap)));
  if (i >= bound) {
    if (i == 0 && lane == 0) a.plan_hdr[1] = 0;  // no query tokens
    return false;
  }
  const SelfPlan pl = self_plan(r, shape, a.plan_cus, a.plan_resident, a.plan_item_cap, a.plan_entry_cap, lane);
  const int per = pl.splits > 1 ? pl.per : (1 << 30);  // unsplit: no tile reaches past per
  const float rp = rcp_small(per);
  // each row's split tiles (its last ones) and key ranges, a row per lane
  const int sp_l = tiles_over(r.shift, r.q_len, r.tiles, lt, per);
  int rng_l = r.tiles - sp_l;
  for (int t = r.tiles - sp_l; t < r.tiles; ++t) rng_l += ceil_div_small(tile_key_tiles(r.shift, r.q_len, lt, t), per, rp);
  if (i == 0) {
    const int split_units = wave_sum_i(sp_l);
    if (lane == 0) a.plan_hdr[1] = split_units;
  }
  // the row holding item i and the split units of the rows before it
  int rl = -1, off = i, su = 0;
  for (uint64_t b = pl.live; b != 0; b &= b - 1) {
    const int q = __builtin_ctzll(b);
    const int ni = lane_i(rng_l, q) * hb;
    if (off < ni) {
      rl = q;
      break;
    }
    off -= ni;
    su += lane_i(sp_l, q);
  }
  if (rl < 0) return false;  // past the plan's items
  const int shift = lane_i(r.shift, rl), q_len = lane_i(r.q_len, rl), tiles = lane_i(r.tiles, rl);
  const int split_here = lane_i(sp_l, rl);
  // the row's split units, one per lane (lane u: tile tiles - 1 - u): their key ranges
  const int used_l = lane < split_here ? ceil_div_small(tile_key_tiles(shift, q_len, lt, tiles - 1 - lane), per, rp) : 1;
  int k = 0;
  for (; k < split_here; ++k) {
    const int nk = lane_i(used_l, k) * hb;
    if (off < nk) break;
    off -= nk;
  }
  int tile, used = 1;
  if (k < split_here) {
    tile = tiles - 1 - k;
    used = lane_i(used_l, k);
    su += k;
  } else {
    const int u = floor_div_small(off, hb, rhb);  // an unsplit tile: one item per head block
    tile = tiles - 1 - split_here - u;
    off -= u * hb;
  }
  const int nt = tile_key_tiles(shift, q_len, lt, tile);
  const int range = floor_div_small(off, hb, rhb), block = off - range * hb;
  const int len = used > 1 ? per : nt, first = range * len;
  const int q0 = lane_i(r.q0, rl), kv = lane_i(r.kv, rl);
  d0 = i32x4{q0, q_len, kv, rl | (range << 16) | (pl.splits << 24)};
  d1 = i32x4{tile | (block << 16), first, min(nt, first + len), used > 1 ? su * hb + block : -1};
  if (used > 1 && range == 0 && block == 0 && lane == 0) {
    a.plan_units[2 * su] = i32x4{q0, q_len, kv, rl};
    a.plan_units[2 * su + 1] = i32x4{tile << lt, used, pl.splits, su * hb};
  }
  return true;
}

// kWork: how workgroups map to work (each a separate instance, so that the one-kernel instances
// keep their code).
template <int D, int kPages, int kWaves, int kWork>
__global__ __launch_bounds__(64 * kWaves, 8 / kWaves) void context_attn(ContextArgs a) {
  constexpr bool kSplit = kWork == kWorkSplit;
  constexpr bool kPlan = kWork == kWorkPlan || kWork == kWorkSelfPlan;  // items from a plan
  constexpr int kCtxWaves = kWaves;
  constexpr int kCtxThreads = 64 * kWaves;
  constexpr int KS = D / 16;            // MFMA k-steps over the head dim (S^T)
  constexpr int DB = D / 32;            // 32-dim blocks of O^T
  constexpr int KROW = D + 8;           // bf16 per LDS key row (+16 B: conflict-free A reads)
  constexpr int VROW = D + 16;          // bf16 per LDS value row (+32 B: conflict-free column reads)
  constexpr int CPR = D / 8;            // 16-byte chunks per key / value row
  constexpr int LOADS = kTileP * CPR / kCtxThreads;  // 16-byte chunks per thread per tile, each of K and V
  // Two tile buffers each of keys and values: with the software pipeline, the next tile's keys are
  // read while this tile's values are. Four separate arrays, so that the compiler's wait insertion
  // tells a buffer that an LDS DMA load is filling from the ones being read.
  __shared__ __align__(16) uint16_t k_lds0[kTileP * KROW];
  __shared__ __align__(16) uint16_t k_lds1[kTileP * KROW];
  __shared__ __align__(16) uint16_t v_lds0[kTileP * VROW];
  __shared__ __align__(16) uint16_t v_lds1[kTileP * VROW];
  const auto klds = [&](int b) { return b ? k_lds1 : k_lds0; };
  const auto vlds = [&](int b) { return b ? v_lds1 : v_lds0; };

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id_uniform();
  __builtin_assume(wave >= 0 && wave < kCtxWaves);  // lets the LDS DMA dealing fold its bounds
  const int n = lane & 31, hf = lane >> 5;  // this lane's query row (token) and lane half
  const int hgroups = (a.group + a.heads_per_wg - 1) / a.heads_per_wg;
  // A planned launch's item. Unsplit plans are the grid launch's workgroups in row order (each row's
  // longest tiles first), taken from the workgroup id: their lengths are loaded in the same round
  // trip as the plan's counts (row clamped to the last), as the grid launch loads them, and no item
  // is read. Split plans' items
  // are read from the plan; workgroups past the plan's count exit (the item array holds one slot
  // per workgroup of the grid, so the load stays inside it).
  i32x4 d0{}, d1{};
  if constexpr (kWork == kWorkSelfPlan) {
    // wavefront 0 lays the plan out and hands the item to the others through LDS: the plan's uniform
    // arithmetic runs on the CU's one scalar unit, which every wavefront on the CU shares
    __shared__ i32x4 item_lds[2];
    __shared__ int item_ok;
    if (wave == 0) {
      i32x4 e0{}, e1{};
      const bool ok = self_plan_item<D>(a, lane, static_cast<int>(blockIdx.x), e0, e1);
      if (lane == 0) {
        item_ok = ok ? 1 : 0;
        item_lds[0] = e0;
        item_lds[1] = e1;
      }
    }
    __syncthreads();
    if (item_ok == 0) return;  // uniform over the workgroup
    d0 = item_lds[0];
    d1 = item_lds[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      d0[e] = __builtin_amdgcn_readfirstlane(d0[e]);
      d1[e] = __builtin_amdgcn_readfirstlane(d1[e]);
    }
  } else if constexpr (kPlan) {
    const int n_items = a.plan_hdr[0], plan_splits = a.plan_hdr[2];
    const unsigned per_row = static_cast<unsigned>(a.plan_gy) * (a.hk * hgroups);
    const unsigned grid_row = blockIdx.x / per_row, rem = blockIdx.x - grid_row * per_row;
    const int row_ld = static_cast<int>(min(grid_row, static_cast<unsigned>(a.plan_rows - 1)));
    const int cu0 = a.cu_seqlens_q[row_ld], cu1 = a.cu_seqlens_q[row_ld + 1], len = a.seq_lens[row_ld];
    if (static_cast<int>(blockIdx.x) >= n_items) return;
    if (plan_splits == 1) {
      const unsigned y = rem / (a.hk * hgroups), block = rem - y * (a.hk * hgroups);
      const int tile = a.plan_gy - 1 - static_cast<int>(y);
      d0 = i32x4{cu0, cu1 - cu0, len, row_ld | (1 << 24)};
      d1 = i32x4{tile | static_cast<int>(block << 16), 0, INT32_MAX, -1};
    } else {
      d0 = a.plan_items[2 * blockIdx.x];
      d1 = a.plan_items[2 * blockIdx.x + 1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        d0[e] = __builtin_amdgcn_readfirstlane(d0[e]);
        d1[e] = __builtin_amdgcn_readfirstlane(d1[e]);
      }
    }
  }
  const unsigned head_block = kPlan ? static_cast<unsigned>(d1[0]) >> 16 : blockIdx.x;
  const int kvh = head_block / hgroups, hg = head_block - kvh * hgroups;
  // Token tiles are launched in reverse: workgroups are dispatched in id order, and the last tiles
  // reach the most positions, so they start first. The grid launch is (head block, token tile,
  // row), or with tile_major (head block, row, token tile): then every row's longest tiles start
  // first and the short ones end the launch (longest first over the whole grid where the rows share
  // their cached lengths), which the host picks when one row's work would not cover the time of
  // its longest tile. The split launch is (head block, token tile, row x split).
  const bool tile_major = !kSplit && a.tile_major != 0;
  const unsigned tile_id = tile_major ? blockIdx.z : blockIdx.y;
  const int grid_tiles = static_cast<int>(tile_major ? gridDim.z : gridDim.y);
  const int row = kPlan ? d0[3] & 0xffff : (kSplit ? blockIdx.z / a.kv_splits : (tile_major ? blockIdx.y : blockIdx.z));
  const int split = kPlan ? (d0[3] >> 16) & 0xff : (kSplit ? blockIdx.z - row * a.kv_splits : 0);
  const int q0 = kPlan ? d0[0] : a.cu_seqlens_q[row];
  const int q_len = kPlan ? d0[1] : a.cu_seqlens_q[row + 1] - q0;
  const int tokens_per_wg = kRowsPerWave * (kCtxWaves / a.heads_per_wg);
  const int tile_idx = kPlan ? d1[0] & 0xffff : grid_tiles - 1 - static_cast<int>(tile_id);
  const int tile_tok = tile_idx * tokens_per_wg;
  if (tile_tok >= q_len) return;  // uniform over the workgroup
  // kv_len clamped to the block table's reach; a kv_len below q_len leaves the first tokens with
  // negative positions: they see no key and get zeros.
  const int64_t cap = a.max_blocks << a.log2_page;
  const int64_t raw_len = kPlan ? d0[2] : a.seq_lens[row];
  // Error bits are reported at the end: a global atomic before the tile loop would keep the
  // compiler from reading the block table through the scalar cache.
  // also flagged: a row with more query tokens than the grid covers (max_q_len too small); the
  // tokens past the grid are left unwritten. The planner reports these for planned launches.
  const bool len_bad =
      !kPlan && (raw_len < q_len || raw_len > cap || q_len > grid_tiles * tokens_per_wg);
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
  // This workgroup's key tiles: all of them, or its split's share (a planned item carries its range).
  const bool split_tile = kPlan ? d1[3] >= 0 : kSplit && ntiles >= a.split_from;
  const int per_split = split_tile && !kPlan ? split_tiles(ntiles, a.kv_splits) : ntiles;
  const int it_begin = kPlan ? max(d1[1], 0) : (kSplit ? split * per_split : 0);
  const int it_end = kPlan ? min(d1[2], ntiles)
                           : (!split_tile || split == a.kv_splits - 1 ? ntiles : min(ntiles, it_begin + per_split));
  // an empty split (uniform), which the merge skips; split 0 of a tile that is not split goes on,
  // to write its output (zeros for a tile that reaches no key)
  if (kSplit && it_begin >= it_end && (split_tile || split > 0)) {
    if (len_bad && tid == 0 && blockIdx.x == 0 && tile_idx == 0 && split == 0) report(a.err, MAS_ERRBIT_POSITION);
    return;
  }

  float m_run = kNegInf, l_run = 0.f;  // token n's running max (raw score units) and this half's sum
  f32x16 acc[DB];                      // O^T: element j of block db holds O[token n][32 db + 8 (j/4) + 4 hf + j%4]
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};

  const int32_t* bt = a.block_tables + row * a.bt_stride;
  const int pmask = (1 << a.log2_page) - 1;
  // kPagesLane, a thread's chunks of a tile: chunk c = tid + T u (T threads) -> position tid / CPR +
  // (T / CPR) u, head-dim chunk tid % CPR (the same for every u). The rows' validity flags are kept
  // so that the loads themselves are not waited on before the stores.
  constexpr int kPosStep = kCtxThreads / CPR;
  const int dcol = tid % CPR, prow = tid / CPR;
  struct TileRegs {
    u32x4 k[LOADS], v[LOADS];
    bool lok[LOADS];
    bool full;  // every chunk of the tile valid: stores need no zeroing
  };
  bool page_bad = false;  // a real position's page id outside the cache (reported once, at the end)
  const int last_page = kv_len > 0 ? (kv_len - 1) >> a.log2_page : 0;  // the sequence's last block-table entry

  // ---- Pages of at least 8 slots (kDirect): the tiles go to LDS by DMA (buffer_load ... lds), with
  // no registers or stores in between. A wavefront's load instruction fills 64 consecutive 16-byte
  // slots of an LDS tile buffer, lane i slot i. The buffers keep their row padding (SK / SV slots per
  // key / value row, the last one or two of them padding), so lane i of an instruction that starts
  // at a row's first slot loads row i / S, head-dim chunk i % S of the rows from there (a padding
  // slot loads the row's last chunk once more). The rows are read through a buffer resource based at
  // the first row of the tile (one-page tiles) or of the page (kMulti) of this kv head, its records
  // ending after the last position below kv_len (none for a page id outside the cache): the rows past
  // them arrive as zeros. The host keeps this mode to layouts whose in-page byte offsets fit 31 bits.
  constexpr bool kMulti = kPages >= kPagesMulti8;
  constexpr bool kDirect = kPages == kPagesTile || kMulti;
  constexpr int SK = KROW / 8, SV = VROW / 8;  // 16-byte slots per LDS key / value row
  constexpr int NK = (SK + kCtxWaves - 1) / kCtxWaves, NV = (SV + kCtxWaves - 1) / kCtxWaves;
  // One-page tiles: instruction ii fills slots 64 ii .. 64 ii + 63 of the buffer, ii = wave + W j for
  // this wavefront's j, and each lane keeps the byte offset of its row and chunk from the tile's
  // first row.
  // kMulti: page q of the tile (PS rows) fills the buffer's slots from q PS S on, in MQ = ceil(PS S /
  // 64) instructions 64 slots apart (the last one with only the lanes inside the page's region).
  // Page q is wavefront q % W's, and each lane keeps the byte offset of its row and chunk from the
  // start of the page for each k < MQ (the same for every page).
  constexpr int PS = kMulti ? (8 << (kPages - kPagesMulti8)) : kTileP;  // rows per page (kMulti)
  constexpr int PT = kTileP / PS;                                         // pages per tile
  constexpr int PPW = (PT + kCtxWaves - 1) / kCtxWaves;                   // pages per wavefront, at most
  constexpr int MQK = kMulti ? (PS * SK + 63) / 64 : NK, MQV = kMulti ? (PS * SV + 63) / 64 : NV;
  int koff[MQK], voff[MQV];
  if constexpr (kDirect) {
    auto place = [&](int s, int S) {
      return static_cast<int>((s / S) * a.entry_stride) * 2 + 16 * min(s % S, CPR - 1);
    };
#pragma unroll
    for (int j = 0; j < MQK; ++j) koff[j] = place(64 * (kMulti ? j : wave + kCtxWaves * j) + lane, SK);
#pragma unroll
    for (int j = 0; j < MQV; ++j) voff[j] = place(64 * (kMulti ? j : wave + kCtxWaves * j) + lane, SV);
  }
  struct TileRsrc {
    __amdgpu_buffer_rsrc_t k, v;
  };
  // The block table through the constant address space: a scalar load (the DMA instructions would
  // otherwise keep the compiler from proving the table unwritten, and it would load the page id
  // with a vector load and wait on every load in flight).
  const auto bt_const = (const __attribute__((address_space(4))) int32_t*)(bt);
  auto tile_rsrc = [&](int base) {
    const int32_t page = bt_const[base >> a.log2_page];
    const bool ok = page >= 0 && page < a.num_pages;
    page_bad |= !ok;
    const int64_t off = (ok ? static_cast<int64_t>(page) : 0) * a.page_stride +
                        static_cast<int64_t>(base & pmask) * a.entry_stride + kvh * a.head_stride;
    const int bytes = ok ? static_cast<int>(min(kTileP, kv_len - base) * a.entry_stride) * 2 : 0;
    return TileRsrc{make_rsrc(a.k_cache + off, bytes), make_rsrc(a.v_cache + off, bytes)};
  };
  // kMulti: the resource of page q of the tile at `base` (pages start at multiples of their size,
  // and tiles at multiples of 64): based at the page's first row of this kv head, its records ending
  // after the page's last position below kv_len. A page wholly past kv_len has no records (its
  // block-table entry, read clamped to the sequence's last one, is not used).
  auto page_rsrc = [&](const uint16_t* cache, int base, int q) {
    const int pos = base + q * PS;
    // (readfirstlane: the clamp is selected as a vector med3, and a resource dword in a vector
    // register would make the compiler loop over its distinct values)
    const int rows = __builtin_amdgcn_readfirstlane(max(0, min(kv_len - pos, PS)));
    const int32_t page = bt_const[min(pos >> a.log2_page, last_page)];
    const bool ok = page >= 0 && page < a.num_pages;
    page_bad |= rows > 0 && !ok;
    const int64_t off = (ok ? static_cast<int64_t>(page) : 0) * a.page_stride + kvh * a.head_stride;
    return make_rsrc(cache + off, ok ? static_cast<int>(rows * a.entry_stride) * 2 : 0);
  };
  // One tile's keys or values into `dst`, this wavefront's instructions. The LDS addresses are
  // formed where the loads issue (the opaque copy of the buffer's address keeps the compiler from
  // hoisting twenty of them out of the tile loop into spilled registers).
  auto dma_part = [&](bool keys, int base, uint16_t* dst) {
    const uint16_t* cache = keys ? a.k_cache : a.v_cache;
    uint16_t* d = dst;
    asm volatile("" : "+s"(d));
    if constexpr (kMulti) {
#pragma unroll
      for (int pj = 0; pj < PPW; ++pj) {
        const int q = wave + kCtxWaves * pj;
        if (q >= PT) continue;  // wavefront-uniform
        const __amdgpu_buffer_rsrc_t r = page_rsrc(cache, base, q);
        const int S = keys ? SK : SV;
        uint16_t* dq = d + 8 * q * PS * S;
        constexpr int MQ = MQK > MQV ? MQK : MQV;
#pragma unroll
        for (int k = 0; k < MQ; ++k) {
          if (k >= (keys ? MQK : MQV)) continue;
          const int nact = min(64, PS * S - 64 * k);  // a constant
          const int off = keys ? koff[k] : voff[k];
          if (nact == 64 || lane < nact) dma16(r, dq + 512 * k, off);
        }
      }
    } else {
      const TileRsrc t = tile_rsrc(base);
      constexpr int N = NK > NV ? NK : NV;
#pragma unroll
      for (int j = 0; j < N; ++j) {
        if (keys ? j >= NK : j >= NV) continue;
        const int m = wave + kCtxWaves * j;
        if (m >= (keys ? SK : SV)) continue;
        dma16(keys ? t.k : t.v, d + 512 * m, keys ? koff[j] : voff[j]);
      }
    }
  };
  auto dma_keys = [&](int base, uint16_t* dst) { dma_part(true, base, dst); };
  auto dma_values = [&](int base, uint16_t* dst) { dma_part(false, base, dst); };

  // kPagesLane: each lane reads the page of each of its rows; rows past kv_len load the sequence's
  // last row and are zeroed when staged, as are rows on a page id outside the cache (page 0 read).
  auto issue_tile = [&](TileRegs& tr, int base) {
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
  };
  // The tile in `tr` into LDS buffer `buf` (rows past kv_len or on a bad page zeroed).
  auto stage = [&](const TileRegs& tr, int buf) {
    uint16_t* k_lds = klds(buf);
    uint16_t* v_lds = vlds(buf);
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
    const uint16_t* k_lds = klds(buf);
    bf16x8 ka[KS][2];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
        ka[ks][pb] = *reinterpret_cast<const bf16x8*>(k_lds + (32 * pb + n) * KROW + 16 * ks + 8 * hf);
    s[0] = f32x16{};
    s[1] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) s[pb] = mfma32(ka[ks][pb], qb[ks], s[pb]);
    // the key reads run four ahead of the MFMAs that take them (the compiler's own order kept two in
    // flight; eight ahead spills): 4 reads, then (MFMA, read) pairs, then the last 4 MFMAs
    constexpr int kAhead = 4;
    __builtin_amdgcn_sched_group_barrier(0x100, kAhead, 0);  // DS reads
#pragma unroll
    for (int i = 0; i < 2 * KS - kAhead; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // an MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // a DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, kAhead, 0);
  };
  // ---- causal mask, only on tiles that cross the diagonal of the wavefront's first row or the end
  // of the sequence (a wavefront-uniform branch)
  auto mask = [&](f32x16 (&s)[2], int base) {
    if (base + kTileP - 1 > shift + tok || base + kTileP > kv_len) {
      // position kp is masked past min(this lane's query position, kv_len - 1); element j of s[pb]
      // sits at kp = base + 4 hf + (32 pb + 8 (j / 4) + j % 4), the bracket a constant
      const int lim = min(shift + tok + n, kv_len - 1) - base - 4 * hf;
#pragma unroll
      for (int pb = 0; pb < 2; ++pb)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (32 * pb + 8 * (j >> 2) + (j & 3) > lim) s[pb][j] = kNegInf;
    }
  };
  // ---- online softmax per query row; scores stay in raw units, the scale enters the exponent
  // through one fma: p = 2^(s c - m c). The reference point m is lazy: a row moves it only to a max
  // more than kLazyLog2 above it (in exponent units), so p stays below 2^kLazyLog2 and O and l are
  // rescaled (64 multiplies per lane) only when some row of the wavefront moved from a finite m;
  // otherwise the stale m holds. bf16 P and the fp32 sums carry the same relative precision at any
  // such magnitude, and O / l does not depend on m. The split partials carry this m with their sums.
  // A row's 64 scores of a tile sit in lanes n and n + 32 (32 each). Whether any row must move its m
  // is decided from each lane's own half (max(a, b) c exceeds a bound iff a c or b c does, c > 0), so
  // the two halves exchange their maxima only on the seldom path that moves some m; each lane keeps
  // its half's sum in l_run, and the halves are added once, after the last tile.
  // P^T is packed to bf16 as the B operands of O^T += V^T P^T: k-step kk = positions 16 kk ..
  // 16 kk + 15, lane half hf holding 16 kk + 4 hf + e (e < 4) and 16 kk + 8 + 4 hf + e - 4 (e >= 4),
  // i.e. elements 8 (kk % 2) .. + 7 of s[kk / 2].
  auto softmax = [&](f32x16 (&s)[2], bf16x8 (&pbo)[4]) {
    float mh = kNegInf;  // this lane's half of the row
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int j = 0; j < 16; ++j) mh = fmaxf(mh, s[pb][j]);
    // a row's first finite score (m = -inf) always moves it; -inf against -inf does not
    const float bound = m_run * c + kLazyLog2;
    if (__builtin_amdgcn_ballot_w64(mh * c > bound) != 0) {  // wavefront-uniform
      const float mx = fmaxf(mh, __shfl_xor(mh, 32));        // the row's max, the same in both halves
      const bool grow = mx * c > bound;
      // rows that had no finite score have O = 0 and l = 0: their factor is 1
      const float alpha = grow && m_run != kNegInf ? __builtin_amdgcn_exp2f(__builtin_fmaf(m_run, c, -(mx * c))) : 1.f;
      if (grow) m_run = mx;
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db) acc[db] *= alpha;
      }
    }
    const float mc = (m_run == kNegInf ? 0.f : m_run) * c;
    float sum = 0.f;
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        s[pb][j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[pb][j], c, -mc));
        sum += s[pb][j];
      }
    l_run += sum;  // this half's share
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int o = 8 * (kk & 1);
      const f32x16& sv = s[kk >> 1];
      const u32x4 packed = {pack_bf16x2(sv[o], sv[o + 1]), pack_bf16x2(sv[o + 2], sv[o + 3]),
                            pack_bf16x2(sv[o + 4], sv[o + 5]), pack_bf16x2(sv[o + 6], sv[o + 7])};
      pbo[kk] = __builtin_bit_cast(bf16x8, packed);
    }
  };
  // ---- O^T += V^T P^T: A = V^T[32 dims][16 positions], read transposed from the row-major value
  // tile in the position order of pbo
  auto pv = [&](int buf, const bf16x8 (&pbo)[4]) {
    const uint16_t* v_lds = vlds(buf);
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
  // Buffer (it - it_begin) & 1 holds tile it, the other one tile it + 1 (staged after the barrier
  // that ends every read of tile it - 1, which used that buffer). The parity is counted from the
  // workgroup's first tile, so that it is a constant at each call of step even where the first tile
  // is not known at compile time (split ranges): LDS addresses then fold into the instructions.
  // With LDS DMA (kDirect) the keys run a tile ahead of the values: in step it, key buffer buf ^ 1
  // holds tile it + 1 and the DMA fills key buffer buf (tile it's keys, read in step it - 1) with
  // tile it + 2 and value buffer buf ^ 1 (tile it - 1's values) with tile it + 1. One barrier per
  // step, after this wavefront's DMA of the previous step has landed, covers both: every wavefront's
  // loads are in LDS, and every read of the buffers refilled next is done.
  f32x16 s_a[2], s_b[2];
  if (it_begin < it_end) {
    if constexpr (kDirect) {
      dma_keys(it_begin * kTileP, klds(0));
      dma_values(it_begin * kTileP, vlds(0));
      if (it_begin + 1 < it_end) dma_keys((it_begin + 1) * kTileP, klds(1));
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      __syncthreads();
    } else {
      issue_tile(tr, it_begin * kTileP);
      stage(tr, 0);
      __syncthreads();
      if (it_begin + 1 < it_end) issue_tile(tr, (it_begin + 1) * kTileP);
    }
    if (wave_live) scores(0, s_a);
  }
  // One tile in buffer `buf`; `cur` holds its scores, `nxt` receives the next tile's. Called with
  // the two score arrays in turn (no copy between them).
  auto step = [&](int it, int buf, f32x16 (&cur)[2], f32x16 (&nxt)[2]) {
    if constexpr (kDirect) {
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      __syncthreads();
      if (it + 1 < it_end) dma_values((it + 1) * kTileP, vlds(buf ^ 1));
      if (it + 2 < it_end) dma_keys((it + 2) * kTileP, klds(buf));
    } else {
      __syncthreads();  // tile it - 1's reads (of buffer buf ^ 1) are done
      if (it + 1 < it_end) stage(tr, buf ^ 1);
      __syncthreads();
      if (it + 2 < it_end) issue_tile(tr, (it + 2) * kTileP);
    }
    if (wave_live) {
      mask(cur, it * kTileP);
      bf16x8 pbo[4];
      scores(buf ^ 1, nxt);  // the next tile's (stale buffer contents after the last tile: unused)
      softmax(cur, pbo);
      pv(buf, pbo);
    }
  };
  int it = it_begin;
  for (; it + 1 < it_end; it += 2) {
    step(it, 0, s_a, s_b);
    step(it + 1, 1, s_b, s_a);
  }
  if (it < it_end) step(it, 0, s_a, s_b);
  if (__builtin_amdgcn_ballot_w64(page_bad) != 0 && lane == 0) report(a.err, MAS_ERRBIT_PAGE);
  // reported by the workgroup of token tile 0, which every row with a query token has
  if (len_bad && tid == 0 && blockIdx.x == 0 && tile_idx == 0) report(a.err, MAS_ERRBIT_POSITION);

  if (!wave_live) return;
  l_run += __shfl_xor(l_run, 32);  // the row's sum: both halves' shares
  const int t = tok + n;
  if (t >= q_len) return;
  if (split_tile) {
    // ---- this split's partial: O row (lane half hf holds columns 32 db + 8 q + 4 hf .. + 3) and
    // (max, sum), both halves holding the same (max, sum)
    const int64_t pi =
        kPlan ? ((static_cast<int64_t>(d1[3]) * tokens_per_wg + (t - tile_tok)) * a.heads_per_wg + hsub) *
                        ((d0[3] >> 24) & 0xff) + split
              : ((static_cast<int64_t>(row) * a.row_tokens + t) * a.hq + h) * a.kv_splits + split;
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

// Merges one (token, query head)'s nsplit partials, stored from index `base` on, with weights
// 2^(c (m_s - max m)) (c = bmm1_scale * log2 e, maxima in raw score units as the split kernel keeps
// them) and writes O / l * bmm2_scale as bf16, or its fp8 quantize, to output token `token`, head
// `h`. Every load is issued in one round trip: lane s reads split s's (max, sum) and 16 (32 past 16
// splits) partial O rows are loaded (indices past the last split clamped to it, weighted 0) before
// the max is known. A token that sees no position (all maxima -inf) gets zeros.
template <int D>
__device__ __forceinline__ void merge_partials(const ContextArgs& a, int64_t base, int nsplit, int64_t token, int h,
                                               int lane) {
  constexpr int DPL = D / 64;  // head-dim elements per lane
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
  const int64_t at = token * a.out_stride + h * a.out_head_stride + DPL * lane;
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

// One wavefront per (row, token, query head) of a split-KV launch: merges the token's non-empty
// splits (merge_partials).
template <int D>
__global__ __launch_bounds__(64) void context_combine(ContextArgs a, int tokens_per_wg) {
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
  merge_partials<D>(a, base, nsplit, q0 + t, h, lane);
}

// The merge of a planned launch: its split units' (token, query head) pairs, one per wavefront in
// turn (a fixed grid: the plan's size is known only on the device).
constexpr int kMergeWaves = 8;  // wavefronts per workgroup of the planned merge

template <int D>
__global__ __launch_bounds__(64 * kMergeWaves) void context_combine_plan(ContextArgs a, int tokens_per_wg) {
  const int lane = threadIdx.x & 63;
  const int n_units = a.plan_hdr[1];
  const int per_unit = tokens_per_wg * a.hq;  // pairs per split unit; n_units * per_unit <= 2^31 - 1 (host-checked)
  const int total = n_units * per_unit;
  const int hgroups = (a.group + a.heads_per_wg - 1) / a.heads_per_wg;
  const int waves = static_cast<int>(gridDim.x) * kMergeWaves;
  for (int m = static_cast<int>(blockIdx.x) * kMergeWaves + wave_id_uniform(); m < total; m += waves) {
    const int su = m / per_unit, r = m - su * per_unit;
    const int j = r / a.hq, h = r - j * a.hq;  // token of the unit's tile, query head
    const i32x4 u0 = a.plan_units[2 * su], u1 = a.plan_units[2 * su + 1];
    const int q0 = __builtin_amdgcn_readfirstlane(u0[0]), q_len = __builtin_amdgcn_readfirstlane(u0[1]);
    const int t = __builtin_amdgcn_readfirstlane(u1[0]) + j;
    if (t >= q_len) continue;
    const int nsplit = __builtin_amdgcn_readfirstlane(u1[1]), splits = __builtin_amdgcn_readfirstlane(u1[2]);
    const int kvh = h / a.group, g = h - kvh * a.group, hg = g / a.heads_per_wg, hs = g - hg * a.heads_per_wg;
    const int slot = __builtin_amdgcn_readfirstlane(u1[3]) + kvh * hgroups + hg;
    const int64_t base = ((static_cast<int64_t>(slot) * tokens_per_wg + j) * a.heads_per_wg + hs) * splits;
    merge_partials<D>(a, base, nsplit, q0 + t, h, lane);
  }
}

// ---- the planner of planned launches ----------------------------------------------------------

struct PlanArgs {
  const int32_t* cu_seqlens_q;
  const int32_t* seq_lens;
  int rows, gy, tokens_per_wg, heads_per_wg, head_blocks, hq, head_dim;
  int64_t cap;         // positions the block table reaches
  int64_t cus, resident;
  int64_t item_cap;    // items the main grid has workgroups for
  int64_t entry_cap;   // partial entries ((token, head, split)) the workspace holds
  int* hdr;
  i32x4* items;
  i32x4* units;
  uint32_t* err;
};

// Exclusive prefix sum of v[0..n) in place, v[n] = the total, which every thread gets back.
__device__ int plan_scan(int* v, int n, int* slots) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __syncthreads();  // v written, slots free
  const int per = (n + kPlanThreads - 1) / kPlanThreads;
  const int lo = min(n, tid * per), hi = min(n, lo + per);
  int sum = 0;
  for (int i = lo; i < hi; ++i) sum += v[i];
  int x = sum;  // inclusive scan over the wavefront
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  if (lane == 63) slots[wave] = x;
  __syncthreads();
  int run = x - sum, total = 0;
#pragma unroll
  for (int w = 0; w < kPlanThreads / 64; ++w) {
    if (w < wave) run += slots[w];
    total += slots[w];
  }
  for (int i = lo; i < hi; ++i) {
    const int c = v[i];
    v[i] = run;
    run += c;
  }
  if (tid == 0) v[n] = total;
  __syncthreads();
  return total;
}

__device__ int plan_max(int x, int* slots) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) x = max(x, __shfl_xor(x, d));
  __syncthreads();
  if ((tid & 63) == 0) slots[tid >> 6] = x;
  __syncthreads();
  int m = slots[0];
#pragma unroll
  for (int w = 1; w < kPlanThreads / 64; ++w) m = max(m, slots[w]);
  return m;
}

// The estimate for k > 1 splits (infinite if the grid or the workspace would not hold them); the
// unit lengths are read from LDS, the same address in every lane.
__device__ float plan_split_cost(const PlanModel& m, const int* u_nt, int k) {
  const int per = plan_per(m, k);
  if (per == 0 || per >= m.longest) return __builtin_huge_valf();
  int split = 0;  // units longer than per
  for (int u = 0; u < m.units; ++u) split += u_nt[u] > per ? 1 : 0;
  const int64_t wgs = static_cast<int64_t>(m.units + split * (k - 1)) * m.head_blocks;  // at most
  const int64_t entries = static_cast<int64_t>(split) * m.entries_per_unit * k;
  if (wgs > m.item_cap || entries > m.entry_cap) return __builtin_huge_valf();
  return plan_time(m, static_cast<int>(wgs), per) + 5.0f +
         fmaxf(static_cast<float>(entries) * m.entry_us, static_cast<float>(split) * m.pair_us);
}

// The split count, lane l weighing l + 2 splits: the smallest count of least estimate if it beats
// one kernel by 20%, else 1.
__device__ int plan_best_splits(const PlanModel& m, const int* u_nt, int lane) {
  const float c = plan_split_cost(m, u_nt, lane + 2);
  float low = c;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) low = fminf(low, __shfl_xor(low, d));
  if (!(low < 0.8f * plan_time(m, m.units * m.head_blocks, m.longest))) return 1;
  return __builtin_ctzll(__ballot(c == low)) + 2;
}

// Lays out a planned launch from the real lengths (one workgroup). Units are a row's token tiles,
// longest reach first. The split count comes from PlanModel's estimate; a unit longer than the
// split length is cut into ranges of that length, each range an item per head block, and its
// partials get a slot per head block; every other unit is one item per head block that writes its
// output. Rows' length errors are reported here, as the grid launch reports them (a row with query
// tokens: kv_len below q_len or past the block table, or more tokens than the grid's token tiles
// cover, which are left unwritten).
__global__ __launch_bounds__(kPlanThreads) void context_plan(PlanArgs p) {
  __shared__ int r_q0[kPlanMaxRows], r_qlen[kPlanMaxRows], r_kv[kPlanMaxRows], r_unit[kPlanMaxRows + 1];
  __shared__ int u_row[kPlanMaxUnits], u_tile[kPlanMaxUnits], u_nt[kPlanMaxUnits];
  __shared__ int u_item[kPlanMaxUnits + 1], u_slot[kPlanMaxUnits + 1];
  __shared__ int slots[kPlanThreads / 64];
  __shared__ int params[1];
  const int tid = threadIdx.x;

  // rows: lengths and token tiles
  bool bad = false;
  int reach_bound = 0;  // key tiles of the longest row: no unit reaches more
  for (int r = tid; r < p.rows; r += kPlanThreads) {
    const int q0 = p.cu_seqlens_q[r];
    const int64_t q_len = static_cast<int64_t>(p.cu_seqlens_q[r + 1]) - q0;
    const int64_t raw = p.seq_lens[r];
    int tiles = 0;
    if (q_len > 0) {
      const int64_t covered = static_cast<int64_t>(p.gy) * p.tokens_per_wg;
      tiles = static_cast<int>((min(q_len, covered) + p.tokens_per_wg - 1) / p.tokens_per_wg);
      bad = bad || raw < q_len || raw > p.cap || q_len > covered;
    }
    r_q0[r] = q0;
    r_qlen[r] = q_len > 0 ? static_cast<int>(q_len) : 0;
    r_kv[r] = static_cast<int>(raw < 0 ? 0 : (raw > p.cap ? p.cap : raw));
    r_unit[r] = tiles;
    if (tiles > 0) reach_bound = max(reach_bound, (r_kv[r] + kTileP - 1) / kTileP);
  }
  if (__syncthreads_or(bad) && tid == 0) report(p.err, MAS_ERRBIT_POSITION);
  // short rows: an unsplit plan without laying out the units
  if (plan_never_splits(plan_max(reach_bound, slots))) {
    if (tid == 0) {
      p.hdr[0] = p.rows * p.gy * p.head_blocks;
      p.hdr[1] = 0;
      p.hdr[2] = 1;
    }
    return;
  }
  const int units = plan_scan(r_unit, p.rows, slots);  // <= rows * gy <= kPlanMaxUnits (host-checked)

  // units: each row's token tiles, the last (longest reach) first
  int longest = 0;
  for (int r = tid; r < p.rows; r += kPlanThreads) {
    const int first = r_unit[r], tiles = r_unit[r + 1] - first;
    const int q_len = r_qlen[r], shift = r_kv[r] - q_len;
    for (int i = 0; i < tiles; ++i) {
      const int tile = tiles - 1 - i;
      const int reach = shift + min((tile + 1) * p.tokens_per_wg, q_len);
      const int nt = reach > 0 ? (reach + kTileP - 1) / kTileP : 0;
      u_row[first + i] = r;
      u_tile[first + i] = tile;
      u_nt[first + i] = nt;
      longest = max(longest, nt);
    }
  }
  longest = plan_max(longest, slots);

  // the split count (wavefront 0, a split count per lane) and its split length
  if (tid < 64) {
    int best = 1;
    if (units > 0 && units * p.head_blocks < p.cus) {
      PlanModel m{};
      m.units = units;
      m.head_blocks = p.head_blocks;
      m.longest = longest;
      m.cus = static_cast<int>(p.cus);
      m.resident = static_cast<int>(p.resident);
      m.item_cap = static_cast<int>(p.item_cap);
      m.entry_cap = p.entry_cap;
      m.entries_per_unit = p.head_blocks * p.tokens_per_wg * p.heads_per_wg;
      m.pair_us = static_cast<float>(p.tokens_per_wg) * p.hq * 9.0e-4f;
      m.entry_us = (p.head_dim + 2) * 4.f / 5.0e6f;
      best = plan_best_splits(m, u_nt, tid);
    }
    if (tid == 0) params[0] = best;
  }
  __syncthreads();
  int splits = params[0];
  const int per = splits > 1 ? max(4, (longest + splits - 1) / splits) : 0;  // units longer than per split

  // items and partial slots per unit; no split if the grid or the workspace would not hold them
  int items = 0, split_units = 0;
  if (splits > 1) {
    for (int u = tid; u < units; u += kPlanThreads) {
      const int nt = u_nt[u];
      const int used = nt > per ? (nt + per - 1) / per : 1;  // <= splits
      u_item[u] = used * p.head_blocks;
      u_slot[u] = used > 1 ? 1 : 0;
    }
    items = plan_scan(u_item, units, slots);
    split_units = plan_scan(u_slot, units, slots);
    const bool fits = items <= p.item_cap &&
                      static_cast<int64_t>(split_units) * p.head_blocks * p.tokens_per_wg * p.heads_per_wg * splits <=
                          p.entry_cap;
    if (!fits) splits = 1;  // the same totals in every thread
  }

  if (splits == 1) {
    // No split: the launch is the grid launch, each workgroup finding its (head block, token tile,
    // row) from its id and loading its row's lengths itself; no items are written.
    split_units = 0;
    items = p.rows * p.gy * p.head_blocks;  // <= item_cap (host-checked)
  } else {
    // items in unit order: unit u's items are its key ranges x head blocks (head block fastest),
    // from u_item[u] on; one thread per (unit, head block) writes that block's ranges
    for (int j = tid; j < units * p.head_blocks; j += kPlanThreads) {
      const int u = j / p.head_blocks, block = j - u * p.head_blocks;
      const int used = (u_item[u + 1] - u_item[u]) / p.head_blocks;
      const int r = u_row[u], nt = u_nt[u];
      const int len = used > 1 ? per : nt;
      const int slot = used > 1 ? u_slot[u] * p.head_blocks + block : -1;
      for (int range = 0; range < used; ++range) {
        const int i = u_item[u] + range * p.head_blocks + block, first = range * len;
        p.items[2 * i] = i32x4{r_q0[r], r_qlen[r], r_kv[r], r | (range << 16) | (splits << 24)};
        p.items[2 * i + 1] = i32x4{u_tile[u] | (block << 16), first, min(nt, first + len), slot};
      }
    }
  }
  // split units, for the merge
  for (int u = tid; u < units && split_units > 0; u += kPlanThreads) {
    const int used = (u_item[u + 1] - u_item[u]) / p.head_blocks;
    if (used > 1) {
      const int su = u_slot[u], r = u_row[u];
      p.units[2 * su] = i32x4{r_q0[r], r_qlen[r], r_kv[r], r};
      p.units[2 * su + 1] = i32x4{u_tile[u] * p.tokens_per_wg, used, splits, su * p.head_blocks};
    }
  }
  if (tid == 0) {
    p.hdr[0] = items;
    p.hdr[1] = split_units;
    p.hdr[2] = splits;
  }
}

template <int D, int kWaves, int kWork>
void launch_context_mode(int mode, dim3 grid, dim3 block, hipStream_t stream, const ContextArgs& a) {
  if (mode == kPagesTile) hipLaunchKernelGGL((context_attn<D, kPagesTile, kWaves, kWork>), grid, block, 0, stream, a);
  else if (mode == kPagesMulti8)
    hipLaunchKernelGGL((context_attn<D, kPagesMulti8, kWaves, kWork>), grid, block, 0, stream, a);
  else if (mode == kPagesMulti16)
    hipLaunchKernelGGL((context_attn<D, kPagesMulti16, kWaves, kWork>), grid, block, 0, stream, a);
  else if (mode == kPagesMulti32)
    hipLaunchKernelGGL((context_attn<D, kPagesMulti32, kWaves, kWork>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((context_attn<D, kPagesLane, kWaves, kWork>), grid, block, 0, stream, a);
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

template <int kWork>
void launch_context(int64_t head_dim, int waves, int mode, dim3 grid, dim3 block, hipStream_t stream,
                    const ContextArgs& a) {
  if (head_dim == 64) {
    if (waves == 8) launch_context_mode<64, 8, kWork>(mode, grid, block, stream, a);
    else launch_context_mode<64, 4, kWork>(mode, grid, block, stream, a);
  } else {
    if (waves == 8) launch_context_mode<128, 8, kWork>(mode, grid, block, stream, a);
    else launch_context_mode<128, 4, kWork>(mode, grid, block, stream, a);
  }
}

// The workspace of a planned launch: the plan's counts (256 bytes), its items (32 bytes per
// workgroup of the grid), its split units (32 bytes per unit), then the partials.
struct PlanLayout {
  int64_t item_cap, units_bound, partial_off;
};

// A self-planned launch's workspace: the plan's counts (256 bytes), its split units (32 bytes
// each, at most one per (row, token tile)), then the partials.
int64_t self_plan_partial_off(int64_t units_bound) { return 256 + 32 * units_bound; }

PlanLayout plan_layout(int64_t units_bound, int64_t head_blocks, int64_t resident) {
  // items: at most one per (unit, head block) unsplit; split, the estimate keeps the grid within
  // two rounds of resident workgroups (best_splits)
  const int64_t item_cap = std::max(units_bound * head_blocks, 2 * resident);
  return {item_cap, units_bound, 256 + 32 * item_cap + 32 * units_bound};
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
  // the block table's reach) only sizes the estimate that picks the split count (SplitModel).
  // Whole rounds matter: one row of 256 new tokens after 2048 (64 workgroups) took 39 us in 8
  // splits (512 workgroups, one round of two per CU) and 49 us in 9. The merge's per-(token, head)
  // cost decides for many short rows: 24 rows of 32 new tokens after 512 took 26.6 us unsplit and
  // 44.9 in 2 splits. A grid with a workgroup on every CU gains nothing (4 rows of 256 after
  // 8192: 256 workgroups, 237 us either way) and is not split.
  //
  // Planned: a grid sized for kPlanMinRows or more rows of up to kPlanMaxTokens query tokens that
  // holds a workgroup per CU or more may still be mostly empty (a graph captured with padded prompt
  // rows and the step's whole token count as max_q_len; the rows' real lengths are on the device). When
  // the smallest grid it could hold (one token tile) would split at the hint's reach, context_plan
  // lays the launch out from the real lengths first: the same estimate on the real grid, one
  // workgroup per item, and a merge over the split tiles only.
  const int64_t row_tokens = gy * tokens_per_wg;
  const int64_t entry_bytes = (head_dim + 2) * 4;
  const int64_t units_bound = num_rows * gy;
  int64_t kv_splits = 1, split_from = INT32_MAX;
  const int64_t base_wgs = gx * gy * num_rows;
  bool planned = false;
  PlanLayout plan{};
  int64_t plan_entries = 0;
  bool self_plan = false;
  int cus = 0;
  int64_t resident = 0;
  if (workspace != nullptr && workspace_bytes > 0 && (reinterpret_cast<uintptr_t>(workspace) & 15u) == 0) {
    if (const int st = device_cu_count(&cus); st != MAS_OK) return st;
    resident = static_cast<int64_t>(cus) * (8 / waves);
    const int64_t max_tiles = cdiv(cap, kTileP);
    const int64_t hint_tiles = max_kv_len > 0 ? std::min(max_tiles, cdiv(max_kv_len, kTileP)) : max_tiles;
    if (base_wgs < cus && num_rows * row_tokens * num_q_heads <= INT32_MAX) {
      SplitModel m{};
      m.base = base_wgs;
      m.cus = cus;
      m.resident = resident;
      m.merges = static_cast<double>(num_rows * row_tokens * num_q_heads);
      m.partial_per_split = context_partial_bytes(num_rows, row_tokens, num_q_heads, head_dim, 1);
      m.capacity = workspace_bytes;
      m.max_splits = 65535 / num_rows;
      kv_splits = best_splits(m, hint_tiles);
      if (kv_splits > 1) split_from = split_from_reach(m, hint_tiles);
    } else if (base_wgs >= cus && num_rows >= kPlanMinRows && num_rows <= kPlanMaxRows && units_bound <= kPlanMaxUnits &&
               row_tokens <= kPlanMaxTokens && gx <= 32767 && units_bound * tokens_per_wg * num_q_heads <= INT32_MAX) {
      plan = plan_layout(units_bound, gx, resident);
      // a self-planned launch (up to kSelfPlanMaxRows rows) keeps only the plan's counts and split
      // units in the workspace, no items
      // (the kernels' small-operand quotients need the grid and the reach in key tiles below 2^22)
      self_plan = num_rows <= kSelfPlanMaxRows && plan.item_cap < (int64_t{1} << 22) && cap <= (int64_t{1} << 27);
      const int64_t plan_off = self_plan ? self_plan_partial_off(units_bound) : plan.partial_off;
      if (workspace_bytes > plan_off) {
        plan_entries = (workspace_bytes - plan_off) / entry_bytes;
        SplitModel m{};
        m.base = gx;
        m.cus = cus;
        m.resident = resident;
        m.merges = static_cast<double>(tokens_per_wg * num_q_heads);
        m.partial_per_split = gx * tokens_per_wg * heads_per_wg * entry_bytes;
        m.capacity = plan_entries * entry_bytes;
        m.max_splits = kMaxCtxSplits;
        planned = best_splits(m, hint_tiles) > 1;
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
  // Page mode: LDS DMA by tile or by page, or per-lane reads staged through registers.
  // One-page tiles load by LDS DMA through buffer resources: 31-bit byte offsets and record counts
  // from the tile's first row, and rows whose validity a record count can express (a position's
  // row of one kv head inside its entry).
  const bool tile_offsets_fit =
      entry_stride >= head_dim && head_stride >= 0 &&
      (kTileP * entry_stride + (num_kv_heads - 1) * head_stride + head_dim) * 2 < (int64_t{1} << 31);
  // Pages of 8-32 slots: the same by page (offsets and records from a page's first row).
  const bool page_offsets_fit = entry_stride >= head_dim && head_stride >= 0 &&
                                page_size * entry_stride * 2 < (int64_t{1} << 31);
  const int mode = page_size >= kTileP && tile_offsets_fit                     ? kPagesTile
                   : page_size >= 8 && page_size < kTileP && page_offsets_fit
                       ? (page_size == 8 ? kPagesMulti8 : page_size == 16 ? kPagesMulti16 : kPagesMulti32)
                                                                                 : kPagesLane;
  const dim3 block(static_cast<uint32_t>(64 * waves));
  if (planned && self_plan) {
    // every workgroup lays the plan out itself (no planner launch) and writes what the merge reads:
    // the plan's counts, then its split units, then the partials
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    a.plan_hdr = reinterpret_cast<int*>(ws);
    a.plan_units = reinterpret_cast<i32x4*>(ws + 256);
    a.plan_rows = static_cast<int>(num_rows);
    a.plan_gy = static_cast<int>(gy);
    a.plan_cus = cus;
    a.plan_resident = static_cast<int>(resident);
    a.plan_lt = __builtin_ctzll(static_cast<uint64_t>(tokens_per_wg));
    a.plan_hb = static_cast<int>(gx);
    a.plan_item_cap = plan.item_cap;
    a.plan_entry_cap = plan_entries;
    a.plan_cap = cap;
    a.part_o = reinterpret_cast<float*>(ws + self_plan_partial_off(units_bound));
    a.part_ml = a.part_o + plan_entries * head_dim;
    launch_context<kWorkSelfPlan>(head_dim, waves, mode, dim3(static_cast<uint32_t>(plan.item_cap)), block, stream, a);
    if (const int st = launch_status(); st != MAS_OK) return st;
  } else if (planned) {
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    PlanArgs pa{};
    pa.cu_seqlens_q = cu_seqlens_q;
    pa.seq_lens = seq_lens;
    pa.rows = static_cast<int>(num_rows);
    pa.gy = static_cast<int>(gy);
    pa.tokens_per_wg = static_cast<int>(tokens_per_wg);
    pa.heads_per_wg = heads_per_wg;
    pa.head_blocks = static_cast<int>(gx);
    pa.hq = static_cast<int>(num_q_heads);
    pa.head_dim = static_cast<int>(head_dim);
    pa.cap = cap;
    pa.cus = cus;
    pa.resident = resident;
    pa.item_cap = plan.item_cap;
    pa.entry_cap = plan_entries;
    pa.hdr = reinterpret_cast<int*>(ws);
    pa.items = reinterpret_cast<i32x4*>(ws + 256);
    pa.units = reinterpret_cast<i32x4*>(ws + 256 + 32 * plan.item_cap);
    pa.err = err;
    a.plan_hdr = pa.hdr;
    a.plan_items = pa.items;
    a.plan_units = pa.units;
    a.plan_rows = pa.rows;
    a.plan_gy = pa.gy;
    a.part_o = reinterpret_cast<float*>(ws + plan.partial_off);
    a.part_ml = a.part_o + plan_entries * head_dim;
    hipLaunchKernelGGL(context_plan, dim3(1), dim3(kPlanThreads), 0, stream, pa);
    if (const int st = launch_status(); st != MAS_OK) return st;
    launch_context<kWorkPlan>(head_dim, waves, mode, dim3(static_cast<uint32_t>(plan.item_cap)), block, stream, a);
    if (const int st = launch_status(); st != MAS_OK) return st;
  }
  if (planned) {
    // each wavefront takes (token, head) pairs of the split units in turn; 24 per CU (6 per SIMD,
    // as many as the merge's registers allow: 12,288 pairs merged in 9.6 us against 11.1 with 16)
    const int64_t pairs = units_bound * tokens_per_wg * num_q_heads;
    const dim3 merge_grid(
        static_cast<uint32_t>(std::min<int64_t>(cdiv(pairs, kMergeWaves), 24 * static_cast<int64_t>(cus) / kMergeWaves)));
    const dim3 merge_block(64 * kMergeWaves);
    if (head_dim == 64)
      hipLaunchKernelGGL(context_combine_plan<64>, merge_grid, merge_block, 0, stream, a, static_cast<int>(tokens_per_wg));
    else
      hipLaunchKernelGGL(context_combine_plan<128>, merge_grid, merge_block, 0, stream, a, static_cast<int>(tokens_per_wg));
    return launch_status();
  }
  if (kv_splits > 1) {
    const dim3 grid(static_cast<uint32_t>(gx), static_cast<uint32_t>(gy), static_cast<uint32_t>(num_rows * kv_splits));
    launch_context<kWorkSplit>(head_dim, waves, mode, grid, block, stream, a);
  } else {
    // Rows in turn (their tiles longest first) keep a row's key / value tiles warm in L2 while its
    // workgroups run, but the last row's longest tiles then start late: the launch ends on them.
    // Tile-major order starts every row's longest tiles first and ends on short ones, at the cost
    // of those cache hits. It is taken when the longest tile (kv_max positions) is at least 30% of
    // the launch's time per resident workgroup, the rows taken as long as the longest (max_q_len
    // new tokens, kv_max positions): measured on MI355X, 24B heads 4 x 2048 tokens (48%) -4%,
    // 4 x 512 after 2048 cached (110%) -5%, 16 x 1024 (24%) -2%, 8 x 2048 (24%) even; 32 x 512
    // (22%) +3%; 123B heads 16 x 512 (15%) +4%, 4 x 4096 (8%) +0.7%. Only for fewer than
    // kPlanMinRows rows: a grid of more may be a captured graph's padded layout (17 rows, 1-3 real
    // ones far shorter than max_q_len), where tile-major order dispatches every row's empty last
    // tiles before any real work (3 x 100 tokens after 2000 in the 17-row layout: 62 -> 85 us).
    if (cus == 0) {
      if (const int st = device_cu_count(&cus); st != MAS_OK) return st;
    }
    const int64_t resident_wgs = static_cast<int64_t>(cus) * (8 / waves);
    const int64_t kv_max = max_kv_len > 0 ? std::min(cap, max_kv_len) : cap;
    // a workgroup's mean reach in positions: the cached ones plus half the new tokens
    const int64_t mean_reach = std::max(kv_max - max_q_len / 2 + tokens_per_wg / 2, tokens_per_wg);
    a.tile_major = num_rows < kPlanMinRows &&
                   10.0 * static_cast<double>(kv_max) * static_cast<double>(resident_wgs) >=
                       3.0 * static_cast<double>(num_rows * gx * gy) * static_cast<double>(mean_reach);
    const dim3 grid = a.tile_major
                          ? dim3(static_cast<uint32_t>(gx), static_cast<uint32_t>(num_rows), static_cast<uint32_t>(gy))
                          : dim3(static_cast<uint32_t>(gx), static_cast<uint32_t>(gy), static_cast<uint32_t>(num_rows));
    launch_context<kWorkGrid>(head_dim, waves, mode, grid, block, stream, a);
  }
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
