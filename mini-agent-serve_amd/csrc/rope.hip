// rope.hip - rotary embedding applied in place to q and k heads from a cos/sin table.
//
// Semantics (miniagentserve/models/devstral2/devstral2.py:163-166,
// flashinfer.rope.apply_rope_with_cos_sin_cache_inplace with is_neox=True; table layout from
// _yarn_cos_sin_cache at devstral2.py:44-90: row p = [cos(p*f_0..f_{R/2-1}), sin(...)] * scaling):
//   c = T[pos, i], s = T[pos, R/2 + i]
//   NeoX  (is_neox):  a = x[i], b = x[i + R/2]
//   GPT-J (!is_neox): a = x[2i], b = x[2i + 1]
//   a' = bf16(a*c - b*s), b' = bf16(b*c + a*s)      (fp32 products, fp32 subtract / add)
//
// Work item: one wavefront rotates PASSES x (64 / LPH) heads of one token, LPH = R/16 lanes per
// head, each lane owning 8 rotation pairs: two 16-byte head loads and stores plus 8 cos and
// 8 sin from the table row (read once per wavefront). Heads 0..Hq-1 are q heads, the rest k
// heads; q and k are independent strided views (for the model they are column slices of one
// fused qkv row). The token's position is wave-uniform and comes through the scalar cache.
#include "device.h"

namespace mas {
namespace {

constexpr int kBlock = 256;  // threads per workgroup (64..512 measured equal on MI355X)
constexpr int kWavesPerBlock = kBlock / kWave;

struct RopeArgs {
  uint16_t* q;
  int64_t q_stride, q_head_stride;
  uint16_t* k;
  int64_t k_stride, k_head_stride;
  const void* positions;
  const float* table;
  int64_t table_stride, table_rows;
  int64_t rows;
  int num_q_heads, num_heads;
  int groups_per_token;
  uint32_t* err;
};

template <int LPH, bool kNeox, bool kPos64, int PASSES>
__global__ __launch_bounds__(kBlock) void rope_inplace(RopeArgs a) {
  constexpr int kHeadsPerPass = kWave / LPH;
  constexpr int kHalf = LPH * 8;  // R / 2
  const int lane = threadIdx.x & (kWave - 1);
  const int slot = lane / LPH;
  const int chunk = lane % LPH;
  // Workgroups go to the 8 XCDs round-robin by id; token t's wavefronts all run on XCD t % 8, so
  // its cos/sin row is fetched into one L2.
  const int64_t xcd = blockIdx.x % kXcds;
  const int64_t work = static_cast<int64_t>(blockIdx.x / kXcds) * kWavesPerBlock + wave_id_uniform();
  const int64_t tx = work / a.groups_per_token;
  const int64_t t = tx * kXcds + xcd;
  if (t >= a.rows) return;
  const int group = static_cast<int>(work - tx * a.groups_per_token);

  // Offsets of the two 16-byte vectors this lane owns inside a head.
  const int off_a = kNeox ? chunk * 8 : chunk * 16;
  const int off_b = kNeox ? kHalf + chunk * 8 : chunk * 16 + 8;

  // The head data does not depend on the position: load it first (head indices past the last head
  // are clamped to it and their stores skipped), then fetch the position and its table row.
  uint16_t* ptr[PASSES];
  u32x4 va[PASSES], vb[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    int h = (group * PASSES + p) * kHeadsPerPass + slot;
    h = h < a.num_heads ? h : a.num_heads - 1;
    ptr[p] = h < a.num_q_heads ? a.q + t * a.q_stride + h * a.q_head_stride
                               : a.k + t * a.k_stride + (h - a.num_q_heads) * a.k_head_stride;
    va[p] = load_stream(ptr[p] + off_a);
    vb[p] = load_stream(ptr[p] + off_b);
  }
  load_fence();

  const int64_t pos = kPos64 ? static_cast<const int64_t*>(a.positions)[t]
                             : static_cast<int64_t>(static_cast<const int32_t*>(a.positions)[t]);
  if (pos < 0 || pos >= a.table_rows) {
    if (lane == 0 && group == 0) report(a.err, MAS_ERRBIT_POSITION);
    return;
  }
  const float* trow = a.table + pos * a.table_stride + chunk * 8;
  const f32x4 c0 = load_cached_f4(trow), c1 = load_cached_f4(trow + 4);
  const f32x4 s0 = load_cached_f4(trow + kHalf), s1 = load_cached_f4(trow + kHalf + 4);
  // Keeps the head rows' unpacking below the table loads: hoisted above them, it would make the
  // table loads wait for the head rows to arrive.
  load_fence();
  const float cs[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};

#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int h = (group * PASSES + p) * kHeadsPerPass + slot;
    if (h >= a.num_heads) continue;
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
      // 16 consecutive elements = 8 interleaved pairs; pair i uses cos/sin column chunk*8 + i.
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
    store_stream(ptr[p] + off_a, pack8(ya));
    store_stream(ptr[p] + off_b, pack8(yb));
  }
}

template <int LPH, bool kNeox, bool kPos64, int PASSES>
int launch_rope(RopeArgs a, hipStream_t s) {
  constexpr int kHeadsPerWave = (kWave / LPH) * PASSES;
  a.groups_per_token = static_cast<int>(cdiv(a.num_heads, kHeadsPerWave));
  const int64_t blocks = kXcds * cdiv(cdiv(a.rows, kXcds) * a.groups_per_token, kWavesPerBlock);
  if (blocks > INT32_MAX) return MAS_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((rope_inplace<LPH, kNeox, kPos64, PASSES>), dim3(static_cast<uint32_t>(blocks)), dim3(kBlock),
                     0, s, a);
  return launch_status();
}

// Few tokens: one pass per wavefront for the most parallelism. Many tokens: two passes per
// wavefront (measured best on MI355X for 40 and 104 heads of 128, ahead of 1, 3, 4 and 5).
template <int LPH, bool kNeox, bool kPos64>
int pick_passes(RopeArgs a, int cus, hipStream_t s) {
  constexpr int kHeadsPerPass = kWave / LPH;
  const int64_t passes = cdiv(a.num_heads, kHeadsPerPass);
  if (a.rows * passes < static_cast<int64_t>(cus) * 16) return launch_rope<LPH, kNeox, kPos64, 1>(a, s);
  return launch_rope<LPH, kNeox, kPos64, 2>(a, s);
}

template <int LPH>
int dispatch_layout(RopeArgs a, bool neox, bool pos64, int cus, hipStream_t s) {
  if (neox) return pos64 ? pick_passes<LPH, true, true>(a, cus, s) : pick_passes<LPH, true, false>(a, cus, s);
  return pos64 ? pick_passes<LPH, false, true>(a, cus, s) : pick_passes<LPH, false, false>(a, cus, s);
}

}  // namespace
}  // namespace mas

extern "C" int mas_rope_cos_sin_cache_bf16(void* q, int64_t q_stride, int64_t q_head_stride, int64_t num_q_heads,
                                           void* k, int64_t k_stride, int64_t k_head_stride, int64_t num_k_heads,
                                           const void* positions, int pos_is_int64, const float* table,
                                           int64_t table_stride, int64_t table_rows, int64_t rows, int64_t head_dim,
                                           int64_t rotary_dim, int is_neox, uint32_t* err, hipStream_t stream) {
  using namespace mas;
  if (rows < 0 || num_q_heads < 0 || num_k_heads < 0 || head_dim <= 0 || table_rows < 0)
    return MAS_ERR_INVALID_VALUE;
  if (rotary_dim != 32 && rotary_dim != 64 && rotary_dim != 128 && rotary_dim != 256 && rotary_dim != 512)
    return MAS_ERR_UNSUPPORTED;
  if (rotary_dim > head_dim) return MAS_ERR_INVALID_VALUE;
  if (num_q_heads + num_k_heads > INT32_MAX) return MAS_ERR_UNSUPPORTED;
  if (rows == 0 || num_q_heads + num_k_heads == 0) return MAS_OK;
  if (positions == nullptr || table == nullptr) return MAS_ERR_INVALID_VALUE;
  if (num_q_heads > 0 && q == nullptr) return MAS_ERR_INVALID_VALUE;
  if (num_k_heads > 0 && k == nullptr) return MAS_ERR_INVALID_VALUE;
  if (table_stride < rotary_dim && table_rows > 1) return MAS_ERR_INVALID_VALUE;
  // 16-byte head vectors and table rows.
  const bool q_ok = num_q_heads == 0 || (aligned16(q) && q_stride % 8 == 0 && q_head_stride % 8 == 0);
  const bool k_ok = num_k_heads == 0 || (aligned16(k) && k_stride % 8 == 0 && k_head_stride % 8 == 0);
  if (!q_ok || !k_ok || !aligned16(table) || table_stride % 4 != 0) return MAS_ERR_MISALIGNED;
  int cus = 0;
  if (const int st = device_cu_count(&cus); st != MAS_OK) return st;

  RopeArgs a{static_cast<uint16_t*>(q), q_stride, q_head_stride, static_cast<uint16_t*>(k), k_stride, k_head_stride,
             positions, table, table_stride, table_rows, rows, static_cast<int>(num_q_heads),
             static_cast<int>(num_q_heads + num_k_heads), 0, err};
  const bool neox = is_neox != 0, pos64 = pos_is_int64 != 0;
  switch (rotary_dim) {
    case 32: return dispatch_layout<2>(a, neox, pos64, cus, stream);
    case 64: return dispatch_layout<4>(a, neox, pos64, cus, stream);
    case 128: return dispatch_layout<8>(a, neox, pos64, cus, stream);
    case 256: return dispatch_layout<16>(a, neox, pos64, cus, stream);
    case 512: return dispatch_layout<32>(a, neox, pos64, cus, stream);
    default: return MAS_ERR_UNSUPPORTED;
  }
}
