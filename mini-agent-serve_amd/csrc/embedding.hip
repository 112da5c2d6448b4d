// embedding.hip - token-embedding gather, out[t, :] = weight[ids[t], :].
//
// Semantics: nn.Embedding.forward at miniagentserve/models/devstral2/devstral2.py:260,282 (ids are
// int64, miniagentserve/engine/model_runner.py:45). A bit copy of one table row per token.
//
// Grid: x = groups of 4 tokens (one wavefront each), y = chunks of 64 * kUnroll 16-byte vectors
// of the row, so short batches still spread over many CUs. The id is wave-uniform and read
// through the scalar cache; an id outside [0, vocab) zero-fills its row and sets
// MAS_ERRBIT_TOKEN_ID (torch raises on such an id; the table is never read out of bounds).
#include "device.h"

namespace mas {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kUnroll = 8;
constexpr int kChunkVec = kWave * kUnroll;

__global__ __launch_bounds__(kBlock) void embedding_gather(uint16_t* __restrict__ out, int64_t out_stride,
                                                           const uint16_t* __restrict__ weight, int64_t weight_stride,
                                                           int64_t vocab, const int64_t* __restrict__ ids,
                                                           int64_t rows, int nvec, uint32_t* err) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_id_uniform();
  if (t >= rows) return;
  const int64_t id = ids[t];
  const int v0 = blockIdx.y * kChunkVec + lane;
  uint16_t* dst = out + t * out_stride;
  if (id < 0 || id >= vocab) {
    if (lane == 0 && blockIdx.y == 0) report(err, MAS_ERRBIT_TOKEN_ID);
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {
      const int v = v0 + j * kWave;
      if (v < nvec) store_stream(dst + 8 * v, zero);
    }
    return;
  }
  const uint16_t* src = weight + id * weight_stride;
  // Unconditional loads (indices past the row end clamped to its last vector) so they issue
  // back to back; only the stores are guarded.
  u32x4 x[kUnroll];
#pragma unroll
  for (int j = 0; j < kUnroll; ++j) {
    const int v = v0 + j * kWave;
    x[j] = load_stream(src + 8 * (v < nvec ? v : nvec - 1));
  }
  load_fence();
#pragma unroll
  for (int j = 0; j < kUnroll; ++j) {
    const int v = v0 + j * kWave;
    if (v < nvec) store_stream(dst + 8 * v, x[j]);
  }
}

__global__ __launch_bounds__(kBlock) void embedding_gather_scalar(uint16_t* __restrict__ out, int64_t out_stride,
                                                                  const uint16_t* __restrict__ weight,
                                                                  int64_t weight_stride, int64_t vocab,
                                                                  const int64_t* __restrict__ ids, int64_t rows,
                                                                  int64_t hidden, uint32_t* err) {
  for (int64_t t = blockIdx.x; t < rows; t += gridDim.x) {
    const int64_t id = ids[t];
    const bool ok = id >= 0 && id < vocab;
    if (!ok) {
      if (threadIdx.x == 0) report(err, MAS_ERRBIT_TOKEN_ID);
      for (int64_t i = threadIdx.x; i < hidden; i += kBlock) out[t * out_stride + i] = 0;
      continue;
    }
    for (int64_t i = threadIdx.x; i < hidden; i += kBlock) out[t * out_stride + i] = weight[id * weight_stride + i];
  }
}

}  // namespace
}  // namespace mas

extern "C" int mas_embedding_bf16(void* out, int64_t out_stride, const void* weight, int64_t weight_stride,
                                  int64_t vocab, const int64_t* ids, int64_t rows, int64_t hidden, uint32_t* err,
                                  hipStream_t stream) {
  using namespace mas;
  if (rows < 0 || hidden < 0 || vocab < 0) return MAS_ERR_INVALID_VALUE;
  if (rows == 0 || hidden == 0) return MAS_OK;
  if (out == nullptr || ids == nullptr || (vocab > 0 && weight == nullptr)) return MAS_ERR_INVALID_VALUE;
  if (rows > 1 && out_stride < hidden) return MAS_ERR_INVALID_VALUE;
  if (vocab > 1 && weight_stride < hidden) return MAS_ERR_INVALID_VALUE;
  const bool vec_ok = hidden % 8 == 0 && aligned16(out) && aligned16(weight) && out_stride % 8 == 0 &&
                      weight_stride % 8 == 0 && hidden / 8 <= INT32_MAX;
  if (vec_ok) {
    const int nvec = static_cast<int>(hidden / 8);
    const int64_t gx = cdiv(rows, kWavesPerBlock);
    const int64_t gy = cdiv(nvec, kChunkVec);
    if (gx > INT32_MAX || gy > 65535) return MAS_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(embedding_gather, dim3(static_cast<uint32_t>(gx), static_cast<uint32_t>(gy)), dim3(kBlock), 0,
                       stream, static_cast<uint16_t*>(out), out_stride, static_cast<const uint16_t*>(weight),
                       weight_stride, vocab, ids, rows, nvec, err);
    return launch_status();
  }
  const int64_t grid = rows < 65536 ? rows : 65536;
  hipLaunchKernelGGL(embedding_gather_scalar, dim3(static_cast<uint32_t>(grid)), dim3(kBlock), 0, stream,
                     static_cast<uint16_t*>(out), out_stride, static_cast<const uint16_t*>(weight), weight_stride,
                     vocab, ids, rows, hidden, err);
  return launch_status();
}
