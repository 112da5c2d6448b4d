// embedding.hip - token-embedding gather, out[t, :] = weight[ids[t], :].
//
// Semantics: nn.Embedding.forward at miniagentserve/models/devstral2/devstral2.py:260,282 (ids are
// int64, miniagentserve/engine/model_runner.py:45). A bit copy of one table row per token.
//
// Grid: x = token, y = chunks of 64 * kVpl 16-byte vectors of the row; one wavefront per
// workgroup, so a 64-token decode step spreads over 640 wavefronts (hidden 5120), as many as a plain
// copy of the same bytes. The id is wave-uniform and read through the scalar cache; an id outside
// [0, vocab) zero-fills its row and sets MAS_ERRBIT_TOKEN_ID (torch raises on such an id; the table
// is never read out of bounds).
//
// Placeholder form (the step-input path at miniagentserve/engine/model_runner.py:149-154 fused with
// the gather): an id -1 - r stands for row r of the previous step's samples (int32, still on the
// GPU). The kernel resolves it, writes the resolved id back into ids as fill_placeholders does, and
// gathers that row - one launch instead of fill_placeholders' five plus the gather. A placeholder
// whose row r is past the samples zero-fills its row, keeps its id and sets MAS_ERRBIT_PLACEHOLDER.
// Several workgroups may resolve the same token (one per row chunk); they read either the
// placeholder or the id another one wrote back, and resolve both to the same row.
#include "device.h"

namespace mas {
namespace {

constexpr int kBlock = 256;          // scalar-path and fill-only workgroups
constexpr int kVpl = 1;              // 16-byte vectors per lane in the vector path

// Resolves a placeholder id (-1 - r -> last[r]); writes the resolved id back when `write` is set.
// Returns -1 (and reports) for a placeholder past the samples.
__device__ __forceinline__ int64_t resolve_id(int64_t* ids, int64_t t, int64_t id, const int32_t* last,
                                              int64_t num_last, bool write, uint32_t* err) {
  if (id >= 0) return id;
  const int64_t r = -1 - id;
  if (r >= num_last) {
    if (write) report(err, MAS_ERRBIT_PLACEHOLDER);
    return -1;
  }
  const int64_t resolved = last[r];
  if (write) ids[t] = resolved;
  return resolved;
}

template <bool kFill>
__global__ __launch_bounds__(kWave) void embedding_gather(uint16_t* __restrict__ out, int64_t out_stride,
                                                          const uint16_t* __restrict__ weight, int64_t weight_stride,
                                                          int64_t vocab, int64_t* ids, int64_t rows, int nvec,
                                                          const int32_t* __restrict__ last, int64_t num_last,
                                                          uint32_t* err) {
  const int lane = threadIdx.x;
  const int64_t t = blockIdx.x;
  int64_t id = ids[t];
  const bool leader = lane == 0 && blockIdx.y == 0;
  bool placeholder_bad = false;
  if constexpr (kFill) {
    if (id < 0) {
      placeholder_bad = -1 - id >= num_last;
      id = resolve_id(ids, t, id, last, num_last, leader, err);
    }
  }
  const int v0 = blockIdx.y * (kWave * kVpl) + lane;
  uint16_t* dst = out + t * out_stride;
  if (id < 0 || id >= vocab) {
    if (leader && !placeholder_bad) report(err, MAS_ERRBIT_TOKEN_ID);
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < kVpl; ++j) {
      const int v = v0 + j * kWave;
      if (v < nvec) store_stream(dst + 8 * v, zero);
    }
    return;
  }
  const uint16_t* src = weight + id * weight_stride;
  // Unconditional loads (indices past the row end clamped to its last vector) so they issue
  // back to back; only the stores are guarded.
  u32x4 x[kVpl];
#pragma unroll
  for (int j = 0; j < kVpl; ++j) {
    const int v = v0 + j * kWave;
    x[j] = load_stream(src + 8 * (v < nvec ? v : nvec - 1));
  }
  load_fence();
#pragma unroll
  for (int j = 0; j < kVpl; ++j) {
    const int v = v0 + j * kWave;
    if (v < nvec) store_stream(dst + 8 * v, x[j]);
  }
}

__global__ __launch_bounds__(kBlock) void embedding_gather_scalar(uint16_t* __restrict__ out, int64_t out_stride,
                                                                  const uint16_t* __restrict__ weight,
                                                                  int64_t weight_stride, int64_t vocab, int64_t* ids,
                                                                  int64_t rows, int64_t hidden,
                                                                  const int32_t* __restrict__ last, int64_t num_last,
                                                                  uint32_t* err) {
  for (int64_t t = blockIdx.x; t < rows; t += gridDim.x) {
    int64_t id = ids[t];
    bool placeholder_bad = false;
    if (last != nullptr && id < 0) {
      placeholder_bad = -1 - id >= num_last;
      id = resolve_id(ids, t, id, last, num_last, threadIdx.x == 0, err);
    }
    const bool ok = id >= 0 && id < vocab;
    if (!ok) {
      if (threadIdx.x == 0 && !placeholder_bad) report(err, MAS_ERRBIT_TOKEN_ID);
      for (int64_t i = threadIdx.x; i < hidden; i += kBlock) out[t * out_stride + i] = 0;
      continue;
    }
    for (int64_t i = threadIdx.x; i < hidden; i += kBlock) out[t * out_stride + i] = weight[id * weight_stride + i];
  }
}

// Placeholder resolution alone (no gather): one lane per token.
__global__ __launch_bounds__(kBlock) void fill_placeholders(int64_t* ids, int64_t rows, const int32_t* __restrict__ last,
                                                            int64_t num_last, uint32_t* err) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (t < rows) {
    const int64_t id = ids[t];
    if (id < 0) resolve_id(ids, t, id, last, num_last, true, err);
  }
}

int gather(void* out, int64_t out_stride, const void* weight, int64_t weight_stride, int64_t vocab, int64_t* ids,
           int64_t rows, int64_t hidden, const int32_t* last, int64_t num_last, uint32_t* err, hipStream_t stream) {
  if (rows > 1 && out_stride < hidden) return MAS_ERR_INVALID_VALUE;
  if (vocab > 1 && weight_stride < hidden) return MAS_ERR_INVALID_VALUE;
  const bool vec_ok = hidden % 8 == 0 && aligned16(out) && aligned16(weight) && out_stride % 8 == 0 &&
                      weight_stride % 8 == 0 && hidden / 8 <= INT32_MAX;
  if (vec_ok) {
    const int nvec = static_cast<int>(hidden / 8);
    const int64_t gy = cdiv(nvec, kWave * kVpl);
    if (rows > INT32_MAX || gy > 65535) return MAS_ERR_UNSUPPORTED;
    const dim3 grid(static_cast<uint32_t>(rows), static_cast<uint32_t>(gy));
    if (last != nullptr) {
      hipLaunchKernelGGL(embedding_gather<true>, grid, dim3(kWave), 0, stream, static_cast<uint16_t*>(out),
                         out_stride, static_cast<const uint16_t*>(weight), weight_stride, vocab, ids, rows, nvec, last,
                         num_last, err);
    } else {
      hipLaunchKernelGGL(embedding_gather<false>, grid, dim3(kWave), 0, stream, static_cast<uint16_t*>(out),
                         out_stride, static_cast<const uint16_t*>(weight), weight_stride, vocab, ids, rows, nvec, last,
                         num_last, err);
    }
    return launch_status();
  }
  const int64_t grid = rows < 65536 ? rows : 65536;
  hipLaunchKernelGGL(embedding_gather_scalar, dim3(static_cast<uint32_t>(grid)), dim3(kBlock), 0, stream,
                     static_cast<uint16_t*>(out), out_stride, static_cast<const uint16_t*>(weight), weight_stride,
                     vocab, ids, rows, hidden, last, num_last, err);
  return launch_status();
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
  // Without samples no id is written: the cast only lets both forms share the kernel.
  return gather(out, out_stride, weight, weight_stride, vocab, const_cast<int64_t*>(ids), rows, hidden, nullptr, 0,
                err, stream);
}

extern "C" int mas_embedding_fill_placeholders_bf16(void* out, int64_t out_stride, const void* weight,
                                                    int64_t weight_stride, int64_t vocab, int64_t* ids, int64_t rows,
                                                    int64_t hidden, const int32_t* last_tokens, int64_t num_last,
                                                    uint32_t* err, hipStream_t stream) {
  using namespace mas;
  if (rows < 0 || hidden < 0 || vocab < 0 || num_last < 0) return MAS_ERR_INVALID_VALUE;
  if (rows == 0) return MAS_OK;
  if (ids == nullptr || (num_last > 0 && last_tokens == nullptr)) return MAS_ERR_INVALID_VALUE;
  // A null pointer for samples is the plain gather, so pass a valid one even when there are none.
  const int32_t* last = last_tokens != nullptr ? last_tokens : reinterpret_cast<const int32_t*>(ids);
  if (out == nullptr || hidden == 0) {
    const int64_t blocks = cdiv(rows, kBlock);
    if (blocks > INT32_MAX) return MAS_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(fill_placeholders, dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, stream, ids, rows,
                       last, num_last, err);
    return launch_status();
  }
  if (vocab > 0 && weight == nullptr) return MAS_ERR_INVALID_VALUE;
  return gather(out, out_stride, weight, weight_stride, vocab, ids, rows, hidden, last, num_last, err, stream);
}
