// silu_and_mul.hip - SiluAndMul gating over the gate_up projection output.
//
// Semantics (miniagentserve/models/devstral2/devstral2.py:223-224, flashinfer.activation.silu_and_mul;
// gate first, up second by the concat order at devstral2.py:364):
//   g = f32(in[r, i]), u = f32(in[r, I + i]);  out[r, i] = bf16((g / (1 + exp(-g))) * u)
//
// Streaming kernel: each workgroup owns a tile of 256 * UNROLL 128-bit output vectors of one
// row; each lane issues all of its gate and up loads before any arithmetic, so 2 * UNROLL
// 16-byte loads per lane are in flight. 6 bytes move per output element (read 4, write 2).
// At decode sizes the per-element arithmetic is part of the critical path, so it is kept short.
#include "device.h"

namespace mas {
namespace {

constexpr int kBlock = 256;
constexpr int kVecBlock = 64;

// silu(g) * u with the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32): a few fp32 ulps from
// the correctly rounded g / (1 + e^-g), far below the bf16 rounding of the result, at a quarter
// of the instructions of an IEEE divide. Limits: g -> -inf gives 1 / inf = 0 (so -0 * u), g -> +inf
// gives exp2 -> 0 and g * u, NaN propagates.
__device__ __forceinline__ float silu_mul(float g, float u) {
  constexpr float kLog2e = 1.4426950408889634f;
  const float e = __builtin_amdgcn_exp2f(-g * kLog2e);
  return (g * __builtin_amdgcn_rcpf(1.0f + e)) * u;
}

template <int UNROLL>
__global__ __launch_bounds__(kVecBlock) void silu_and_mul_vec(void* __restrict__ out, int64_t out_stride,
                                                           const void* __restrict__ in, int64_t in_stride,
                                                           int64_t rows, int64_t inter) {
  const int64_t nvec = inter >> 3;
  const int64_t v0 = static_cast<int64_t>(blockIdx.x) * (kVecBlock * UNROLL) + threadIdx.x;
  for (int64_t row = blockIdx.y; row < rows; row += gridDim.y) {
    const uint16_t* g = static_cast<const uint16_t*>(in) + row * in_stride;
    const uint16_t* u = g + inter;
    uint16_t* o = static_cast<uint16_t*>(out) + row * out_stride;

    // Loads are unconditional (indices past the row end are clamped to its last vector) so the
    // compiler issues them back to back; only the stores are guarded.
    u32x4 gv[UNROLL], uv[UNROLL];
#pragma unroll
    for (int j = 0; j < UNROLL; ++j) {
      const int64_t v = v0 + j * kVecBlock;
      const int64_t vl = v < nvec ? v : nvec - 1;
      gv[j] = load_stream(g + 8 * vl);
      uv[j] = load_stream(u + 8 * vl);
    }
    load_fence();
#pragma unroll
    for (int j = 0; j < UNROLL; ++j) {
      const int64_t v = v0 + j * kVecBlock;
      if (v < nvec) {
        float gf[8], uf[8], y[8];
        unpack8(gv[j], gf);
        unpack8(uv[j], uf);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = silu_mul(gf[e], uf[e]);
        store_stream(o + 8 * v, pack8(y));
      }
    }
  }
}

// SiluAndMul with the fp8 quantize of the down_proj input fused in (miniagentserve/models/
// devstral2/devstral2.py:93-95,110-111,224): y = bf16(silu(g) * u) as the unfused op writes it, then
// out = e4m3fn(clamp(f32(y) / scale, -448, 448)). Reads 4 bytes and writes 1 per element instead of
// the unfused 6 + 3.
__global__ __launch_bounds__(kVecBlock) void silu_and_mul_quant_vec(void* __restrict__ out, int64_t out_stride,
                                                                 const void* __restrict__ in, int64_t in_stride,
                                                                 int64_t rows, int64_t inter,
                                                                 const float* __restrict__ scale_dev, float scale_host) {
  const int64_t nvec = inter >> 3;
  const int64_t v = static_cast<int64_t>(blockIdx.x) * kVecBlock + threadIdx.x;
  for (int64_t row = blockIdx.y; row < rows; row += gridDim.y) {
    const uint16_t* g = static_cast<const uint16_t*>(in) + row * in_stride;
    const int64_t vl = v < nvec ? v : nvec - 1;
    const u32x4 gv = load_stream(g + 8 * vl);
    const u32x4 uv = load_stream(g + inter + 8 * vl);
    load_fence();
    const float scale = scale_dev != nullptr ? *scale_dev : scale_host;
    const float rcp = 1.0f / scale;
    if (v < nvec) {
      float gf[8], uf[8];
      unpack8(gv, gf);
      unpack8(uv, uf);
      float qf[8];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const uint32_t y2 = pack_bf16x2(silu_mul(gf[e], uf[e]), silu_mul(gf[e + 1], uf[e + 1]));
        qf[e] = div_by_scale(bf16_lo(y2), scale, rcp);
        qf[e + 1] = div_by_scale(bf16_hi(y2), scale, rcp);
      }
      u32x2 q;
      q[0] = fp8x4_saturate_encode(qf[0], qf[1], qf[2], qf[3]);
      q[1] = fp8x4_saturate_encode(qf[4], qf[5], qf[6], qf[7]);
      store_stream(static_cast<uint8_t*>(out) + row * out_stride + 8 * v, q);
    }
  }
}

__global__ __launch_bounds__(kBlock) void silu_and_mul_quant_scalar(void* __restrict__ out, int64_t out_stride,
                                                                    const void* __restrict__ in, int64_t in_stride,
                                                                    int64_t rows, int64_t inter,
                                                                    const float* __restrict__ scale_dev,
                                                                    float scale_host) {
  const float scale = scale_dev != nullptr ? *scale_dev : scale_host;
  const int64_t total = rows * inter;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kBlock) {
    const int64_t row = i / inter, col = i - row * inter;
    const uint16_t* g = static_cast<const uint16_t*>(in) + row * in_stride;
    const uint32_t y = pack_bf16x2(silu_mul(bf16_lo(g[col]), bf16_lo(g[inter + col])), 0.f);
    static_cast<uint8_t*>(out)[row * out_stride + col] = static_cast<uint8_t>(fp8_saturate_encode(bf16_lo(y) / scale));
  }
}

__global__ __launch_bounds__(kBlock) void silu_and_mul_scalar(void* __restrict__ out, int64_t out_stride,
                                                              const void* __restrict__ in, int64_t in_stride,
                                                              int64_t rows, int64_t inter) {
  const int64_t total = rows * inter;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kBlock) {
    const int64_t row = i / inter, col = i - row * inter;
    const uint16_t* g = static_cast<const uint16_t*>(in) + row * in_stride;
    const float y = silu_mul(bf16_lo(g[col]), bf16_lo(g[inter + col]));
    static_cast<uint16_t*>(out)[row * out_stride + col] = static_cast<uint16_t>(pack_bf16x2(y, 0.f));
  }
}

// Grid of (tiles of one row) x (rows): the row comes from blockIdx.y, so no lane divides by the
// tile count. Rows past the grid's y extent (65535) are covered by a uniform stride loop.
dim3 row_tile_grid(int64_t tiles_per_row, int64_t rows) {
  return dim3(static_cast<uint32_t>(tiles_per_row), static_cast<uint32_t>(rows < 65535 ? rows : 65535));
}

// One vector per lane and a grid covering every vector once: measured best on MI355X at every size
// from the 64-token decode to 16384 x 28672 (more waves in flight beat 2 and 4 vectors per lane).
int launch_vec(void* out, int64_t out_stride, const void* in, int64_t in_stride, int64_t rows, int64_t inter,
               hipStream_t s) {
  hipLaunchKernelGGL((silu_and_mul_vec<1>), row_tile_grid(cdiv(inter / 8, kVecBlock), rows), dim3(kVecBlock), 0, s, out,
                     out_stride, in, in_stride, rows, inter);
  return launch_status();
}

}  // namespace
}  // namespace mas

extern "C" int mas_silu_and_mul_bf16(void* out, int64_t out_stride, const void* input, int64_t input_stride,
                                     int64_t rows, int64_t inter, hipStream_t stream) {
  using namespace mas;
  if (rows < 0 || inter < 0) return MAS_ERR_INVALID_VALUE;
  if (rows == 0 || inter == 0) return MAS_OK;
  if (out == nullptr || input == nullptr) return MAS_ERR_INVALID_VALUE;
  if (rows > 1 && (out_stride < inter || input_stride < 2 * inter)) return MAS_ERR_INVALID_VALUE;
  if (inter > (int64_t{1} << 40)) return MAS_ERR_UNSUPPORTED;
  int cus = 0;
  if (const int st = device_cu_count(&cus); st != MAS_OK) return st;
  const bool vec_ok = inter % 8 == 0 && aligned16(out) && aligned16(input) && out_stride % 8 == 0 &&
                      input_stride % 8 == 0;
  if (!vec_ok) {
    const int64_t blocks = cdiv(rows * inter, kBlock);
    const int64_t grid = blocks < 8 * cus ? blocks : 8 * cus;
    hipLaunchKernelGGL(silu_and_mul_scalar, dim3(static_cast<uint32_t>(grid)), dim3(kBlock), 0, stream, out,
                       out_stride, input, input_stride, rows, inter);
    return launch_status();
  }
  return launch_vec(out, out_stride, input, input_stride, rows, inter, stream);
}

extern "C" int mas_silu_and_mul_quant_fp8(void* out, int64_t out_stride, const void* input, int64_t input_stride,
                                          int64_t rows, int64_t inter, const float* scale_dev, float scale_host,
                                          hipStream_t stream) {
  using namespace mas;
  if (rows < 0 || inter < 0) return MAS_ERR_INVALID_VALUE;
  if (rows == 0 || inter == 0) return MAS_OK;
  if (out == nullptr || input == nullptr) return MAS_ERR_INVALID_VALUE;
  if (rows > 1 && (out_stride < inter || input_stride < 2 * inter)) return MAS_ERR_INVALID_VALUE;
  if (inter > (int64_t{1} << 40)) return MAS_ERR_UNSUPPORTED;
  int cus = 0;
  if (const int st = device_cu_count(&cus); st != MAS_OK) return st;
  const bool vec_ok = inter % 8 == 0 && (reinterpret_cast<uintptr_t>(out) & 7u) == 0 && aligned16(input) &&
                      out_stride % 8 == 0 && input_stride % 8 == 0;
  if (!vec_ok) {
    const int64_t blocks = cdiv(rows * inter, kBlock);
    const int64_t grid = blocks < 8 * cus ? blocks : 8 * cus;
    hipLaunchKernelGGL(silu_and_mul_quant_scalar, dim3(static_cast<uint32_t>(grid)), dim3(kBlock), 0, stream, out,
                       out_stride, input, input_stride, rows, inter, scale_dev, scale_host);
    return launch_status();
  }
  hipLaunchKernelGGL(silu_and_mul_quant_vec, row_tile_grid(cdiv(inter / 8, kVecBlock), rows), dim3(kVecBlock), 0, stream,
                     out, out_stride, input, input_stride, rows, inter, scale_dev, scale_host);
  return launch_status();
}
