// rmsnorm.hip - fused residual add + RMSNorm, bf16 (in place) and fp8-e4m3fn epilogues.
//
// Semantics (miniagentserve/models/devstral2/devstral2.py:241-252 and 305-307, the
// flashinfer.norm.fused_add_rmsnorm / fused_add_rmsnorm_quant calls):
//   s = f32(x) + f32(r)               per element, exact fp32 add of two bf16
//   r <- bf16(s)                      the updated residual stream
//   rstd = rsqrt(sum(s*s) / H + eps)  the hardware reciprocal square root (v_rsq_f32, within 1 ulp
//                                     of 1 / sqrt: 0.1 us less latency per row than the IEEE pair)
//   y = (s * rstd) * f32(w)
//   bf16 epilogue: x <- bf16(y)       fp8 epilogue: out <- e4m3fn(clamp(y / scale, +-448))
//
// Fast path: one workgroup per row. The row is held in registers as VPT 128-bit vectors per
// lane (8 bf16 each), so x and r are read from HBM once and every output is written once; each
// workgroup loads its weight slice once. Row sum of squares: DPP wavefront sum, then one LDS slot
// per wavefront, read back in four 16-byte reads.
// Generic path (hidden not a multiple of 8, unaligned rows, or rows wider than 65536): two
// passes over the row with scalar accesses, the second recomputing s from x and r.
#include "device.h"

namespace mas {
namespace {

struct NormArgs {
  void* out;  // bf16: the input rows themselves; fp8: the quantized output
  int64_t out_stride;
  const void* input;
  int64_t in_stride;
  void* residual;
  int64_t res_stride;
  const void* weight;
  const float* scale_dev;
  float scale_host;
  int64_t rows;
  int hidden;
  float eps;
};

__device__ __forceinline__ float norm_scale(const NormArgs& a) {
  return a.scale_dev != nullptr ? *a.scale_dev : a.scale_host;
}

// Largest workgroup each register tile is launched with; the launch bound lets the compiler give
// the wider tiles up to 256 VGPRs without spilling.
constexpr int max_threads_for(int vpt) { return vpt <= 4 ? 1024 : (vpt <= 6 ? 512 : 256); }

template <int VPT, bool kFp8>
__global__ __launch_bounds__(max_threads_for(VPT)) void fused_add_rmsnorm_tile(NormArgs a) {
  __shared__ __align__(16) float slots[2][16];
  const int nvec = a.hidden >> 3;
  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const float hidden_f = static_cast<float>(a.hidden);

  // Vector indices past the row end are clamped to its last vector, so every load is in bounds
  // and unconditional (the compiler then issues them back to back); those lanes contribute zero
  // to the sum and store nothing. The weight slice is loaded once, ahead of the rows: measured
  // faster on MI355X than loading it in each row's group (3.10 vs 3.25 us for 64 x 5120).
  u32x4 w[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int v = tid + j * nthr;
    w[j] = load_cached(static_cast<const uint16_t*>(a.weight) + 8 * (v < nvec ? v : nvec - 1));
  }

  int parity = 0;
  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const uint16_t* x = static_cast<const uint16_t*>(a.input) + row * a.in_stride;
    uint16_t* r = static_cast<uint16_t*>(a.residual) + row * a.res_stride;

    u32x4 xv[VPT], rv[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = tid + j * nthr;
      const int vl = v < nvec ? v : nvec - 1;
      xv[j] = load_stream(x + 8 * vl);
      rv[j] = load_stream(r + 8 * vl);
    }
    load_fence();
    const float scale = kFp8 ? norm_scale(a) : 1.0f;
    const float rcp = 1.0f / scale;

    float s[VPT][8];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const bool valid = tid + j * nthr < nvec;
      float xf[8], rf[8];
      unpack8(xv[j], xf);
      unpack8(rv[j], rf);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s[j][e] = valid ? xf[e] + rf[e] : 0.f;
        ss = fmaf(s[j][e], s[j][e], ss);
      }
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = tid + j * nthr;
      if (v < nvec) store_stream(r + 8 * v, pack8(s[j]));
    }

    const float total = block_sum(ss, slots[parity]);
    parity ^= 1;
    const float rstd = __builtin_amdgcn_rsqf(total / hidden_f + a.eps);

#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = tid + j * nthr;
      if (v < nvec) {
        float wf[8], y[8];
        unpack8(w[j], wf);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = (s[j][e] * rstd) * wf[e];
        if constexpr (kFp8) {
          u32x2 q;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            q[h] = fp8x4_saturate_encode(div_by_scale(y[4 * h], scale, rcp), div_by_scale(y[4 * h + 1], scale, rcp),
                                         div_by_scale(y[4 * h + 2], scale, rcp), div_by_scale(y[4 * h + 3], scale, rcp));
          }
          store_stream(static_cast<uint8_t*>(a.out) + row * a.out_stride + 8 * v, q);
        } else {
          store_stream(static_cast<uint16_t*>(a.out) + row * a.out_stride + 8 * v, pack8(y));
        }
      }
    }
  }
}

template <bool kFp8>
__global__ __launch_bounds__(256) void fused_add_rmsnorm_generic(NormArgs a) {
  __shared__ __align__(16) float slots[2][16];
  const float hidden_f = static_cast<float>(a.hidden);
  const float scale = kFp8 ? norm_scale(a) : 1.0f;
  const uint16_t* w = static_cast<const uint16_t*>(a.weight);
  int parity = 0;
  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const uint16_t* x = static_cast<const uint16_t*>(a.input) + row * a.in_stride;
    uint16_t* r = static_cast<uint16_t*>(a.residual) + row * a.res_stride;
    float ss = 0.f;
    for (int i = threadIdx.x; i < a.hidden; i += blockDim.x) {
      const float s = bf16_lo(x[i]) + bf16_lo(r[i]);
      ss = fmaf(s, s, ss);
    }
    const float total = block_sum(ss, slots[parity]);
    parity ^= 1;
    const float rstd = __builtin_amdgcn_rsqf(total / hidden_f + a.eps);
    for (int i = threadIdx.x; i < a.hidden; i += blockDim.x) {
      const float s = bf16_lo(x[i]) + bf16_lo(r[i]);
      const float y = (s * rstd) * bf16_lo(w[i]);
      r[i] = static_cast<uint16_t>(pack_bf16x2(s, 0.f));
      if constexpr (kFp8) {
        static_cast<uint8_t*>(a.out)[row * a.out_stride + i] = static_cast<uint8_t>(fp8_saturate_encode(y / scale));
      } else {
        static_cast<uint16_t*>(a.out)[row * a.out_stride + i] = static_cast<uint16_t>(pack_bf16x2(y, 0.f));
      }
    }
  }
}

constexpr int kVpts[] = {1, 2, 3, 4, 5, 6, 8};

// Picks the register tile: VPT vectors per lane and a multiple of 64 lanes covering the row, with
// at most 12.5% padding. The most lanes per row wins, at every row count: measured on MI355X,
// 640 lanes beat 320 and 128 for hidden 5120, and 768 beat 512, 384 and 256 for hidden 12288
// (more waves in flight per CU, fewer registers per lane).
bool choose_tile(int64_t nvec, int* vpt, int* threads) {
  int best_v = 0, best_t = 0;
  int64_t best_score = INT64_MAX;
  for (int v : kVpts) {
    const int64_t t = cdiv(cdiv(nvec, v), kWave) * kWave;
    if (t > max_threads_for(v)) continue;
    const int64_t waste = t * v - nvec;
    if (waste * 8 > nvec) continue;  // more than 12.5% idle lanes
    const int64_t score = -t * 1024 + waste;
    if (score < best_score) {
      best_score = score;
      best_v = v;
      best_t = static_cast<int>(t);
    }
  }
  if (best_v == 0) {
    // Short rows (fewer than 64 vectors): one vector per lane beats the scalar path.
    const int64_t t = cdiv(nvec, kWave) * kWave;
    if (t > max_threads_for(1)) return false;
    best_v = 1;
    best_t = static_cast<int>(t);
  }
  *vpt = best_v;
  *threads = best_t;
  return true;
}

template <bool kFp8>
int launch_tile(int vpt, dim3 grid, dim3 block, hipStream_t s, const NormArgs& a) {
  switch (vpt) {
    case 1: hipLaunchKernelGGL((fused_add_rmsnorm_tile<1, kFp8>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((fused_add_rmsnorm_tile<2, kFp8>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((fused_add_rmsnorm_tile<3, kFp8>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((fused_add_rmsnorm_tile<4, kFp8>), grid, block, 0, s, a); break;
    case 5: hipLaunchKernelGGL((fused_add_rmsnorm_tile<5, kFp8>), grid, block, 0, s, a); break;
    case 6: hipLaunchKernelGGL((fused_add_rmsnorm_tile<6, kFp8>), grid, block, 0, s, a); break;
    case 8: hipLaunchKernelGGL((fused_add_rmsnorm_tile<8, kFp8>), grid, block, 0, s, a); break;
    default: return MAS_ERR_UNSUPPORTED;
  }
  return launch_status();
}

template <bool kFp8>
int run_norm(const NormArgs& a, int out_elem_bytes, hipStream_t stream) {
  if (a.rows < 0 || a.hidden < 0) return MAS_ERR_INVALID_VALUE;
  if (a.rows == 0 || a.hidden == 0) return MAS_OK;
  if (a.out == nullptr || a.input == nullptr || a.residual == nullptr || a.weight == nullptr)
    return MAS_ERR_INVALID_VALUE;
  if (a.rows > 1 && (a.in_stride < a.hidden || a.res_stride < a.hidden || a.out_stride < a.hidden))
    return MAS_ERR_INVALID_VALUE;
  if (!(a.eps >= 0.f)) return MAS_ERR_INVALID_VALUE;

  const int64_t nvec = a.hidden / 8;
  // 16-byte rows: hidden % 8 == 0, every base pointer and row stride keeps 16-byte alignment
  // (the fp8 output rows need 8-byte alignment: 8 codes per vector).
  const bool vec_ok = (a.hidden % 8 == 0) && aligned16(a.input) && aligned16(a.residual) && aligned16(a.weight) &&
                      (reinterpret_cast<uintptr_t>(a.out) % (8 * out_elem_bytes) == 0) && (a.in_stride % 8 == 0) &&
                      (a.res_stride % 8 == 0) && (a.out_stride % 8 == 0);
  int vpt = 0, threads = 0;
  const int64_t grid = a.rows < INT32_MAX ? a.rows : INT32_MAX;
  if (vec_ok && choose_tile(nvec, &vpt, &threads)) {
    return launch_tile<kFp8>(vpt, dim3(static_cast<uint32_t>(grid)), dim3(threads), stream, a);
  }
  hipLaunchKernelGGL((fused_add_rmsnorm_generic<kFp8>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0, stream,
                     a);
  return launch_status();
}

}  // namespace
}  // namespace mas

extern "C" int mas_fused_add_rmsnorm_bf16(void* input, int64_t input_stride, void* residual,
                                          int64_t residual_stride, const void* weight, int64_t rows,
                                          int64_t hidden, float eps, hipStream_t stream) {
  if (hidden > INT32_MAX) return MAS_ERR_UNSUPPORTED;
  mas::NormArgs a{input, input_stride, input, input_stride, residual, residual_stride, weight, nullptr, 1.0f,
                  rows, static_cast<int>(hidden), eps};
  return mas::run_norm<false>(a, 2, stream);
}

extern "C" int mas_fused_add_rmsnorm_quant_fp8(void* out, int64_t out_stride, const void* input,
                                               int64_t input_stride, void* residual, int64_t residual_stride,
                                               const void* weight, const float* scale_dev, float scale_host,
                                               int64_t rows, int64_t hidden, float eps, hipStream_t stream) {
  if (hidden > INT32_MAX) return MAS_ERR_UNSUPPORTED;
  mas::NormArgs a{out, out_stride, input, input_stride, residual, residual_stride, weight, scale_dev, scale_host,
                  rows, static_cast<int>(hidden), eps};
  return mas::run_norm<true>(a, 1, stream);
}
