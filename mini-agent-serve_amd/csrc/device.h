// device.h - gfx950 device helpers shared by the layer kernels: 128-bit vector memory access,
// bf16 / fp8-e4m3fn conversions, DPP wavefront reductions and launch-time device queries.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mas_kernels.h"

namespace mas {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kWave = 64;
constexpr int kXcds = 8;  // MI355X: workgroups go to its 8 XCDs (each with its own L2) round-robin by id

// ---- memory ------------------------------------------------------------------------------
// Streaming accesses carry the non-temporal hint: every byte these kernels move is touched once.
__device__ __forceinline__ u32x4 load_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void store_stream(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ void store_stream(void* p, u32x2 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x2*>(p));
}
// Keeps the compiler's scheduler from moving instructions across this point: placed after a
// kernel's group of loads so that all of them issue before the first instruction that waits on one.
__device__ __forceinline__ void load_fence() { __builtin_amdgcn_sched_barrier(0); }

// Cached access, for data re-read by other waves (norm weights, cos/sin rows, index tables).
__device__ __forceinline__ u32x4 load_cached(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ f32x4 load_cached_f4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

// ---- bf16 ----------------------------------------------------------------------------------
// A bf16 value is the high half of an fp32, so widening is a shift.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two fp32 -> packed bf16 pair, round-to-nearest-even (one v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Unpack 8 bf16 (one 128-bit vector) into fp32.
__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(v[i]);
    f[2 * i + 1] = bf16_hi(v[i]);
  }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return v;
}

// ---- fp8 e4m3fn (OCP: bias 7, no infinities, max 448, NaN = S.1111.111) -------------------
// Saturating encode of four fp32 values, code i in byte i: |v| > 448 -> +-448, otherwise round to
// nearest even, NaN -> 0x7f with the input's sign. gfx950's v_cvt_pk_fp8_f32 does the rounding
// (OCP e4m3 on this target) on inputs clamped beforehand; it writes 0xff for every NaN, so the
// sign bits are put back with two byte permutes. Matches the integer-arithmetic encoder
// (clamp, then RNE at mantissa bit 20, subnormals as m * 2^-9) on all 2^32 fp32 inputs.
// IEEE 754-2019 maximum/minimum (v_maximum3_f32 / v_minimum3_f32 on gfx950): NaN passes through.
__device__ __forceinline__ float fp8_clamp(float v) {
  return __builtin_elementwise_minimum(__builtin_elementwise_maximum(v, -448.0f), 448.0f);
}

__device__ __forceinline__ uint32_t fp8x4_saturate_encode(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(fp8_clamp(a), fp8_clamp(b), 0, false);
  const uint32_t codes =
      static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(fp8_clamp(c), fp8_clamp(d), lo, true));
  const uint32_t signs = __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x0c0c0703u) |
                         __builtin_amdgcn_perm(__float_as_uint(d), __float_as_uint(c), 0x07030c0cu);
  return codes & (signs | 0x7f7f7f7fu);
}

__device__ __forceinline__ uint32_t fp8_saturate_encode(float v) { return fp8x4_saturate_encode(v, v, v, v) & 0xffu; }

// y / s rounded as IEEE division rounds it, from r = 1/s (one division per thread), for the fp8
// epilogues: q0 = y * r is within an ulp of the quotient, the residual q0 * s - y is exact in one
// fma, and q0 minus the residual times r rounds to the correctly rounded quotient (Markstein, IBM J.
// Res. Dev. 34(1), 1990). Holds while the residual does not underflow, i.e. for every
// |y / s| >= 2^-100 - far below fp8's smallest subnormal 2^-9. Before the correction q0 is clamped
// to +-896 (one v_med3): values that far out saturate to +-448 whatever their rounding, and the
// clamp keeps the residual finite when y * r overflows or y is infinite (the result is then
// +-inf or a value past 896, which the fp8 clamp saturates). A NaN y returns NaN through -y. The
// residual is formed as q0 * s - y so that a zero quotient keeps its sign (-0 - (+0) * r = -0).
// s must be a positive normal number (an activation scale).
__device__ __forceinline__ float div_by_scale(float y, float s, float r) {
  const float q0 = __builtin_amdgcn_fmed3f(y * r, -896.0f, 896.0f);
  const float e = __builtin_fmaf(q0, s, -y);
  return __builtin_fmaf(-e, r, q0);
}

// ---- wavefront / block reductions ----------------------------------------------------------
template <int kCtrl>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf,
                                                               false));
}

// Max / sum over each row of 16 lanes; every lane of the row receives the result.
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

// Sum over the 64 lanes of a wavefront; every lane receives the total. Rows of 16 lanes reduce
// through DPP (quad_perm xor1, xor2, row_half_mirror, row_mirror), then the four row sums are
// read out and added in a fixed order.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_move<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  v += dpp_move<0x140>(v);  // row_mirror
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Sum over the block (at most 16 wavefronts); `slots` is a 16-float, 16-byte aligned LDS array.
// Each wavefront's sum goes to its slot and the unused slots are zeroed, then every lane reads all
// 16 back with four 16-byte reads and adds them as a fixed tree: no loop over the wavefront count
// after the barrier. The caller alternates between two slot arrays on consecutive calls, so one
// barrier per call is enough.
__device__ __forceinline__ float block_sum(float v, float* slots) {
  v = wave_sum(v);
  const int nwaves = blockDim.x / kWave;
  if (nwaves == 1) return v;
  const int tid = threadIdx.x;
  if ((tid & (kWave - 1)) == 0) slots[tid / kWave] = v;
  if (tid >= nwaves && tid < 16) slots[tid] = 0.f;
  __syncthreads();
  const f32x4 a0 = *reinterpret_cast<const f32x4*>(slots), a1 = *reinterpret_cast<const f32x4*>(slots + 4);
  const f32x4 a2 = *reinterpret_cast<const f32x4*>(slots + 8), a3 = *reinterpret_cast<const f32x4*>(slots + 12);
  return (((a0[0] + a0[1]) + (a0[2] + a0[3])) + ((a1[0] + a1[1]) + (a1[2] + a1[3]))) +
         (((a2[0] + a2[1]) + (a2[2] + a2[3])) + ((a3[0] + a3[1]) + (a3[2] + a3[3])));
}

// Four values of one column of a row-major bf16 tile in LDS (rows vrow elements apart) from four
// consecutive rows, with gfx950's transposing LDS read: in each group of 16 lanes, lane k points
// at row first + k / 4, columns col0 + 4 (k % 4) .. + 3; lane n then holds rows first .. first + 3
// of column col0 + n.
__device__ __forceinline__ i16x4 read_column4(const uint16_t* lds_tile, int vrow, int first, int col0, int k) {
  const uint16_t* p = lds_tile + (first + (k >> 2)) * vrow + col0 + 4 * (k & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(__attribute__((address_space(3))) uint16_t*)(p));
}

__device__ __forceinline__ void report(uint32_t* err, uint32_t bit) {
  if (err != nullptr) __hip_atomic_fetch_or(err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int wave_id_uniform() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
}

// ---- host-side helpers ---------------------------------------------------------------------
// Compute units of the current device (cached per device after the first query).
int device_cu_count(int* cus);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MAS_OK : static_cast<int>(e);
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace mas
