// stream_skeleton.hip - memory skeletons of the layer kernels, built into a separate library that
// only the benchmark loads (libmas_bench.so); nothing in the product path calls it.
//
// A skeleton moves the bytes of one layer kernel over the same buffers - the same rows, row
// strides and read / write mix - with no arithmetic: each lane loads one 16-byte vector from every
// source stream (non-temporal, as the kernels do) and stores one to every destination stream. Timed
// beside the kernel in the same run and under the same protocol, it is the practical ceiling for a
// kernel of that size and shape, launch ramp-up and drain included (a 1 GiB copy amortises those,
// a 12 MB decode kernel cannot).
#include "../csrc/device.h"

namespace mas {
namespace {

struct SkeletonStreams {
  const uint16_t* src[2];
  int64_t src_stride[2];  // elements between rows
  uint16_t* dst[2];
  int64_t dst_stride[2];
};

// kSrc == kDst: source j is copied to destination j. kSrc = 2, kDst = 1: the destination gets the
// XOR of the two sources (SiluAndMul's two-reads-per-write mix).
template <int kSrc, int kDst>
__global__ __launch_bounds__(256) void stream_skeleton(SkeletonStreams s, int64_t row_vecs) {
  const int64_t v = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = blockIdx.y;
  if (v >= row_vecs) return;
  u32x4 x[kSrc];
#pragma unroll
  for (int j = 0; j < kSrc; ++j) x[j] = load_stream(s.src[j] + row * s.src_stride[j] + 8 * v);
  if constexpr (kSrc == kDst) {
#pragma unroll
    for (int j = 0; j < kDst; ++j) store_stream(s.dst[j] + row * s.dst_stride[j] + 8 * v, x[j]);
  } else {
    store_stream(s.dst[0] + row * s.dst_stride[0] + 8 * v, x[0] ^ x[1]);
  }
}

// The fused RoPE + KV append kernel's streams: each token's qkv row is read once; its q and k
// vectors are written back in place, k also to a key-cache row and v to a value-cache row (cache
// rows consecutive per token, as the KV skeleton writes them). The in-place write-back goes through
// `qkv_out`, the same address passed as a second pointer: a store of a just-loaded value through
// the pointer it was loaded from would be removed by the compiler, with its load.
__global__ __launch_bounds__(256) void rope_append_skeleton(const uint16_t* qkv, uint16_t* qkv_out, int64_t qkv_stride,
                                                            int64_t qk_vecs, int64_t kv_vecs, uint16_t* k_cache,
                                                            uint16_t* v_cache, int64_t cache_stride) {
  const int64_t v = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = blockIdx.y;
  if (v >= qk_vecs + kv_vecs) return;
  const u32x4 x = load_stream(qkv + row * qkv_stride + 8 * v);
  if (v < qk_vecs) {
    store_stream(qkv_out + row * qkv_stride + 8 * v, x);
    if (v >= qk_vecs - kv_vecs) store_stream(k_cache + row * cache_stride + 8 * (v - (qk_vecs - kv_vecs)), x);
  } else {
    store_stream(v_cache + row * cache_stride + 8 * (v - qk_vecs), x);
  }
}

}  // namespace
}  // namespace mas

// rows x row_elems bf16 elements per stream; src1 / dst1 null for one stream. Supported mixes:
// 1 -> 1, 2 -> 2 (pairwise copies) and 2 -> 1. Rows up to 65535 (one grid row each); row_elems a
// multiple of 8 and every pointer and stride 16-byte aligned. `block_threads`: threads per
// workgroup, 64 or 256 (neither shape is the faster one at every size, so the benchmark times both).
extern "C" int mas_bench_stream_skeleton(const void* src0, int64_t src0_stride, const void* src1,
                                         int64_t src1_stride, void* dst0, int64_t dst0_stride, void* dst1,
                                         int64_t dst1_stride, int64_t rows, int64_t row_elems, int64_t block_threads,
                                         hipStream_t stream) {
  using namespace mas;
  if (rows < 0 || row_elems < 0 || rows > 65535 || (block_threads != 64 && block_threads != 256))
    return MAS_ERR_INVALID_VALUE;
  if (rows == 0 || row_elems == 0) return MAS_OK;
  if (src0 == nullptr || dst0 == nullptr || (dst1 != nullptr && src1 == nullptr)) return MAS_ERR_INVALID_VALUE;
  if (row_elems % 8 != 0 || !aligned16(src0) || !aligned16(dst0) || src0_stride % 8 != 0 || dst0_stride % 8 != 0)
    return MAS_ERR_INVALID_VALUE;
  if ((src1 != nullptr && (!aligned16(src1) || src1_stride % 8 != 0)) ||
      (dst1 != nullptr && (!aligned16(dst1) || dst1_stride % 8 != 0)))
    return MAS_ERR_INVALID_VALUE;
  SkeletonStreams s{{static_cast<const uint16_t*>(src0), static_cast<const uint16_t*>(src1)},
                    {src0_stride, src1_stride},
                    {static_cast<uint16_t*>(dst0), static_cast<uint16_t*>(dst1)},
                    {dst0_stride, dst1_stride}};
  const int64_t row_vecs = row_elems / 8;
  const int block = row_vecs >= block_threads ? static_cast<int>(block_threads)
                                              : static_cast<int>(cdiv(row_vecs, kWave) * kWave);
  const dim3 grid(static_cast<uint32_t>(cdiv(row_vecs, block)), static_cast<uint32_t>(rows));
  if (src1 == nullptr)
    hipLaunchKernelGGL((stream_skeleton<1, 1>), grid, dim3(block), 0, stream, s, row_vecs);
  else if (dst1 != nullptr)
    hipLaunchKernelGGL((stream_skeleton<2, 2>), grid, dim3(block), 0, stream, s, row_vecs);
  else
    hipLaunchKernelGGL((stream_skeleton<2, 1>), grid, dim3(block), 0, stream, s, row_vecs);
  return launch_status();
}

// The fused RoPE + KV append's memory skeleton: rows of [q | k | v] (qk_elems + kv_elems elements
// each, the last kv_elems of the q|k part being k) read once; q|k written back in place, k to
// k_cache and v to v_cache rows of cache_stride elements. Rows up to 65535; every size a multiple
// of 8 and every pointer and stride 16-byte aligned. `block_threads`: 64 or 256.
extern "C" int mas_bench_rope_append_skeleton(void* qkv, int64_t qkv_stride, int64_t qk_elems, int64_t kv_elems,
                                              void* k_cache, void* v_cache, int64_t cache_stride, int64_t rows,
                                              int64_t block_threads, hipStream_t stream) {
  using namespace mas;
  if (rows < 0 || rows > 65535 || qk_elems < kv_elems || kv_elems < 0 ||
      (block_threads != 64 && block_threads != 256))
    return MAS_ERR_INVALID_VALUE;
  if (rows == 0 || qk_elems == 0) return MAS_OK;
  if (qkv == nullptr || k_cache == nullptr || v_cache == nullptr) return MAS_ERR_INVALID_VALUE;
  if (qk_elems % 8 != 0 || kv_elems % 8 != 0 || qkv_stride % 8 != 0 || cache_stride % 8 != 0 ||
      qkv_stride < qk_elems + kv_elems || cache_stride < kv_elems || !aligned16(qkv) || !aligned16(k_cache) ||
      !aligned16(v_cache))
    return MAS_ERR_INVALID_VALUE;
  const int64_t vecs = (qk_elems + kv_elems) / 8;
  const dim3 grid(static_cast<uint32_t>(cdiv(vecs, block_threads)), static_cast<uint32_t>(rows));
  hipLaunchKernelGGL(rope_append_skeleton, grid, dim3(static_cast<uint32_t>(block_threads)), 0, stream,
                     static_cast<const uint16_t*>(qkv), static_cast<uint16_t*>(qkv), qkv_stride, qk_elems / 8,
                     kv_elems / 8,
                     static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), cache_stride);
  return launch_status();
}
