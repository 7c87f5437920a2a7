// compressed-tensors "pack-quantized" export of one quantized layer.
//
// utils/compressed_tensors_utils.py:22-45 (compress) turns the compensation's
// per-element integer codes and scales into the checkpoint tensors:
//   weight_packed = pack_to_int32(W_int.to(int8), bits)   (compressed-tensors
//                   0.18.0, compressors/quantized_compressors/pack_quantized):
//                   each code offset by 2^(bits−1) to an unsigned field, 32/bits
//                   consecutive input columns per int32, the first column in the
//                   lowest bits, columns past the end zero;
//   weight_scale  = the first scale of every group, cast to the weight dtype,
//                   after asserting that every scale of a group is that one.
// Both are HBM-bound single passes: one thread per packed word (reading its
// 32/bits codes as one contiguous run), and one thread per scale element
// (comparing it with its group's first scale, and writing the group's value
// from the group's first column).
#include <algorithm>

#include "common.hpp"

namespace g2ptq {
namespace {

__device__ __forceinline__ uint16_t f2bf_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__global__ void pack_codes_kernel(const float* __restrict__ codes, int64_t ldc, int64_t rows,
                                  int64_t cols, int bits, int32_t* __restrict__ packed,
                                  int64_t ldp, int64_t words) {
  const int pf = 32 / bits;
  const uint32_t off = 1u << (bits - 1), mask = (1u << bits) - 1u;
  const int64_t n = rows * words;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / words, w = e - r * words;
    const float* src = codes + r * ldc + w * pf;
    const int64_t left = cols - w * pf;
    uint32_t acc = 0;
    for (int i = 0; i < pf; ++i) {
      if (i >= left) break;
      // float code → int8 (truncation, as torch's .to(int8) for integral values)
      const int c = (int)(int8_t)(int)src[i];
      acc |= (((uint32_t)(c + (int)off)) & mask) << (bits * i);
    }
    packed[r * ldp + w] = (int32_t)acc;
  }
}

__global__ void group_scale_kernel(const float* __restrict__ scale, int64_t lds, int64_t rows,
                                   int64_t cols, int64_t g, void* out, int dtype, int64_t ldo,
                                   int* flags) {
  const int64_t n = rows * cols;
  int bad = 0;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / cols, j = e - r * cols;
    const int64_t k = j / g, j0 = k * g;
    const float v = scale[r * lds + j];
    const float f = scale[r * lds + j0];
    // torch's == on the group: NaN never equals, so a NaN scale fails the check
    bad |= !(v == f);
    if (j == j0) {
      const int64_t o = r * ldo + k;
      if (dtype == 0) static_cast<uint16_t*>(out)[o] = f2bf_rne(f);
      else if (dtype == 1) static_cast<_Float16*>(out)[o] = (_Float16)f;
      else static_cast<float*>(out)[o] = f;
    }
  }
  bad = __any(bad);
  if (bad && (threadIdx.x & 63) == 0 && flags) atomicOr(flags, G2PTQ_FLAG_GROUP_SCALE);
}

unsigned grid_of(int64_t n) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, 256), 16384));
}

}  // namespace
}  // namespace g2ptq

using namespace g2ptq;

extern "C" int g2ptq_pack_quantized(void* stream, const float* codes, int64_t ldc,
                                    const float* scale, int64_t lds, int64_t rows, int64_t cols,
                                    int bits, int64_t groupsize, int32_t* packed, int64_t ldp,
                                    void* scale_out, int dtype, int64_t ldo, int* flags) {
  G2PTQ_CHECK(bits >= 1 && bits <= 8, "pack_quantized: bits=%d unsupported (1..8)", bits);
  G2PTQ_CHECK(rows >= 0 && cols >= 0, "pack_quantized: bad sizes");
  G2PTQ_CHECK(dtype >= 0 && dtype <= 2, "pack_quantized: dtype code %d", dtype);
  if (rows == 0 || cols == 0) return G2PTQ_OK;
  const int64_t pf = 32 / bits;
  const int64_t words = cdiv(cols, pf);
  G2PTQ_CHECK(codes && packed && ldc >= cols && ldp >= words, "pack_quantized: bad codes/packed");
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(pack_codes_kernel, dim3(grid_of(rows * words)), dim3(256), 0, st, codes, ldc,
                     rows, cols, bits, packed, ldp, words);
  G2PTQ_LAUNCHED();
  if (scale_out) {
    G2PTQ_CHECK(scale && groupsize >= 1 && cols % groupsize == 0 && lds >= cols &&
                    ldo >= cols / groupsize,
                "pack_quantized: group size %lld must divide %lld columns", (long long)groupsize,
                (long long)cols);
    hipLaunchKernelGGL(group_scale_kernel, dim3(grid_of(rows * cols)), dim3(256), 0, st, scale,
                       lds, rows, cols, groupsize, scale_out, dtype, ldo, flags);
    G2PTQ_LAUNCHED();
  }
  return G2PTQ_OK;
}
