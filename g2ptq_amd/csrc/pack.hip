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
//
// MoE expert stacking (utils/models/mixins.py:93-144) turns the per-expert
// tensors of a layer into 3-D checkpoint tensors with torch.stack of
// torch.cat's; here one launch copies every expert's tensor to its place
// (concat_kernel: workgroup column y copies source y, 16-byte vectors when
// both ends are aligned).
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

constexpr int64_t kConcatChunk = 256 * 16 * 8;  // bytes per workgroup pass

__global__ __launch_bounds__(256) void concat_kernel(const uint64_t* __restrict__ src,
                                                     const int64_t* __restrict__ off,
                                                     unsigned char* __restrict__ dst) {
  const int64_t b = blockIdx.y;
  const int64_t lo = off[b], size = off[b + 1] - lo;
  const unsigned char* s = reinterpret_cast<const unsigned char*>(src[b]);
  unsigned char* d = dst + lo;
  const bool vec = ((reinterpret_cast<uintptr_t>(s) | reinterpret_cast<uintptr_t>(d)) & 15) == 0;
  for (int64_t c0 = (int64_t)blockIdx.x * kConcatChunk; c0 < size;
       c0 += (int64_t)gridDim.x * kConcatChunk) {
    const int64_t c1 = c0 + kConcatChunk < size ? c0 + kConcatChunk : size;
    int64_t i = c0;
    if (vec) {
      const int64_t v1 = c0 + (c1 - c0) / 16 * 16;
#pragma unroll 8
      for (int64_t k = c0 + 16 * (int64_t)threadIdx.x; k < v1; k += 16 * 256)
        *reinterpret_cast<uint4*>(d + k) = *reinterpret_cast<const uint4*>(s + k);
      i = v1;
    }
    for (int64_t k = i + threadIdx.x; k < c1; k += 256) d[k] = s[k];
  }
}

unsigned grid_of(int64_t n) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, 256), 16384));
}

}  // namespace
}  // namespace g2ptq

using namespace g2ptq;

extern "C" int g2ptq_concat(void* stream, const uint64_t* src, const int64_t* off, int64_t n,
                            int64_t max_bytes, void* dst) {
  G2PTQ_CHECK(n >= 0 && n < 65536, "concat: %lld buffers (at most 65535)", (long long)n);
  G2PTQ_CHECK(max_bytes >= 0, "concat: negative size");
  if (n == 0 || max_bytes == 0) return G2PTQ_OK;
  G2PTQ_CHECK(src && off && dst, "concat: null pointer");
  // enough workgroups per source to cover the largest one, at most ~4096 in all
  const int64_t per = std::max<int64_t>(1, std::min<int64_t>(cdiv(max_bytes, kConcatChunk),
                                                             cdiv(4096, n)));
  hipLaunchKernelGGL(concat_kernel, dim3((unsigned)per, (unsigned)n), dim3(256), 0,
                     as_stream(stream), src, off, static_cast<unsigned char*>(dst));
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

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
