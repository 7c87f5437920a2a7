// Calibration statistics that feed add_batch (G2PTQ / GuidedQuant).
//
// SaliencyCache.grad_hook (gptq_utils/g2ptq_utils.py:604-618): for the
// gradient of a linear's output (n tokens × hidden), the mean over each of G
// equal channel groups of grad², one (n, G) fp32 saliency per batch.
//   group_mean_square_kernel: one wave per (token, group); lanes stride the
//   group's columns (coalesced), a butterfly sums the squares, and the mean is
//   sum · fp32(1/gs), the product torch's mean reduction forms on the GPU.
//
// GradientCache.cache_gradient (:704-714): the per-token running mean of the
// weight gradient, cache ← cache·(k/(k+1)) + grad/(n·(k+1)).
//   running_mean_kernel: one elementwise HBM pass, in the reference's fp32
//   operation order; the division by the Python number n·(k+1) is, in torch
//   on the GPU, a multiplication by its fp32 reciprocal, and so it is here.
#include <algorithm>

#include "common.hpp"

// Every product and sum is rounded on its own, as torch evaluates these
// expressions: no fused multiply-adds.  The __f*_rn helpers are plain
// operators in the HIP headers, so this translation unit is built with
// -ffp-contract=off (the pragma covers this file's own code).
#pragma clang fp contract(off)

namespace g2ptq {
namespace {

__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
  if (dtype == 0) return __uint_as_float((uint32_t) static_cast<const uint16_t*>(p)[i] << 16);
  if (dtype == 1) return (float)static_cast<const _Float16*>(p)[i];
  return static_cast<const float*>(p)[i];
}

__global__ __launch_bounds__(256) void group_mean_square_kernel(const void* __restrict__ x,
                                                                int dtype, int64_t rows,
                                                                int64_t ldx, int64_t groups,
                                                                int64_t gs, float inv_gs,
                                                                float* __restrict__ out) {
  const int64_t pair = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (pair >= rows * groups) return;  // whole waves: no barrier below
  const int64_t t = pair / groups, g = pair - t * groups;
  const int64_t base = t * ldx + g * gs;
  float acc = 0.f;
  for (int64_t c = lane; c < gs; c += 64) {
    const float v = load_any(x, base + c, dtype);
    acc = __fadd_rn(acc, __fmul_rn(v, v));  // grad.float().pow(2), then the sum
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if (lane == 0) out[pair] = __fmul_rn(acc, inv_gs);
}

__global__ __launch_bounds__(256) void running_mean_kernel(float* __restrict__ cache,
                                                           const void* __restrict__ grad,
                                                           int dtype, int64_t n, float keep,
                                                           float inv_count, int first) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float d = __fmul_rn(load_any(grad, i, dtype), inv_count);
    // first call: the cache is the Python int 0, so cache·keep + d is 0.0 + d
    const float c = first ? 0.f : __fmul_rn(cache[i], keep);
    cache[i] = __fadd_rn(c, d);
  }
}

}  // namespace
}  // namespace g2ptq

using namespace g2ptq;

extern "C" int g2ptq_group_mean_square(void* stream, const void* x, int dtype, int64_t rows,
                                       int64_t cols, int64_t ldx, int64_t groups, float* out) {
  G2PTQ_CHECK(dtype >= 0 && dtype <= 2, "group_mean_square: dtype code %d", dtype);
  G2PTQ_CHECK(rows >= 0 && cols >= 0 && groups >= 1, "group_mean_square: bad sizes");
  G2PTQ_CHECK(cols % groups == 0, "group_mean_square: %lld columns do not split into %lld groups",
              (long long)cols, (long long)groups);
  if (rows == 0 || cols == 0) return G2PTQ_OK;
  G2PTQ_CHECK(x && out && ldx >= cols, "group_mean_square: bad operands");
  const int64_t gs = cols / groups;
  const int64_t waves = rows * groups;
  G2PTQ_CHECK(cdiv(waves, (int64_t)4) < (1ll << 31), "group_mean_square: too many rows");
  hipLaunchKernelGGL(group_mean_square_kernel, dim3((unsigned)cdiv(waves, (int64_t)4)), dim3(256),
                     0, as_stream(stream), x, dtype, rows, ldx, groups, gs, 1.0f / (float)gs,
                     out);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

extern "C" int g2ptq_running_mean_update(void* stream, float* cache, const void* grad, int dtype,
                                         int64_t n, float keep, float inv_count, int first) {
  G2PTQ_CHECK(dtype >= 0 && dtype <= 2, "running_mean_update: dtype code %d", dtype);
  G2PTQ_CHECK(n >= 0, "running_mean_update: negative size");
  if (n == 0) return G2PTQ_OK;
  G2PTQ_CHECK(cache && grad, "running_mean_update: null pointer");
  const unsigned blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, 256), 8192));
  hipLaunchKernelGGL(running_mean_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), cache,
                     grad, dtype, n, keep, inv_count, first);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}
