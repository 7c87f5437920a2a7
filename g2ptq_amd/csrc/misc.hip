// Hessian preparation, act-order permutation, gathers, casts and the ABI
// identity functions.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace g2ptq {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

namespace {

size_t al256(size_t x) { return (x + 255) / 256 * 256; }

__global__ void fill_kernel(float* p, int64_t n, float v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// nz[b] |= any(diag H[b] != 0): a nonzero diagonal entry settles the test
// below without reading the rest (every real Hessian has one).
__global__ void nonzero_diag_kernel(const float* __restrict__ H, int64_t C, int* nz) {
  const int64_t b = blockIdx.y;
  const float* Hb = H + b * C * C;
  int any = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < C;
       i += (int64_t)gridDim.x * blockDim.x)
    any |= !(Hb[i * C + i] == 0.f);
  any = __any(any);
  if (any && (threadIdx.x & 63) == 0) atomicOr(&nz[b], 1);
}

// nz[b] = any(H[b] != 0)   (NaN counts as nonzero, like `(H == 0).all()` being False);
// only layers whose diagonal is all zero are scanned.
__global__ void nonzero_kernel(const float* __restrict__ H, int64_t CC, int* nz) {
  const int64_t b = blockIdx.y;
  if (nz[b]) return;  // settled by the diagonal (or another workgroup)
  const float* Hb = H + b * CC;
  int any = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < CC;
       i += (int64_t)gridDim.x * blockDim.x)
    any |= !(Hb[i] == 0.f);
  any = __any(any);
  if (any && (threadIdx.x & 63) == 0) atomicOr(&nz[b], 1);
}

// dead[b][i] = H[b] nonzero and H[b][i][i] == 0; anydead[b] = any of them.
__global__ void dead_kernel(const float* __restrict__ H, int64_t C, const int* nz, int* dead,
                            int* anydead) {
  const int64_t b = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= C) return;
  const int d = nz[b] && (H[b * C * C + i * C + i] == 0.f);
  dead[b * C + i] = d;
  if (d) atomicOr(&anydead[b], 1);
}

// An all-zero H[b] becomes the identity; otherwise only dead diagonal entries
// change (to 1), so only the diagonal is visited.
__global__ void fix_h_kernel(float* H, int64_t C, const int* nz, const int* dead) {
  const int64_t b = blockIdx.y;
  const int64_t CC = C * C;
  float* Hb = H + b * CC;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if (!nz[b]) {
    for (int64_t e = t0; e < CC; e += stride) Hb[e] = (e % (C + 1) == 0) ? 1.f : 0.f;
  } else {
    for (int64_t i = t0; i < C; i += stride)
      if (dead[b * C + i]) Hb[i * C + i] = 1.f;
  }
}

// wipe == 0: zero the dead columns of each (rows, C) slice of M (weights, GPTAQ's
// cross term).  wipe == 1: zero the whole slice where H[b] was all zero and leave
// every other slice alone, dead columns included (G2PTQ's gradients:
// g2ptq_utils.py:394-401 clears them only together with an all-zero Hessian).
__global__ void zero_cols_kernel(float* M, int64_t rows, int64_t C, const int* dead, const int* nz,
                                 const int* anydead, int wipe) {
  const int64_t b = blockIdx.y;
  const int64_t n = rows * C;
  float* Mb = M + b * n;
  if (wipe ? nz[b] != 0 : !anydead[b]) return;  // nothing to zero in this slice
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    if (wipe || dead[b * C + (e % C)]) Mb[e] = 0.f;
  }
}

__global__ void order_key_kernel(const float* __restrict__ src, int64_t B, int64_t C, int mode,
                                 float* key) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  float s = 0.f;
  for (int64_t b = 0; b < B; ++b) s += mode == 0 ? src[b * C * C + c * C + c] : src[b * C + c];
  key[c] = s / (float)B;
}

// Descending stable rank: rank[i] = #{j : key[j] > key[i] or (key[j] == key[i] and j < i)}.
__global__ __launch_bounds__(256) void rank_kernel(const float* __restrict__ key, int64_t C,
                                                   int* perm, int* invperm) {
  __shared__ float tile[1024];
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const float ki = i < C ? key[i] : 0.f;
  int64_t rank = 0;
  for (int64_t j0 = 0; j0 < C; j0 += 1024) {
    __syncthreads();
    for (int t = threadIdx.x; t < 1024; t += 256) tile[t] = (j0 + t < C) ? key[j0 + t] : 0.f;
    __syncthreads();
    const int64_t lim = std::min<int64_t>(1024, C - j0);
    for (int64_t t = 0; t < lim; ++t) {
      const float kj = tile[t];
      const int64_t j = j0 + t;
      rank += (kj > ki) || (kj == ki && j < i);
    }
  }
  if (i < C) {
    perm[rank] = (int)i;
    invperm[i] = (int)rank;
  }
}

__global__ void permute_cols_kernel(const float* __restrict__ in, float* __restrict__ out,
                                    int64_t rows, int64_t C, const int* __restrict__ cols) {
  const int64_t n = rows * C;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / C, c = e % C;
    out[e] = in[r * C + cols[c]];
  }
}

__global__ void permute_sym_kernel(const float* __restrict__ in, float* __restrict__ out,
                                   int64_t C, const int* __restrict__ perm) {
  const int64_t b = blockIdx.y;
  const int64_t CC = C * C;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < CC;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / C, j = e % C;
    out[b * CC + e] = in[b * CC + (int64_t)perm[i] * C + perm[j]];
  }
}

__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__global__ void cast_check_kernel(const float* __restrict__ in, void* out, int64_t n, int dtype,
                                  int* flags) {
  int nan = 0;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const float v = in[e];
    if (dtype == 0) {
      const uint16_t h = f2bf(v);
      static_cast<uint16_t*>(out)[e] = h;
      nan |= ((h & 0x7fff) > 0x7f80);
    } else if (dtype == 1) {
      const _Float16 h = (_Float16)v;
      static_cast<_Float16*>(out)[e] = h;
      nan |= (h != h);
    } else {
      static_cast<float*>(out)[e] = v;
      nan |= (v != v);
    }
  }
  nan = __any(nan);
  if (nan && (threadIdx.x & 63) == 0 && flags) atomicOr(flags, FLAG_NAN_OUTPUT);
}

__global__ void to_f32_kernel(const void* in, float* out, int64_t n, int dtype) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    if (dtype == 0)
      out[e] = __uint_as_float((uint32_t) static_cast<const uint16_t*>(in)[e] << 16);
    else if (dtype == 1)
      out[e] = (float)static_cast<const _Float16*>(in)[e];
    else
      out[e] = static_cast<const float*>(in)[e];
  }
}

// The bf16 cases on 8 elements (16 bytes of bf16) per step: the same
// conversion per element, with 16-byte loads and stores.
__global__ void bf16_to_f32_vec_kernel(const uint4* __restrict__ in, float4* __restrict__ out,
                                       int64_t n8) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n8;
       e += (int64_t)gridDim.x * blockDim.x) {
    const uint4 u = in[e];
    out[2 * e] = make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                             __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
    out[2 * e + 1] = make_float4(__uint_as_float(u.z << 16), __uint_as_float(u.z & 0xffff0000u),
                                 __uint_as_float(u.w << 16), __uint_as_float(u.w & 0xffff0000u));
  }
}

__global__ void cast_check_bf16_vec_kernel(const float4* __restrict__ in, uint4* __restrict__ out,
                                           int64_t n8, int* flags) {
  int nan = 0;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n8;
       e += (int64_t)gridDim.x * blockDim.x) {
    const float4 a = in[2 * e], b = in[2 * e + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t h[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      h[k] = f2bf(v[k]);
      nan |= ((h[k] & 0x7fff) > 0x7f80);
    }
    out[e] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                        h[6] | (h[7] << 16));
  }
  nan = __any(nan);
  if (nan && (threadIdx.x & 63) == 0 && flags) atomicOr(flags, FLAG_NAN_OUTPUT);
}

bool vec8(const void* a, const void* b, int64_t n) {
  return n % 8 == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(b) & 15) == 0;
}

unsigned grid_for(int64_t n) { return (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(n, 256), 16384)); }

}  // namespace

int fill_f32(hipStream_t s, float* p, int64_t n, float v) {
  if (n <= 0) return G2PTQ_OK;
  hipLaunchKernelGGL(fill_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, n, v);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

}  // namespace g2ptq

using namespace g2ptq;

extern "C" int g2ptq_abi_version(void) { return 1; }

extern "C" const char* g2ptq_status_string(int status) {
  switch (status) {
    case G2PTQ_OK: return "ok";
    case G2PTQ_ERR_ARG: return "invalid argument";
    case G2PTQ_ERR_HIP: return "HIP runtime error";
    case G2PTQ_ERR_WORKSPACE: return "workspace too small";
    case G2PTQ_ERR_UNSUPPORTED: return "unsupported";
    default: return "unknown status";
  }
}

extern "C" const char* g2ptq_last_error(void) { return g_last_error; }

extern "C" int g2ptq_prepare_hessian(void* stream, float* H, int64_t B, int64_t C, float* W,
                                     int64_t R, float* Dx, float* Grad, int64_t Rg, void* ws,
                                     size_t ws_bytes) {
  G2PTQ_CHECK(H && W, "prepare_hessian: null pointer");
  G2PTQ_CHECK(B >= 1 && B < 65536 && C >= 1, "prepare_hessian: bad sizes");
  const size_t need = al256((size_t)B * 8) + al256((size_t)B * C * 4);
  G2PTQ_CHECK(ws && ws_bytes >= need, "prepare_hessian: workspace %zu < %zu", ws_bytes, need);
  hipStream_t s = as_stream(stream);
  int* nz = static_cast<int*>(ws);  // B flags, then B "any dead column" flags
  int* anydead = nz + B;
  int* dead = reinterpret_cast<int*>(static_cast<char*>(ws) + al256((size_t)B * 8));
  // Flags start at zero: cleared by a kernel so the call can be graph-captured.
  G2PTQ_TRY(fill_f32(s, reinterpret_cast<float*>(nz), 2 * B, 0.f));
  const int64_t CC = C * C;
  hipLaunchKernelGGL(nonzero_diag_kernel, dim3((unsigned)std::min<int64_t>(cdiv(C, 256), 64), (unsigned)B),
                     dim3(256), 0, s, H, C, nz);
  G2PTQ_LAUNCHED();
  hipLaunchKernelGGL(nonzero_kernel, dim3(std::min<unsigned>(grid_for(CC), 1024), (unsigned)B),
                     dim3(256), 0, s, H, CC, nz);
  G2PTQ_LAUNCHED();
  hipLaunchKernelGGL(dead_kernel, dim3((unsigned)cdiv(C, 256), (unsigned)B), dim3(256), 0, s, H,
                     C, nz, dead, anydead);
  G2PTQ_LAUNCHED();
  hipLaunchKernelGGL(fix_h_kernel, dim3(std::min<unsigned>(grid_for(CC), 4096), (unsigned)B),
                     dim3(256), 0, s, H, C, nz, dead);
  G2PTQ_LAUNCHED();
  hipLaunchKernelGGL(zero_cols_kernel, dim3(std::min<unsigned>(grid_for(R * C), 4096), (unsigned)B),
                     dim3(256), 0, s, W, R, C, dead, nz, anydead, 0);
  G2PTQ_LAUNCHED();
  if (Dx) {
    hipLaunchKernelGGL(zero_cols_kernel, dim3(std::min<unsigned>(grid_for(CC), 4096), (unsigned)B),
                       dim3(256), 0, s, Dx, C, C, dead, nz, anydead, 0);
    G2PTQ_LAUNCHED();
  }
  if (Grad) {
    hipLaunchKernelGGL(zero_cols_kernel,
                       dim3(std::min<unsigned>(grid_for(Rg * C), 4096), (unsigned)B), dim3(256), 0,
                       s, Grad, Rg, C, dead, nz, anydead, 1);
    G2PTQ_LAUNCHED();
  }
  return G2PTQ_OK;
}

extern "C" int g2ptq_act_order(void* stream, const float* src, int64_t B, int64_t C, int key_mode,
                               int* perm, int* invperm, void* ws, size_t ws_bytes) {
  G2PTQ_CHECK(src && perm && invperm, "act_order: null pointer");
  G2PTQ_CHECK(ws && ws_bytes >= (size_t)C * 4, "act_order: workspace too small");
  G2PTQ_CHECK(C < (1ll << 31), "act_order: C too large");
  hipStream_t s = as_stream(stream);
  float* key = static_cast<float*>(ws);
  hipLaunchKernelGGL(order_key_kernel, dim3((unsigned)cdiv(C, 256)), dim3(256), 0, s, src, B, C,
                     key_mode, key);
  G2PTQ_LAUNCHED();
  hipLaunchKernelGGL(rank_kernel, dim3((unsigned)cdiv(C, 256)), dim3(256), 0, s, key, C, perm,
                     invperm);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

extern "C" int g2ptq_permute_cols(void* stream, const float* in, float* out, int64_t rows,
                                  int64_t C, const int* cols) {
  G2PTQ_CHECK(in && out && cols && in != out, "permute_cols: bad pointers");
  const int64_t n = rows * C;
  if (n <= 0) return G2PTQ_OK;
  hipLaunchKernelGGL(permute_cols_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), in,
                     out, rows, C, cols);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

extern "C" int g2ptq_permute_sym(void* stream, const float* in, float* out, int64_t B, int64_t C,
                                 const int* perm) {
  G2PTQ_CHECK(in && out && perm && in != out, "permute_sym: bad pointers");
  if (B <= 0 || C <= 0) return G2PTQ_OK;
  hipLaunchKernelGGL(permute_sym_kernel, dim3(std::min<unsigned>(grid_for(C * C), 4096), (unsigned)B),
                     dim3(256), 0, as_stream(stream), in, out, C, perm);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

extern "C" int g2ptq_cast_check(void* stream, const float* in, void* out, int64_t n, int dtype,
                                int* flags) {
  G2PTQ_CHECK(in && out, "cast_check: null pointer");
  G2PTQ_CHECK(dtype >= 0 && dtype <= 2, "cast_check: dtype code %d", dtype);
  if (n <= 0) return G2PTQ_OK;
  if (dtype == 0 && vec8(in, out, n))
    hipLaunchKernelGGL(cast_check_bf16_vec_kernel, dim3(grid_for(n / 8)), dim3(256), 0,
                       as_stream(stream), reinterpret_cast<const float4*>(in),
                       static_cast<uint4*>(out), n / 8, flags);
  else
    hipLaunchKernelGGL(cast_check_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), in,
                       out, n, dtype, flags);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

extern "C" int g2ptq_to_f32(void* stream, const void* in, float* out, int64_t n, int dtype) {
  G2PTQ_CHECK(in && out, "to_f32: null pointer");
  G2PTQ_CHECK(dtype >= 0 && dtype <= 2, "to_f32: dtype code %d", dtype);
  if (n <= 0) return G2PTQ_OK;
  if (dtype == 0 && vec8(in, out, n))
    hipLaunchKernelGGL(bf16_to_f32_vec_kernel, dim3(grid_for(n / 8)), dim3(256), 0,
                       as_stream(stream), static_cast<const uint4*>(in),
                       reinterpret_cast<float4*>(out), n / 8);
  else
    hipLaunchKernelGGL(to_f32_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), in, out,
                       n, dtype);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}
