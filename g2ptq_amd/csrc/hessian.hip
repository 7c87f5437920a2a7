// Streaming Hessian accumulation on CDNA4 bf16 matrix cores.
//
//   H = beta·H + alpha·XᵀX          (GPTQ,  gptq_utils.py:115-126)
//   H, Dx = ..., Dx = beta·Dx + alpha·(X_fp − X)ᵀX   (GPTAQ, gptaq_utils.py:130-148)
//   H[g] = beta·H[g] + alpha·Σ_t S[t,g] x_t x_tᵀ     (G2PTQ / GuidedQuant)
//
// X arrives token-major (T × C bf16, the hook payload).  A transpose pass
// writes Xᵀ (Cp × Tp, zero padded to tile multiples) into the workspace so
// that both MFMA operands read K-contiguous 16-byte runs.  The Gram kernel
// then computes 128×128 output tiles with v_mfma_f32_32x32x16_bf16 (fp32
// accumulation of exact bf16 products), K staged through LDS 64 tokens at a
// time with register prefetch.  The Hessian is symmetric: only tiles I <= J
// are computed and each is stored to both triangles.
#include "common.hpp"

namespace g2ptq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int GT = 128;  // output tile
constexpr int GK = 64;   // tokens per LDS stage
constexpr int GP = 72;   // LDS row pitch in bf16 elements (64 + 8)

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// X (T × C, ld ldx) → XT (Cp × Tp), zero padded.  64×64 tiles through LDS.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const uint16_t* __restrict__ X,
                                                             int64_t T, int64_t C, int64_t ldx,
                                                             uint16_t* __restrict__ XT,
                                                             int64_t Tp) {
  __shared__ uint16_t tile[64][66];
  const int64_t t0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t t = t0 + ty + 4 * i, c = c0 + tx;
    tile[ty + 4 * i][tx] = (t < T && c < C) ? X[t * ldx + c] : (uint16_t)0;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t c = c0 + ty + 4 * i, t = t0 + tx;
    XT[c * Tp + t] = tile[tx][ty + 4 * i];
  }
}

// S (T × G fp32, ld lds) → ST (G × Tp), zero padded.
__global__ void transpose_sal_kernel(const float* __restrict__ S, int64_t T, int64_t G,
                                     int64_t lds, float* __restrict__ ST, int64_t Tp) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= G * Tp) return;
  const int64_t g = i / Tp, t = i % Tp;
  ST[i] = t < T ? S[t * lds + g] : 0.f;
}

// act = act_beta·act + act_alpha·Σ_t x[t,c]² over XT rows (one wave per feature).
__global__ __launch_bounds__(256) void act_square_kernel(const uint16_t* __restrict__ XT,
                                                         int64_t C, int64_t Tp, float* act,
                                                         float act_alpha, float act_beta) {
  const int64_t c = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (c >= C) return;
  float s = 0.f;
  const uint16_t* row = XT + c * Tp;
  for (int64_t t = lane; t < Tp; t += 64) {
    const float v = bf16_to_f32(row[t]);
    s += v * v;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) act[c] = act_beta * act[c] + act_alpha * s;
}

struct GramArgs {
  const uint16_t* XT;   // Cp × Tp
  const uint16_t* FT;   // GPTAQ: X_fp transposed
  const float* ST;      // weighted: G × Tp saliencies
  int64_t Tp, C, nt;
  float alpha, beta;
  float* H; int64_t ldh; int64_t sH;  // sH: stride between group Hessians
  float* D; int64_t ldd;
};

// Upper-triangular tile index → (I, J), I <= J.
__device__ __forceinline__ void tri_tile(int64_t idx, int64_t nt, int64_t& I, int64_t& J) {
  int64_t i = 0, row_len = nt;
  while (idx >= row_len) {
    idx -= row_len;
    ++i;
    --row_len;
  }
  I = i;
  J = i + idx;
}

// MODE 0: H (upper tiles, mirrored).  MODE 1: GPTAQ, all tiles: Dx from the
// exact fp32 difference x_fp − x split into bf16 hi + lo operands (two MFMAs),
// and, for I <= J, H.  MODE 2: saliency weighted, upper tiles, group g = blockIdx.y,
// scaled operand split into bf16 hi + lo parts (two MFMAs per step).
template <int MODE>
__global__ __launch_bounds__(256) void gram_kernel(GramArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[GT * GP];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[GT * GP];
  __shared__ __attribute__((aligned(16))) uint16_t A2s[(MODE == 0) ? 8 : GT * GP];
  __shared__ __attribute__((aligned(16))) uint16_t A3s[(MODE == 1) ? GT * GP : 8];

  int64_t I, J;
  if (MODE == 1) {
    I = blockIdx.x / a.nt;
    J = blockIdx.x % a.nt;
  } else {
    tri_tile(blockIdx.x, a.nt, I, J);
  }
  const int g = (MODE == 2) ? blockIdx.y : 0;
  const int64_t i0 = I * GT, j0 = J * GT;
  const bool diag_tile = (I == J);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const uint16_t* Arow = a.XT + i0 * a.Tp;
  const uint16_t* Frow = (MODE == 1) ? a.FT + i0 * a.Tp : nullptr;
  const uint16_t* Brow = a.XT + j0 * a.Tp;
  const float* Sg = (MODE == 2) ? a.ST + (int64_t)g * a.Tp : nullptr;

  uint4 ra[4], rb[4], rf[4];
  float4 rs[4][2];

  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + i * 256;
      const int row = c >> 3, col8 = (c & 7) * 8;
      const int64_t off = (int64_t)row * a.Tp + k0 + col8;
      ra[i] = *reinterpret_cast<const uint4*>(Arow + off);
      if (!diag_tile || MODE == 1 || MODE == 2) rb[i] = *reinterpret_cast<const uint4*>(Brow + off);
      if (MODE == 1) rf[i] = *reinterpret_cast<const uint4*>(Frow + off);
      if (MODE == 2) {
        rs[i][0] = *reinterpret_cast<const float4*>(Sg + k0 + col8);
        rs[i][1] = *reinterpret_cast<const float4*>(Sg + k0 + col8 + 4);
      }
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + i * 256;
      const int row = c >> 3, col8 = (c & 7) * 8;
      uint4* pa = reinterpret_cast<uint4*>(As + row * GP + col8);
      uint4* pb = reinterpret_cast<uint4*>(Bs + row * GP + col8);
      if (MODE == 2) {
        // hi/lo split of s_t * x[t, i] for 8 consecutive tokens.
        const uint16_t* xs = reinterpret_cast<const uint16_t*>(&ra[i]);
        const float sv[8] = {rs[i][0].x, rs[i][0].y, rs[i][0].z, rs[i][0].w,
                             rs[i][1].x, rs[i][1].y, rs[i][1].z, rs[i][1].w};
        uint16_t hi[8], lo[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float v = bf16_to_f32(xs[e]) * sv[e];
          hi[e] = f32_to_bf16_rne(v);
          lo[e] = f32_to_bf16_rne(v - bf16_to_f32(hi[e]));
        }
        *pa = *reinterpret_cast<const uint4*>(hi);
        *reinterpret_cast<uint4*>(A2s + row * GP + col8) = *reinterpret_cast<const uint4*>(lo);
        *pb = rb[i];
      } else if (MODE == 1) {
        // d = x_fp - x exactly in fp32, split into bf16 hi + lo.
        const uint16_t* xs = reinterpret_cast<const uint16_t*>(&ra[i]);
        const uint16_t* fs = reinterpret_cast<const uint16_t*>(&rf[i]);
        uint16_t hi[8], lo[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = bf16_to_f32(fs[e]) - bf16_to_f32(xs[e]);
          hi[e] = f32_to_bf16_rne(d);
          lo[e] = f32_to_bf16_rne(d - bf16_to_f32(hi[e]));
        }
        *pa = ra[i];
        *pb = rb[i];
        *reinterpret_cast<uint4*>(A2s + row * GP + col8) = *reinterpret_cast<const uint4*>(hi);
        *reinterpret_cast<uint4*>(A3s + row * GP + col8) = *reinterpret_cast<const uint4*>(lo);
      } else {
        *pa = ra[i];
        if (!diag_tile) *pb = rb[i];
      }
    }
  };

  f32x16 acc[2][2], acc2[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        acc[i][j][v] = 0.f;
        acc2[i][j][v] = 0.f;
      }
    }

  // For MODE 0 diagonal tiles the B operand equals the A operand.
  const uint16_t* Bsrc = (MODE == 0 && diag_tile) ? As : Bs;
  const int nk = (int)(a.Tp / GK);
  if (nk > 0) gload(0);
  for (int kt = 0; kt < nk; ++kt) {
    __syncthreads();
    lstore();
    __syncthreads();
    if (kt + 1 < nk) gload((int64_t)(kt + 1) * GK);
#pragma unroll
    for (int ks = 0; ks < GK / 16; ++ks) {
      bf16x8 av[2], bv[2], fv[2], lv[2];
      const int kof = ks * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int row = wm * 64 + mt * 32 + (lane & 31);
        av[mt] = *reinterpret_cast<const bf16x8*>(As + row * GP + kof);
        if (MODE != 0) fv[mt] = *reinterpret_cast<const bf16x8*>(A2s + row * GP + kof);
        if (MODE == 1) lv[mt] = *reinterpret_cast<const bf16x8*>(A3s + row * GP + kof);
      }
#pragma unroll
      for (int nt2 = 0; nt2 < 2; ++nt2) {
        const int row = wn * 64 + nt2 * 32 + (lane & 31);
        bv[nt2] = *reinterpret_cast<const bf16x8*>(Bsrc + row * GP + kof);
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt2 = 0; nt2 < 2; ++nt2) {
          acc[mt][nt2] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[mt], bv[nt2], acc[mt][nt2], 0, 0, 0);
          if (MODE != 0)
            acc2[mt][nt2] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(fv[mt], bv[nt2], acc2[mt][nt2], 0, 0, 0);
          if (MODE == 1)
            acc2[mt][nt2] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(lv[mt], bv[nt2], acc2[mt][nt2], 0, 0, 0);
        }
    }
  }

  // Epilogue.  32×32 MFMA output: lane holds rows 8*(v/4) + 4*(lane/32) + v%4,
  // column lane%32.
  float* H = a.H + (int64_t)g * a.sH;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt2 = 0; nt2 < 2; ++nt2)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t i = i0 + wm * 64 + mt * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int64_t j = j0 + wn * 64 + nt2 * 32 + (lane & 31);
        if (i >= a.C || j >= a.C) continue;
        if (MODE == 1) {
          const float d = acc2[mt][nt2][v];
          float* pd = a.D + i * a.ldd + j;
          *pd = (a.beta != 0.f ? a.beta * *pd : 0.f) + a.alpha * d;
          if (I > J) continue;
        }
        if (diag_tile && i > j) continue;
        const float s = (MODE == 2) ? acc[mt][nt2][v] + acc2[mt][nt2][v] : acc[mt][nt2][v];
        float* ph = H + i * a.ldh + j;
        const float val = (a.beta != 0.f ? a.beta * *ph : 0.f) + a.alpha * s;
        *ph = val;
        if (i != j) H[j * a.ldh + i] = val;
      }
}

struct HessWs {
  int64_t Tp, Cp;
  size_t xt_bytes, ft_bytes, st_bytes;
};

HessWs hess_ws(int64_t T, int64_t C, int kind, int64_t G) {
  HessWs w;
  w.Tp = cdiv(T, GK) * GK;
  w.Cp = cdiv(C, GT) * GT;
  w.xt_bytes = (size_t)(w.Cp * w.Tp * 2 + 255) / 256 * 256;
  w.ft_bytes = kind == 1 ? w.xt_bytes : 0;
  w.st_bytes = kind == 2 ? (size_t)(G * w.Tp * 4 + 255) / 256 * 256 : 0;
  return w;
}

int transpose_into(hipStream_t st, const uint16_t* X, int64_t T, int64_t C, int64_t ldx,
                   uint16_t* XT, const HessWs& w) {
  dim3 grid((unsigned)(w.Tp / 64), (unsigned)(w.Cp / 64));
  hipLaunchKernelGGL(transpose_bf16_kernel, grid, dim3(256), 0, st, X, T, C, ldx, XT, w.Tp);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

int check_sizes(int64_t T, int64_t C) {
  G2PTQ_CHECK(T >= 0 && C > 0, "hessian: bad sizes T=%lld C=%lld", (long long)T, (long long)C);
  G2PTQ_CHECK(C <= (1ll << 20), "hessian: C too large");
  return G2PTQ_OK;
}

}  // namespace
}  // namespace g2ptq

using namespace g2ptq;

extern "C" int g2ptq_hessian_workspace(int64_t T, int64_t C, int kind, size_t* bytes) {
  G2PTQ_CHECK(bytes != nullptr, "hessian_workspace: null out");
  if (kind == 0) {
    *bytes = gram_update_ws_bytes(T, C);
    return G2PTQ_OK;
  }
  const HessWs w = hess_ws(T, C, kind, 8);
  *bytes = w.xt_bytes + w.ft_bytes + w.st_bytes;
  return G2PTQ_OK;
}

extern "C" int g2ptq_gptaq_update(void* stream, const uint16_t* X, const uint16_t* Xfp, int64_t T,
                                  int64_t C, int64_t ldx, int64_t ldxf, float alpha, float beta,
                                  float* H, float* Dx, int64_t ld, void* ws, size_t ws_bytes) {
  G2PTQ_TRY(check_sizes(T, C));
  G2PTQ_CHECK(H && Dx && ((X && Xfp) || T == 0), "gptaq_update: null pointer");
  const HessWs w = hess_ws(T, C, 1, 0);
  G2PTQ_CHECK(ws != nullptr && ws_bytes >= w.xt_bytes + w.ft_bytes,
              "gptaq_update: workspace too small");
  hipStream_t st = as_stream(stream);
  uint16_t* XT = static_cast<uint16_t*>(ws);
  uint16_t* FT = reinterpret_cast<uint16_t*>(static_cast<char*>(ws) + w.xt_bytes);
  if (w.Tp > 0) {
    G2PTQ_TRY(transpose_into(st, X, T, C, ldx, XT, w));
    G2PTQ_TRY(transpose_into(st, Xfp, T, C, ldxf, FT, w));
  }
  GramArgs a{};
  a.XT = XT; a.FT = FT; a.Tp = w.Tp; a.C = C; a.nt = w.Cp / GT;
  a.alpha = alpha; a.beta = beta; a.H = H; a.ldh = ld; a.D = Dx; a.ldd = ld;
  hipLaunchKernelGGL(gram_kernel<1>, dim3((unsigned)(a.nt * a.nt)), dim3(256), 0, st, a);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

extern "C" int g2ptq_weighted_hessian_update(void* stream, const uint16_t* X, int64_t T,
                                             int64_t C, int64_t ldx, const float* S, int64_t G,
                                             int64_t lds, float alpha, float beta, float* H,
                                             int64_t ldh, int64_t sH, float* act,
                                             float act_alpha, float act_beta, void* ws,
                                             size_t ws_bytes) {
  G2PTQ_TRY(check_sizes(T, C));
  G2PTQ_CHECK(G >= 1 && G <= 64, "weighted_hessian_update: G=%lld unsupported", (long long)G);
  G2PTQ_CHECK(H && ((X && S) || T == 0), "weighted_hessian_update: null pointer");
  HessWs w = hess_ws(T, C, 2, G);
  G2PTQ_CHECK(ws != nullptr && ws_bytes >= w.xt_bytes + w.st_bytes,
              "weighted_hessian_update: workspace too small");
  hipStream_t st = as_stream(stream);
  uint16_t* XT = static_cast<uint16_t*>(ws);
  float* ST = reinterpret_cast<float*>(static_cast<char*>(ws) + w.xt_bytes);
  if (w.Tp > 0) {
    G2PTQ_TRY(transpose_into(st, X, T, C, ldx, XT, w));
    const int64_t n = G * w.Tp;
    hipLaunchKernelGGL(transpose_sal_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, S, T,
                       G, lds, ST, w.Tp);
    G2PTQ_LAUNCHED();
  }
  GramArgs a{};
  a.XT = XT; a.ST = ST; a.Tp = w.Tp; a.C = C; a.nt = w.Cp / GT;
  a.alpha = alpha; a.beta = beta; a.H = H; a.ldh = ldh; a.sH = sH;
  const int64_t tiles = a.nt * (a.nt + 1) / 2;
  hipLaunchKernelGGL(gram_kernel<2>, dim3((unsigned)tiles, (unsigned)G), dim3(256), 0, st, a);
  G2PTQ_LAUNCHED();
  if (act) {
    hipLaunchKernelGGL(act_square_kernel, dim3((unsigned)cdiv(C, 4)), dim3(256), 0, st, XT, C,
                       w.Tp, act, act_alpha, act_beta);
    G2PTQ_LAUNCHED();
  }
  return G2PTQ_OK;
}
