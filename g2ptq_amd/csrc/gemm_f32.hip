// Batched fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_16x16x4_f32).
//
// One workgroup = 4 wave64s computing a 128×128 output tile; each wave owns a
// 64×64 quadrant as a 4×4 grid of 16×16 MFMA accumulators.  K advances in
// slabs of 16 staged through LDS with register double buffering.  The same
// kernel serves every fp32 product of the path: block-tail updates of the
// compensation sweep, the Cholesky TRSM/SYRK steps, the triangular-inverse
// levels, GPTAQ's P and the G2PTQ trust-region products.
#include "common.hpp"

namespace g2ptq {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int LDS_P = 144;  // row pitch (floats) of the [k][m] / [k][n] LDS slabs

template <bool B_KCONTIG>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmF32 g, int tiles_n) {
  __shared__ float As[2][BK][LDS_P];
  __shared__ float Bs[2][BK][LDS_P];

  const int z = blockIdx.z;
  const int64_t b1 = z / g.batch2, b2 = z % g.batch2;
  if (g.skip && g.skip[b1]) return;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  if (g.uplo == 1 && n0 > m0 + BM - 1) return;
  if (g.uplo == 2 && m0 > n0 + BN - 1) return;

  const float* A = g.A + b1 * g.sA + b2 * g.sA2;
  const float* B = g.B + b1 * g.sB + b2 * g.sB2;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Global staging registers: 8 A values and 8 B values per thread per slab.
  float ra[8], rb[8];

  // A slab: 128 (m) × 16 (k).  Thread loads m = tid & 127, k = (tid >> 7) * 8 + i.
  auto load_a = [&](int64_t k0) {
    const int m = tid & 127;
    const int kb = (tid >> 7) * 8;
    const int64_t gm = m0 + m;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t gk = k0 + kb + i;
      ra[i] = (gm < g.M && gk < g.K) ? A[gm * g.lda + gk] : 0.f;
    }
  };
  auto store_a = [&](int buf) {
    const int m = tid & 127;
    const int kb = (tid >> 7) * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) As[buf][kb + i][m] = ra[i];
  };
  // B slab: 16 (k) × 128 (n).
  auto load_b = [&](int64_t k0) {
    if (B_KCONTIG) {  // B given as N×K row-major
      const int n = tid & 127;
      const int kb = (tid >> 7) * 8;
      const int64_t gn = n0 + n;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t gk = k0 + kb + i;
        rb[i] = (gn < g.N && gk < g.K) ? B[gn * g.ldb + gk] : 0.f;
      }
    } else {  // B row-major K×N: thread loads k = tid >> 4, n = (tid & 15) * 8 + i
      const int k = tid >> 4;
      const int nb = (tid & 15) * 8;
      const int64_t gk = k0 + k;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t gn = n0 + nb + i;
        rb[i] = (gk < g.K && gn < g.N) ? B[gk * g.ldb + gn] : 0.f;
      }
    }
  };
  auto store_b = [&](int buf) {
    if (B_KCONTIG) {
      const int n = tid & 127;
      const int kb = (tid >> 7) * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) Bs[buf][kb + i][n] = rb[i];
    } else {
      const int k = tid >> 4;
      const int nb = (tid & 15) * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) Bs[buf][k][nb + i] = rb[i];
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = (int)cdiv(g.K, BK);
  if (nk > 0) {
    load_a(0);
    load_b(0);
    store_a(0);
    store_b(0);
  }
  __syncthreads();

  const int lr = lane & 15, lk = lane >> 4;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) {
      load_a((int64_t)(kt + 1) * BK);
      load_b((int64_t)(kt + 1) * BK);
    }
#pragma unroll
    for (int ks = 0; ks < BK / 4; ++ks) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[buf][ks * 4 + lk][wm * 64 + i * 16 + lr];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[buf][ks * 4 + lk][wn * 64 + j * 16 + lr];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) {
      store_a(buf ^ 1);
      store_b(buf ^ 1);
    }
    __syncthreads();
  }

  // Epilogue.  16×16 MFMA output: lane holds rows 4*(lane/16)+v, column lane%16.
  const float* C = g.C ? g.C + b1 * g.sC + b2 * g.sC2 : nullptr;
  const float* X = g.X ? g.X + b1 * g.sX + b2 * g.sX2 : nullptr;
  float* D = g.D + b1 * g.sD + b2 * g.sD2;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t m = m0 + wm * 64 + i * 16 + lk * 4 + v;
        const int64_t n = n0 + wn * 64 + j * 16 + lr;
        if (m >= g.M || n >= g.N) continue;
        if (g.uplo == 1 && n > m) continue;
        if (g.uplo == 2 && m > n) continue;
        float val = g.alpha * acc[i][j][v];
        if (g.beta != 0.f) val += g.beta * C[m * g.ldc + n];
        if (g.gamma != 0.f) val += g.gamma * X[m * g.ldx + n];
        D[m * g.ldd + n] = val;
      }
}

}  // namespace

int gemm_f32(hipStream_t stream, const GemmF32& g) {
  if (g.M <= 0 || g.N <= 0 || g.batch <= 0 || g.batch2 <= 0) return G2PTQ_OK;
  G2PTQ_CHECK(g.K >= 0, "gemm_f32: negative K");
  G2PTQ_CHECK(g.A != nullptr || g.K == 0, "gemm_f32: null A");
  G2PTQ_CHECK(g.B != nullptr || g.K == 0, "gemm_f32: null B");
  G2PTQ_CHECK(g.D != nullptr, "gemm_f32: null D");
  G2PTQ_CHECK(g.beta == 0.f || g.C != nullptr, "gemm_f32: beta != 0 needs C");
  G2PTQ_CHECK(g.gamma == 0.f || g.X != nullptr, "gemm_f32: gamma != 0 needs X");
  const int64_t tm = cdiv(g.M, BM), tn = cdiv(g.N, BN);
  const int64_t nz = g.batch * g.batch2;
  G2PTQ_CHECK(tm * tn < (1ll << 31) && nz < 65536, "gemm_f32: grid too large");
  dim3 grid((unsigned)(tm * tn), 1, (unsigned)nz);
  if (g.b_kcontig)
    hipLaunchKernelGGL(gemm_f32_kernel<true>, grid, dim3(256), 0, stream, g, (int)tn);
  else
    hipLaunchKernelGGL(gemm_f32_kernel<false>, grid, dim3(256), 0, stream, g, (int)tn);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

}  // namespace g2ptq

extern "C" int g2ptq_gemm_f32(void* stream, int64_t M, int64_t N, int64_t K, int64_t batch,
                              const float* A, int64_t lda, int64_t sA, const float* B, int64_t ldb,
                              int64_t sB, int b_trans, const float* C, int64_t ldc, int64_t sC,
                              float* D, int64_t ldd, int64_t sD, float alpha, float beta) {
  g2ptq::GemmF32 g;
  g.M = M; g.N = N; g.K = K; g.batch = batch;
  g.A = A; g.lda = lda; g.sA = sA;
  g.B = B; g.ldb = ldb; g.sB = sB; g.b_kcontig = b_trans;
  g.C = C; g.ldc = ldc; g.sC = sC;
  g.D = D; g.ldd = ldd; g.sD = sD;
  g.alpha = alpha; g.beta = beta;
  return g2ptq::gemm_f32(g2ptq::as_stream(stream), g);
}
