// Dampened inverse-Cholesky factor on CDNA4.
//
// The reference computes U = chol(cholesky_inverse(chol(A)), upper) with
// A = H + p·mean(diag H)·I (gptq_utils.py:295-302): three factorizations'
// worth of work (~4C³/3).  The same unique factor (upper triangular, positive
// diagonal, UᵀU = A⁻¹) is U = J·L̂⁻¹·J where L̂ = chol(J·A·J) and J reverses
// index order: one Cholesky plus one triangular inverse (2C³/3).
//
//   1. reverse-copy Â = J(H + damp·I)J (lower triangle) into the workspace
//   2. blocked right-looking Cholesky of Â in panels of NBO = 256 columns,
//      each factored NB = 64 columns at a time: potrf of the diagonal block
//      in one workgroup (registers), which also inverts it in place;  TRSM
//      as a GEMM with that inverse;  update of the panel's remaining
//      columns;  then one SYRK trailing update per panel (K = 256) as a
//      lower-triangular fp32 MFMA GEMM
//   3. triangular inverse by recursive doubling: diagonal blocks are already
//      inverted; level s joins pairs of s-sized inverses with
//      X21 = −X22·(L21·X11), each level two batched GEMMs
//   4. un-reverse into U (upper, zeros below) with the reference's NaN check.
#include "common.hpp"

namespace g2ptq {
namespace {

constexpr int NB = 64;   // diagonal block width (potrf in registers)
constexpr int NBO = 256; // panel width of the trailing (SYRK) updates
constexpr int TPT = NB / 16;  // rows (and columns) of the per-thread register tile

__global__ void diag_sum_kernel(const float* __restrict__ H, int64_t C, const int* skip,
                                float* sums, int* st, int* info) {
  const int64_t b = blockIdx.x;
  __shared__ float red[256];
  const float* Hb = H + b * C * C;
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < C; i += 256) s += Hb[i * C + i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    sums[b] = red[0];
    const int sk = skip ? skip[b] : 0;
    st[b] = sk;
    if (!sk) info[b] = 0;
  }
}

// Â[i][j] = A[C-1-i][C-1-j] for i >= j (damp on the diagonal), 0 above.
__global__ void reverse_damp_kernel(const float* __restrict__ H, int64_t C, float percdamp,
                                    const float* sums, const int* st, float* __restrict__ WA) {
  const int64_t b = blockIdx.z;
  if (st[b]) return;
  const int64_t i = (int64_t)blockIdx.y * 16 + (threadIdx.x >> 4);
  const int64_t j0 = (int64_t)blockIdx.x * 64;
  const float damp = percdamp * (sums[b] / (float)C);
  const float* Hb = H + b * C * C;
  float* Wb = WA + b * C * C;
  if (i >= C) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t j = j0 + (threadIdx.x & 15) + 16 * q;
    if (j >= C) continue;
    float v = 0.f;
    if (i >= j) {
      v = Hb[(C - 1 - i) * C + (C - 1 - j)];
      if (i == j) v = v + damp;
    }
    Wb[i * C + j] = v;
  }
}

// Cholesky + in-place inverse of the nbk×nbk (nbk <= 64) diagonal block at (k, k).
//
// Right-looking, register resident: the block is split over a 16×16 thread
// grid, each thread holding a 4×4 tile of L and of X = L⁻¹.  At step j the
// owners of column j of L and of row j of X publish them through LDS
// (double-buffered, one barrier per step); every thread then finishes the
// pivot (sqrt, scale by its reciprocal) and applies the rank-1 updates of the
// Cholesky trailing block and of the forward elimination of L·X = I to its
// own tile.  Register tiles are indexed with compile-time indices only.
__global__ __launch_bounds__(256) void potrf_diag_kernel(float* WA, int64_t C, int64_t k, int nbk,
                                                         int* st, int* info) {
  const int64_t b = blockIdx.x;
  if (st[b]) return;
  __shared__ float colL[2][NB];
  __shared__ float rowX[2][NB];
  float* Wb = WA + b * C * C + k * C + k;
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int i0 = ty * TPT, c0 = tx * TPT;
  float l[TPT][TPT], x[TPT][TPT];
#pragma unroll
  for (int r = 0; r < TPT; ++r)
#pragma unroll
    for (int c = 0; c < TPT; ++c) {
      const int i = i0 + r, kk = c0 + c;
      l[r][c] = (kk <= i && i < nbk) ? Wb[(int64_t)i * C + kk] : 0.f;
      x[r][c] = (i == kk) ? 1.f : 0.f;
    }
  int fail = 0;
  for (int j = 0; j < nbk; ++j) {
    const int buf = j & 1;
    const int cj = j % TPT, tj = j / TPT;
    if (tx == tj) {
#pragma unroll
      for (int r = 0; r < TPT; ++r) {
        float v = 0.f;
#pragma unroll
        for (int c = 0; c < TPT; ++c) v = (c == cj) ? l[r][c] : v;
        colL[buf][i0 + r] = v;
      }
    }
    if (ty == tj) {
#pragma unroll
      for (int c = 0; c < TPT; ++c) {
        float v = 0.f;
#pragma unroll
        for (int r = 0; r < TPT; ++r) v = (r == cj) ? x[r][c] : v;
        rowX[buf][c0 + c] = v;
      }
    }
    __syncthreads();
    const float djj = colL[buf][j];
    if (!(djj > 0.f)) {  // also catches NaN; every thread sees the same value
      fail = j + 1;
      break;
    }
    const float d = __fsqrt_rn(djj);
    const float rd = 1.f / d;
    // Unconditional LDS reads (rows above the pivot hold stale values that the
    // selects discard), so no divergent branch separates the loads.
    float li[TPT], lk[TPT], xr[TPT];
#pragma unroll
    for (int r = 0; r < TPT; ++r) {
      const float v = colL[buf][i0 + r];
      li[r] = (i0 + r > j) ? v * rd : 0.f;
    }
#pragma unroll
    for (int c = 0; c < TPT; ++c) {
      const float v = colL[buf][c0 + c];
      const float xv = rowX[buf][c0 + c];
      lk[c] = (c0 + c > j) ? v * rd : 0.f;
      xr[c] = (c0 + c <= j) ? xv * rd : 0.f;
    }
    // li[r] = 0 for rows i <= j and lk[c] = 0 for columns <= j, so the rank-1
    // updates need no masks; only the strict upper triangle of the L tile is
    // written with values nobody reads.
#pragma unroll
    for (int r = 0; r < TPT; ++r) {
      const bool diag_row = (i0 + r == j);
#pragma unroll
      for (int c = 0; c < TPT; ++c) {
        l[r][c] -= li[r] * lk[c];
        x[r][c] = diag_row ? xr[c] : x[r][c] - li[r] * xr[c];
      }
    }
    if (tx == tj) {
#pragma unroll
      for (int r = 0; r < TPT; ++r) {
        const float v = (i0 + r == j) ? d : li[r];
#pragma unroll
        for (int c = 0; c < TPT; ++c)
          if (c == cj) l[r][c] = v;
      }
    }
  }
  if (fail) {
    if (tid == 0) {
      info[b] = (int)(k + fail);
      st[b] = 1;
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < TPT; ++r)
#pragma unroll
    for (int c = 0; c < TPT; ++c) {
      const int i = i0 + r, kk = c0 + c;
      if (i < nbk && kk < nbk) Wb[(int64_t)i * C + kk] = (kk <= i) ? x[r][c] : 0.f;
    }
}

// U[i][j] = X[C-1-i][C-1-j] for i <= j, 0 below; NaN → info = -1.
__global__ void unreverse_kernel(const float* __restrict__ WA, int64_t C, const int* skip,
                                 int* info, float* __restrict__ U) {
  const int64_t b = blockIdx.z;
  if ((skip && skip[b]) || info[b] > 0) return;
  const int64_t i = (int64_t)blockIdx.y * 16 + (threadIdx.x >> 4);
  const int64_t j0 = (int64_t)blockIdx.x * 64;
  if (i >= C) return;
  const float* Wb = WA + b * C * C;
  float* Ub = U + b * C * C;
  bool nan = false;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t j = j0 + (threadIdx.x & 15) + 16 * q;
    if (j >= C) continue;
    float v = 0.f;
    if (i <= j) {
      v = Wb[(C - 1 - i) * C + (C - 1 - j)];
      nan |= (v != v);
    }
    Ub[i * C + j] = v;
  }
  if (nan) atomicCAS(&info[b], 0, -1);
}

struct FactorWs {
  size_t wa, wt, sums, st, total;
};

FactorWs factor_ws(int64_t B, int64_t C) {
  FactorWs w;
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  w.wa = al((size_t)B * C * C * 4);
  const int64_t half = (C + 1) / 2;
  w.wt = al((size_t)B * half * half * 4 + 4);
  w.sums = al((size_t)B * 4);
  w.st = al((size_t)B * 4);
  w.total = w.wa + w.wt + w.sums + w.st;
  return w;
}

}  // namespace
}  // namespace g2ptq

using namespace g2ptq;

extern "C" int g2ptq_factor_workspace(int64_t B, int64_t C, size_t* bytes) {
  G2PTQ_CHECK(bytes != nullptr, "factor_workspace: null out");
  *bytes = factor_ws(B, C).total;
  return G2PTQ_OK;
}

extern "C" int g2ptq_inv_chol_upper(void* stream, const float* H, int64_t B, int64_t C,
                                    float percdamp, const int* skip, float* U, int* info, void* ws,
                                    size_t ws_bytes) {
  G2PTQ_CHECK(H && U && info, "inv_chol_upper: null pointer");
  G2PTQ_CHECK(B >= 1 && B < 65536 && C >= 1, "inv_chol_upper: bad sizes");
  const FactorWs w = factor_ws(B, C);
  G2PTQ_CHECK(ws != nullptr && ws_bytes >= w.total, "inv_chol_upper: workspace %zu < %zu",
              ws_bytes, w.total);
  hipStream_t s = as_stream(stream);
  char* base = static_cast<char*>(ws);
  float* WA = reinterpret_cast<float*>(base);
  float* WT = reinterpret_cast<float*>(base + w.wa);
  float* sums = reinterpret_cast<float*>(base + w.wa + w.wt);
  int* st = reinterpret_cast<int*>(base + w.wa + w.wt + w.sums);
  const int64_t CC = C * C;

  hipLaunchKernelGGL(diag_sum_kernel, dim3((unsigned)B), dim3(256), 0, s, H, C, skip, sums, st,
                     info);
  G2PTQ_LAUNCHED();
  dim3 cgrid((unsigned)cdiv(C, 64), (unsigned)cdiv(C, 16), (unsigned)B);
  hipLaunchKernelGGL(reverse_damp_kernel, cgrid, dim3(256), 0, s, H, C, percdamp, sums, st, WA);
  G2PTQ_LAUNCHED();

  // Blocked Cholesky of Â (lower) with inverted diagonal blocks, two levels:
  // panels of NBO columns are factored NB columns at a time (potrf + TRSM +
  // update of the panel's own remaining columns), then the trailing matrix
  // receives the whole panel in one SYRK with K = NBO instead of NBO/NB
  // passes with K = NB (a quarter of the trailing-matrix traffic).
  for (int64_t k = 0; k < C; k += NBO) {
    const int64_t kb = std::min<int64_t>(NBO, C - k);
    for (int64_t j = k; j < k + kb; j += NB) {
      const int nbk = (int)std::min<int64_t>(NB, k + kb - j);
      hipLaunchKernelGGL(potrf_diag_kernel, dim3((unsigned)B), dim3(256), 0, s, WA, C, j, nbk,
                         st, info);
      G2PTQ_LAUNCHED();
      const int64_t rest = C - j - nbk;
      if (rest <= 0) break;
      GemmF32 t;  // panel ← panel · inv(L_jj)ᵀ
      t.M = rest; t.N = nbk; t.K = nbk; t.batch = B;
      t.A = WA + (j + nbk) * C + j; t.lda = C; t.sA = CC;
      t.B = WA + j * C + j; t.ldb = C; t.sB = CC; t.b_kcontig = 1;
      t.D = WA + (j + nbk) * C + j; t.ldd = C; t.sD = CC;
      t.skip = st;
      G2PTQ_TRY(gemm_f32(s, t));
      const int64_t pw = k + kb - (j + nbk);  // panel columns still to factor
      if (pw <= 0) continue;
      GemmF32 y;  // panel remainder ← remainder − L[:, j] · L[panel rows, j]ᵀ (lower)
      y.M = rest; y.N = pw; y.K = nbk; y.batch = B;
      y.A = WA + (j + nbk) * C + j; y.lda = C; y.sA = CC;
      y.B = WA + (j + nbk) * C + j; y.ldb = C; y.sB = CC; y.b_kcontig = 1;
      y.C = WA + (j + nbk) * C + (j + nbk); y.ldc = C; y.sC = CC;
      y.D = WA + (j + nbk) * C + (j + nbk); y.ldd = C; y.sD = CC;
      y.alpha = -1.f; y.beta = 1.f; y.uplo = 1; y.skip = st;
      G2PTQ_TRY(gemm_f32(s, y));
    }
    const int64_t rest = C - k - kb;
    if (rest <= 0) break;
    GemmF32 y;  // trailing ← trailing − panel · panelᵀ (lower), K = panel width
    y.M = rest; y.N = rest; y.K = kb; y.batch = B;
    y.A = WA + (k + kb) * C + k; y.lda = C; y.sA = CC;
    y.B = WA + (k + kb) * C + k; y.ldb = C; y.sB = CC; y.b_kcontig = 1;
    y.C = WA + (k + kb) * C + (k + kb); y.ldc = C; y.sC = CC;
    y.D = WA + (k + kb) * C + (k + kb); y.ldd = C; y.sD = CC;
    y.alpha = -1.f; y.beta = 1.f; y.uplo = 1; y.skip = st;
    G2PTQ_TRY(gemm_f32(s, y));
  }

  // Triangular inverse by recursive doubling (diagonal NB blocks already inverted).
  for (int64_t sz = NB; sz < C; sz *= 2) {
    const int64_t full = C / (2 * sz);             // pairs with a full second block
    const int64_t tail_i = full * 2 * sz;          // start of a possible ragged pair
    const int64_t tail_n2 = C - tail_i - sz;       // its second block size (if > 0)
    for (int part = 0; part < 2; ++part) {
      int64_t npairs, i0, n2;
      if (part == 0) {
        npairs = full; i0 = 0; n2 = sz;
      } else {
        npairs = tail_n2 > 0 ? 1 : 0; i0 = tail_i; n2 = tail_n2;
      }
      if (npairs == 0) continue;
      const int64_t pstride = 2 * sz * (C + 1);
      GemmF32 t;  // T = L21 · X11
      t.M = n2; t.N = sz; t.K = sz; t.batch = B; t.batch2 = npairs;
      t.A = WA + (i0 + sz) * C + i0; t.lda = C; t.sA = CC; t.sA2 = pstride;
      t.B = WA + i0 * C + i0; t.ldb = C; t.sB = CC; t.sB2 = pstride;
      t.D = WT; t.ldd = sz; t.sD = npairs * n2 * sz; t.sD2 = n2 * sz;
      t.skip = st;
      G2PTQ_TRY(gemm_f32(s, t));
      GemmF32 x;  // X21 = −X22 · T
      x.M = n2; x.N = sz; x.K = n2; x.batch = B; x.batch2 = npairs;
      x.A = WA + (i0 + sz) * C + (i0 + sz); x.lda = C; x.sA = CC; x.sA2 = pstride;
      x.B = WT; x.ldb = sz; x.sB = npairs * n2 * sz; x.sB2 = n2 * sz;
      x.D = WA + (i0 + sz) * C + i0; x.ldd = C; x.sD = CC; x.sD2 = pstride;
      x.alpha = -1.f; x.skip = st;
      G2PTQ_TRY(gemm_f32(s, x));
    }
  }

  hipLaunchKernelGGL(unreverse_kernel, cgrid, dim3(256), 0, s, WA, C, skip, info, U);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}
