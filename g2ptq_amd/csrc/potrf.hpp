// Diagonal-block Cholesky + inverse for the factor (device code, gfx950).
#pragma once
#include "common.hpp"

namespace g2ptq {
namespace {

// Cholesky + inverse of a diagonal block of the factor (nbk×nbk, nbk <= 64),
// shared by factor.hip's potrf kernel and the GEMM's fused variant (the panel
// update that produces the block factors it as soon as it is written).
//
// Two wave64s do the work (further waves of the workgroup only keep the
// barrier count); rows at or past nbk are identity rows.  Lane i of
// wave 0 holds row i of the trailing matrix A, lane i of wave 1 column i of
// the inverse X = L⁻¹ being formed, both as a register array v rotated so
// that entry 0 is always the current pivot column / row: before step j,
// wave 0 has v[c] = A[i][j + c] and wave 1 v[c] = (e_i − Σ_{k<j} L[·][k]·X[k][i])[j + c].
// Step j:
//   wave 0: pivot d = sqrt(A[j][j]) (read from lane j), m = l_ij = A[i][j]/d
//           (i > j); publishes column j of L below the diagonal and 1/d
//           through LDS (double buffered by step parity);
//   barrier;
//   wave 1: m = X[j][i] = v[0]/d;
//   both:   v[c] ← v[c+1] − m·L[j+1+c][j]
// i.e. the right-looking Cholesky and the forward substitution of L·x = e_i
// sharing the broadcast column, one per wave so each runs half the FMAs.
// Entries that correspond to columns past the block hold finite leftovers
// that are never read.
//
// The step code is a loop, not unrolled: a wave executing straight-line code
// once per launch is bound by instruction fetch.  The 64 steps run as four
// 16-step phases over 64, 48, 32 and 16 live entries (the rotated arrays
// shrink by one column per step), so the compiled kernel stays a few KB.  A
// non-positive (or NaN) pivot is recorded and the block is not stored.
constexpr int POT_NB = 64;          // block edge
constexpr int XP = POT_NB + 1;      // LDS row pitch of the X / load staging buffer

// Wave 0's pivot step for column j: d = sqrt(v[0] of lane j), m = l_ij, and
// column j of L below the diagonal plus 1/d published in LDS buffer j & 1.
__device__ __forceinline__ float chol_pivot(float v0, int j, int i, float (*colL)[POT_NB], float* rdl,
                                            int& fail) {
  const float djj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v0), j));
  fail = (fail == 0 && !(djj > 0.f)) ? j + 1 : fail;  // also catches NaN
  // 1/sqrt from the hardware reciprocal square root (about 1 ulp): the factor
  // is held to fp32 tolerance, not to correctly rounded bits.
  const float rd = __builtin_amdgcn_rsqf(djj);
  const float m = (i > j) ? v0 * rd : 0.f;
  if (i > j) colL[j & 1][i - j - 1] = m;
  if (i == 0) rdl[j & 1] = rd;
  return m;
}

// Steps j0 .. j0+15 over LEN live entries.  Wave 0 enters step j with its
// multiplier m already computed and column j published; it updates v[0] (the
// next pivot column) first and publishes column j+1 before the rest of step
// j's updates, so the LDS write latency and the pivot chain overlap the bulk
// FMAs.  Buffers alternate by step parity: column j+1 goes to the buffer that
// wave 1 finished reading before the barrier of step j.
template <int LEN>
__device__ __forceinline__ void chol_inv_phase(float (&v)[POT_NB], int j0, int i, int w,
                                               float (*colL)[POT_NB], float* rdl, float* Xs, float& m,
                                               int& fail) {
#pragma clang loop unroll(disable)
  for (int jj = 0; jj < 16; ++jj) {
    const int j = j0 + jj;
    const int buf = j & 1;
    __syncthreads();  // column j and 1/d_j are published
    float mm = m;
    if (w == 1) {
      mm = v[0] * rdl[buf];
      Xs[j * XP + i] = mm;
    }
    float cl[LEN];
#pragma unroll
    for (int q = 0; q < LEN / 4; ++q) {
      const float4 u = *reinterpret_cast<const float4*>(&colL[buf][4 * q]);
      cl[4 * q] = u.x; cl[4 * q + 1] = u.y; cl[4 * q + 2] = u.z; cl[4 * q + 3] = u.w;
    }
    v[0] = v[1] - mm * cl[0];
    if (w == 0 && j + 1 < POT_NB) m = chol_pivot(v[0], j + 1, i, colL, rdl, fail);
#pragma unroll
    for (int c = 1; c + 1 < LEN; ++c) v[c] = v[c + 1] - mm * cl[c];
    v[LEN - 1] = 0.f;
  }
}


// The steps on a block staged in Xs (lower triangle, identity padded), by
// every thread of the workgroup (waves past the first two are passive).
// Leaves X = L⁻¹ in Xs (rows, lower triangle) and returns the failing pivot
// index + 1, or 0.
__device__ __forceinline__ int potrf_core(float* Xs, float (*colL)[POT_NB], float* rdl,
                                          int* fail_s) {
  const int i = threadIdx.x & 63, w = threadIdx.x >> 6;
  float v[POT_NB];
#pragma unroll
  for (int c = 0; c < POT_NB; ++c) v[c] = (w == 0) ? Xs[i * XP + c] : (c == i ? 1.f : 0.f);
  if (w < 2) colL[w][i] = 0.f;
  __syncthreads();  // Xs is reused for X below
  int fail = 0;
  float m = 0.f;
  if (w == 0) m = chol_pivot(v[0], 0, i, colL, rdl, fail);
  chol_inv_phase<64>(v, 0, i, w, colL, rdl, Xs, m, fail);
  chol_inv_phase<48>(v, 16, i, w, colL, rdl, Xs, m, fail);
  chol_inv_phase<32>(v, 32, i, w, colL, rdl, Xs, m, fail);
  chol_inv_phase<16>(v, 48, i, w, colL, rdl, Xs, m, fail);
  if (threadIdx.x == 0) *fail_s = fail;
  __syncthreads();
  return *fail_s;
}

}  // namespace
}  // namespace g2ptq
