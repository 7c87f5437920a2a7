// Diagonal-block Cholesky + inverse for the factor (device code, gfx950).
#pragma once
#include "common.hpp"

namespace g2ptq {
namespace {

// Cholesky + inverse of a diagonal block of the factor (nbk×nbk, nbk <= 64),
// shared by factor.hip's potrf kernel and its panel step (the workgroup that
// updates the next diagonal block factors it as soon as it is written).
//
// Blocked right-looking Cholesky in four 16-column panels on a 256-thread
// workgroup (rows at or past nbk are identity rows), and the inverse
// X = L⁻¹ by forward substitution, block row by block row:
//   panel p (wave 0, lane i = row i): the 16 pivots of columns
//     [16p, 16p + 16) in turn, each d = A[j][j] read from lane j,
//     l_ij = A[i][j]·rsqrt(d), and the rank-1 update of the panel's own
//     later columns with the multipliers of rows j + 1.. broadcast from
//     their lanes (no LDS round trip, no barrier);
//   trailing update (all waves): A[i][c] −= Σ_t l_it·l_ct over the panel's
//     16 columns for 16p + 16 <= c <= i, 2×2 entries per thread;
//   inverse rows [16p, 16p + 16) (wave 1, lane i = column i, beside the next
//     panel): acc_r = δ_ri − Σ_{j<r} X[j][i]·l_rj, X[r][i] = acc_r·rsqrt(d_r).
// Every entry receives its updates one fused multiply-add at a time in
// increasing column order, as in the unblocked right-looking algorithm (and
// the column-at-a-time forward substitution), so the block factor is that
// algorithm's to the bit; the blocking only moves the bulk of each step's
// work off the 64-step pivot chain.  1/sqrt comes from the hardware
// reciprocal square root (about 1 ulp): the factor is held to fp32
// tolerance, not to correctly rounded bits.  A non-positive (or NaN) pivot is
// recorded (its index + 1) and the steps run on.
constexpr int POT_NB = 64;          // block edge
constexpr int XP = POT_NB + 1;      // LDS row pitch of the block / X buffer
constexpr int LP = POT_NB + 4;      // LDS row pitch of L (16-byte rows)
constexpr int PB = 16;              // panel width

__device__ __forceinline__ float lane_val(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Panel P's 16 pivot steps on wave 0: rows from As, L columns to Lm, 1/sqrt
// of the pivots to rdv.
template <int P>
__device__ __forceinline__ void pot_panel(const float* As, float* Lm, float* rdv, int i, int& fail) {
  constexpr int k0 = P * PB;
  float a[PB];
#pragma unroll
  for (int c = 0; c < PB; ++c) a[c] = As[i * XP + k0 + c];
#pragma unroll
  for (int j = 0; j < PB; ++j) {
    const float d = lane_val(a[j], k0 + j);
    fail = (fail == 0 && !(d > 0.f)) ? k0 + j + 1 : fail;  // also catches NaN
    const float rd = __builtin_amdgcn_rsqf(d);
    const float m = (i > k0 + j) ? a[j] * rd : 0.f;
    if (i > k0 + j) Lm[i * LP + k0 + j] = m;
    if (i == 0) rdv[k0 + j] = rd;
#pragma unroll
    for (int c = j + 1; c < PB; ++c) a[c] = __builtin_fmaf(-m, lane_val(m, k0 + c), a[c]);
  }
}

// Trailing update by panel P of the lower entries at or past column 16P + 16.
template <int P>
__device__ __forceinline__ void pot_trail(float* As, const float* Lm) {
  constexpr int k0 = P * PB, t0 = k0 + PB, NBK = (POT_NB - t0) / 2;
  constexpr int NLOW = NBK * (NBK + 1) / 2;  // 2×2 blocks on or below the diagonal
  for (int q = threadIdx.x; q < NLOW; q += 256) {
    int ib = (int)((sqrtf(8.f * (float)q + 1.f) - 1.f) * 0.5f);
    while (ib * (ib + 1) / 2 > q) --ib;
    while ((ib + 1) * (ib + 2) / 2 <= q) ++ib;
    const int cb = q - ib * (ib + 1) / 2;
    const int r0 = t0 + 2 * ib, c0 = t0 + 2 * cb;
    float acc[2][2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[r][c] = As[(r0 + r) * XP + c0 + c];
#pragma unroll
    for (int t4 = 0; t4 < PB; t4 += 4) {
      float4 li[2], lc[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        li[r] = *reinterpret_cast<const float4*>(&Lm[(r0 + r) * LP + k0 + t4]);
        lc[r] = *reinterpret_cast<const float4*>(&Lm[(c0 + r) * LP + k0 + t4]);
      }
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          acc[r][c] = __builtin_fmaf(-li[r].x, lc[c].x, acc[r][c]);
          acc[r][c] = __builtin_fmaf(-li[r].y, lc[c].y, acc[r][c]);
          acc[r][c] = __builtin_fmaf(-li[r].z, lc[c].z, acc[r][c]);
          acc[r][c] = __builtin_fmaf(-li[r].w, lc[c].w, acc[r][c]);
        }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int c = 0; c < 2; ++c)
        if (c0 + c <= r0 + r) As[(r0 + r) * XP + c0 + c] = acc[r][c];
  }
}

// Rows [16P, 16P + 16) of X = L⁻¹ into Xs, lane i = column i (one wave);
// rows above are final in Xs.
template <int P>
__device__ __forceinline__ void pot_inv(float* Xs, const float* Lm, const float* rdv, int i) {
  constexpr int r0 = P * PB;
  float acc[PB];
#pragma unroll
  for (int q = 0; q < PB; ++q) acc[q] = (r0 + q == i) ? 1.f : 0.f;
#pragma unroll 1
  for (int j4 = 0; j4 < r0; j4 += 4) {
    float x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = Xs[(j4 + u) * XP + i];
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      const float4 l = *reinterpret_cast<const float4*>(&Lm[(r0 + q) * LP + j4]);
      acc[q] = __builtin_fmaf(-x[0], l.x, acc[q]);
      acc[q] = __builtin_fmaf(-x[1], l.y, acc[q]);
      acc[q] = __builtin_fmaf(-x[2], l.z, acc[q]);
      acc[q] = __builtin_fmaf(-x[3], l.w, acc[q]);
    }
  }
#pragma unroll
  for (int q = 0; q < PB; ++q) {
    const float x = acc[q] * rdv[r0 + q];
    Xs[(r0 + q) * XP + i] = x;
#pragma unroll
    for (int q2 = q + 1; q2 < PB; ++q2)
      acc[q2] = __builtin_fmaf(-x, Lm[(r0 + q2) * LP + r0 + q], acc[q2]);
  }
}

// The factor of the block staged in Xs (lower triangle, identity padded),
// by a 256-thread workgroup.  Lm (64·LP floats) and rdv (64) are scratch.
// Leaves X = L⁻¹ in Xs (rows, lower triangle; what lies above is not
// defined) and returns the failing pivot index + 1, or 0.
__device__ __forceinline__ int potrf_core(float* Xs, float* Lm, float* rdv, int* fail_s) {
  const int i = threadIdx.x & 63, w = threadIdx.x >> 6;
  int fail = 0;
  if (w == 0) pot_panel<0>(Xs, Lm, rdv, i, fail);
  __syncthreads();
  pot_trail<0>(Xs, Lm);
  __syncthreads();
  if (w == 0) pot_panel<1>(Xs, Lm, rdv, i, fail);
  else if (w == 1) pot_inv<0>(Xs, Lm, rdv, i);
  __syncthreads();
  pot_trail<1>(Xs, Lm);
  __syncthreads();
  if (w == 0) pot_panel<2>(Xs, Lm, rdv, i, fail);
  else if (w == 1) pot_inv<1>(Xs, Lm, rdv, i);
  __syncthreads();
  pot_trail<2>(Xs, Lm);
  __syncthreads();
  if (w == 0) pot_panel<3>(Xs, Lm, rdv, i, fail);
  else if (w == 1) pot_inv<2>(Xs, Lm, rdv, i);
  __syncthreads();
  if (w == 1) pot_inv<3>(Xs, Lm, rdv, i);
  if (threadIdx.x == 0) *fail_s = fail;
  __syncthreads();
  return *fail_s;
}

}  // namespace
}  // namespace g2ptq
