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
//     later columns: the next two with the multipliers of their rows read
//     from those lanes (v_readlane, on the pivot chain), the rest with the
//     multipliers the panel rows wrote to LDS (one store and a few
//     broadcast reads instead of a v_readlane per column; no barrier, the
//     wave's LDS accesses complete in order);
//   trailing update (all waves): A[i][c] −= Σ_t l_it·l_ct over the panel's
//     16 columns for 16p + 16 <= c <= i, 4×2 or 2×2 entries per thread;
//   inverse rows [16p, 16p + 16) (one of waves 1 to 3, lane i = column i,
//     beside the later panels): acc_r = δ_ri − Σ_{j<r} X[j][i]·l_rj,
//     X[r][i] = acc_r·rsqrt(d_r).
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
// of the pivots to rdv.  The multipliers and pivots stay in registers until
// the panel is done (Lm gets whole 16-byte rows, zeros on and above the
// diagonal, which nothing reads), so the pivot chain carries no stores.
template <int P>
__device__ __forceinline__ void pot_panel(const float* As, float* Lm, float* rdv, int i, int& fail) {
  constexpr int k0 = P * PB;
  constexpr int LA = 2;  // columns after the pivot updated through v_readlane
  float* Mb = rdv + POT_NB;  // per pivot, the panel rows' multipliers (LDS)
  float a[PB], l[PB];
  float rdl = 0.f;  // lane j: 1/sqrt of pivot k0 + j
#pragma unroll
  for (int c = 0; c < PB; ++c) a[c] = As[i * XP + k0 + c];
#pragma unroll
  for (int j = 0; j < PB; ++j) {
    const float d = lane_val(a[j], k0 + j);
    fail = (fail == 0 && !(d > 0.f)) ? k0 + j + 1 : fail;  // also catches NaN
    const float rd = __builtin_amdgcn_rsqf(d);
    const float m = (i > k0 + j) ? a[j] * rd : 0.f;
    l[j] = m;
    rdl = (i == j) ? rd : rdl;
    if (j + LA + 1 < PB && i >= k0 && i < k0 + PB) Mb[j * PB + (i - k0)] = m;
#pragma unroll
    for (int c = j + 1; c < PB && c <= j + LA; ++c)
      a[c] = __builtin_fmaf(-m, lane_val(m, k0 + c), a[c]);
#pragma unroll
    for (int c = j + LA + 1; c < PB; ++c) a[c] = __builtin_fmaf(-m, Mb[j * PB + c], a[c]);
  }
#pragma unroll
  for (int c4 = 0; c4 < PB; c4 += 4)
    *reinterpret_cast<float4*>(&Lm[i * LP + k0 + c4]) = make_float4(l[c4], l[c4 + 1], l[c4 + 2], l[c4 + 3]);
  if (i < PB) rdv[k0 + i] = rdl;
}

// Trailing update by panel P of the lower entries at or past column 16P + 16,
// in blocks of RB rows × 2 columns on or below the diagonal, one per thread:
// 4-row blocks where 2×2 blocks would not fit in one pass of the 256 threads
// (panel 0: 156 blocks of 4×2 instead of 300 of 2×2), 2×2 otherwise.
template <int P>
__device__ __forceinline__ void pot_trail(float* As, const float* Lm) {
  constexpr int k0 = P * PB, t0 = k0 + PB, W = POT_NB - t0;
  constexpr int RB = (W / 2) * (W / 2 + 1) / 2 > 256 ? 4 : 2;
  constexpr int NR = W / RB;  // row blocks; row block ib has RB / 2·ib + RB / 2 column pairs
  constexpr int NLOW = RB == 4 ? NR * (NR + 1) : NR * (NR + 1) / 2;
  static_assert(NLOW <= 256, "one pass");
  const int q = threadIdx.x;
  if (q >= NLOW) return;
  // blocks before row block ib: ib·(ib + 1) (RB = 4) or ib·(ib + 1)/2 (RB = 2)
  const float qf = RB == 4 ? (float)q : 2.f * (float)q;
  int ib = (int)((sqrtf(4.f * qf + 1.f) - 1.f) * 0.5f);
  auto before = [](int v) { return RB == 4 ? v * (v + 1) : v * (v + 1) / 2; };
  while (before(ib) > q) --ib;
  while (before(ib + 1) <= q) ++ib;
  const int cb = q - before(ib);
  const int r0 = t0 + RB * ib, c0 = t0 + 2 * cb;
  float acc[RB][2];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[r][c] = As[(r0 + r) * XP + c0 + c];
#pragma unroll
  for (int t4 = 0; t4 < PB; t4 += 4) {
    float4 li[RB], lc[2];
#pragma unroll
    for (int r = 0; r < RB; ++r) li[r] = *reinterpret_cast<const float4*>(&Lm[(r0 + r) * LP + k0 + t4]);
#pragma unroll
    for (int c = 0; c < 2; ++c) lc[c] = *reinterpret_cast<const float4*>(&Lm[(c0 + c) * LP + k0 + t4]);
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        acc[r][c] = __builtin_fmaf(-li[r].x, lc[c].x, acc[r][c]);
        acc[r][c] = __builtin_fmaf(-li[r].y, lc[c].y, acc[r][c]);
        acc[r][c] = __builtin_fmaf(-li[r].z, lc[c].z, acc[r][c]);
        acc[r][c] = __builtin_fmaf(-li[r].w, lc[c].w, acc[r][c]);
      }
  }
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int c = 0; c < 2; ++c)
      if (c0 + c <= r0 + r) As[(r0 + r) * XP + c0 + c] = acc[r][c];
}

// Rows [16P, 16P + 16) of X = L⁻¹, lane i = column i (one wave), in three
// parts so that the bulk of the later block rows runs beside the panels:
//   pot_inv_init: acc_q = δ(16P + q, i);
//   pot_inv_bulk: acc_q −= Σ_{jlo <= j < jhi} X[j][i]·l_{16P+q, j}, j in
//     increasing order (X rows below jhi final in Xs);
//   pot_inv_fin:  the block's own triangle and the rows into Xs.
// Each entry receives the same fused multiply-adds in the same order however
// the j range is split, so the split is invisible in the results.
template <int P>
__device__ __forceinline__ void pot_inv_init(float (&acc)[PB], int i) {
  constexpr int r0 = P * PB;
#pragma unroll
  for (int q = 0; q < PB; ++q) acc[q] = (r0 + q == i) ? 1.f : 0.f;
}

template <int P, int JLO, int JHI>
__device__ __forceinline__ void pot_inv_bulk(float (&acc)[PB], const float* Xs, const float* Lm,
                                             int i) {
  constexpr int r0 = P * PB;
  static_assert(JHI <= r0 && JLO % 4 == 0 && JHI % 4 == 0, "bulk columns left of the block");
#pragma unroll 1
  for (int j4 = JLO; j4 < JHI; j4 += 4) {
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
}

template <int P>
__device__ __forceinline__ void pot_inv_fin(float (&acc)[PB], float* Xs, const float* Lm,
                                            const float* rdv, int i) {
  constexpr int r0 = P * PB;
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
// by a 256-thread workgroup.  Lm (64·LP floats) and rdv (64 + 16·16) are scratch.
// Leaves X = L⁻¹ in Xs (rows, lower triangle; what lies above is not
// defined) and returns the failing pivot index + 1, or 0.
// Schedule (waves w0..w3, `|` a barrier; the trailing updates occupy the
// first 156, 136 and 36 threads):
//   panel0 | trail0, inv0 (w3) |
//   panel1, inv2[j < 16] (w1), inv3[j < 16] (w2), inv1[j < 16] (w3) |
//   trail1, inv1 triangle (w3) |
//   panel2, inv2[16 <= j < 32] (w1), inv3[16 <= j < 32] (w2) |
//   trail2, inv2 triangle (w1) | panel3, inv3[32 <= j < 48] (w2) | inv3 triangle (w2)
// so only the last block row's triangle follows the last panel.
__device__ __forceinline__ int potrf_core(float* Xs, float* Lm, float* rdv, int* fail_s) {
  const int i = threadIdx.x & 63, w = threadIdx.x >> 6;
  int fail = 0;
  float acc[PB];  // the wave's inverse block row (waves 1 to 3)
  if (w == 0) pot_panel<0>(Xs, Lm, rdv, i, fail);
  __syncthreads();
  pot_trail<0>(Xs, Lm);
  if (w == 3) {
    pot_inv_init<0>(acc, i);
    pot_inv_fin<0>(acc, Xs, Lm, rdv, i);
  }
  __syncthreads();
  if (w == 0) {
    pot_panel<1>(Xs, Lm, rdv, i, fail);
  } else if (w == 1) {
    pot_inv_init<2>(acc, i);
    pot_inv_bulk<2, 0, 16>(acc, Xs, Lm, i);
  } else if (w == 2) {
    pot_inv_init<3>(acc, i);
    pot_inv_bulk<3, 0, 16>(acc, Xs, Lm, i);
  } else {
    pot_inv_init<1>(acc, i);
    pot_inv_bulk<1, 0, 16>(acc, Xs, Lm, i);
  }
  __syncthreads();
  pot_trail<1>(Xs, Lm);
  if (w == 3) pot_inv_fin<1>(acc, Xs, Lm, rdv, i);
  __syncthreads();
  if (w == 0) {
    pot_panel<2>(Xs, Lm, rdv, i, fail);
  } else if (w == 1) {
    pot_inv_bulk<2, 16, 32>(acc, Xs, Lm, i);
  } else if (w == 2) {
    pot_inv_bulk<3, 16, 32>(acc, Xs, Lm, i);
  }
  __syncthreads();
  pot_trail<2>(Xs, Lm);
  if (w == 1) pot_inv_fin<2>(acc, Xs, Lm, rdv, i);
  __syncthreads();
  if (w == 0) {
    pot_panel<3>(Xs, Lm, rdv, i, fail);
  } else if (w == 2) {
    pot_inv_bulk<3, 32, 48>(acc, Xs, Lm, i);
  }
  __syncthreads();
  if (w == 2) pot_inv_fin<3>(acc, Xs, Lm, rdv, i);
  if (threadIdx.x == 0) *fail_s = fail;
  __syncthreads();
  return *fail_s;
}

}  // namespace
}  // namespace g2ptq
