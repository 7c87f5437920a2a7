// Quantizer grid kernels and the fused lazy-batch block sweep.
//
// Rounding contract (bit-exact with the reference's torch backend):
//   q   = clamp(rint(x / s) + z, -(maxq+1), maxq)      IEEE div, half-to-even
//   deq = s * (q - z)
//   err = (x - deq [- gh]) / U_jj                       IEEE div
//   w_k = w_k - round(U_jk * err)                       no FMA contraction
// which is what torch's elementwise ops and its K=1 baddbmm compute.  hipcc
// contracts a*b+c into FMA by default, even across the __f*_rn helpers of the
// HIP headers, so this translation unit is built with -ffp-contract=off.
#include "sweep.hpp"

#pragma clang fp contract(off)

namespace g2ptq {
namespace {

template <bool B>
struct ExactTag {
  static constexpr bool value = B;
};

// NaN-propagating clamp (torch.clamp semantics).
__device__ __forceinline__ float clamp_nan(float v, float lo, float hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// a / b correctly rounded, from y = RN(1/b): Markstein's sequence
// q = RN(a·y), r = a − b·q (exact through the FMA), RN(q + r·y) (P. Markstein,
// "Computation of elementary functions on the IBM RISC System/6000
// processor", IBM J. Res. Dev. 34(1), 1990).  It equals the IEEE quotient
// whenever r is exactly representable and nothing overflows, which holds for
// |a|, |q| in [2^-100, 2^100].  It also gives the IEEE quotient for a = +0
// whenever y is finite and nonzero (q = ±0 with the quotient's sign, r = +0,
// q + r·y = q), which is what dead columns and exactly representable values
// produce.  Any lane outside those cases (−0, tiny, huge, infinite or NaN
// operands, a zero or infinite divisor) takes the IEEE division, on a
// wave-uniform branch that real data never enters.  Three dependent
// operations instead of the eleven of the IEEE division sequence on the
// sweep's per-column chain.
__device__ __forceinline__ bool recip_div_exact(float a, float q, float y) {
  const float aa = fabsf(a), aq = fabsf(q), ay = fabsf(y);
  const bool pos_zero = __float_as_uint(a) == 0u && ay > 0.f && ay < __builtin_inff();
  return pos_zero || (aa >= 0x1p-100f && aa <= 0x1p100f && aq >= 0x1p-100f && aq <= 0x1p100f);
}
// Markstein's sequence alone: the IEEE quotient when recip_div_exact(a, RN(a·y), y).
__device__ __forceinline__ float div_markstein(float a, float b, float y) {
  const float q = __fmul_rn(a, y);
  const float r = __fmaf_rn(-b, q, a);
  return __fmaf_rn(r, y, q);
}
__device__ __forceinline__ float div_rn_recip(float a, float b, float y) {
  const float q = __fmul_rn(a, y);
  const float r = __fmaf_rn(-b, q, a);
  float res = __fmaf_rn(r, y, q);
  const bool slow = !recip_div_exact(a, q, y);
  if (__builtin_amdgcn_ballot_w64(slow) != 0) {
    asm volatile("" ::: "memory");  // keeps the branch: the division is not speculated
    res = slow ? __fdiv_rn(a, b) : res;
  }
  return res;
}

// ---------------------------------------------------------------------------
// find_params: one quantization group per row, 16 lanes per row.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void params_from_minmax(float mn, float mx, bool has_nan, int maxq,
                                                   int sym, float& s, float& z) {
  const float minq = (float)(-(maxq + 1));
  const float bit_range = (float)(2 * maxq + 1);
  float xmin = has_nan ? __builtin_nanf("") : fminf(mn, 0.f);
  float xmax = has_nan ? __builtin_nanf("") : fmaxf(mx, 0.f);
  if (sym) {
    const float m = has_nan ? xmin : fmaxf(fabsf(xmin), xmax);
    s = __fdiv_rn(m, 0.5f * bit_range);
    z = 0.f;
  } else {
    s = __fdiv_rn(__fsub_rn(xmax, xmin), bit_range);
    float t = rintf(__fsub_rn(minq, __fdiv_rn(xmin, s)));
    z = rintf(clamp_nan(t, minq, (float)maxq));
  }
}

__global__ __launch_bounds__(256) void find_params_kernel(const float* __restrict__ x,
                                                          int64_t rows, int64_t cols, int64_t ldx,
                                                          int maxq, int sym, float* scale,
                                                          float* zero, int64_t ldp, int* flags) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid >> 4;
  const int sub = threadIdx.x & 15;
  float mn = INFINITY, mx = -INFINITY;
  int nan = 0;
  if (row < rows) {
    const float* xr = x + row * ldx;
    for (int64_t c = sub; c < cols; c += 16) {
      const float v = xr[c];
      nan |= (v != v);
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, o, 16));
    mx = fmaxf(mx, __shfl_xor(mx, o, 16));
    nan |= __shfl_xor(nan, o, 16);
  }
  if (sub == 0 && row < rows) {
    float s, z;
    params_from_minmax(mn, mx, nan != 0, maxq, sym, s, z);
    scale[row * ldp] = s;
    zero[row * ldp] = z;
    if (!(s > 0.f) && flags) atomicOr(flags, FLAG_BAD_SCALE);
  }
}

// ---------------------------------------------------------------------------
// MSE clip search (quant_utils.py:406-425): one wave per row.  Candidate
// (i, j) shrinks xmin by (1 - i/grid) and xmax by (1 - j/grid); the error is
// sum(|fq - x|^norm), or with Hessian-diagonal weights sum((fq - x)^2 * h)
// (_quant_err, :84-105); a candidate replaces the incumbent only when
// strictly better, scanning i-major exactly like the reference loop.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void find_params_mse_kernel(const float* __restrict__ x,
                                                             int64_t rows, int64_t cols,
                                                             int64_t ldx, int maxq, int sym,
                                                             float norm, int grid, int steps,
                                                             HDiag hd, float* scale, float* zero,
                                                             int64_t ldp, int* flags) {
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  const float* xr = x + row * ldx;
  // The weights are dropped (plain |err|^norm search) when every entry of the
  // given H_diag is equal (quant_utils.py:393-397: min == max, which a NaN
  // never satisfies).  Every wave checks the whole H_diag (nblocks·gpr·cols
  // values, L2-resident) against the search's steps² passes over its row.
  const float* hr = nullptr;
  if (hd.h) {
    const int64_t hc = hd.gpr * cols;
    float hmn = INFINITY, hmx = -INFINITY;
    int hnan = 0;
    for (int64_t b = 0; b < hd.nblocks; ++b)
      for (int64_t c = lane; c < hc; c += 64) {
        const float v = hd.h[b * hd.ld + c];
        hnan |= (v != v);
        hmn = fminf(hmn, v);
        hmx = fmaxf(hmx, v);
      }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      hmn = fminf(hmn, __shfl_xor(hmn, o));
      hmx = fmaxf(hmx, __shfl_xor(hmx, o));
      hnan |= __shfl_xor(hnan, o);
    }
    if (hnan || hmn != hmx) {
      const int64_t orow = row / hd.gpr, k = row - orow * hd.gpr;
      const int64_t share = rows / hd.gpr / hd.nblocks;  // original rows per block
      hr = hd.h + (orow / share) * hd.ld + k * cols;
    }
  }
  float mn = INFINITY, mx = -INFINITY;
  int nan = 0;
  for (int64_t c = lane; c < cols; c += 64) {
    const float v = xr[c];
    nan |= (v != v);
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, o));
    mx = fmaxf(mx, __shfl_xor(mx, o));
    nan |= __shfl_xor(nan, o);
  }
  const float xmin = nan ? __builtin_nanf("") : fminf(mn, 0.f);
  const float xmax = nan ? __builtin_nanf("") : fmaxf(mx, 0.f);
  float best_s, best_z;
  params_from_minmax(mn, mx, nan != 0, maxq, sym, best_s, best_z);
  float best = INFINITY;
  const float minq = (float)(-(maxq + 1)), fmaxq = (float)maxq;
  const float bit_range = (float)(2 * maxq + 1);
  for (int i = 0; i < steps; ++i) {
    // (1 - i/grid) is a python float product with a fp32 tensor: the factor is
    // rounded to fp32 once and multiplied in fp32.
    const float fi = (float)(1.0 - (double)i / (double)grid);
    const float xmin1 = __fmul_rn(fi, xmin);
    for (int j = 0; j < steps; ++j) {
      const float fj = (float)(1.0 - (double)j / (double)grid);
      const float xmax1 = __fmul_rn(fj, xmax);
      float s1, z1;
      if (sym) {
        s1 = __fdiv_rn(fmaxf(fabsf(xmin1), xmax1), 0.5f * bit_range);
        z1 = 0.f;
      } else {
        s1 = __fdiv_rn(__fsub_rn(xmax1, xmin1), bit_range);
        z1 = clamp_nan(rintf(__fsub_rn(minq, __fdiv_rn(xmin1, s1))), minq, fmaxq);
      }
      float err = 0.f;
      for (int64_t c = lane; c < cols; c += 64) {
        const float v = xr[c];
        const float q = clamp_nan(__fadd_rn(rintf(__fdiv_rn(v, s1)), z1), minq, fmaxq);
        const float fq = __fmul_rn(s1, __fsub_rn(q, z1));
        const float d = __fsub_rn(fq, v);
        err += hr ? __fmul_rn(__fmul_rn(d, d), hr[c]) : powf(fabsf(d), norm);
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) err += __shfl_xor(err, o);
      if (err < best) {
        best = err;
        best_s = s1;
        best_z = z1;
      }
    }
  }
  if (lane == 0) {
    scale[row * ldp] = best_s;
    zero[row * ldp] = rintf(best_z);
    if (!(best_s > 0.f) && flags) atomicOr(flags, FLAG_BAD_SCALE);
  }
}

__global__ __launch_bounds__(256) void fake_quantize_kernel(
    const float* __restrict__ x, int64_t rows, int64_t cols, int64_t ldx, int64_t gsize,
    const float* __restrict__ scale, const float* __restrict__ zero, int64_t ldp, int maxq,
    float* q_out, int64_t ldq, float* int_out, int64_t ldi) {
  const int64_t n = rows * cols;
  const float minq = (float)(-(maxq + 1)), fmaxq = (float)maxq;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols, c = i % cols;
    const int64_t gidx = gsize > 0 ? c / gsize : 0;
    const float s = scale[r * ldp + gidx], z = zero[r * ldp + gidx];
    const float v = x[r * ldx + c];
    const float q = clamp_nan(__fadd_rn(rintf(__fdiv_rn(v, s)), z), minq, fmaxq);
    q_out[r * ldq + c] = __fmul_rn(s, __fsub_rn(q, z));
    if (int_out) int_out[r * ldi + c] = q;
  }
}

// ---------------------------------------------------------------------------
// Fused block sweep.
//
// One wave64 owns 64 rows of one layer (lane = row) for a block of n <= 128
// columns.  The block's upper-triangular U (and P) is staged once into LDS in
// packed row order and read with wave-uniform (broadcast) LDS loads.  The
// block is walked in panels of PW columns whose values live in VGPRs; updates
// from earlier panels are replayed from the per-lane error history kept in
// LDS, in increasing column order, so every element sees the reference's
// exact sequence of updates.  VEC: every per-row operand is contiguous along
// columns and 16-byte aligned (the native (B, R, C) layout), so panel loads
// and result stores move 4 columns per instruction.
// ---------------------------------------------------------------------------
constexpr int kTri = kMaxBlock * (kMaxBlock + 1) / 2;

// Packed upper triangle: element (j, k >= j) lives at tri_base(j, n) + k.
__device__ __forceinline__ int tri_base(int j, int n) { return j * n - (j * (j - 1)) / 2 - j; }

template <int V, int PW, bool VEC, bool FULL>
__global__ __launch_bounds__(64) void sweep_kernel(SweepArgs a) {
  __shared__ float Us[kTri];
  __shared__ float Ps[(V == 1) ? kTri : 1];
  __shared__ float e_s[kMaxBlock * 64];
  __shared__ float t_s[(V == 1) ? kMaxBlock * 64 : 1];
  __shared__ float z_s[(V == 2) ? kMaxBlock * 64 : 1];

  const int lane = threadIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t r0 = (int64_t)blockIdx.x * 64 + lane;
  const bool act = r0 < a.R;
  const int64_t r = act ? r0 : 0;
  const int n = a.n;
  const float minq = (float)(-(a.maxq + 1)), fmaxq = (float)a.maxq;

  {
    // Stage the upper triangle: 8 independent loads in flight per lane per batch.
    const float* U = a.U + b * a.ub;
    const float* P = (V == 1) ? a.P + b * a.ub : nullptr;
    const int nn = n * n;
    for (int base = 0; base < nn; base += 64 * 8) {
      float uv[8], pv[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int idx = base + q * 64 + lane;
        const int j = idx / n, k = idx - j * n;
        const bool need = idx < nn && k >= j;
        uv[q] = need ? U[(int64_t)j * a.uj + k] : 0.f;
        if (V == 1) pv[q] = need ? P[(int64_t)j * a.uj + k] : 0.f;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int idx = base + q * 64 + lane;
        const int j = idx / n, k = idx - j * n;
        if (idx < nn && k >= j) {
          Us[tri_base(j, n) + k] = uv[q];
          if (V == 1) Ps[tri_base(j, n) + k] = pv[q];
        }
      }
    }
  }
  __syncthreads();

  const float* Win = a.W + b * a.wb + r * a.wr;
  const float* Sp = a.S + b * a.sb + r * a.sr;
  const float* Zp = a.Z0 + b * a.sb + r * a.sr;
  const float* Zg = (V == 2) ? a.Zg + b * a.zb + r * a.zr : nullptr;
  const float* GH = (V == 2) ? a.GH + b * a.gb + r * a.gr : nullptr;
  float* GHo = (V == 2 && a.GHout) ? a.GHout + b * a.gb + r * a.gr : nullptr;
  float* Qo = a.Q + b * a.qb + r * a.qr;
  float* Io = a.I ? a.I + b * a.ib + r * a.ir : nullptr;
  float* Eo = a.E ? a.E + b * a.eb + r * a.er : nullptr;
  float* So = a.Sc ? a.Sc + b * a.cb + r * a.cr : nullptr;
  float* E2 = (V == 2 && a.E2) ? a.E2 + b * a.e2b + r * a.e2r : nullptr;
  float* E3 = (V == 2 && a.E3) ? a.E3 + b * a.e3b + r * a.e3r : nullptr;

  int bad = 0;
  float last_x = 0.f;

  for (int p0 = 0; p0 < n; p0 += PW) {
    const int np = FULL ? PW : min(PW, n - p0);
    // ---- panel inputs, all issued before any store of this panel -------------
    float w[PW], gh[PW], sv[PW], zv[PW], zg[PW];
#pragma unroll
    for (int jj = 0; jj < PW; ++jj) {
      const bool in = FULL || jj < np;
      const int j = p0 + jj;
      int gidx = 0;
      if (a.colgroup) gidx = a.colgroup[in ? j : 0];
      else if (a.gsize > 0) gidx = (int)((int)a.col0 + j) / (int)a.gsize;
      if (!in) gidx = 0;
      sv[jj] = Sp[(int64_t)gidx * a.sg];
      zv[jj] = Zp[(int64_t)gidx * a.sg];
      if (V == 2) zg[jj] = Zg[(int64_t)(in ? j : 0) * a.zc];
    }
    if (VEC) {
#pragma unroll
      for (int kk = 0; kk < PW; kk += 4) {
        const int off = (FULL || kk < np) ? p0 + kk : 0;
        const float4 v = *reinterpret_cast<const float4*>(Win + off);
        w[kk] = v.x; w[kk + 1] = v.y; w[kk + 2] = v.z; w[kk + 3] = v.w;
        if (V == 2) {
          const float4 g4 = *reinterpret_cast<const float4*>(GH + off);
          gh[kk] = g4.x; gh[kk + 1] = g4.y; gh[kk + 2] = g4.z; gh[kk + 3] = g4.w;
        }
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < PW; ++kk) {
        const int c = (FULL || kk < np) ? p0 + kk : 0;
        w[kk] = Win[(int64_t)c * a.wc];
        if (V == 2) gh[kk] = GH[(int64_t)c * a.gc];
      }
    }
    // ---- replay updates of the columns swept in earlier panels (LDS only) ---
    for (int j = 0; j < p0; ++j) {
      const float e = e_s[j * 64 + lane];
      float t = 0.f, zj = 0.f;
      if (V == 1) t = t_s[j * 64 + lane];
      if (V == 2) zj = z_s[j * 64 + lane];
      const float* Uj = Us + tri_base(j, n) + p0;
      const float* Pj = (V == 1) ? Ps + tri_base(j, n) + p0 : nullptr;
#pragma unroll
      for (int kk = 0; kk < PW; ++kk) {
        if (FULL || kk < np) {
          const float u = Uj[kk];
          if (V == 0) {
            w[kk] = __fsub_rn(w[kk], __fmul_rn(u, e));
          } else if (V == 1) {
            w[kk] = __fadd_rn(__fsub_rn(w[kk], __fmul_rn(u, e)), __fmul_rn(Pj[kk], t));
          } else {
            w[kk] = __fsub_rn(__fsub_rn(w[kk], gh[kk]), __fmul_rn(u, e));
            gh[kk] = __fsub_rn(gh[kk], __fmul_rn(u, zj));
          }
        }
      }
    }
    // ---- sweep this panel column by column (registers + LDS only) -----------
    float qb[PW], ib[PW], gb[PW];
#pragma unroll
    for (int jj = 0; jj < PW; ++jj) {
      if (FULL || jj < np) {
        const int j = p0 + jj;
        const float x = w[jj];
        const float s = sv[jj];
        const float z0 = zv[jj];
        const float q = clamp_nan(__fadd_rn(rintf(__fdiv_rn(x, s)), z0), minq, fmaxq);
        const float deq = __fmul_rn(s, __fsub_rn(q, z0));
        const float d = Us[tri_base(j, n) + j];
        float err;
        float zj = 0.f;
        if (V == 2) {
          err = __fdiv_rn(__fsub_rn(__fsub_rn(x, deq), gh[jj]), d);
          zj = zg[jj];
          z_s[j * 64 + lane] = zj;
          gb[jj] = gh[jj];
        } else {
          err = __fdiv_rn(__fsub_rn(x, deq), d);
        }
        bad |= !(s > 0.f);
        qb[jj] = deq;
        ib[jj] = q;
        e_s[j * 64 + lane] = err;
        if (V == 1) t_s[j * 64 + lane] = x;
        last_x = x;
        const float* Uj = Us + tri_base(j, n) + p0;
        const float* Pj = (V == 1) ? Ps + tri_base(j, n) + p0 : nullptr;
#pragma unroll
        for (int kk = jj + 1; kk < PW; ++kk) {
          if (FULL || kk < np) {
            const float u = Uj[kk];
            if (V == 0) {
              w[kk] = __fsub_rn(w[kk], __fmul_rn(u, err));
            } else if (V == 1) {
              w[kk] = __fadd_rn(__fsub_rn(w[kk], __fmul_rn(u, err)), __fmul_rn(Pj[kk], x));
            } else {
              w[kk] = __fsub_rn(__fsub_rn(w[kk], gh[kk]), __fmul_rn(u, err));
              gh[kk] = __fsub_rn(gh[kk], __fmul_rn(u, zj));
            }
          }
        }
      }
    }
    // ---- panel outputs ------------------------------------------------------
    if (act) {
      if (VEC) {
#pragma unroll
        for (int kk = 0; kk < PW; kk += 4) {
          if (FULL || kk < np) {
            const int c = p0 + kk;
            *reinterpret_cast<float4*>(Qo + c) = make_float4(qb[kk], qb[kk + 1], qb[kk + 2], qb[kk + 3]);
            if (Io) *reinterpret_cast<float4*>(Io + c) = make_float4(ib[kk], ib[kk + 1], ib[kk + 2], ib[kk + 3]);
            if (So) *reinterpret_cast<float4*>(So + c) = make_float4(sv[kk], sv[kk + 1], sv[kk + 2], sv[kk + 3]);
            float ev[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) ev[q] = e_s[(c + q) * 64 + lane];
            if (Eo) *reinterpret_cast<float4*>(Eo + c) = make_float4(ev[0], ev[1], ev[2], ev[3]);
            if (V == 2 && E2) {
              float e2[4];
#pragma unroll
              for (int q = 0; q < 4; ++q)
                e2[q] = __fsub_rn(ev[q], __fmul_rn(zg[kk + q], (float)(a.dist0 - (c + q))));
              *reinterpret_cast<float4*>(E2 + c) = make_float4(e2[0], e2[1], e2[2], e2[3]);
            }
            if (V == 2 && E3) {
              float e3[4];
#pragma unroll
              for (int q = 0; q < 4; ++q)
                e3[q] = __fsub_rn(ev[q], __fmul_rn(zg[kk + q], (float)(a.dist3 - (c + q))));
              *reinterpret_cast<float4*>(E3 + c) = make_float4(e3[0], e3[1], e3[2], e3[3]);
            }
          }
        }
      } else {
#pragma unroll
        for (int jj = 0; jj < PW; ++jj) {
          if (FULL || jj < np) {
            const int j = p0 + jj;
            const float ev = e_s[j * 64 + lane];
            Qo[(int64_t)j * a.qc] = qb[jj];
            if (Io) Io[(int64_t)j * a.ic] = ib[jj];
            if (Eo) Eo[(int64_t)j * a.ec] = ev;
            if (So) So[(int64_t)j * a.cc] = sv[jj];
            if (V == 2 && E2)
              E2[(int64_t)j * a.e2c] = __fsub_rn(ev, __fmul_rn(zg[jj], (float)(a.dist0 - j)));
            if (V == 2 && E3)
              E3[(int64_t)j * a.e2c] = __fsub_rn(ev, __fmul_rn(zg[jj], (float)(a.dist3 - j)));
            if (V == 2 && GHo) GHo[(int64_t)j * a.gc] = gb[jj];
          }
        }
      }
    }
  }
  if (V == 1 && a.CW && act) a.CW[b * a.cwb + r * a.cwr] = last_x;
  if (bad && act && a.flags) atomicOr(a.flags, FLAG_BAD_SCALE);
}

// Split sweep: the same computation, with each row split over L lanes (a quad,
// L = 4: 16 rows per wave; or a 16-lane DPP row, L = 16: 4 rows per wave).  In
// every 32-column panel lane `sub` of a row's group owns columns L·s + sub
// (s < 32/L).  Column jj's quantisation runs on all L lanes but only its owner
// (sub == jj % L) holds the column, and its error (and x, z) reach the other
// lanes with a DPP broadcast (quad_perm, or row_newbcast for L = 16); every
// lane then applies the rank-1 update to the columns it owns.  Each element
// still receives exactly the reference's sequence of rounded products and
// differences, in the same order, so the results equal sweep_kernel's bit for
// bit.  The per-row dependency chain (two divisions per column) is the same
// for every L; a larger L spreads a block's rows over more waves and gives
// each lane fewer columns to update, which pays when the block has few rows
// (a wave per SIMD at most), while L = 4 does less redundant chain work per
// row when rows are plentiful.  A workgroup of four waves (256/L rows) stages
// the block's U triangle once for all of them.
template <int O>
__device__ __forceinline__ float quad_bcast_c(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), O * 0x55, 0xf, 0xf, false));
}
__device__ __forceinline__ float quad_bcast(float v, int o) {
  switch (o & 3) {
    case 0: return quad_bcast_c<0>(v);
    case 1: return quad_bcast_c<1>(v);
    case 2: return quad_bcast_c<2>(v);
    default: return quad_bcast_c<3>(v);
  }
}
// Lane o of each 16-lane row to the whole row (DPP row_newbcast:o).
template <int O>
__device__ __forceinline__ float row_bcast_c(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + O, 0xf, 0xf, false));
}
template <int L>
__device__ __forceinline__ float group_bcast(float v, int o) {
  if (L == 4) return quad_bcast(v, o);
  switch (o & 15) {
    case 0: return row_bcast_c<0>(v);
    case 1: return row_bcast_c<1>(v);
    case 2: return row_bcast_c<2>(v);
    case 3: return row_bcast_c<3>(v);
    case 4: return row_bcast_c<4>(v);
    case 5: return row_bcast_c<5>(v);
    case 6: return row_bcast_c<6>(v);
    case 7: return row_bcast_c<7>(v);
    case 8: return row_bcast_c<8>(v);
    case 9: return row_bcast_c<9>(v);
    case 10: return row_bcast_c<10>(v);
    case 11: return row_bcast_c<11>(v);
    case 12: return row_bcast_c<12>(v);
    case 13: return row_bcast_c<13>(v);
    case 14: return row_bcast_c<14>(v);
    default: return row_bcast_c<15>(v);
  }
}

template <int V, int L, bool F, bool SBM = false>
__global__ __launch_bounds__(256) void sweep4_kernel(SweepArgs a) {
  constexpr int PW = 32, RW = 256 / L;  // panel width, rows per workgroup
  constexpr int NS = PW / L;            // panel columns per lane
  // The triangles plus one spare word per lane (the full-block staging's
  // sink for entries left of the diagonal).
  __shared__ __attribute__((aligned(16))) float Us[kTri + 64];
  __shared__ float Ps[(V == 1) ? kTri + 64 : 1];
  __shared__ float e_s[kMaxBlock * RW];
  __shared__ float t_s[(V == 1) ? kMaxBlock * RW : 1];
  __shared__ float z_s[(V == 2) ? kMaxBlock * RW : 1];
  __shared__ __attribute__((aligned(16))) float rdiag[kMaxBlock];  // RN(1 / U_jj)
  __shared__ __attribute__((aligned(16))) float dg[kMaxBlock];     // U_jj

  const int64_t b = blockIdx.y;
  const float minq = (float)(-(a.maxq + 1)), fmaxq = (float)a.maxq;

  int bad = 0;
  float last_x = 0.f;
  const int nblk = SBM ? a.nblk : 1;
#pragma clang loop unroll(disable)
  for (int bi = 0; bi < nblk; ++bi) {
  const int64_t cofs = (int64_t)bi * kMaxBlock;  // the block's first column in the super-block
  // In a super-block launch the thread index and block width are re-read
  // opaquely per block, so the compiler cannot hoist the block's many
  // derived addresses out of the block loop (which would cost a wave
  // occupancy in registers).
  int tid = threadIdx.x, n = a.n;
  if (SBM) {
    asm volatile("" : "+v"(tid));
    asm volatile("" : "+s"(n));
  }
  const int rr = tid / L, sub = tid % L;
  const int64_t r0 = (int64_t)blockIdx.x * RW + rr;
  const bool act = r0 < a.R;
  const int64_t r = act ? r0 : 0;
  {
    // Stage the block's upper triangle (shared by the four waves): rows of U
    // as 16-byte chunks, all of a thread's loads in flight before its stores.
    const float* U = a.U + b * a.ub + cofs * a.uj + cofs;
    const float* P = (V == 1) ? a.P + b * a.ub + cofs * a.uj + cofs : nullptr;
    const int nc = (n + 3) >> 2;              // 4-column chunks per row
    const int total = n * nc;
    const bool vec = ((a.uj & 3) == 0) && ((reinterpret_cast<uintptr_t>(U) & 15) == 0) &&
                     (V != 1 || (reinterpret_cast<uintptr_t>(P) & 15) == 0);
    if (n == kMaxBlock && vec) {
      // Full block: chunk q of thread tid is row j = 8q + tid/32, columns
      // k..k+3 = 4·(tid % 32), all in bounds (entries left of the diagonal
      // are U's zeros); those entries are stored to the thread's spare word
      // instead of branching around the store.
      static_assert(kMaxBlock == 128, "full-block staging covers 128 rows in 16 chunks of 8");
      float4 uv[16], pv[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int j = q * 8 + (tid >> 5), k = (tid & 31) * 4;
        uv[q] = *reinterpret_cast<const float4*>(U + (int64_t)j * a.uj + k);
        if (V == 1) pv[q] = *reinterpret_cast<const float4*>(P + (int64_t)j * a.uj + k);
      }
      const int sink = kTri + (tid & 63);
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int j = q * 8 + (tid >> 5), k = (tid & 31) * 4;
        const int t0 = tri_base(j, kMaxBlock);
        const float ue[4] = {uv[q].x, uv[q].y, uv[q].z, uv[q].w};
        const float pe[4] = {pv[q].x, pv[q].y, pv[q].z, pv[q].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int at = (k + e >= j) ? t0 + k + e : sink;
          Us[at] = ue[e];
          if (V == 1) Ps[at] = pe[e];
        }
      }
    } else {
      for (int base = 0; base < total; base += 256 * 16) {
        float4 uv[16], pv[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int idx = base + q * 256 + tid;
          const int j = idx / nc, k = (idx - j * nc) * 4;
          float4 u = make_float4(0.f, 0.f, 0.f, 0.f), pp = u;
          if (idx < total && k + 3 >= j) {
            const float* pu = U + (int64_t)j * a.uj + k;
            const float* ppp = (V == 1) ? P + (int64_t)j * a.uj + k : nullptr;
            if (vec && k + 3 < n) {
              u = *reinterpret_cast<const float4*>(pu);
              if (V == 1) pp = *reinterpret_cast<const float4*>(ppp);
            } else {
              if (k >= j && k < n) { u.x = pu[0]; if (V == 1) pp.x = ppp[0]; }
              if (k + 1 >= j && k + 1 < n) { u.y = pu[1]; if (V == 1) pp.y = ppp[1]; }
              if (k + 2 >= j && k + 2 < n) { u.z = pu[2]; if (V == 1) pp.z = ppp[2]; }
              if (k + 3 >= j && k + 3 < n) { u.w = pu[3]; if (V == 1) pp.w = ppp[3]; }
            }
          }
          uv[q] = u;
          if (V == 1) pv[q] = pp;
        }
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int idx = base + q * 256 + tid;
          const int j = idx / nc, k = (idx - j * nc) * 4;
          if (idx >= total) continue;
          const int t0 = tri_base(j, n);
          const float ue[4] = {uv[q].x, uv[q].y, uv[q].z, uv[q].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (k + e >= j && k + e < n) Us[t0 + k + e] = ue[e];
          }
          if (V == 1) {
            const float pe[4] = {pv[q].x, pv[q].y, pv[q].z, pv[q].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (k + e >= j && k + e < n) Ps[t0 + k + e] = pe[e];
            }
          }
        }
      }
    }
  }
  __syncthreads();
  if (tid < n) {
    const float d = Us[tri_base(tid, n) + tid];
    dg[tid] = d;
    rdiag[tid] = __fdiv_rn(1.f, d);
  }
  __syncthreads();

  const float* Win = a.W + b * a.wb + r * a.wr + cofs * a.wc;
  const float* Sp = a.S + b * a.sb + r * a.sr;
  const float* Zp = a.Z0 + b * a.sb + r * a.sr;
  const float* Zg = (V == 2) ? a.Zg + b * a.zb + r * a.zr + cofs * a.zc : nullptr;
  const float* GH = (V == 2) ? a.GH + b * a.gb + r * a.gr + cofs * a.gc : nullptr;
  float* GHo = (V == 2 && a.GHout) ? a.GHout + b * a.gb + r * a.gr + cofs * a.gc : nullptr;
  float* Qo = a.Q + b * a.qb + r * a.qr + cofs * a.qc;
  float* Io = a.I ? a.I + b * a.ib + r * a.ir + cofs * a.ic : nullptr;
  float* Eo = a.E ? a.E + b * a.eb + r * a.er + cofs * a.ec : nullptr;
  float* So = a.Sc ? a.Sc + b * a.cb + r * a.cr + cofs * a.cc : nullptr;
  float* E2 = (V == 2 && a.E2) ? a.E2 + b * a.e2b + r * a.e2r + cofs * a.e2c : nullptr;
  float* E3 = (V == 2 && a.E3) ? a.E3 + b * a.e3b + r * a.e3r + cofs * a.e2c : nullptr;
  const int* colgroup = a.colgroup ? a.colgroup + cofs : nullptr;
  const int64_t col0 = a.col0 + cofs;

  float fs = 0.f, fz = 0.f;  // fused group parameters of the current group

  for (int p0 = 0; p0 < n; p0 += PW) {
    if (F && p0 % (int)a.fuse == 0) {
      // find_params_kernel's fit of the group [p0, p0 + fuse) from the
      // block's input values (nothing in this kernel writes W): min and max
      // are exact in any order, NaN is tracked on the side.
      const int ge = min(p0 + (int)a.fuse, n);
      float mn = INFINITY, mx = -INFINITY;
      int nan = 0;
      if constexpr (L == 16) {
        // the lane's (at most eight) values loaded together, then reduced
        constexpr int KG = kMaxBlock / L;
        float v[KG];
#pragma unroll
        for (int k = 0; k < KG; ++k) {
          const int j = p0 + sub + L * k;
          v[k] = j < ge ? Win[(int64_t)j * a.wc] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < KG; ++k) {
          if (p0 + sub + L * k < ge) {
            nan |= (v[k] != v[k]);
            mn = fminf(mn, v[k]);
            mx = fmaxf(mx, v[k]);
          }
        }
      } else {
        for (int j = p0 + sub; j < ge; j += L) {
          const float v = Win[(int64_t)j * a.wc];
          nan |= (v != v);
          mn = fminf(mn, v);
          mx = fmaxf(mx, v);
        }
      }
#pragma unroll
      for (int o = L / 2; o > 0; o >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, o, L));
        mx = fmaxf(mx, __shfl_xor(mx, o, L));
        nan |= __shfl_xor(nan, o, L);
      }
      params_from_minmax(mn, mx, nan != 0, a.maxq, a.sym, fs, fz);
      if (act && sub == 0) {
        const int64_t gidx = (col0 + p0) / a.gsize;
        a.FS[b * a.sb + r * a.sr + gidx * a.sg] = fs;
        a.FZ[b * a.sb + r * a.sr + gidx * a.sg] = fz;
      }
    }
    // ---- panel inputs of the lane's NS columns -------------------------------
    float w[NS], gh[NS], sv[NS], zv[NS], zg[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int j = p0 + L * s + sub;
      if (F) {
        sv[s] = fs;
        zv[s] = fz;
      } else {
        int gidx = 0;
        if (colgroup) gidx = colgroup[j];
        else if (a.gsize > 0) gidx = (int)((int)col0 + j) / (int)a.gsize;
        sv[s] = Sp[(int64_t)gidx * a.sg];
        zv[s] = Zp[(int64_t)gidx * a.sg];
      }
      if (V == 2) zg[s] = Zg[(int64_t)j * a.zc];
    }
    // The panel's weights (and GH) as the earlier panels leave them: loaded
    // from the block's input (nothing in this kernel writes it) and updated
    // with the earlier panels' errors from LDS.  Called again, from opaque
    // copies of its index bases, when the panel is swept a second time.
    auto load_panel = [&](int sub, int rr, int p0) __attribute__((always_inline)) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int j = p0 + L * s + sub;
        w[s] = Win[(int64_t)j * a.wc];
        if (V == 2) gh[s] = GH[(int64_t)j * a.gc];
      }
      // Replay of the columns swept in earlier panels (LDS only), eight
      // columns at a time: their LDS operands are all read before the
      // updates, which then run in the reference's column order.  Sixteen
      // at a time where the registers allow (16 lanes per row, no P), so
      // fewer LDS round trips stay exposed; row j + 1 of the packed triangle
      // starts n − j − 1 entries after row j.
      constexpr int RB = (L == 16 && V != 1) ? 16 : 8;
      for (int j0 = 0; j0 < p0; j0 += RB) {
        float e[RB], t[RB], zj[RB], u[RB][NS], pu[RB][NS];
        const int row0 = tri_base(j0, n) + p0 + sub, step = n - j0 - 1;
#pragma unroll
        for (int q = 0; q < RB; ++q) {
          const int j = j0 + q;
          e[q] = e_s[j * RW + rr];
          if (V == 1) t[q] = t_s[j * RW + rr];
          if (V == 2) zj[q] = z_s[j * RW + rr];
          const int off = row0 + q * step - q * (q - 1) / 2;  // tri_base(j, n) + p0 + sub
          const float* Uj = Us + off;
          const float* Pj = (V == 1) ? Ps + off : nullptr;
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            u[q][s] = Uj[L * s];
            if (V == 1) pu[q][s] = Pj[L * s];
          }
        }
#pragma unroll
        for (int q = 0; q < RB; ++q) {
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            if (V == 0) {
              w[s] = __fsub_rn(w[s], __fmul_rn(u[q][s], e[q]));
            } else if (V == 1) {
              w[s] = __fadd_rn(__fsub_rn(w[s], __fmul_rn(u[q][s], e[q])), __fmul_rn(pu[q][s], t[q]));
            } else {
              w[s] = __fsub_rn(__fsub_rn(w[s], gh[s]), __fmul_rn(u[q][s], e[q]));
              gh[s] = __fsub_rn(gh[s], __fmul_rn(u[q][s], zj[q]));
            }
          }
        }
      }
    };
    load_panel(sub, rr, p0);
    // ---- sweep the panel column by column -----------------------------------
    // The panel's pivots and their reciprocals are read up front, and each
    // column's U row one column ahead, so the per-column dependency chain
    // (quantise, error, broadcast, update) never waits for LDS.
    float qb[NS], ib[NS], eb[NS], gb[NS], ysv[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) ysv[s] = __fdiv_rn(1.f, sv[s]);
    // The divisions of the column chain run as Markstein's sequence with no
    // per-column range test (a test and branch per division cost the chain
    // its scheduling).  After the panel each lane re-derives, for the columns
    // it owns, both divisions' operands and first quotients from the values
    // it kept (x, deq, gh) and tests their range; if any lane of the wave
    // fails, the wave reloads the panel and sweeps it again with
    // div_rn_recip, which takes the IEEE division where needed.  The results
    // therefore equal a sweep with div_rn_recip on every column.
    float xo[NS], xs[(V == 1) ? NS : 1];
    auto sweep_panel = [&](auto exact_tag, int sub, int rr, int p0) __attribute__((always_inline)) {
      constexpr bool EXACT = decltype(exact_tag)::value;
      float dcol[PW], ycol[PW];
#pragma unroll
      for (int q4 = 0; q4 < PW / 4; ++q4) {
        const float4 dv = *reinterpret_cast<const float4*>(&dg[p0 + 4 * q4]);
        const float4 yv = *reinterpret_cast<const float4*>(&rdiag[p0 + 4 * q4]);
        dcol[4 * q4] = dv.x; dcol[4 * q4 + 1] = dv.y; dcol[4 * q4 + 2] = dv.z; dcol[4 * q4 + 3] = dv.w;
        ycol[4 * q4] = yv.x; ycol[4 * q4 + 1] = yv.y; ycol[4 * q4 + 2] = yv.z; ycol[4 * q4 + 3] = yv.w;
      }
      float uc[NS], pc[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        uc[s] = Us[tri_base(p0, n) + p0 + sub + L * s];
        if (V == 1) pc[s] = Ps[tri_base(p0, n) + p0 + sub + L * s];
      }
#pragma unroll
      for (int jj = 0; jj < PW; ++jj) {
        const int sl = jj / L, o = jj % L;
        const bool own = sub == o;
        const int j = p0 + jj;
        float un[NS], pn[NS];
        if (jj + 1 < PW) {
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            un[s] = Us[tri_base(j + 1, n) + p0 + sub + L * s];
            if (V == 1) pn[s] = Ps[tri_base(j + 1, n) + p0 + sub + L * s];
          }
        }
        const float x = w[sl];  // meaningful on the owner lane
        const float sc = sv[sl];
        const float z0 = zv[sl];
        const float t = EXACT ? div_rn_recip(x, sc, ysv[sl]) : div_markstein(x, sc, ysv[sl]);
        // The fast pass clamps with max/min (no compare-and-select hazard on
        // the column chain): they differ from the NaN-propagating clamp only
        // for a NaN, and a NaN anywhere in a column's quotients fails the
        // owner's range test after the panel, which sweeps the panel again
        // with the exact pass.
        const float qv = __fadd_rn(rintf(t), z0);
        const float q = EXACT ? clamp_nan(qv, minq, fmaxq) : fminf(fmaxf(qv, minq), fmaxq);
        const float deq = __fmul_rn(sc, __fsub_rn(q, z0));
        const float d = dcol[jj];
        const float yd = ycol[jj];
        const float a2 = (V == 2) ? __fsub_rn(__fsub_rn(x, deq), gh[sl]) : __fsub_rn(x, deq);
        const float err0 = EXACT ? div_rn_recip(a2, d, yd) : div_markstein(a2, d, yd);
        const float err = group_bcast<L>(err0, o);
        const float xb = (V == 1 || jj == PW - 1) ? group_bcast<L>(x, o) : 0.f;
        const float zj = (V == 2) ? group_bcast<L>(zg[sl], o) : 0.f;
        bad |= own && !(sc > 0.f);
        qb[sl] = own ? deq : qb[sl];
        ib[sl] = own ? q : ib[sl];
        eb[sl] = own ? err0 : eb[sl];
        if (!EXACT) xo[sl] = own ? x : xo[sl];
        if (V == 1) xs[sl] = own ? x : xs[sl];
        if (V == 2) gb[sl] = own ? gh[sl] : gb[sl];
        if (jj == PW - 1) last_x = xb;
        // With 16 lanes every column of a slot that is not wholly done takes
        // the update, the done ones too (the owner's and earlier columns):
        // nothing reads their values again, and no lane mask is needed.  (A
        // quad per row measured faster with the mask.)
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          if (L * s + L - 1 <= jj) continue;       // every column of the slot is done
          const bool upd = L == 16 || L * s > jj || sub > jj - L * s;
          const float u = uc[s];
          if (V == 0) {
            const float nw = __fsub_rn(w[s], __fmul_rn(u, err));
            w[s] = upd ? nw : w[s];
          } else if (V == 1) {
            const float nw = __fadd_rn(__fsub_rn(w[s], __fmul_rn(u, err)), __fmul_rn(pc[s], xb));
            w[s] = upd ? nw : w[s];
          } else {
            const float nw = __fsub_rn(__fsub_rn(w[s], gh[s]), __fmul_rn(u, err));
            const float ng = __fsub_rn(gh[s], __fmul_rn(u, zj));
            w[s] = upd ? nw : w[s];
            gh[s] = upd ? ng : gh[s];
          }
        }
        if (jj + 1 < PW) {
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            uc[s] = un[s];
            if (V == 1) pc[s] = pn[s];
          }
        }
      }
    };
    // (16 lanes per row only: with a quad per row the owned values kept for
    // the test cost the second wave per SIMD.)
    if constexpr (L != 16) {
      sweep_panel(ExactTag<true>{}, sub, rr, p0);
    } else {
      sweep_panel(ExactTag<false>{}, sub, rr, p0);
      bool inexact = false;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int c = p0 + L * s + sub;
        const float a1 = xo[s];
        const float a2 = (V == 2) ? __fsub_rn(__fsub_rn(a1, qb[s]), gb[s]) : __fsub_rn(a1, qb[s]);
        inexact |= !recip_div_exact(a1, __fmul_rn(a1, ysv[s]), ysv[s]) ||
                   !recip_div_exact(a2, __fmul_rn(a2, rdiag[c]), rdiag[c]);
      }
      if (__builtin_amdgcn_ballot_w64(inexact) != 0) {
        // The second sweep recomputes its addresses from opaque copies of
        // their bases and reloads its operands: keeping the first pass's
        // addresses and loads live for it would cost a wave's worth of
        // registers.
        int sub2 = sub, rr2 = rr, p02 = p0;
        asm volatile("" : "+v"(sub2), "+v"(rr2), "+s"(p02)::"memory");
        load_panel(sub2, rr2, p02);
        sweep_panel(ExactTag<true>{}, sub2, rr2, p02);
      }
    }
    // The panel's errors (and GPTAQ's x, G2PTQ's z), read by the replay of
    // later panels and by the near tails: each lane stores the columns it
    // owns, once, after the panel (the column chain broadcasts them between
    // lanes and never reads them back from LDS).
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int j = p0 + L * s + sub;
      e_s[j * RW + rr] = eb[s];
      if (V == 1) t_s[j * RW + rr] = xs[s];
      if (V == 2) z_s[j * RW + rr] = zg[s];
    }
    // ---- panel outputs ------------------------------------------------------
    if (act) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int j = p0 + L * s + sub;
        Qo[(int64_t)j * a.qc] = qb[s];
        if (Io) Io[(int64_t)j * a.ic] = ib[s];
        if (Eo) Eo[(int64_t)j * a.ec] = eb[s];
        if (So) So[(int64_t)j * a.cc] = sv[s];
        if (V == 2 && E2) E2[(int64_t)j * a.e2c] = __fsub_rn(eb[s], __fmul_rn(zg[s], (float)(a.dist0 - j)));
        if (V == 2 && E3) E3[(int64_t)j * a.e2c] = __fsub_rn(eb[s], __fmul_rn(zg[s], (float)(a.dist3 - j)));
        if (V == 2 && GHo) GHo[(int64_t)j * a.gc] = gb[s];
      }
    }
  }
    if (SBM && bi + 1 < nblk) {
      // Near tail of the super-block: W[row, c] −= Σ_k e_k·U[cofs + k, c] for
      // the columns c of the later blocks, 64 at a time (the triangle's LDS
      // holds the U slab, k-major), four consecutive columns per lane.
      float* Wr = a.Wsb + b * a.wb + r * a.wr;
      const float* Ub = a.U + b * a.ub + cofs * a.uj;
      // A thread's eight 16-byte pieces of a slab are all loaded before any
      // is stored: one memory round trip per slab, not eight.
      static_assert(kMaxBlock * 16 == 8 * 256, "a slab is eight 16-byte pieces per thread");
      // thread tid's piece i: row k = tid/16 + 16i of the slab, columns 4·(tid%16)..+3
      const int k0 = tid >> 4, c4 = (tid & 15) * 4;
      for (int c0 = (int)cofs + kMaxBlock; c0 < nblk * kMaxBlock; c0 += 64) {
        const float* us = Ub + (int64_t)k0 * a.uj + c0 + c4;
        const int64_t st16 = 16 * a.uj;
#define G2_LDU(i) const float4 u##i = *reinterpret_cast<const float4*>(us + (i) * st16)
        G2_LDU(0); G2_LDU(1); G2_LDU(2); G2_LDU(3); G2_LDU(4); G2_LDU(5); G2_LDU(6); G2_LDU(7);
#undef G2_LDU
        __syncthreads();  // the sweep's (or the previous slab's) LDS reads are done
        float* ud = &Us[k0 * 64 + c4];
#define G2_STU(i) *reinterpret_cast<float4*>(ud + (i) * 16 * 64) = u##i
        G2_STU(0); G2_STU(1); G2_STU(2); G2_STU(3); G2_STU(4); G2_STU(5); G2_STU(6); G2_STU(7);
#undef G2_STU
        __syncthreads();
        if (act) {
          float4 w = *reinterpret_cast<const float4*>(Wr + c0 + 4 * sub);
          float t[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll 4
          for (int k = 0; k < kMaxBlock; k += 2) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const float e = e_s[(k + h) * RW + rr];
              const float4 u = *reinterpret_cast<const float4*>(&Us[(k + h) * 64 + 4 * sub]);
              t[h][0] = __builtin_fmaf(e, u.x, t[h][0]);
              t[h][1] = __builtin_fmaf(e, u.y, t[h][1]);
              t[h][2] = __builtin_fmaf(e, u.z, t[h][2]);
              t[h][3] = __builtin_fmaf(e, u.w, t[h][3]);
            }
          }
          w.x = __fsub_rn(w.x, __fadd_rn(t[0][0], t[1][0]));
          w.y = __fsub_rn(w.y, __fadd_rn(t[0][1], t[1][1]));
          w.z = __fsub_rn(w.z, __fadd_rn(t[0][2], t[1][2]));
          w.w = __fsub_rn(w.w, __fadd_rn(t[0][3], t[1][3]));
          *reinterpret_cast<float4*>(Wr + c0 + 4 * sub) = w;
        }
      }
    }
    if (SBM) __syncthreads();  // the next block's staging overwrites the LDS
  }  // block bi of the super-block
  const int rr = threadIdx.x / L, sub = threadIdx.x % L;
  const int64_t r0 = (int64_t)blockIdx.x * RW + rr;
  const bool act = r0 < a.R;
  if (V == 1 && a.CW && act && sub == 0) a.CW[b * a.cwb + r0 * a.cwr] = last_x;
  if (bad && act && a.flags) atomicOr(a.flags, FLAG_BAD_SCALE);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Whether every per-row operand is column-contiguous with 16-byte aligned rows.
bool sweep_vec_ok(const SweepArgs& a) {
  if (a.n % 32 != 0) return false;
  auto ok = [](const void* p, int64_t sb, int64_t sr, int64_t sc) {
    return p == nullptr || (sc == 1 && sr % 4 == 0 && sb % 4 == 0 && aligned16(p));
  };
  return ok(a.W, a.wb, a.wr, a.wc) && ok(a.Q, a.qb, a.qr, a.qc) && ok(a.I, a.ib, a.ir, a.ic) &&
         ok(a.E, a.eb, a.er, a.ec) && ok(a.Sc, a.cb, a.cr, a.cc) &&
         ok(a.E2, a.e2b, a.e2r, a.e2c) && ok(a.E3, a.e3b, a.e3r, a.e2c) &&
         ok(a.GH, a.gb, a.gr, a.gc) && a.GHout == nullptr;
}

// 16 lanes per row up to 16384 rows in the launch (four waves per SIMD at
// two resident), a quad of lanes beyond: measured on GPTQ loops of 4096
// columns, 16 lanes were 6–9 % faster at 12288 and 14336 rows and 12 % slower
// at 28672 (GPTAQ loops: 10–13 % slower at 28672 and 57344).  G2PTQ takes 16
// lanes at any row count (launch_variant).
bool lanes16(int64_t B, int64_t R) { return B * R <= 16384; }

template <int V>
void launch_variant(hipStream_t stream, const SweepArgs& a, dim3 grid, bool vec) {
  const bool full = (a.n % 32) == 0;
  if (full) {
    // 16 lanes per row while that keeps the block within about two waves per
    // SIMD (1024 SIMDs), else a quad per row.  G2PTQ always takes 16 lanes:
    // its quad sweep needs 312–328 VGPRs (one workgroup per CU) where 16
    // lanes need 244–249 (two), and its loops of 4096 columns ran 9–17 %
    // faster with 16 lanes at 20000, 28672 and 57344 rows.
    if (V == 2 || lanes16(grid.y, a.R)) {
      dim3 g16((unsigned)cdiv(a.R, (int64_t)16), grid.y);
      if constexpr (V == 0) {
        if (a.nblk > 1) {
          if (a.fuse > 0)
            hipLaunchKernelGGL((sweep4_kernel<V, 16, true, true>), g16, dim3(256), 0, stream, a);
          else
            hipLaunchKernelGGL((sweep4_kernel<V, 16, false, true>), g16, dim3(256), 0, stream, a);
          return;
        }
      }
      if (a.fuse > 0)
        hipLaunchKernelGGL((sweep4_kernel<V, 16, true>), g16, dim3(256), 0, stream, a);
      else
        hipLaunchKernelGGL((sweep4_kernel<V, 16, false>), g16, dim3(256), 0, stream, a);
    } else if constexpr (V != 2) {
      dim3 g4((unsigned)cdiv(a.R, (int64_t)64), grid.y);
      if (a.fuse > 0)
        hipLaunchKernelGGL((sweep4_kernel<V, 4, true>), g4, dim3(256), 0, stream, a);
      else
        hipLaunchKernelGGL((sweep4_kernel<V, 4, false>), g4, dim3(256), 0, stream, a);
    }
    return;
  }
  if (vec && full)
    hipLaunchKernelGGL((sweep_kernel<V, 32, true, true>), grid, dim3(64), 0, stream, a);
  else if (full)
    hipLaunchKernelGGL((sweep_kernel<V, 32, false, true>), grid, dim3(64), 0, stream, a);
  else
    hipLaunchKernelGGL((sweep_kernel<V, 32, false, false>), grid, dim3(64), 0, stream, a);
}

}  // namespace

bool sweep_superblock_ok(const SweepArgs& a, int64_t B) {
  return a.n == kMaxBlock && lanes16(B, a.R) && sweep_vec_ok(a) && a.uj % 4 == 0 &&
         aligned16(a.U) && a.P == nullptr && a.Zg == nullptr;
}

int launch_sweep(hipStream_t stream, int variant, const SweepArgs& a, int64_t B) {
  G2PTQ_CHECK(a.n >= 1 && a.n <= kMaxBlock, "block sweep: block width %d not in [1, %d]", a.n,
              kMaxBlock);
  if (a.R <= 0 || B <= 0) return G2PTQ_OK;
  G2PTQ_CHECK(B < 65536, "block sweep: batch too large");
  G2PTQ_CHECK(a.fuse == 0 || (a.n % 32 == 0 && a.fuse % 32 == 0 && a.gsize == a.fuse &&
                              a.col0 % a.fuse == 0 && a.colgroup == nullptr && a.FS && a.FZ),
              "block sweep: fused group parameters need 32-column panels and aligned groups");
  dim3 grid((unsigned)cdiv(a.R, 64), (unsigned)B);
  const bool vec = sweep_vec_ok(a);
  G2PTQ_CHECK(a.nblk <= 1 || (variant == G2PTQ_VARIANT_GPTQ && sweep_superblock_ok(a, B) &&
                              a.Wsb == a.W && a.nblk * kMaxBlock <= 1 << 20),
              "block sweep: a super-block launch needs GPTQ, full blocks and 16 lanes per row");
  switch (variant) {
    case G2PTQ_VARIANT_GPTQ:
      launch_variant<0>(stream, a, grid, vec);
      break;
    case G2PTQ_VARIANT_GPTAQ:
      G2PTQ_CHECK(a.P != nullptr, "GPTAQ sweep needs P");
      launch_variant<1>(stream, a, grid, vec);
      break;
    case G2PTQ_VARIANT_G2PTQ:
      G2PTQ_CHECK(a.Zg != nullptr && a.GH != nullptr, "G2PTQ sweep needs z and ghinv");
      launch_variant<2>(stream, a, grid, vec);
      break;
    default:
      G2PTQ_CHECK(false, "unknown compensation variant %d", variant);
  }
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

int launch_find_params(hipStream_t stream, const float* x, int64_t rows, int64_t cols, int64_t ldx,
                       int maxq, int sym, float* scale, float* zero, int64_t ldp, int* flags) {
  if (rows <= 0) return G2PTQ_OK;
  G2PTQ_CHECK(cols > 0, "find_params: empty group");
  const int64_t threads = rows * 16;
  hipLaunchKernelGGL(find_params_kernel, dim3((unsigned)cdiv(threads, 256)), dim3(256), 0, stream,
                     x, rows, cols, ldx, maxq, sym, scale, zero, ldp, flags);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

int launch_find_params_mse(hipStream_t stream, const float* x, int64_t rows, int64_t cols,
                           int64_t ldx, int maxq, int sym, float norm, int grid, float maxshrink,
                           const HDiag& hd, float* scale, float* zero, int64_t ldp, int* flags) {
  G2PTQ_CHECK(grid > 0, "find_params_mse: grid must be positive");
  if (rows <= 0) return G2PTQ_OK;
  G2PTQ_CHECK(cols > 0, "find_params_mse: empty group");
  G2PTQ_CHECK(rows < (1ll << 31), "find_params_mse: too many rows");
  if (hd.h) {
    G2PTQ_CHECK(hd.nblocks >= 1 && hd.gpr >= 1 && hd.ld >= hd.gpr * cols,
                "find_params_mse: bad H_diag layout (%lld blocks, %lld groups per row, ld %lld)",
                (long long)hd.nblocks, (long long)hd.gpr, (long long)hd.ld);
    G2PTQ_CHECK(rows % hd.gpr == 0 && (rows / hd.gpr) % hd.nblocks == 0,
                "find_params_mse: %lld rows do not split into %lld H_diag blocks",
                (long long)(rows / hd.gpr), (long long)hd.nblocks);
  }
  // int(self.maxshrink * self.grid) with Python's float product.
  const int steps = (int)((double)maxshrink * (double)grid);
  hipLaunchKernelGGL(find_params_mse_kernel, dim3((unsigned)rows), dim3(64), 0, stream, x, rows,
                     cols, ldx, maxq, sym, norm, grid, steps, hd, scale, zero, ldp, flags);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

}  // namespace g2ptq

using namespace g2ptq;

extern "C" int g2ptq_find_params(void* stream, const float* x, int64_t rows, int64_t cols,
                                 int64_t ldx, int bits, int sym, float* scale, float* zero,
                                 int64_t ldp, int* flags) {
  G2PTQ_CHECK(bits >= 2 && bits <= 16, "find_params: bits=%d unsupported", bits);
  G2PTQ_CHECK(x && scale && zero, "find_params: null pointer");
  const int maxq = (1 << (bits - 1)) - 1;
  return launch_find_params(as_stream(stream), x, rows, cols, ldx, maxq, sym, scale, zero, ldp,
                            flags);
}

extern "C" int g2ptq_find_params_mse(void* stream, const float* x, int64_t rows, int64_t cols,
                                     int64_t ldx, int bits, int sym, float norm, int grid,
                                     float maxshrink, const float* hdiag, int64_t ldh,
                                     int64_t hblocks, int64_t groups_per_row, float* scale,
                                     float* zero, int64_t ldp, int* flags) {
  G2PTQ_CHECK(bits >= 2 && bits <= 16, "find_params_mse: bits=%d unsupported", bits);
  G2PTQ_CHECK(x && scale && zero, "find_params_mse: null pointer");
  const int maxq = (1 << (bits - 1)) - 1;
  HDiag hd;
  hd.h = hdiag; hd.ld = ldh; hd.nblocks = hblocks; hd.gpr = groups_per_row;
  return launch_find_params_mse(as_stream(stream), x, rows, cols, ldx, maxq, sym, norm, grid,
                                maxshrink, hd, scale, zero, ldp, flags);
}

extern "C" int g2ptq_fake_quantize(void* stream, const float* x, int64_t rows, int64_t cols,
                                   int64_t ldx, int64_t groupsize, const float* scale,
                                   const float* zero, int64_t ldp, int bits, float* q_out,
                                   int64_t ldq, float* int_out, int64_t ldi, int* flags) {
  (void)flags;
  G2PTQ_CHECK(bits >= 2 && bits <= 16, "fake_quantize: bits=%d unsupported", bits);
  G2PTQ_CHECK(x && scale && zero && q_out, "fake_quantize: null pointer");
  if (rows <= 0 || cols <= 0) return G2PTQ_OK;
  const int maxq = (1 << (bits - 1)) - 1;
  const int64_t n = rows * cols;
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(n, 256), 65536);
  hipLaunchKernelGGL(fake_quantize_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), x, rows,
                     cols, ldx, groupsize, scale, zero, ldp, maxq, q_out, ldq, int_out, ldi);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

extern "C" int g2ptq_block_sweep(void* stream, int variant, int64_t B, int64_t bs, int64_t R,
                                 int maxq, float* weight, const float* hinv, const float* p,
                                 const float* scale, const float* zero, const float* z,
                                 float* ghinv, float* column_weight, float* int_weight,
                                 float* error, int* flags) {
  G2PTQ_CHECK(weight && hinv && scale && zero && int_weight && error,
              "block_sweep: null pointer");
  // Transposed block layout (B, bs, R): element (b, row r, column j) at b*bs*R + j*R + r.
  SweepArgs a{};
  a.R = R;
  a.n = (int)bs;
  a.maxq = maxq;
  const int64_t sb = bs * R;
  a.W = weight; a.wb = sb; a.wr = 1; a.wc = R;
  a.U = hinv; a.ub = bs * bs; a.uj = bs;
  a.P = p;
  a.Zg = z; a.zb = sb; a.zr = 1; a.zc = R;
  a.GH = ghinv; a.GHout = ghinv; a.gb = sb; a.gr = 1; a.gc = R;
  // Per-element scale/zero: use the column index as the "group".
  a.S = scale; a.Z0 = zero; a.sb = sb; a.sr = 1; a.sg = R;
  a.colgroup = nullptr; a.col0 = 0; a.gsize = 1;
  a.Q = weight; a.qb = sb; a.qr = 1; a.qc = R;
  a.I = int_weight; a.ib = sb; a.ir = 1; a.ic = R;
  a.E = error; a.eb = sb; a.er = 1; a.ec = R;
  a.Sc = nullptr;
  a.CW = column_weight; a.cwb = R; a.cwr = 1;
  a.E2 = nullptr;
  a.flags = flags;
  return launch_sweep(as_stream(stream), variant, a, B);
}
