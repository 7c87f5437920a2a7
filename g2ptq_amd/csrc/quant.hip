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

// NaN-propagating clamp (torch.clamp semantics).
__device__ __forceinline__ float clamp_nan(float v, float lo, float hi) {
  return v < lo ? lo : (v > hi ? hi : v);
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
// sum(|fq - x|^norm); a candidate replaces the incumbent only when strictly
// better, scanning i-major exactly like the reference loop.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void find_params_mse_kernel(const float* __restrict__ x,
                                                             int64_t rows, int64_t cols,
                                                             int64_t ldx, int maxq, int sym,
                                                             float norm, int grid, int steps,
                                                             float* scale, float* zero,
                                                             int64_t ldp, int* flags) {
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  const float* xr = x + row * ldx;
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
        err += powf(fabsf(__fsub_rn(fq, v)), norm);
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
// columns.  The block is walked in panels of PW columns whose values live in
// VGPRs; updates from earlier panels are replayed from the per-lane error
// history kept in LDS, in increasing column order, so every element sees the
// reference's exact sequence of updates.  U (and P) rows are wave-uniform and
// read through the scalar path.
// ---------------------------------------------------------------------------
template <int V, int PW>
__global__ __launch_bounds__(64) void sweep_kernel(SweepArgs a) {
  __shared__ float e_s[kMaxBlock * 64];
  __shared__ float t_s[(V == 1) ? kMaxBlock * 64 : 1];

  const int lane = threadIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t r0 = (int64_t)blockIdx.x * 64 + lane;
  const bool act = r0 < a.R;
  const int64_t r = act ? r0 : 0;
  const int n = a.n;
  const float minq = (float)(-(a.maxq + 1)), fmaxq = (float)a.maxq;

  const float* __restrict__ U = a.U + b * a.ub;
  const float* __restrict__ P = (V == 1) ? a.P + b * a.ub : nullptr;
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

  int bad = 0;
  float last_x = 0.f;

  for (int p0 = 0; p0 < n; p0 += PW) {
    const int np = min(PW, n - p0);
    float w[PW], gh[PW];
#pragma unroll
    for (int kk = 0; kk < PW; ++kk) {
      w[kk] = (kk < np) ? Win[(int64_t)(p0 + kk) * a.wc] : 0.f;
      if (V == 2) gh[kk] = (kk < np) ? GH[(int64_t)(p0 + kk) * a.gc] : 0.f;
    }
    // Replay updates of the columns already swept in earlier panels.
    for (int j = 0; j < p0; ++j) {
      const float e = e_s[j * 64 + lane];
      float t = 0.f, zj = 0.f;
      if (V == 1) t = t_s[j * 64 + lane];
      if (V == 2) zj = Zg[(int64_t)j * a.zc];
      const float* Uj = U + (int64_t)j * a.uj + p0;
      const float* Pj = (V == 1) ? P + (int64_t)j * a.uj + p0 : nullptr;
#pragma unroll
      for (int kk = 0; kk < PW; ++kk) {
        if (kk < np) {
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
    // Sweep this panel column by column.
#pragma unroll
    for (int jj = 0; jj < PW; ++jj) {
      if (jj < np) {
        const int j = p0 + jj;
        const float x = w[jj];
        const int64_t gidx = a.colgroup ? a.colgroup[j]
                                        : (a.gsize > 0 ? (int64_t)(a.col0 + j) / a.gsize : 0);
        const float s = Sp[gidx * a.sg];
        const float z0 = Zp[gidx * a.sg];
        const float q = clamp_nan(__fadd_rn(rintf(__fdiv_rn(x, s)), z0), minq, fmaxq);
        const float deq = __fmul_rn(s, __fsub_rn(q, z0));
        const float d = U[(int64_t)j * a.uj + j];
        float err;
        float zj = 0.f;
        if (V == 2) {
          err = __fdiv_rn(__fsub_rn(__fsub_rn(x, deq), gh[jj]), d);
          zj = Zg[(int64_t)j * a.zc];
        } else {
          err = __fdiv_rn(__fsub_rn(x, deq), d);
        }
        bad |= !(s > 0.f);
        if (act) {
          Qo[(int64_t)j * a.qc] = deq;
          if (Io) Io[(int64_t)j * a.ic] = q;
          if (Eo) Eo[(int64_t)j * a.ec] = err;
          if (So) So[(int64_t)j * a.cc] = s;
          if (V == 2) {
            if (GHo) GHo[(int64_t)j * a.gc] = gh[jj];
            if (E2) E2[(int64_t)j * a.e2c] = __fsub_rn(err, __fmul_rn(zj, (float)(a.dist0 - j)));
          }
        }
        e_s[j * 64 + lane] = err;
        if (V == 1) t_s[j * 64 + lane] = x;
        last_x = x;
        const float* Uj = U + (int64_t)j * a.uj + p0;
        const float* Pj = (V == 1) ? P + (int64_t)j * a.uj + p0 : nullptr;
#pragma unroll
        for (int kk = jj + 1; kk < PW; ++kk) {
          if (kk < np) {
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
  }
  if (V == 1 && a.CW && act) a.CW[b * a.cwb + r * a.cwr] = last_x;
  if (bad && act && a.flags) atomicOr(a.flags, FLAG_BAD_SCALE);
}

}  // namespace

int launch_sweep(hipStream_t stream, int variant, const SweepArgs& a, int64_t B) {
  G2PTQ_CHECK(a.n >= 1 && a.n <= kMaxBlock, "block sweep: block width %d not in [1, %d]", a.n,
              kMaxBlock);
  if (a.R <= 0 || B <= 0) return G2PTQ_OK;
  G2PTQ_CHECK(B < 65536, "block sweep: batch too large");
  dim3 grid((unsigned)cdiv(a.R, 64), (unsigned)B);
  switch (variant) {
    case G2PTQ_VARIANT_GPTQ:
      hipLaunchKernelGGL((sweep_kernel<0, 32>), grid, dim3(64), 0, stream, a);
      break;
    case G2PTQ_VARIANT_GPTAQ:
      G2PTQ_CHECK(a.P != nullptr, "GPTAQ sweep needs P");
      hipLaunchKernelGGL((sweep_kernel<1, 32>), grid, dim3(64), 0, stream, a);
      break;
    case G2PTQ_VARIANT_G2PTQ:
      G2PTQ_CHECK(a.Zg != nullptr && a.GH != nullptr, "G2PTQ sweep needs z and ghinv");
      hipLaunchKernelGGL((sweep_kernel<2, 32>), grid, dim3(64), 0, stream, a);
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
                           float* scale, float* zero, int64_t ldp, int* flags) {
  G2PTQ_CHECK(grid > 0, "find_params_mse: grid must be positive");
  if (rows <= 0) return G2PTQ_OK;
  G2PTQ_CHECK(cols > 0, "find_params_mse: empty group");
  G2PTQ_CHECK(rows < (1ll << 31), "find_params_mse: too many rows");
  // int(self.maxshrink * self.grid) with Python's float product.
  const int steps = (int)((double)maxshrink * (double)grid);
  hipLaunchKernelGGL(find_params_mse_kernel, dim3((unsigned)rows), dim3(64), 0, stream, x, rows,
                     cols, ldx, maxq, sym, norm, grid, steps, scale, zero, ldp, flags);
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
                                     float maxshrink, float* scale, float* zero, int64_t ldp,
                                     int* flags) {
  G2PTQ_CHECK(bits >= 2 && bits <= 16, "find_params_mse: bits=%d unsupported", bits);
  G2PTQ_CHECK(x && scale && zero, "find_params_mse: null pointer");
  const int maxq = (1 << (bits - 1)) - 1;
  return launch_find_params_mse(as_stream(stream), x, rows, cols, ldx, maxq, sym, norm, grid,
                                maxshrink, scale, zero, ldp, flags);
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
