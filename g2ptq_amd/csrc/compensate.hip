// Per-layer lazy-batch compensation driver, GPTAQ's P and the G2PTQ trust region.
//
// The block loop stays on the host (it is a dependency chain of kernels);
// each block is: fit the parameters of groups that start in the block
// (dynamic groups; min/max groups that tile the block in 32-column multiples
// are fitted by the sweep itself) → fused sweep (one launch for every row of
// every layer in the batch) → block-tail update of the remaining columns as
// fp32 MFMA GEMMs.
#include <mutex>
#include <numeric>

#include "sweep.hpp"

namespace g2ptq {
namespace {

size_t al256(size_t x) { return (x + 255) / 256 * 256; }

// GPTAQ: zero the lower triangle including the diagonal (torch.triu(t, 1)).
__global__ void triu1_kernel(float* t, int64_t C) {
  const int64_t b = blockIdx.z;
  const int64_t i = (int64_t)blockIdx.y * 16 + (threadIdx.x >> 4);
  const int64_t j0 = (int64_t)blockIdx.x * 64;
  if (i >= C) return;
  float* tb = t + b * C * C;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t j = j0 + (threadIdx.x & 15) + 16 * q;
    if (j < C && j <= i) tb[i * C + j] = 0.f;
  }
}

// Ut[j][i] = U[i][j] for the 64×64 tiles on and above U's diagonal (Ut's
// tiles below its diagonal are not written): the block tails read the
// factor as N×K rows, k-contiguous, which the GEMM stages and splits once
// per workgroup (faster than splitting a K×N operand per wave).
__global__ __launch_bounds__(256) void transpose_upper_kernel(const float* __restrict__ U,
                                                              int64_t C, float* __restrict__ Ut) {
  const int64_t bi = blockIdx.y, bj = blockIdx.x, b = blockIdx.z;
  if (bi > bj) return;
  __shared__ float t[64][65];
  const float* Ub = U + b * C * C;
  float* Tb = Ut + b * C * C;
  const int c = threadIdx.x & 63, r0 = threadIdx.x >> 6;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int r = r0 + 4 * q;
    const int64_t i = bi * 64 + r, j = bj * 64 + c;
    t[r][c] = (i < C && j < C) ? Ub[i * C + j] : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int r = r0 + 4 * q;
    const int64_t j = bj * 64 + r, i = bi * 64 + c;
    if (i < C && j < C) Tb[j * C + i] = t[c][r];
  }
}

// diag(A⁻¹)[c] = Σ_i U[i][c]² (A⁻¹ = UᵀU): a workgroup per 64 columns,
// four row phases per column (rows i ≡ p mod 4, four loads in flight per
// thread), the phases summed in a fixed order.
__global__ __launch_bounds__(256) void inv_diag_kernel(const float* __restrict__ U, int64_t C,
                                                       float* dA) {
  __shared__ float part[4][64];
  const int64_t b = blockIdx.y;
  const int cl = threadIdx.x & 63, ph = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + cl;
  const float* Ub = U + b * C * C;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  if (c < C) {
    int64_t i = ph;
    for (; i + 12 <= c; i += 16) {
      const float u0 = Ub[i * C + c], u1 = Ub[(i + 4) * C + c];
      const float u2 = Ub[(i + 8) * C + c], u3 = Ub[(i + 12) * C + c];
      s0 += u0 * u0; s1 += u1 * u1; s2 += u2 * u2; s3 += u3 * u3;
    }
    for (; i <= c; i += 4) {
      const float u = Ub[i * C + c];
      s0 += u * u;
    }
  }
  part[ph][cl] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (ph == 0 && c < C)
    dA[b * C + c] = (part[0][cl] + part[1][cl]) + (part[2][cl] + part[3][cl]);
}

__device__ float block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s += red[i];
  return s;
}

// One workgroup per output row of a row group: β from the row statistics,
// then Z = β·T1 and GH = β·GA in place (Z holds T1, GH holds GA on entry).
__global__ __launch_bounds__(256) void trust_row_kernel(const float* __restrict__ Grad,
                                                        const float* __restrict__ Q0,
                                                        const float* __restrict__ W0,
                                                        const float* __restrict__ dA, int64_t Rg,
                                                        int64_t C, float two_alpha, float* beta,
                                                        float* Z, float* GH) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;  // over BG*Rg
  const int64_t bg = row / Rg;
  const float* g = Grad + row * C;
  const float* q0 = Q0 + row * C;
  const float* w0 = W0 + row * C;
  const float* da = dA + bg * C;
  float* z = Z + row * C;
  float* gh = GH + row * C;
  float cs = 0.f;
  for (int64_t j = threadIdx.x; j < C; j += 256) cs += g[j] * gh[j];
  const float crow = block_sum(cs, red);
  const float tiny = 1.17549435e-38f;  // torch.finfo(torch.float32).tiny
  float bs = 0.f;
  for (int64_t j = threadIdx.x; j < C; j += 256) {
    const float ga = gh[j], d = da[j];
    const float e = q0[j] - w0[j];
    const float loss = fabsf((e * ga + (e * e) / 2.f) / d);
    const float tl = two_alpha * loss;
    float c = crow - (ga * ga) / d;
    c = c < tl ? tl : c;
    c = c < tiny ? tiny : c;
    float u = 1.f - tl / c;
    u = u < 0.f ? 0.f : u;
    bs += 1.f - sqrtf(u);
  }
  const float bsum = block_sum(bs, red);
  const float bt = bsum / (float)C;
  if (threadIdx.x == 0) beta[row] = bt;
  for (int64_t j = threadIdx.x; j < C; j += 256) {
    z[j] = z[j] * bt;
    gh[j] = gh[j] * bt;
  }
}

}  // namespace
}  // namespace g2ptq

using namespace g2ptq;

// Columns per super-block of the compensation loop.  Inside a super-block the
// tail of every 128-column block is applied right away to the super-block's
// remaining columns (K = bs); the columns after it receive the errors of the
// whole super-block in one product (K = super-block width).  This is the
// reference's right-looking update regrouped: every column still receives
// every earlier block's error term before it is quantized, and a dynamic
// group never straddles a super-block boundary (the width is a multiple of
// the group size), so find_params sees the same, fully updated columns.
// G2PTQ's block tail also subtracts bs·GH with a GH that every block's own
// tail updates (GH −= Z_b·U_b).  Summed over the m blocks of a super-block,
// the columns after it receive
//   m·bs·GH₀ + Σ_b (E2_b − bs·(m−1−b)·Z_b)·U_b   and   GH −= Σ_b Z_b·U_b,
// with GH₀ their GH at the super-block's start (the blocks' own tails touch
// only the super-block's columns) and E2_b = err − z·(bs−1−j) the block
// operand of g2ptq_utils.py:329-346: so the sweep also writes
// E3_b = err − z·(bs−1−j + bs·(m−1−b)), and the far tail is one K = m·bs
// product with γ = −m·bs, like the other variants'.
static int64_t super_block(int variant, int64_t bs, int64_t groupsize, int static_groups) {
  (void)variant;
  int64_t unit = bs;
  if (groupsize > 0 && !static_groups) unit = bs / std::gcd(bs, groupsize) * groupsize;
  return unit >= 512 ? unit : unit * (512 / unit);
}

extern "C" int g2ptq_compensate_workspace(int variant, int64_t B, int64_t R, int64_t C,
                                          int64_t blocksize, size_t* bytes) {
  G2PTQ_CHECK(bytes != nullptr, "compensate_workspace: null out");
  // The super-block width depends on the group layout; size for the widest
  // (a dynamic group size that is coprime to the block size is bounded by C),
  // three times: the error columns of consecutive super-blocks rotate over
  // three buffers so that the far tails of the two before run on the side
  // stream while the next is swept.
  // G2PTQ adds one block's near-tail operand (E2, below).
  // Then the factor transposed (Ut, B·C² floats), which lets every block
  // tail read it k-contiguous.
  const int64_t bs = std::max<int64_t>(blocksize, 1);
  const int64_t widest = std::max<int64_t>(512, bs);
  *bytes = 3 * al256((size_t)B * R * widest * 4) +
           (variant == G2PTQ_VARIANT_G2PTQ ? al256((size_t)B * R * bs * 4) : 0) +
           al256((size_t)B * C * C * 4);
  return G2PTQ_OK;
}

// The lazy-batch loop behind g2ptq_compensate and g2ptq_compensate_noalloc.
// ws holds the error columns of one super-block (two or three with overlap
// allowed); every column of it is written by a sweep before a tail reads it,
// so it needs no clearing.
static int compensate_impl(hipStream_t s, int variant, int64_t B, int64_t R, int64_t C,
                           int64_t bs, float* W, const float* U, const float* P, const float* Z,
                           float* GH, int bits, int sym, int64_t groupsize, int static_groups,
                           int mse_grid, float mse_norm, float mse_maxshrink, const float* hdiag,
                           int64_t hblocks, const int* colgroup, float* scale_tab,
                           float* zero_tab, float* Q, float* Wint, float* Scale, int* flags,
                           void* ws, size_t ws_bytes, bool allow_overlap,
                           bool allow_transpose) {
  G2PTQ_CHECK(W && U && scale_tab && zero_tab && Q, "compensate: null pointer");
  G2PTQ_CHECK(bits >= 2 && bits <= 16, "compensate: bits=%d unsupported", bits);
  G2PTQ_CHECK(bs >= 1 && bs <= kMaxBlock, "compensate: blocksize %lld not in [1, %d]",
              (long long)bs, kMaxBlock);
  G2PTQ_CHECK(groupsize == -1 || groupsize > 0, "compensate: bad groupsize");
  G2PTQ_CHECK(variant != G2PTQ_VARIANT_GPTAQ || P, "compensate: GPTAQ needs P");
  G2PTQ_CHECK(variant != G2PTQ_VARIANT_G2PTQ || (Z && GH), "compensate: G2PTQ needs Z and GH");
  G2PTQ_CHECK(B >= 1 && B < 65536 && R >= 1 && C >= 1, "compensate: bad sizes");
  const int maxq = (1 << (bits - 1)) - 1;
  const bool dynamic = groupsize > 0 && !static_groups;
  int64_t SB = std::min(super_block(variant, bs, groupsize, static_groups),
                        cdiv(C, bs) * bs);
  // G2PTQ with super-blocks: the near tails read each block's E2 from a
  // buffer of its own; the super-block buffer holds the far-tail E3.
  const bool g2 = variant == G2PTQ_VARIANT_G2PTQ;
  size_t need = al256((size_t)B * R * SB * 4);
  size_t need2 = (g2 && SB > bs) ? al256((size_t)B * R * bs * 4) : 0;
  if (ws_bytes < need + need2 && SB > bs) {  // a smaller workspace: per-block tails
    SB = bs;
    need = al256((size_t)B * R * SB * 4);
    need2 = 0;
  }
  G2PTQ_CHECK(ws && ws_bytes >= need + need2, "compensate: workspace %zu < %zu", ws_bytes,
              need + need2);
  // Workspace layout: E (one super-block's error columns), E2 (G2PTQ), then,
  // as far as the workspace reaches, Ut (the factor transposed, for
  // k-contiguous tail products) and a second and third E buffer (lookahead).
  const size_t need_t = al256((size_t)B * C * C * 4);
  const bool transposed = allow_transpose && ws_bytes >= need + need2 + need_t;
  // Lookahead: with room for two error buffers, and outside graph capture,
  // the tail of a super-block beyond the next super-block's columns (the
  // "far" tail) runs on the side stream while the next super-block is swept.
  // With a third buffer the far tail goes out in two launches, the columns
  // of the super-block after next first: the caller's stream then waits only
  // for that part (and the side stream's earlier work), and the rest of the
  // far tail runs beside two sweeps instead of one.
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  G2PTQ_HIP(hipStreamIsCapturing(s, &capture));
  const size_t base = need + need2 + (transposed ? need_t : 0);
  const bool overlap = allow_overlap && ws_bytes >= base + need &&
                       capture == hipStreamCaptureStatusNone && SB < C;
  const bool deep = overlap && ws_bytes >= base + 2 * need;
  const int nbuf = deep ? 3 : overlap ? 2 : 1;
  SideStream side;
  if (overlap) G2PTQ_TRY(side_stream(s, side));
  char* wsb = static_cast<char*>(ws);
  float* Ebuf[3] = {reinterpret_cast<float*>(wsb),
                    reinterpret_cast<float*>(wsb + (overlap ? base : 0)),
                    reinterpret_cast<float*>(wsb + (deep ? base + need : 0))};
  float* E2buf = need2 ? reinterpret_cast<float*>(wsb + need) : nullptr;
  float* Ut = transposed ? reinterpret_cast<float*>(wsb + need + need2) : nullptr;
  const int64_t RC = R * C, CC = C * C;
  if (Ut) {
    const unsigned nt = (unsigned)cdiv(C, (int64_t)64);
    hipLaunchKernelGGL(transpose_upper_kernel, dim3(nt, nt, (unsigned)B), dim3(256), 0, s, U, C,
                       Ut);
    G2PTQ_LAUNCHED();
  }

  // W[:, :, c0:c1] -= Ecols · U[k0:k1, c0:c1]  (+ GPTAQ: += Q[:, :, k0:k1] · P[k0:k1, c0:c1]),
  // on stream q.  Every tail reads and writes only its own columns c0..c1.
  auto tail_on = [&](hipStream_t q, const float* Ecols, int64_t lde, int64_t k0, int64_t k1,
                     int64_t c0, int64_t c1) -> int {
    GemmF32 t;
    t.M = R; t.N = c1 - c0; t.K = k1 - k0; t.batch = B;
    t.A = Ecols; t.lda = lde; t.sA = R * lde;
    if (Ut) {  // U[k0:k1, c0:c1] as rows of Ut (every c > every k: Ut's written tiles)
      t.B = Ut + c0 * C + k0; t.ldb = C; t.sB = CC; t.b_kcontig = 1;
    } else {
      t.B = U + k0 * C + c0; t.ldb = C; t.sB = CC;
    }
    t.C = W + c0; t.ldc = C; t.sC = RC;
    t.D = W + c0; t.ldd = C; t.sD = RC;
    t.alpha = -1.f; t.beta = 1.f;
    if (variant == G2PTQ_VARIANT_G2PTQ) {
      // W -= (k1 − k0)·GH[:, c0:] + E·U_slab: a block's tail with E = E2
      // (k1 − k0 = bs), a super-block's with E = E3.
      t.X = GH + c0; t.ldx = C; t.sX = RC; t.gamma = -(float)(k1 - k0);
    }
    G2PTQ_TRY(gemm_f32(q, t));
    if (variant == G2PTQ_VARIANT_GPTAQ) {
      GemmF32 p = t;  // W += Q1 · P[k0:k1, c0:c1]
      p.A = Q + k0; p.lda = C; p.sA = RC;
      p.B = P + k0 * C + c0; p.ldb = C; p.sB = CC; p.b_kcontig = 0;
      p.alpha = 1.f;
      G2PTQ_TRY(gemm_f32(q, p));
    } else if (variant == G2PTQ_VARIANT_G2PTQ) {
      GemmF32 z = t;  // GH[:, c0:c1] -= Z1 · U_slab
      z.A = Z + k0; z.lda = C; z.sA = RC;
      z.C = GH + c0; z.D = GH + c0;
      z.X = nullptr; z.gamma = 0.f;
      G2PTQ_TRY(gemm_f32(q, z));
    }
    return G2PTQ_OK;
  };
  auto tail = [&](const float* Ecols, int64_t lde, int64_t k0, int64_t k1, int64_t c0,
                  int64_t c1) -> int { return tail_on(s, Ecols, lde, k0, k1, c0, c1); };

  // Every column receives the tails of the super-blocks before it in order:
  // the far tail of super-block p (columns from p + 2 on, side stream) lands
  // before the near tail of p + 1 (columns of p + 2, caller's stream), which
  // waits for it (for its first launch, with three buffers: the columns of
  // p + 2; the side stream runs its launches in order, so everything issued
  // there before is done too); that wait also frees the error buffer that
  // p + 1's successor overwrites (p's with two buffers, p − 1's with three).
  bool far_pending = false, side_used = false;
  for (int64_t s0 = 0, sbi = 0; s0 < C; s0 += SB, ++sbi) {
    const int64_t s1 = std::min(s0 + SB, C);
    float* E = Ebuf[sbi % nbuf];
    // GPTQ with full 128-column blocks, 16 lanes per row and groups fitted in
    // the sweep (or static): one launch sweeps the whole super-block and
    // applies its near tails itself.
    const bool sb_groups = !dynamic || (mse_grid == 0 && groupsize % 32 == 0 &&
                                        bs % groupsize == 0);
    const int nblk = (variant == G2PTQ_VARIANT_GPTQ && bs == kMaxBlock && sb_groups &&
                      (s1 - s0) % bs == 0 && s1 - s0 > bs)
                         ? (int)((s1 - s0) / bs) : 1;
    for (int64_t i1 = s0; i1 < s1; i1 += bs) {
      const int64_t i2 = std::min(i1 + bs, C), n = i2 - i1;
      // Min/max groups that tile the block in 32-column multiples are fitted
      // inside the sweep from the same block values.
      const bool fuse = dynamic && mse_grid == 0 && groupsize % 32 == 0 && bs % groupsize == 0 &&
                        n % 32 == 0;
      if (dynamic && !fuse) {
        for (int64_t gs = (i1 + groupsize - 1) / groupsize * groupsize; gs < i2; gs += groupsize) {
          const int64_t gi = gs / groupsize;
          const int64_t width = std::min(groupsize, C - gs);
          if (mse_grid > 0) {
            HDiag hd;  // H_diag[:, gs:gs + width] (hblocks × C)
            if (hdiag) { hd.h = hdiag + gs; hd.ld = C; hd.nblocks = hblocks; }
            G2PTQ_TRY(launch_find_params_mse(s, W + gs, B * R, width, C, maxq, sym, mse_norm,
                                             mse_grid, mse_maxshrink, hd, scale_tab + gi * B * R,
                                             zero_tab + gi * B * R, 1, flags));
          }
          else
            G2PTQ_TRY(launch_find_params(s, W + gs, B * R, width, C, maxq, sym,
                                         scale_tab + gi * B * R, zero_tab + gi * B * R, 1, flags));
        }
      }
      float* Eb = E + (i1 - s0);  // this block's error columns (ld SB)
      SweepArgs a{};
      a.R = R; a.n = (int)n; a.maxq = maxq;
      a.W = W + i1; a.wb = RC; a.wr = C; a.wc = 1;
      a.U = U + i1 * C + i1; a.ub = CC; a.uj = C;
      a.P = P ? P + i1 * C + i1 : nullptr;
      a.Zg = Z ? Z + i1 : nullptr; a.zb = RC; a.zr = C; a.zc = 1;
      a.GH = GH ? GH + i1 : nullptr; a.GHout = nullptr; a.gb = RC; a.gr = C; a.gc = 1;
      a.S = scale_tab; a.Z0 = zero_tab; a.sb = R; a.sr = 1; a.sg = B * R;
      a.colgroup = colgroup ? colgroup + i1 : nullptr;
      a.col0 = i1;
      a.gsize = groupsize > 0 ? groupsize : 0;
      if (fuse) {
        a.fuse = groupsize; a.sym = sym;
        a.FS = scale_tab; a.FZ = zero_tab;
      }
      a.Q = Q + i1; a.qb = RC; a.qr = C; a.qc = 1;
      a.I = Wint ? Wint + i1 : nullptr; a.ib = RC; a.ir = C; a.ic = 1;
      a.Sc = Scale ? Scale + i1 : nullptr; a.cb = RC; a.cr = C; a.cc = 1;
      a.CW = nullptr;
      if (variant == G2PTQ_VARIANT_G2PTQ) {
        a.E = nullptr;
        a.dist0 = bs - 1;
        if (E2buf) {
          a.E2 = E2buf; a.e2b = R * bs; a.e2r = bs; a.e2c = 1;
          a.E3 = Eb; a.e3b = R * SB; a.e3r = SB;
          a.dist3 = bs - 1 + (s1 - i2);
        } else {
          a.E2 = Eb; a.e2b = R * SB; a.e2r = SB; a.e2c = 1;
        }
      } else {
        a.E = Eb; a.eb = R * SB; a.er = SB; a.ec = 1;
        a.E2 = nullptr;
      }
      a.flags = flags;
      if (nblk > 1 && i1 == s0 && sweep_superblock_ok(a, B)) {
        a.nblk = nblk;
        a.Wsb = W + i1;
        G2PTQ_TRY(launch_sweep(s, variant, a, B));
        break;  // the launch swept every block of the super-block
      }
      G2PTQ_TRY(launch_sweep(s, variant, a, B));
      // The block's tail inside the super-block.
      if (i2 < s1) G2PTQ_TRY(E2buf ? tail(E2buf, bs, i1, i2, i2, s1) : tail(Eb, SB, i1, i2, i2, s1));
    }
    // The super-block's errors applied to every later column at once.
    if (s1 < C) {
      if (!overlap) {
        G2PTQ_TRY(tail(E, SB, s0, s1, s1, C));
        continue;
      }
      const int64_t nxt = std::min(s1 + SB, C);  // end of the next super-block's columns
      const int64_t nxt2 = std::min(nxt + SB, C);  // ... and of the one after
      if (far_pending) G2PTQ_HIP(hipStreamWaitEvent(s, side.tailed, 0));
      far_pending = nxt < C;
      if (far_pending) {
        G2PTQ_HIP(hipEventRecord(side.swept, s));
        G2PTQ_HIP(hipStreamWaitEvent(side.stream, side.swept, 0));
        G2PTQ_TRY(tail_on(side.stream, E, SB, s0, s1, nxt, deep ? nxt2 : C));
        G2PTQ_HIP(hipEventRecord(side.tailed, side.stream));
        if (deep && nxt2 < C) G2PTQ_TRY(tail_on(side.stream, E, SB, s0, s1, nxt2, C));
        side_used = true;
      }
      G2PTQ_TRY(tail(E, SB, s0, s1, s1, nxt));
    }
  }
  if (side_used) {  // the side stream's last launches (the event marks only a first part)
    G2PTQ_HIP(hipEventRecord(side.tailed, side.stream));
    G2PTQ_HIP(hipStreamWaitEvent(s, side.tailed, 0));
  }
  return G2PTQ_OK;
}

extern "C" int g2ptq_compensate(void* stream, int variant, int64_t B, int64_t R, int64_t C,
                                int64_t bs, float* W, const float* U, const float* P,
                                const float* Z, float* GH, int bits, int sym, int64_t groupsize,
                                int static_groups, int mse_grid, float mse_norm,
                                float mse_maxshrink, const float* hdiag, int64_t hblocks,
                                const int* colgroup,
                                float* scale_tab, float* zero_tab, float* Q, float* Wint,
                                float* Scale, int* flags, void* ws, size_t ws_bytes) {
  return compensate_impl(as_stream(stream), variant, B, R, C, bs, W, U, P, Z, GH, bits, sym,
                         groupsize, static_groups, mse_grid, mse_norm, mse_maxshrink, hdiag,
                         hblocks, colgroup, scale_tab, zero_tab, Q, Wint, Scale, flags, ws,
                         ws_bytes, true, true);
}

// Scratch memory of g2ptq_compensate_noalloc: the error columns of the loop,
// in a file-scope device array instead of a caller workspace.  Each device
// that runs the entry point holds its own copy until the process ends, and
// every call on a device shares it.  In host code `scratch` is only a symbol
// handle: its device address comes from hipGetSymbolAddress, once per device.
static constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

static int scratch_address(void** out) {
  static std::mutex mu;
  static void* addr[64] = {};
  int dev = 0;
  G2PTQ_HIP(hipGetDevice(&dev));
  G2PTQ_CHECK(dev >= 0 && dev < 64, "compensate_noalloc: device index %d", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    G2PTQ_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    G2PTQ_CHECK(p != nullptr, "compensate_noalloc: no device address for the scratch array");
    addr[dev] = p;
  }
  *out = addr[dev];
  return G2PTQ_OK;
}

extern "C" int g2ptq_compensate_noalloc(void* stream, int variant, int64_t B, int64_t R,
                                        int64_t C, int64_t bs, float* W, const float* U,
                                        const float* P, const float* Z, float* GH, int bits,
                                        int sym, int64_t groupsize, int static_groups,
                                        int mse_grid, float mse_norm, float mse_maxshrink,
                                        const float* hdiag, int64_t hblocks, const int* colgroup,
                                        float* scale_tab, float* zero_tab, float* Q, float* Wint,
                                        float* Scale, int* flags) {
  G2PTQ_CHECK(B >= 1 && R >= 1 && bs >= 1 && bs <= kMaxBlock, "compensate_noalloc: bad sizes");
  const size_t need = al256((size_t)B * R * bs * 4);
  G2PTQ_CHECK(need <= kScratchBytes,
              "compensate_noalloc: B*R*blocksize*4 = %zu bytes exceeds the %zu-byte scratch "
              "array (at most %lld rows at blocksize %lld); use g2ptq_compensate",
              need, kScratchBytes, (long long)(kScratchBytes / (4 * (size_t)bs)), (long long)bs);
  void* ws = nullptr;
  G2PTQ_TRY(scratch_address(&ws));
  return compensate_impl(as_stream(stream), variant, B, R, C, bs, W, U, P, Z, GH, bits, sym,
                         groupsize, static_groups, mse_grid, mse_norm, mse_maxshrink, hdiag,
                         hblocks, colgroup, scale_tab, zero_tab, Q, Wint, Scale, flags, ws,
                         kScratchBytes, false, false);
}

extern "C" int g2ptq_gptaq_p(void* stream, const float* Dx, const float* U, int64_t B, int64_t C,
                             float alpha, float* P, void* ws, size_t ws_bytes) {
  G2PTQ_CHECK(Dx && U && P, "gptaq_p: null pointer");
  const size_t need = al256((size_t)B * C * C * 4);
  G2PTQ_CHECK(ws && ws_bytes >= need, "gptaq_p: workspace %zu < %zu", ws_bytes, need);
  hipStream_t s = as_stream(stream);
  float* T = static_cast<float*>(ws);
  const int64_t CC = C * C;
  GemmF32 a;  // T = Dx · Uᵀ, upper tiles only (triu(T, 1) is all that is used)
  a.M = C; a.N = C; a.K = C; a.batch = B;
  a.A = Dx; a.lda = C; a.sA = CC;
  a.B = U; a.ldb = C; a.sB = CC; a.b_kcontig = 1;
  a.D = T; a.ldd = C; a.sD = CC;
  a.uplo = 2;
  a.tri = 2;  // Uᵀ[k][n] = U[n][k] = 0 for k < n
  G2PTQ_TRY(gemm_f32(s, a));
  dim3 grid((unsigned)cdiv(C, 64), (unsigned)cdiv(C, 16), (unsigned)B);
  hipLaunchKernelGGL(triu1_kernel, grid, dim3(256), 0, s, T, C);
  G2PTQ_LAUNCHED();
  GemmF32 b;  // P = alpha · triu(T, 1) · U
  b.M = C; b.N = C; b.K = C; b.batch = B;
  b.A = T; b.lda = C; b.sA = CC;
  b.B = U; b.ldb = C; b.sB = CC;
  b.D = P; b.ldd = C; b.sD = CC;
  b.alpha = alpha;
  // triu(T, 1)[m][k] = 0 for k <= m, U[k][n] = 0 for k > n: tile (m, n) sums
  // k in [m0, n0 + BN) only, and tiles below the diagonal write zeros.
  b.tri = 4 | 8;
  G2PTQ_TRY(gemm_f32(s, b));
  return G2PTQ_OK;
}

extern "C" int g2ptq_trust_region_workspace(int64_t BG, int64_t Rg, int64_t C, size_t* bytes) {
  (void)Rg;
  G2PTQ_CHECK(bytes != nullptr, "trust_region_workspace: null out");
  *bytes = al256((size_t)BG * C * 4);
  return G2PTQ_OK;
}

extern "C" int g2ptq_trust_region(void* stream, const float* Grad, const float* U,
                                  const float* Q0, const float* W0, int64_t BG, int64_t Rg,
                                  int64_t C, float alpha, int enabled, float* beta, float* Z,
                                  float* GH, void* ws, size_t ws_bytes) {
  G2PTQ_CHECK(beta && Z && GH, "trust_region: null output");
  hipStream_t s = as_stream(stream);
  const int64_t n = BG * Rg * C;
  if (!enabled) {
    G2PTQ_TRY(fill_f32(s, beta, BG * Rg, 0.f));
    G2PTQ_TRY(fill_f32(s, Z, n, 0.f));
    G2PTQ_TRY(fill_f32(s, GH, n, 0.f));
    return G2PTQ_OK;
  }
  G2PTQ_CHECK(Grad && U && Q0 && W0, "trust_region: null input");
  size_t need = 0;
  g2ptq_trust_region_workspace(BG, Rg, C, &need);
  G2PTQ_CHECK(ws && ws_bytes >= need, "trust_region: workspace %zu < %zu", ws_bytes, need);
  float* dA = static_cast<float*>(ws);
  const int64_t CC = C * C, RC = Rg * C;
  GemmF32 a;  // Z ← T1 = Grad · Uᵀ
  a.M = Rg; a.N = C; a.K = C; a.batch = BG;
  a.A = Grad; a.lda = C; a.sA = RC;
  a.B = U; a.ldb = C; a.sB = CC; a.b_kcontig = 1;
  a.D = Z; a.ldd = C; a.sD = RC;
  a.tri = 2;  // B(k, n) = U[n][k] is zero for k < n
  G2PTQ_TRY(gemm_f32(s, a));
  GemmF32 b;  // GH ← GA = T1 · U = Grad · A⁻¹
  b.M = Rg; b.N = C; b.K = C; b.batch = BG;
  b.A = Z; b.lda = C; b.sA = RC;
  b.B = U; b.ldb = C; b.sB = CC;
  b.D = GH; b.ldd = C; b.sD = RC;
  b.tri = 8;  // B = U is zero below the diagonal
  G2PTQ_TRY(gemm_f32(s, b));
  hipLaunchKernelGGL(inv_diag_kernel, dim3((unsigned)cdiv(C, 64), (unsigned)BG), dim3(256), 0, s,
                     U, C, dA);
  G2PTQ_LAUNCHED();
  hipLaunchKernelGGL(trust_row_kernel, dim3((unsigned)(BG * Rg)), dim3(256), 0, s, Grad, Q0, W0,
                     dA, Rg, C, (float)(2.0 * (double)alpha), beta, Z, GH);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}
