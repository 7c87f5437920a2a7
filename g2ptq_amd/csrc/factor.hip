// Dampened inverse-Cholesky factor on CDNA4.
//
// The reference computes U = chol(cholesky_inverse(chol(A)), upper) with
// A = H + p·mean(diag H)·I (gptq_utils.py:295-302): three factorizations'
// worth of work (~4C³/3).  The same unique factor (upper triangular, positive
// diagonal, UᵀU = A⁻¹) is U = J·L̂⁻¹·J where L̂ = chol(J·A·J) and J reverses
// index order: one Cholesky plus one triangular inverse (2C³/3).
//
//   1. reverse-copy Â = J(H + damp·I)J (lower triangle) into the workspace
//   2. blocked right-looking Cholesky of Â in panels of NBO = 512 columns,
//      each factored NB = 64 columns at a time: potrf of the diagonal block
//      in one workgroup (registers), which also inverts it in place;  TRSM
//      with that inverse and update of the panel's remaining columns in one
//      launch (panel_step_kernel, whose first tile factors the next diagonal
//      block);  then one SYRK trailing update per panel (K = 512) as a
//      lower-triangular fp32 GEMM
//   3. the triangular inverse X = L̂⁻¹ panel by panel, as soon as each is
//      factored, on a third stream beside the Cholesky: the diagonal block
//      by recursive doubling from the NB inverses, then the block row
//      X[p, 0:p] = −X_pp·(L[p, 0:p]·X[0:p, 0:p]) as two GEMMs, the first
//      reading X[0:p, 0:p] from a transposed copy kept as the rows finish
//   4. un-reverse into U (upper, zeros below) with the reference's NaN check.
#include <map>
#include <mutex>

#include "common.hpp"
#include "potrf.hpp"

namespace g2ptq {
namespace {

constexpr int NB = 64;   // diagonal block width (potrf in registers)
constexpr int NBO = 512; // panel width of the trailing (SYRK) updates
constexpr int64_t SYRK_CHUNK = 2048;  // columns per launch of the far trailing update

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

// Cholesky + in-place inverse of the nbk×nbk (nbk <= 64) diagonal block at
// (k, k) of each layer: load, potrf_core (potrf.hpp), store X = L⁻¹ (lower,
// zeros above) or record the failing pivot.
__global__ __launch_bounds__(256) void potrf_diag_kernel(float* WA, int64_t C, int64_t k, int nbk,
                                                        int* st, int* info) {
  const int64_t b = blockIdx.x;
  __shared__ __attribute__((aligned(16))) float Xs[POT_NB * XP];
  __shared__ __attribute__((aligned(16))) float Lm[POT_NB * LP];
  __shared__ __attribute__((aligned(16))) float rdv[POT_NB + PB * PB];  // + the panels' multipliers
  __shared__ int fail_s;
  float* Wb = WA + b * C * C + k * C + k;
  const int i = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int skip = st[b];
  // Lower triangle of the block: row r through lane i of wave r & 3
  // (coalesced; addresses clamped into the block so the loads need no
  // branches), all 16 rows of a wave in flight together.
  {
    const int ci = i < nbk ? i : nbk - 1;
    float x[POT_NB / 4];
#pragma unroll
    for (int h = 0; h < POT_NB / 4; ++h) {
      const int r = 4 * h + w;
      const int rr = r < nbk ? r : nbk - 1;
      x[h] = Wb[(int64_t)rr * C + ci];
    }
#pragma unroll
    for (int h = 0; h < POT_NB / 4; ++h) {
      const int r = 4 * h + w;
      Xs[r * XP + i] = (r < nbk && i < nbk) ? (i <= r ? x[h] : 0.f) : (r == i ? 1.f : 0.f);
    }
  }
  __syncthreads();
  const int fail = potrf_core(Xs, Lm, rdv, &fail_s);
  // Layers already done (a damp retry) run the steps on whatever the block
  // holds and store nothing: testing the flag only here lets its load overlap
  // the block loads instead of preceding them.
  if (skip) return;
  if (fail) {
    if (threadIdx.x == 0) {
      info[b] = (int)(k + fail);
      st[b] = 1;
    }
    return;
  }
  if (i < nbk) {
#pragma unroll 4
    for (int r = w; r < nbk; r += 4) Wb[(int64_t)r * C + i] = (i <= r) ? Xs[r * XP + i] : 0.f;
  }
}

// ---- Panel steps: TRSM, remainder update and the next diagonal block in one launch ----
//
// Column block [j, j + nbk) of the panel [k, pe), its diagonal block already
// inverted in place (X_jj = L_jj⁻¹, lower):
//   L[r, j:j+nbk] = Â[r, j:j+nbk]·X_jjᵀ           rows r >= r0 = j + nbk
//   Â[r, c]      −= Σ_t L[r, j+t]·L[c, j+t]        r0 <= c < pe, c <= r
// and the workgroup of tile (r0, r0) factors and inverts the next diagonal
// block.  A workgroup owns one 64×64 tile (i, n) of the update and forms the
// two L blocks it multiplies (rows of tile-row i and of tile-column n) itself
// from the raw column block, so the TRSM needs no launch of its own.  The raw
// column block is therefore read while the step runs, and L cannot go back in
// place: workgroups of tile-column 0 write their L rows to a panel buffer
// (Lp, rows × NBO), and the panel's last step (panel_finish_kernel) copies it
// into Â.
//
// The products use v_mfma_f32_32x32x2_f32 in the order of gemm_f32's fp32
// path (32-k slabs; k-octet o, lane half h holding k = 8o + 4h + c in the c-th
// of four MFMAs), and its epilogue arithmetic (alpha·acc + beta·C with
// alpha = 1, beta = 0 for L and alpha = −1, beta = 1 for the update), so the
// factor is bit-identical to a TRSM launch followed by an update launch of
// gemm_f32 (the scheme this replaced: measured on MI355X, same bits for
// C = 64 … 14336).
constexpr int SLP = 68;  // LDS row pitch (floats) of the 64-wide k tiles
static_assert(SLP >= LP, "the panel step's tiles hold the potrf scratch");
typedef float f32x16 __attribute__((ext_vector_type(16)));

// A 64×64 block of Â (rows row0.., columns col0.., only rows < nrows and
// columns < ncols nonzero): thread t's four 16-byte pieces (rows t/16 + 16q,
// columns 4·(t%16)..+3) into registers, then into LDS [row][SLP] by
// panel_put.  panel_fetch_vec (16-byte aligned rows, the thread's four
// columns inside the block) issues its loads unconditionally: row0 is a row of
// Â, so a piece below the block reads from row0, and panel_put zeroes it.  A
// caller fetching several blocks calls it for all of them before putting any,
// so their loads are in flight together.
__device__ __forceinline__ void panel_fetch_vec(float4 (&v)[4], const float* Wb, int64_t C,
                                                int64_t row0, int64_t col0, int64_t nrows) {
  const int t = threadIdx.x;
  const int c4 = (t & 15) * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (t >> 4) + 16 * q;
    v[q] = *reinterpret_cast<const float4*>(Wb + (row0 + (r < nrows ? r : 0)) * C + col0 + c4);
  }
}

__device__ __forceinline__ void panel_fetch_any(float4 (&v)[4], const float* Wb, int64_t C,
                                                int64_t row0, int64_t col0, int64_t nrows,
                                                int ncols) {
  const int t = threadIdx.x;
  const int c4 = (t & 15) * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (t >> 4) + 16 * q;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r < nrows) {
      const float* p = Wb + (row0 + r) * C + col0 + c4;
      if (c4 < ncols) x.x = p[0];
      if (c4 + 1 < ncols) x.y = p[1];
      if (c4 + 2 < ncols) x.z = p[2];
      if (c4 + 3 < ncols) x.w = p[3];
    }
    v[q] = x;
  }
}

// Whether thread t's pieces take panel_fetch_vec.
__device__ __forceinline__ bool panel_vec(bool vec, int ncols) {
  return vec && (threadIdx.x & 15) * 4 + 3 < ncols;
}

__device__ __forceinline__ void panel_put(float* Ls, const float4 (&v)[4], int64_t nrows) {
  const int t = threadIdx.x;
  const int c4 = (t & 15) * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (t >> 4) + 16 * q;
    *reinterpret_cast<float4*>(&Ls[r * SLP + c4]) =
        r < nrows ? v[q] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// One wave's 32×32 block of Σ_k Ap[ar + ·][k]·Bp[br + ·][k] over 64 k.
__device__ __forceinline__ f32x16 panel_mma(const float* Ap, const float* Bp, int ar, int br) {
  const int lane = threadIdx.x & 63, lr = lane & 31, lh = lane >> 5;
  f32x16 acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.f;
#pragma unroll
  for (int o = 0; o < 8; ++o) {
    const float4 a = *reinterpret_cast<const float4*>(Ap + (ar + lr) * SLP + o * 8 + lh * 4);
    const float4 b = *reinterpret_cast<const float4*>(Bp + (br + lr) * SLP + o * 8 + lh * 4);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, acc, 0, 0, 0);
  }
  return acc;
}

// The wave's block of L = (raw)·Xᵀ as gemm_f32 stores it (1·acc + 0), into
// LDS over the raw rows (columns at or past nbk zero).
__device__ __forceinline__ void panel_put_l(float* Ls, const f32x16& acc, int wm, int wn, int nbk) {
  const int lane = threadIdx.x & 63, lr = lane & 31, lh = lane >> 5;
  const int col = wn * 32 + lr;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = wm * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
    Ls[row * SLP + col] = col < nbk ? __builtin_fmaf(1.f, acc[v], 0.f) : 0.f;
  }
}

struct PanelArgs {
  float* WA;         // Â (B × C × C), updated in place
  float* Lp;         // panel buffer (B × C × NBO): L of the panel's column blocks
  int64_t C;
  int64_t k, pe;     // panel [k, pe)
  int64_t j;         // column block [j, j + nbk)
  int nbk;
  int pot_nb;        // next diagonal block's width (0: none)
  int ncb;           // tile-columns of the remainder, cdiv(pe − r0, 64)
  int nrb;           // tile-rows, cdiv(C − r0, 64)
  int* st;
  int* info;
};

__global__ __launch_bounds__(256) void panel_step_kernel(PanelArgs p) {
  __shared__ __attribute__((aligned(16))) float Xj[64 * SLP];
  __shared__ __attribute__((aligned(16))) float Ai[64 * SLP];
  __shared__ __attribute__((aligned(16))) float An[64 * SLP];
  __shared__ int fail_s;
  const int64_t b = blockIdx.y;
  if (p.st[b]) return;
  const int64_t C = p.C, r0 = p.j + p.nbk;
  // Tile id → (i, n): the triangle of tile-rows inside the panel first
  // (id 0 = the diagonal tile that factors the next block), then the
  // rectangle below the panel.
  const int64_t id = blockIdx.x, tri = (int64_t)p.ncb * (p.ncb + 1) / 2;
  int64_t i, n;
  if (id < tri) {
    i = (int64_t)((sqrtf(8.f * (float)id + 1.f) - 1.f) * 0.5f);
    while (i * (i + 1) / 2 > id) --i;
    while ((i + 1) * (i + 2) / 2 <= id) ++i;
    n = id - i * (i + 1) / 2;
  } else {
    i = p.ncb + (id - tri) / p.ncb;
    n = (id - tri) % p.ncb;
  }
  float* Wb = p.WA + b * C * C;
  const bool vec = (C & 3) == 0;
  const int64_t ri = r0 + 64 * i, rn = r0 + 64 * n;  // first row of each L block
  {
    float4 vx[4], va[4], vn[4];
    if (panel_vec(vec, p.nbk)) {
      panel_fetch_vec(vx, Wb, C, p.j, p.j, p.nbk);
      panel_fetch_vec(va, Wb, C, ri, p.j, C - ri);
      panel_fetch_vec(vn, Wb, C, n != i ? rn : ri, p.j, C - (n != i ? rn : ri));
    } else {
      panel_fetch_any(vx, Wb, C, p.j, p.j, p.nbk, p.nbk);
      panel_fetch_any(va, Wb, C, ri, p.j, C - ri, p.nbk);
      panel_fetch_any(vn, Wb, C, n != i ? rn : ri, p.j, C - (n != i ? rn : ri), p.nbk);
    }
    panel_put(Xj, vx, p.nbk);
    panel_put(Ai, va, C - ri);
    if (n != i) panel_put(An, vn, C - rn);
  }
  const int wave = threadIdx.x >> 6, wm = wave >> 1, wn = wave & 1;
  const int lane = threadIdx.x & 63, lr = lane & 31, lh = lane >> 5;
  // The update's Â operand, read with the raw blocks (nothing in this launch
  // writes it before this workgroup's own epilogue).
  const int64_t c = rn + wn * 32 + lr;
  float cv[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t r = ri + wm * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
    cv[v] = (r < C && c < p.pe) ? 1.f * Wb[r * C + c] : 0.f;
  }
  __syncthreads();
  const f32x16 li = panel_mma(Ai, Xj, wm * 32, wn * 32);
  f32x16 ln;
  if (n != i) ln = panel_mma(An, Xj, wm * 32, wn * 32);
  __syncthreads();  // raw blocks and X_jj read
  panel_put_l(Ai, li, wm, wn, p.nbk);
  if (n != i) panel_put_l(An, ln, wm, wn, p.nbk);
  if (n == 0) {
    // L rows of tile-row i into the panel buffer (column j − k on)
    float* Lb = p.Lp + b * C * NBO + (p.j - p.k);
    const int col = wn * 32 + lr;
    if (col < p.nbk) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t r = ri + wm * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
        if (r < C) Lb[r * NBO + col] = __builtin_fmaf(1.f, li[v], 0.f);
      }
    }
  }
  __syncthreads();  // L blocks in LDS
  const float* Ln = (n != i) ? An : Ai;
  const f32x16 acc = panel_mma(Ai, Ln, wm * 32, wn * 32);
  // Epilogue: Â[r][c] = −1·acc + 1·Â[r][c] on the lower part inside the
  // panel; the tile (0, 0) sends the next diagonal block to LDS instead.
  const bool pot = p.pot_nb > 0 && i == 0 && n == 0;
  float* Xs = Xj;  // the potrf staging reuses X_jj's buffer (read above)
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int rl = wm * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
    const int64_t r = ri + rl;
    const float val = __builtin_fmaf(-1.f, acc[v], cv[v]);
    if (pot) {
      const int cl = wn * 32 + lr, nb = p.pot_nb;
      Xs[rl * XP + cl] = (rl < nb && cl < nb) ? (cl <= rl ? val : 0.f) : (rl == cl ? 1.f : 0.f);
      if (rl < nb && cl < nb) continue;
    }
    if (r < C && c < p.pe && c <= r) Wb[r * C + c] = val;
  }
  if (!pot) return;
  __syncthreads();
  const int fail = potrf_core(Xs, Ai, An, &fail_s);  // L and the pivots' 1/sqrt in Ai, An
  if (fail) {
    if (threadIdx.x == 0) {
      p.info[b] = (int)(r0 + fail);
      p.st[b] = 1;
    }
    return;
  }
  const int wv = threadIdx.x >> 6;
  if (lane < p.pot_nb) {
    for (int r = wv; r < p.pot_nb; r += 4)
      Wb[(r0 + r) * C + r0 + lane] = (lane <= r) ? Xs[r * XP + lane] : 0.f;
  }
}

// The panel's last column block [j, pe): workgroup t owns rows
// [k + 64(t + 1), +64).  Rows below the panel get their TRSM for this block in
// place (L = Â·X_jjᵀ; nothing else reads these raw values); every row gets the
// panel buffer's L columns left of its own diagonal block (or of this block)
// copied into Â.
__global__ __launch_bounds__(256) void panel_finish_kernel(PanelArgs p) {
  __shared__ __attribute__((aligned(16))) float Xj[64 * SLP];
  __shared__ __attribute__((aligned(16))) float Ai[64 * SLP];
  const int64_t b = blockIdx.y;
  if (p.st[b]) return;
  const int64_t C = p.C;
  const int64_t R0 = p.k + 64 * ((int64_t)blockIdx.x + 1);
  float* Wb = p.WA + b * C * C;
  const float* Lb = p.Lp + b * C * NBO;
  const bool vec = (C & 3) == 0;
  const int64_t cend = (R0 < p.pe ? R0 : p.j) - p.k;  // buffer columns to copy
  {
    const int nq = (int)(cend >> 2);  // cend is a multiple of 64
    // eight 16-byte pieces per thread and pass, all loaded before any is stored
    constexpr int U = 8;
    for (int q0 = threadIdx.x; q0 < 64 * nq; q0 += 256 * U) {
      float4 x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = q0 + 256 * u;
        const int64_t r = R0 + q / nq;
        const int64_t c4 = (int64_t)(q % nq) * 4;
        if (q < 64 * nq && r < C) {
          const float* s = Lb + r * NBO + c4;
          if (vec) {
            x[u] = *reinterpret_cast<const float4*>(s);
          } else {
            x[u] = make_float4(s[0], s[1], s[2], s[3]);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = q0 + 256 * u;
        const int64_t r = R0 + q / nq;
        const int64_t c4 = (int64_t)(q % nq) * 4;
        if (q < 64 * nq && r < C) {
          float* d = Wb + r * C + p.k + c4;
          if (vec) {
            *reinterpret_cast<float4*>(d) = x[u];
          } else {
            d[0] = x[u].x; d[1] = x[u].y; d[2] = x[u].z; d[3] = x[u].w;
          }
        }
      }
    }
  }
  if (R0 < p.pe) return;
  {
    float4 vx[4], va[4];
    if (panel_vec(vec, p.nbk)) {
      panel_fetch_vec(vx, Wb, C, p.j, p.j, p.nbk);
      panel_fetch_vec(va, Wb, C, R0, p.j, C - R0);
    } else {
      panel_fetch_any(vx, Wb, C, p.j, p.j, p.nbk, p.nbk);
      panel_fetch_any(va, Wb, C, R0, p.j, C - R0, p.nbk);
    }
    panel_put(Xj, vx, p.nbk);
    panel_put(Ai, va, C - R0);
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, wm = wave >> 1, wn = wave & 1;
  const int lane = threadIdx.x & 63, lr = lane & 31, lh = lane >> 5;
  const f32x16 li = panel_mma(Ai, Xj, wm * 32, wn * 32);
  const int col = wn * 32 + lr;
  if (col < p.nbk) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t r = R0 + wm * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
      if (r < C) Wb[r * C + p.j + col] = __builtin_fmaf(1.f, li[v], 0.f);
    }
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

// XT[n][k + m] = X[k + m][n] for the block row [k, k + kb) of X = L̂⁻¹ and
// columns n < k + kb (zeros where n > k + m): the inverse kept transposed, so
// that the next block row's product reads it as a k-contiguous operand.  A
// 64×64 tile per workgroup through LDS (coalesced reads of X's rows, writes
// of XT's rows).
__global__ __launch_bounds__(256) void xt_store_kernel(const float* __restrict__ WA, int64_t C,
                                                       int64_t k, int64_t kb, const int* st,
                                                       float* __restrict__ XT) {
  __shared__ float tile[64][65];
  const int64_t b = blockIdx.z;
  if (st[b]) return;
  const int64_t n0 = (int64_t)blockIdx.x * 64, m0 = (int64_t)blockIdx.y * 64;
  const int64_t kend = k + kb;
  const float* Wb = WA + b * C * C;
  float* Xb = XT + b * C * C;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t m = m0 + ty * 16 + r, n = n0 + tx;  // X[k + m][n]
    float v = 0.f;
    if (m < kb && n < kend && n <= k + m) v = Wb[(k + m) * C + n];
    tile[ty * 16 + r][tx] = v;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t n = n0 + ty * 16 + r, m = m0 + tx;  // XT[n][k + m]
    if (n < kend && m < kb) Xb[n * C + k + m] = tile[tx][ty * 16 + r];
  }
}

struct FactorWs {
  size_t wa, wt, ti, lp, xt, sums, st, total;
};

FactorWs factor_ws(int64_t B, int64_t C) {
  FactorWs w;
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  w.wa = al((size_t)B * C * C * 4);
  const int64_t half = std::min<int64_t>((C + 1) / 2, NBO);
  w.wt = al((size_t)B * half * half * 4 + 4);        // in-panel inverse products
  w.ti = al((size_t)B * NBO * C * 4 + 4);            // inverse block-row products
  w.lp = al((size_t)B * C * NBO * 4);                // a panel's L until its last step
  w.xt = al((size_t)B * C * C * 4);                  // the inverse's finished block rows, transposed
  w.sums = al((size_t)B * 4);
  w.st = al((size_t)B * 4);
  w.total = w.wa + w.wt + w.ti + w.lp + w.xt + w.sums + w.st;
  return w;
}

}  // namespace

int side_stream(hipStream_t caller, SideStream& out) {
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, SideStream> cache;
  int dev = 0;
  G2PTQ_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  SideStream& c = cache[{dev, caller}];
  if (c.stream == nullptr) {
    G2PTQ_HIP(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking));
    G2PTQ_HIP(hipStreamCreateWithFlags(&c.stream2, hipStreamNonBlocking));
    for (hipEvent_t* e : {&c.factored, &c.done[0], &c.done[1], &c.inverted, &c.swept, &c.tailed})
      G2PTQ_HIP(hipEventCreateWithFlags(e, hipEventDisableTiming));
  }
  out = c;
  return G2PTQ_OK;
}

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
  float* TI = reinterpret_cast<float*>(base + w.wa + w.wt);
  float* Lp = reinterpret_cast<float*>(base + w.wa + w.wt + w.ti);
  float* XT = reinterpret_cast<float*>(base + w.wa + w.wt + w.ti + w.lp);
  float* sums = reinterpret_cast<float*>(base + w.wa + w.wt + w.ti + w.lp + w.xt);
  int* st = reinterpret_cast<int*>(base + w.wa + w.wt + w.ti + w.lp + w.xt + w.sums);
  const int64_t CC = C * C;

  hipLaunchKernelGGL(diag_sum_kernel, dim3((unsigned)B), dim3(256), 0, s, H, C, skip, sums, st,
                     info);
  G2PTQ_LAUNCHED();
  dim3 cgrid((unsigned)cdiv(C, 64), (unsigned)cdiv(C, 16), (unsigned)B);
  hipLaunchKernelGGL(reverse_damp_kernel, cgrid, dim3(256), 0, s, H, C, percdamp, sums, st, WA);
  G2PTQ_LAUNCHED();

  // Triangular inverse by recursive doubling over rows/columns [i_base,
  // i_base + n) of Â, whose diagonal blocks of size sz_from are already
  // inverted in place: level sz joins pairs of sz-sized inverses with
  // X21 = −X22·(L21·X11) (two batched GEMMs on stream q), up to blocks of
  // size >= sz_to.
  auto trtri_levels = [&](hipStream_t q, int64_t i_base, int64_t n, int64_t sz_from,
                          int64_t sz_to) -> int {
    for (int64_t sz = sz_from; sz < n && sz < sz_to; sz *= 2) {
      const int64_t full = n / (2 * sz);             // pairs with a full second block
      const int64_t tail_i = full * 2 * sz;          // start of a possible ragged pair
      const int64_t tail_n2 = n - tail_i - sz;       // its second block size (if > 0)
      for (int part = 0; part < 2; ++part) {
        int64_t npairs, i0, n2;
        if (part == 0) {
          npairs = full; i0 = i_base; n2 = sz;
        } else {
          npairs = tail_n2 > 0 ? 1 : 0; i0 = i_base + tail_i; n2 = tail_n2;
        }
        if (npairs == 0) continue;
        const int64_t pstride = 2 * sz * (C + 1);
        GemmF32 t;  // T = L21 · X11
        t.M = n2; t.N = sz; t.K = sz; t.batch = B; t.batch2 = npairs;
        t.A = WA + (i0 + sz) * C + i0; t.lda = C; t.sA = CC; t.sA2 = pstride;
        t.B = WA + i0 * C + i0; t.ldb = C; t.sB = CC; t.sB2 = pstride;
        t.D = WT; t.ldd = sz; t.sD = npairs * n2 * sz; t.sD2 = n2 * sz;
        t.tri = 2;  // X11 is lower triangular
        t.skip = st;
        G2PTQ_TRY(gemm_f32(q, t));
        GemmF32 x;  // X21 = −X22 · T
        x.M = n2; x.N = sz; x.K = n2; x.batch = B; x.batch2 = npairs;
        x.A = WA + (i0 + sz) * C + (i0 + sz); x.lda = C; x.sA = CC; x.sA2 = pstride;
        x.B = WT; x.ldb = sz; x.sB = npairs * n2 * sz; x.sB2 = n2 * sz;
        x.D = WA + (i0 + sz) * C + i0; x.ldd = C; x.sD = CC; x.sD2 = pstride;
        x.alpha = -1.f; x.tri = 1;  // X22 is lower triangular
        x.skip = st;
        G2PTQ_TRY(gemm_f32(q, x));
      }
    }
    return G2PTQ_OK;
  };

  // Blocked Cholesky of Â (lower) with inverted diagonal blocks, two levels:
  // panels of NBO columns are factored NB columns at a time (potrf + TRSM +
  // update of the panel's own remaining columns), and the trailing matrix
  // receives each whole panel in one SYRK with K = NBO.  Lookahead of one
  // panel: the trailing update beyond the next panel runs on a second stream
  // while the next panel (updated first, on the caller's stream) is factored,
  // so the latency-bound panel chain overlaps the MFMA-bound SYRK.  The first
  // diagonal block of a panel is factored by potrf_diag_kernel; every later
  // one by the panel step that produces it (its first workgroup factors the
  // block in LDS right after computing it).  One launch per 64 columns: the
  // step's TRSM and update run together, L of the panel goes to the Lp buffer
  // and reaches Â in the panel's last step.
  // Once a panel is factored, a third stream inverts it into X = L̂⁻¹:
  //   the panel's diagonal block (recursive doubling from the NB inverses,
  //   in place), then, in block-row order so that X[0:k, 0:k] is final,
  //   TI = L[k:kend, 0:k] · X[0:k, 0:k];  X[k:kend, 0:k] = −X_kk · TI,
  //   written over L[k:kend, 0:k], and the finished block row copied
  //   transposed into XT, from which the next block rows' TI products read
  //   X[0:k, 0:k] as a k-contiguous operand (each element still receives the
  //   same products in the same order, so X is unchanged to the bit).
  // The Cholesky reads neither the diagonal block nor the block row again:
  // the trailing updates that read the block row completed before the panel
  // was factored, and those of the panel itself read only the rows below it.
  SideStream side;
  G2PTQ_TRY(side_stream(s, side));
  bool inv_pending = false;  // inverse work queued on stream2
  auto factor_panel = [&](int64_t k, int64_t kb) -> int {
    PanelArgs pa;
    pa.WA = WA; pa.Lp = Lp; pa.C = C; pa.k = k; pa.pe = k + kb; pa.st = st; pa.info = info;
    for (int64_t j = k; j < k + kb; j += NB) {
      const int nbk = (int)std::min<int64_t>(NB, k + kb - j);
      if (j == k) {
        hipLaunchKernelGGL(potrf_diag_kernel, dim3((unsigned)B), dim3(256), 0, s, WA, C, j, nbk,
                           st, info);
        G2PTQ_LAUNCHED();
      }
      pa.j = j; pa.nbk = nbk;
      const int64_t pw = k + kb - (j + nbk);  // panel columns still to factor
      if (pw > 0) {
        // TRSM of the rows below, update of the panel remainder, next diagonal block
        pa.pot_nb = (int)std::min<int64_t>(NB, pw);
        pa.ncb = (int)cdiv(pw, 64);
        pa.nrb = (int)cdiv(C - j - nbk, 64);
        const int64_t tiles = (int64_t)pa.ncb * (pa.ncb + 1) / 2 + (int64_t)(pa.nrb - pa.ncb) * pa.ncb;
        hipLaunchKernelGGL(panel_step_kernel, dim3((unsigned)tiles, (unsigned)B), dim3(256), 0, s,
                           pa);
        G2PTQ_LAUNCHED();
      } else if (C - k > NB) {
        // TRSM of the rows below the panel for its last block; the panel
        // buffer's L into Â
        pa.pot_nb = 0;
        hipLaunchKernelGGL(panel_finish_kernel, dim3((unsigned)cdiv(C - k - NB, 64), (unsigned)B),
                           dim3(256), 0, s, pa);
        G2PTQ_LAUNCHED();
      }
    }
    G2PTQ_HIP(hipEventRecord(side.factored, s));
    G2PTQ_HIP(hipStreamWaitEvent(side.stream2, side.factored, 0));
    inv_pending = true;
    G2PTQ_TRY(trtri_levels(side.stream2, k, kb, NB, NBO));
    if (k > 0) {
      GemmF32 t;  // B = X[0:k, 0:k] read as its transpose XT (N×K, k-contiguous)
      t.M = kb; t.N = k; t.K = k; t.batch = B;
      t.A = WA + k * C; t.lda = C; t.sA = CC;
      t.B = XT; t.ldb = C; t.sB = CC; t.b_kcontig = 1;
      t.D = TI; t.ldd = C; t.sD = NBO * C;
      t.tri = 2;  // X lower triangular: XT[n][kk] = 0 for kk < n
      t.skip = st;
      G2PTQ_TRY(gemm_f32(side.stream2, t));
      GemmF32 x;
      x.M = kb; x.N = k; x.K = kb; x.batch = B;
      x.A = WA + k * C + k; x.lda = C; x.sA = CC;
      x.B = TI; x.ldb = C; x.sB = NBO * C;
      x.D = WA + k * C; x.ldd = C; x.sD = CC;
      x.alpha = -1.f; x.tri = 1;  // X_kk lower triangular
      x.skip = st;
      G2PTQ_TRY(gemm_f32(side.stream2, x));
    }
    if (k + kb < C) {  // later block rows read this one (and its diagonal block) from XT
      hipLaunchKernelGGL(xt_store_kernel, dim3((unsigned)cdiv(k + kb, 64), (unsigned)cdiv(kb, 64),
                                               (unsigned)B),
                         dim3(256), 0, side.stream2, WA, C, k, kb, st, XT);
      G2PTQ_LAUNCHED();
    }
    return G2PTQ_OK;
  };
  // Rows [c0, C) × columns [c0, c1) (lower part) −= panel [k, k + kb) contribution.
  auto syrk1 = [&](hipStream_t q, int64_t k, int64_t kb, int64_t c0, int64_t c1) -> int {
    GemmF32 y;
    y.M = C - c0; y.N = c1 - c0; y.K = kb; y.batch = B;
    y.A = WA + c0 * C + k; y.lda = C; y.sA = CC;
    y.B = WA + c0 * C + k; y.ldb = C; y.sB = CC; y.b_kcontig = 1;
    y.C = WA + c0 * C + c0; y.ldc = C; y.sC = CC;
    y.D = WA + c0 * C + c0; y.ldd = C; y.sD = CC;
    y.alpha = -1.f; y.beta = 1.f; y.uplo = 1; y.skip = st;
    return gemm_f32(q, y);
  };
  // The far trailing update goes out as launches of SYRK_CHUNK columns: the
  // panel chain's kernels on the caller's stream then wait behind one chunk
  // rather than the whole update (the hardware dispatches a queue's kernels
  // in order).
  auto syrk = [&](hipStream_t q, int64_t k, int64_t kb, int64_t c0, int64_t c1) -> int {
    if (q == s) return syrk1(q, k, kb, c0, c1);
    for (int64_t c = c0; c < c1; c += SYRK_CHUNK)
      G2PTQ_TRY(syrk1(q, k, kb, c, std::min(c1, c + SYRK_CHUNK)));
    return G2PTQ_OK;
  };
  G2PTQ_TRY(factor_panel(0, std::min<int64_t>(NBO, C)));
  int pend = -1;  // ping-pong slot of the latest trailing update on the side stream
  for (int64_t k = 0, p = 0; k < C; k += NBO, ++p) {
    const int64_t kb = std::min<int64_t>(NBO, C - k);
    const int64_t next = k + kb;
    if (next >= C) break;
    const int64_t nb2 = std::min<int64_t>(NBO, C - next);
    if (next + nb2 < C) {  // trailing part beyond the next panel, on the side stream
      G2PTQ_HIP(hipEventRecord(side.factored, s));
      G2PTQ_HIP(hipStreamWaitEvent(side.stream, side.factored, 0));
      G2PTQ_TRY(syrk(side.stream, k, kb, next + nb2, C));
    }
    // The next panel's columns also received the previous trailing update.
    if (pend >= 0) G2PTQ_HIP(hipStreamWaitEvent(s, side.done[pend], 0));
    if (next + nb2 < C) {
      pend = (int)(p & 1);
      G2PTQ_HIP(hipEventRecord(side.done[pend], side.stream));
    } else {
      pend = -1;
    }
    G2PTQ_TRY(syrk(s, k, kb, next, next + nb2));
    G2PTQ_TRY(factor_panel(next, nb2));
  }
  if (pend >= 0) G2PTQ_HIP(hipStreamWaitEvent(s, side.done[pend], 0));

  if (inv_pending) {
    G2PTQ_HIP(hipEventRecord(side.inverted, side.stream2));
    G2PTQ_HIP(hipStreamWaitEvent(s, side.inverted, 0));
  }

  hipLaunchKernelGGL(unreverse_kernel, cgrid, dim3(256), 0, s, WA, C, skip, info, U);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}
