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
//      as a GEMM with that inverse;  update of the panel's remaining
//      columns;  then one SYRK trailing update per panel (K = 512) as a
//      lower-triangular fp32 MFMA GEMM
//   3. the triangular inverse X = L̂⁻¹ panel by panel, as soon as each is
//      factored, on a third stream beside the Cholesky: the diagonal block
//      by recursive doubling from the NB inverses, then the block row
//      X[p, 0:p] = −X_pp·(L[p, 0:p]·X[0:p, 0:p]) as two GEMMs
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
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(1, 1))) void potrf_diag_kernel(
    float* WA, int64_t C, int64_t k, int nbk, int* st, int* info) {
  const int64_t b = blockIdx.x;
  __shared__ __attribute__((aligned(16))) float Xs[POT_NB * XP];
  __shared__ __attribute__((aligned(16))) float colL[2][POT_NB];
  __shared__ float rdl[2];
  __shared__ int fail_s;
  float* Wb = WA + b * C * C + k * C + k;
  const int i = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int skip = st[b];
  // Lower triangle of the block: row r through lane i of wave r & 1
  // (coalesced; addresses clamped into the block so the loads need no
  // branches), all 32 rows of a wave in flight together, transposed through
  // LDS so that lane i of wave 0 holds row i.
  {
    const int ci = i < nbk ? i : nbk - 1;
    float x[POT_NB / 2];
#pragma unroll
    for (int h = 0; h < POT_NB / 2; ++h) {
      const int r = 2 * h + w;
      const int rr = r < nbk ? r : nbk - 1;
      x[h] = Wb[(int64_t)rr * C + ci];
    }
#pragma unroll
    for (int h = 0; h < POT_NB / 2; ++h) {
      const int r = 2 * h + w;
      Xs[r * XP + i] = (r < nbk && i < nbk) ? (i <= r ? x[h] : 0.f) : (r == i ? 1.f : 0.f);
    }
  }
  __syncthreads();
  const int fail = potrf_core(Xs, colL, rdl, &fail_s);
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
    for (int r = w; r < nbk; r += 2) Wb[(int64_t)r * C + i] = (i <= r) ? Xs[r * XP + i] : 0.f;
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
  size_t wa, wt, ti, sums, st, total;
};

FactorWs factor_ws(int64_t B, int64_t C) {
  FactorWs w;
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  w.wa = al((size_t)B * C * C * 4);
  const int64_t half = std::min<int64_t>((C + 1) / 2, NBO);
  w.wt = al((size_t)B * half * half * 4 + 4);        // in-panel inverse products
  w.ti = al((size_t)B * NBO * C * 4 + 4);            // inverse block-row products
  w.sums = al((size_t)B * 4);
  w.st = al((size_t)B * 4);
  w.total = w.wa + w.wt + w.ti + w.sums + w.st;
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
  float* sums = reinterpret_cast<float*>(base + w.wa + w.wt + w.ti);
  int* st = reinterpret_cast<int*>(base + w.wa + w.wt + w.ti + w.sums);
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
  // one by the panel-remainder update that produces it (its top-left
  // workgroup factors the block in LDS right after computing it).
  // Once a panel is factored, a third stream inverts it into X = L̂⁻¹:
  //   the panel's diagonal block (recursive doubling from the NB inverses,
  //   in place), then, in block-row order so that X[0:k, 0:k] is final,
  //   TI = L[k:kend, 0:k] · X[0:k, 0:k];  X[k:kend, 0:k] = −X_kk · TI,
  //   written over L[k:kend, 0:k].
  // The Cholesky reads neither the diagonal block nor the block row again:
  // the trailing updates that read the block row completed before the panel
  // was factored, and those of the panel itself read only the rows below it.
  SideStream side;
  G2PTQ_TRY(side_stream(s, side));
  bool inv_pending = false;  // inverse work queued on stream2
  auto factor_panel = [&](int64_t k, int64_t kb) -> int {
    bool fused = false;
    for (int64_t j = k; j < k + kb; j += NB) {
      const int nbk = (int)std::min<int64_t>(NB, k + kb - j);
      if (!fused) {
        hipLaunchKernelGGL(potrf_diag_kernel, dim3((unsigned)B), dim3(128), 0, s, WA, C, j, nbk,
                           st, info);
        G2PTQ_LAUNCHED();
      }
      fused = false;
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
      y.pot_nb = (int)std::min<int64_t>(NB, pw); y.pot_k = j + nbk;
      y.pot_st = st; y.pot_info = info;
      G2PTQ_TRY(gemm_f32(s, y));
      fused = true;
    }
    G2PTQ_HIP(hipEventRecord(side.factored, s));
    G2PTQ_HIP(hipStreamWaitEvent(side.stream2, side.factored, 0));
    inv_pending = true;
    G2PTQ_TRY(trtri_levels(side.stream2, k, kb, NB, NBO));
    if (k > 0) {
      GemmF32 t;
      t.M = kb; t.N = k; t.K = k; t.batch = B;
      t.A = WA + k * C; t.lda = C; t.sA = CC;
      t.B = WA; t.ldb = C; t.sB = CC;
      t.D = TI; t.ldd = C; t.sD = NBO * C;
      t.tri = 2;  // X lower triangular
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
