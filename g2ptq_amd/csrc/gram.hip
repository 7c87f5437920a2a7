// Hessian Gram accumulation H = beta·H + alpha·XᵀX on CDNA4 bf16 matrix cores.
//
// Operands: Xᵀ staged as a (Cp × ldt) bf16 matrix (features × tokens,
// zero padded: Cp multiple of 256, staged token counts multiple of 64), so
// both MFMA operands of an output tile H[I, J] read K-contiguous rows of the
// same buffer.
//
// Kernel shape (gram256_kernel):
//   * one workgroup = 8 wave64s = one 256×256 upper-triangular output tile
//     (I <= J); wave (wm, wn) in a 2×4 grid owns 128×64 = 4×2 tiles of
//     v_mfma_f32_32x32x16_bf16 (fp32 accumulators in AGPRs);
//   * K advances 64 tokens per stage through two LDS buffers (2 × 64 KiB);
//     the next stage's 16-byte global loads are issued before the current
//     stage's MFMAs and written to the other buffer after them, so each stage
//     needs one barrier;
//   * LDS rows are 128 bytes (64 tokens) with the eight 16-byte chunks of
//     row r stored at chunk position c ^ f(r), f(r) = (r & 7) ^ ((r >> 3) & 1),
//     which makes the ds_read_b128 operand fetches of 16 consecutive rows
//     bank-conflict free on 32- and 64-bank LDS;
//   * diagonal tiles read A and B from the same buffer (half the loads).
// When the triangle has too few tiles to fill the GPU, K is split S ways:
// each split writes its raw fp32 tile to a workspace and gram_reduce_kernel
// sums the splits in a fixed order (deterministic) into H.  Every tile is
// stored to both triangles of H, so H stays exactly symmetric.
#include "common.hpp"

namespace g2ptq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int TT = 256;   // output tile edge
constexpr int KS = 64;    // tokens per LDS stage
constexpr int NTH = 512;  // threads per workgroup (8 waves)

__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// X (T × C, ld ldx) → XT[c][t_off + t] (ld ldt) for t < roundup(T, 64),
// zero padded in both directions up to the 64-token / Cp-feature grid.
__global__ __launch_bounds__(256) void stage_kernel(const uint16_t* __restrict__ X, int64_t T,
                                                    int64_t C, int64_t ldx,
                                                    uint16_t* __restrict__ XT, int64_t ldt,
                                                    int64_t t_off) {
  __shared__ uint16_t tile[64][66];
  const int64_t t0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t t = t0 + ty + 4 * i, c = c0 + tx;
    tile[ty + 4 * i][tx] = (t < T && c < C) ? X[t * ldx + c] : (uint16_t)0;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t c = c0 + ty + 4 * i, t = t0 + tx;
    XT[c * ldt + t_off + t] = tile[tx][ty + 4 * i];
  }
}

// Zero columns [k0, k1) of the staged operand (padding up to the split grid).
__global__ void zero_cols_bf16_kernel(uint16_t* XT, int64_t ldt, int64_t rows, int64_t k0,
                                      int64_t k1) {
  const int64_t w = k1 - k0;
  const int64_t n = rows * w;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x)
    XT[(e / w) * ldt + k0 + (e % w)] = 0;
}

struct G2Args {
  const uint16_t* XT;
  int64_t ldt;
  int64_t kc;      // tokens per split (multiple of KS)
  int64_t nt;      // tiles per dimension
  int64_t C;
  int S;           // splits
  float alpha, beta;
  float* H; int64_t ldh;
  float* P;        // split partials: (tile * S + s) * TT*TT
};

__device__ __forceinline__ void tri_tile(int64_t idx, int64_t nt, int64_t& I, int64_t& J) {
  int64_t i = 0, row_len = nt;
  while (idx >= row_len) {
    idx -= row_len;
    ++i;
    --row_len;
  }
  I = i;
  J = i + idx;
}

__global__ __launch_bounds__(NTH) void gram256_kernel(G2Args a) {
  __shared__ __attribute__((aligned(16))) uint16_t Ls[2][2][TT * KS];  // [buf][A/B]

  const int64_t tile = blockIdx.x / a.S;
  const int split = blockIdx.x % a.S;
  int64_t I, J;
  tri_tile(tile, a.nt, I, J);
  const bool diag = (I == J);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;

  const uint16_t* Ag = a.XT + (I * TT) * a.ldt + (int64_t)split * a.kc;
  const uint16_t* Bg = a.XT + (J * TT) * a.ldt + (int64_t)split * a.kc;

  // Chunk q = tid + i*512 of a stage: row q >> 3, 16-byte chunk q & 7.
  // (Macros rather than lambdas: captured arrays would be forced to scratch.)
  uint4 ra0, ra1, ra2, ra3, rb0, rb1, rb2, rb3;
  const int qrow = tid >> 3, qc = tid & 7;  // chunk i adds 64 rows
  const int64_t goff = (int64_t)qrow * a.ldt + qc * 8;
  const int64_t gstep = (int64_t)64 * a.ldt;
#define G2_LOAD(k0)                                                                     \
  do {                                                                                  \
    const uint16_t* pa = Ag + goff + (k0);                                              \
    ra0 = *reinterpret_cast<const uint4*>(pa);                                          \
    ra1 = *reinterpret_cast<const uint4*>(pa + gstep);                                  \
    ra2 = *reinterpret_cast<const uint4*>(pa + 2 * gstep);                              \
    ra3 = *reinterpret_cast<const uint4*>(pa + 3 * gstep);                              \
    if (!diag) {                                                                        \
      const uint16_t* pb = Bg + goff + (k0);                                            \
      rb0 = *reinterpret_cast<const uint4*>(pb);                                        \
      rb1 = *reinterpret_cast<const uint4*>(pb + gstep);                                \
      rb2 = *reinterpret_cast<const uint4*>(pb + 2 * gstep);                            \
      rb3 = *reinterpret_cast<const uint4*>(pb + 3 * gstep);                            \
    }                                                                                   \
  } while (0)
  // LDS position of chunk i: row qrow + 64 i (same swizzle: (r >> 3) & 1 and r & 7
  // do not change when 64 is added).
  const int lpos = qrow * KS + ((qc ^ swz(qrow)) << 3);
#define G2_STORE(buf)                                                                   \
  do {                                                                                  \
    uint16_t* la = &Ls[(buf)][0][lpos];                                                 \
    *reinterpret_cast<uint4*>(la) = ra0;                                                \
    *reinterpret_cast<uint4*>(la + 64 * KS) = ra1;                                      \
    *reinterpret_cast<uint4*>(la + 128 * KS) = ra2;                                     \
    *reinterpret_cast<uint4*>(la + 192 * KS) = ra3;                                     \
    if (!diag) {                                                                        \
      uint16_t* lb = &Ls[(buf)][1][lpos];                                               \
      *reinterpret_cast<uint4*>(lb) = rb0;                                              \
      *reinterpret_cast<uint4*>(lb + 64 * KS) = rb1;                                    \
      *reinterpret_cast<uint4*>(lb + 128 * KS) = rb2;                                   \
      *reinterpret_cast<uint4*>(lb + 192 * KS) = rb3;                                   \
    }                                                                                   \
  } while (0)

  f32x16 acc[4][2];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[m][n][v] = 0.f;

  const int nk = (int)(a.kc / KS);
  G2_LOAD(0);
  G2_STORE(0);
  __syncthreads();
  const int lr = lane & 31, lh = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) G2_LOAD((int64_t)(kt + 1) * KS);
    const uint16_t* As = Ls[buf][0];
    const uint16_t* Bs = diag ? Ls[buf][0] : Ls[buf][1];
#pragma unroll
    for (int ks = 0; ks < KS / 16; ++ks) {
      const int c = ks * 2 + lh;
      bf16x8 av[4], bv[2];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int row = wm * 128 + m * 32 + lr;
        av[m] = *reinterpret_cast<const bf16x8*>(As + row * KS + ((c ^ swz(row)) << 3));
      }
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const int row = wn * 64 + n * 32 + lr;
        bv[n] = *reinterpret_cast<const bf16x8*>(Bs + row * KS + ((c ^ swz(row)) << 3));
      }
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int n = 0; n < 2; ++n)
          acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[m], bv[n], acc[m][n], 0, 0, 0);
    }
    if (kt + 1 < nk) G2_STORE(buf ^ 1);
    __syncthreads();
  }

#undef G2_LOAD
#undef G2_STORE
  // 32×32 MFMA output: lane holds rows 8*(v/4) + 4*(lane/32) + v%4, column lane%32.
  if (a.S == 1) {
    const int64_t i0 = I * TT, j0 = J * TT;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t i = i0 + wm * 128 + m * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
          const int64_t j = j0 + wn * 64 + n * 32 + lr;
          if (i >= a.C || j >= a.C || (diag && i > j)) continue;
          float* ph = a.H + i * a.ldh + j;
          const float val = (a.beta != 0.f ? a.beta * *ph : 0.f) + a.alpha * acc[m][n][v];
          *ph = val;
          if (i != j) a.H[j * a.ldh + i] = val;
        }
  } else {
    float* P = a.P + (tile * a.S + split) * (int64_t)(TT * TT);
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int il = wm * 128 + m * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
          const int jl = wn * 64 + n * 32 + lr;
          P[il * TT + jl] = acc[m][n][v];
        }
  }
}

// H[I,J] = beta·H + alpha·Σ_s partial_s (fixed order), mirrored.
__global__ __launch_bounds__(256) void gram_reduce_kernel(G2Args a) {
  const int64_t tile = blockIdx.y;
  int64_t I, J;
  tri_tile(tile, a.nt, I, J);
  const bool diag = (I == J);
  const int64_t e0 = (int64_t)blockIdx.x * 1024;
  const float* P = a.P + tile * a.S * (int64_t)(TT * TT);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t e = e0 + q * 256 + threadIdx.x;
    const int il = (int)(e / TT), jl = (int)(e % TT);
    const int64_t i = I * TT + il, j = J * TT + jl;
    if (i >= a.C || j >= a.C || (diag && i > j)) continue;
    float s = 0.f;
    for (int sp = 0; sp < a.S; ++sp) s += P[sp * (int64_t)(TT * TT) + e];
    float* ph = a.H + i * a.ldh + j;
    const float val = (a.beta != 0.f ? a.beta * *ph : 0.f) + a.alpha * s;
    *ph = val;
    if (i != j) a.H[j * a.ldh + i] = val;
  }
}

int choose_splits(int64_t tiles, int64_t K) {
  // Aim for >= ~4 workgroups per CU (256 CUs) while keeping >= 8 stages per split.
  int64_t S = cdiv(1024, tiles);
  const int64_t max_s = std::max<int64_t>(1, K / (KS * 8));
  S = std::max<int64_t>(1, std::min<int64_t>(S, max_s));
  return (int)std::min<int64_t>(S, 16);
}

}  // namespace

int64_t gram_padded_features(int64_t C) { return cdiv(C, TT) * TT; }

size_t gram_ws_bytes(int64_t K, int64_t C) {
  const int64_t nt = cdiv(C, TT);
  const int64_t tiles = nt * (nt + 1) / 2;
  const int64_t Kp = cdiv(std::max<int64_t>(K, 1), KS) * KS;
  const int S = choose_splits(tiles, Kp);
  if (S == 1) return 256;
  return (size_t)tiles * S * TT * TT * sizeof(float);
}

int gram_stage(hipStream_t st, const uint16_t* X, int64_t T, int64_t C, int64_t ldx, uint16_t* XT,
               int64_t ldt, int64_t t_off) {
  if (T <= 0) return G2PTQ_OK;
  const int64_t Cp = gram_padded_features(C);
  dim3 grid((unsigned)cdiv(T, 64), (unsigned)(Cp / 64));
  hipLaunchKernelGGL(stage_kernel, grid, dim3(256), 0, st, X, T, C, ldx, XT, ldt, t_off);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

int gram_accumulate(hipStream_t st, uint16_t* XT, int64_t ldt, int64_t K, int64_t C, float alpha,
                    float beta, float* H, int64_t ldh, void* ws, size_t ws_bytes) {
  const int64_t nt = cdiv(C, TT);
  const int64_t Cp = nt * TT;
  const int64_t tiles = nt * (nt + 1) / 2;
  int64_t Kp = cdiv(std::max<int64_t>(K, 1), KS) * KS;
  const int S = choose_splits(tiles, Kp);
  Kp = cdiv(Kp, (int64_t)KS * S) * KS * S;  // every split gets whole stages
  G2PTQ_CHECK(Kp <= ldt, "hessian gram: staged operand too narrow (%lld < %lld)",
              (long long)ldt, (long long)Kp);
  const int64_t K64 = cdiv(std::max<int64_t>(K, 0), KS) * KS;
  if (Kp > K64) {
    const int64_t n = Cp * (Kp - K64);
    hipLaunchKernelGGL(zero_cols_bf16_kernel, dim3((unsigned)std::min<int64_t>(cdiv(n, 256), 4096)),
                       dim3(256), 0, st, XT, ldt, Cp, K64, Kp);
    G2PTQ_LAUNCHED();
  }
  G2Args a{};
  a.XT = XT; a.ldt = ldt; a.kc = Kp / S; a.nt = nt; a.C = C; a.S = S;
  a.alpha = alpha; a.beta = beta; a.H = H; a.ldh = ldh;
  if (S > 1) {
    const size_t need = (size_t)tiles * S * TT * TT * sizeof(float);
    G2PTQ_CHECK(ws != nullptr && ws_bytes >= need, "hessian gram: workspace %zu < %zu", ws_bytes,
                need);
    a.P = static_cast<float*>(ws);
  }
  G2PTQ_CHECK(tiles * S < (1ll << 31), "hessian gram: grid too large");
  hipLaunchKernelGGL(gram256_kernel, dim3((unsigned)(tiles * S)), dim3(NTH), 0, st, a);
  G2PTQ_LAUNCHED();
  if (S > 1) {
    hipLaunchKernelGGL(gram_reduce_kernel, dim3(TT * TT / 1024, (unsigned)tiles), dim3(256), 0, st,
                       a);
    G2PTQ_LAUNCHED();
  }
  return G2PTQ_OK;
}

// One-shot update (stage + accumulate) through a caller workspace laid out as
// [staged Xᵀ: Cp × ldt bf16][split partials].
static int64_t update_ldt(int64_t T, int64_t C) {
  const int64_t nt = cdiv(C, TT);
  const int64_t tiles = nt * (nt + 1) / 2;
  const int64_t K64 = cdiv(std::max<int64_t>(T, 1), KS) * KS;
  const int S = choose_splits(tiles, K64);
  return cdiv(K64, (int64_t)KS * S) * KS * S;
}

size_t gram_update_ws_bytes(int64_t T, int64_t C) {
  const int64_t ldt = update_ldt(T, C);
  const size_t xt = ((size_t)gram_padded_features(C) * ldt * 2 + 255) / 256 * 256;
  return xt + gram_ws_bytes(T, C);
}

}  // namespace g2ptq

using namespace g2ptq;

extern "C" int g2ptq_hessian_update(void* stream, const uint16_t* X, int64_t T, int64_t C,
                                    int64_t ldx, float alpha, float beta, float* H, int64_t ldh,
                                    void* ws, size_t ws_bytes) {
  G2PTQ_CHECK(H != nullptr && (X != nullptr || T == 0) && C > 0 && T >= 0,
              "hessian_update: bad arguments");
  const size_t need = gram_update_ws_bytes(T, C);
  G2PTQ_CHECK(ws != nullptr && ws_bytes >= need, "hessian_update: workspace %zu < %zu", ws_bytes,
              need);
  hipStream_t st = as_stream(stream);
  const int64_t ldt = update_ldt(T, C);
  uint16_t* XT = static_cast<uint16_t*>(ws);
  const size_t xt = ((size_t)gram_padded_features(C) * ldt * 2 + 255) / 256 * 256;
  G2PTQ_TRY(gram_stage(st, X, T, C, ldx, XT, ldt, 0));
  return gram_accumulate(st, XT, ldt, T, C, alpha, beta, H, ldh, static_cast<char*>(ws) + xt,
                         ws_bytes - xt);
}

extern "C" int g2ptq_hessian_stage_rows(int64_t C, int64_t* rows) {
  G2PTQ_CHECK(rows != nullptr && C > 0, "hessian_stage_rows: bad arguments");
  *rows = gram_padded_features(C);
  return G2PTQ_OK;
}

extern "C" int g2ptq_hessian_stage(void* stream, const uint16_t* X, int64_t T, int64_t C,
                                   int64_t ldx, uint16_t* XT, int64_t ldt, int64_t t_off) {
  G2PTQ_CHECK(XT && (X || T == 0) && C > 0 && T >= 0, "hessian_stage: bad arguments");
  G2PTQ_CHECK(t_off % 64 == 0 && t_off + cdiv(T, 64) * 64 <= ldt,
              "hessian_stage: token offset %lld (+%lld) outside the staged width %lld",
              (long long)t_off, (long long)T, (long long)ldt);
  return gram_stage(as_stream(stream), X, T, C, ldx, XT, ldt, t_off);
}

extern "C" int g2ptq_hessian_gram_workspace(int64_t K, int64_t C, size_t* bytes) {
  G2PTQ_CHECK(bytes != nullptr && C > 0, "hessian_gram_workspace: bad arguments");
  *bytes = gram_ws_bytes(K, C);
  return G2PTQ_OK;
}

extern "C" int g2ptq_hessian_gram(void* stream, uint16_t* XT, int64_t ldt, int64_t K, int64_t C,
                                  float alpha, float beta, float* H, int64_t ldh, void* ws,
                                  size_t ws_bytes) {
  G2PTQ_CHECK(XT && H && C > 0 && K >= 0, "hessian_gram: bad arguments");
  return gram_accumulate(as_stream(stream), XT, ldt, K, C, alpha, beta, H, ldh, ws, ws_bytes);
}
