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

// X (T × C, ld ldx) → XT[c][t_off + t] for t < roundup(T, 64), zero padded in
// both directions up to the 64-token / Cp-feature grid.  No LDS: each thread
// loads an 8-token × 8-feature block (eight 16-byte row pieces), transposes
// it in registers with byte permutes, and stores eight 16-byte pieces of
// feature rows.  A wave covers 64 tokens × 64 features; the 8 lanes sharing a
// token row (or a feature row) touch one contiguous 128-byte segment.
constexpr int ST_T = 64, ST_C = 256;  // tokens × features per workgroup (4 waves)

// Low / high 16-bit halves of two words → one word (v_perm_b32 selectors).
__device__ __forceinline__ uint32_t lo_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t hi_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

__global__ __launch_bounds__(256) void stage_kernel(const uint16_t* __restrict__ X, int64_t T,
                                                    int64_t C, int64_t ldx,
                                                    uint16_t* __restrict__ XT, int64_t ldt,
                                                    int64_t t_off, int64_t t_end, int vec) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tb = lane >> 3, fb = lane & 7;
  const int64_t t0 = (int64_t)blockIdx.x * ST_T + tb * 8;
  const int64_t f0 = (int64_t)blockIdx.y * ST_C + wave * 64 + fb * 8;
  // r[i] = features f0..f0+7 of token t0+i (4 words, 2 bf16 each)
  uint32_t r[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t t = t0 + i;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (t < T) {
      if (vec && f0 + 8 <= C) {
        v = *reinterpret_cast<const uint4*>(X + t * ldx + f0);
      } else {
        uint16_t e[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) e[k] = (f0 + k < C) ? X[t * ldx + f0 + k] : (uint16_t)0;
        v.x = e[0] | ((uint32_t)e[1] << 16); v.y = e[2] | ((uint32_t)e[3] << 16);
        v.z = e[4] | ((uint32_t)e[5] << 16); v.w = e[6] | ((uint32_t)e[7] << 16);
      }
    }
    r[i][0] = v.x; r[i][1] = v.y; r[i][2] = v.z; r[i][3] = v.w;
  }
  if (t0 >= t_end) return;  // t_end is a multiple of 8
  // Output row f0 + 2w (+1): tokens t0..t0+7 = low (high) halves of r[0..7][w].
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint4 even = make_uint4(lo_lo(r[0][w], r[1][w]), lo_lo(r[2][w], r[3][w]),
                                  lo_lo(r[4][w], r[5][w]), lo_lo(r[6][w], r[7][w]));
    const uint4 odd = make_uint4(hi_hi(r[0][w], r[1][w]), hi_hi(r[2][w], r[3][w]),
                                 hi_hi(r[4][w], r[5][w]), hi_hi(r[6][w], r[7][w]));
    *reinterpret_cast<uint4*>(XT + (f0 + 2 * w) * ldt + t_off + t0) = even;
    *reinterpret_cast<uint4*>(XT + (f0 + 2 * w + 1) * ldt + t_off + t0) = odd;
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
  int64_t kc;      // tokens per split (an even number of KS stages)
  int64_t nt;      // tiles per dimension
  int64_t tiles;   // nt (nt + 1) / 2
  int64_t C;
  int S;           // splits
  float alpha, beta;
  float* H; int64_t ldh;
  float* P;        // split partials: (tile * S + s) * TT*TT
};

// Upper-triangle tile number idx → (I, J), in row-major order.
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

// Upper-triangle tile number idx → (I, J) in a blocked order: bands of GB
// tile-rows, each band walked column by column (I fastest), so that
// consecutive tiles share their A panels (band rows) and, GB at a time, their
// B panel (column J).
constexpr int GB = 8;
__device__ __forceinline__ void band_tile(int64_t idx, int64_t nt, int64_t& I, int64_t& J) {
  int64_t g0 = 0;
  for (;;) {
    const int64_t h = nt - g0 < GB ? nt - g0 : GB;
    const int64_t tri = h * (h + 1) / 2;
    const int64_t total = tri + (nt - g0 - h) * h;
    if (idx < total) {
      if (idx < tri) {
        int64_t j = 0;
        while (idx > j) {  // column j of the band's triangle holds j + 1 tiles
          idx -= j + 1;
          ++j;
        }
        J = g0 + j;
        I = g0 + idx;
      } else {
        idx -= tri;
        J = g0 + h + idx / h;
        I = g0 + idx % h;
      }
      return;
    }
    idx -= total;
    g0 += h;
  }
}

template <bool HAS_BETA>
__global__ __launch_bounds__(NTH) void gram256_kernel(G2Args a) {
  __shared__ __attribute__((aligned(16))) uint16_t Ls[2][2][TT * KS];  // [buf][A/B]

  // Workgroups are dispatched round-robin over the 8 XCDs (each with its own
  // L2): renumber so that every XCD runs one contiguous range of the work
  // list, split-major and band-ordered, so that the workgroups resident on an
  // XCD read the same panels of the same K range.  A permutation for any grid.
  const int64_t nwg = gridDim.x, bid = blockIdx.x;
  const int64_t q8 = nwg >> 3, r8 = nwg & 7, xcd = bid & 7;
  const int64_t id = xcd * q8 + (xcd < r8 ? xcd : r8) + (bid >> 3);
  const int split = (int)(id / a.tiles);
  const int64_t tile_ord = id - (int64_t)split * a.tiles;
  int64_t I, J;
  band_tile(tile_ord, a.nt, I, J);
  int64_t tile;  // row-major tile number (partials layout)
  tile = I * a.nt - I * (I - 1) / 2 + (J - I);
  const bool diag = (I == J);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;

  const uint16_t* Ag = a.XT + (I * TT) * a.ldt + (int64_t)split * a.kc;
  const uint16_t* Bg = a.XT + (J * TT) * a.ldt + (int64_t)split * a.kc;

  // Chunk q = tid + i*512 of a stage: row q >> 3, 16-byte chunk q & 7.
  // Two register sets carry stages kt+1 and kt+2 while stage kt is multiplied.
  // (Macros rather than lambdas: captured arrays would be forced to scratch.)
  uint4 xa0, xa1, xa2, xa3, xb0, xb1, xb2, xb3;
  uint4 ya0, ya1, ya2, ya3, yb0, yb1, yb2, yb3;
  const int qrow = tid >> 3, qc = tid & 7;  // chunk i adds 64 rows
  const int64_t goff = (int64_t)qrow * a.ldt + qc * 8;
  const int64_t gstep = (int64_t)64 * a.ldt;
  const int nk = (int)(a.kc / KS);
#define G2_LOAD(R, st)                                                                  \
  do {                                                                                  \
    const int64_t k0_ = (int64_t)((st) < nk ? (st) : nk - 1) * KS;                      \
    const uint16_t* pa = Ag + goff + k0_;                                               \
    const uint16_t* pb = Bg + goff + k0_;                                               \
    R##a0 = *reinterpret_cast<const uint4*>(pa);                                        \
    R##a1 = *reinterpret_cast<const uint4*>(pa + gstep);                                \
    R##a2 = *reinterpret_cast<const uint4*>(pa + 2 * gstep);                            \
    R##a3 = *reinterpret_cast<const uint4*>(pa + 3 * gstep);                            \
    R##b0 = *reinterpret_cast<const uint4*>(pb);                                        \
    R##b1 = *reinterpret_cast<const uint4*>(pb + gstep);                                \
    R##b2 = *reinterpret_cast<const uint4*>(pb + 2 * gstep);                            \
    R##b3 = *reinterpret_cast<const uint4*>(pb + 3 * gstep);                            \
  } while (0)
  // LDS position of chunk i: row qrow + 64 i (same swizzle: (r >> 3) & 1 and r & 7
  // do not change when 64 is added).
  const int lpos = qrow * KS + ((qc ^ swz(qrow)) << 3);
#define G2_STORE(R, buf)                                                                \
  do {                                                                                  \
    uint16_t* la = &Ls[(buf)][0][lpos];                                                 \
    uint16_t* lb = &Ls[(buf)][1][lpos];                                                 \
    *reinterpret_cast<uint4*>(la) = R##a0;                                              \
    *reinterpret_cast<uint4*>(la + 64 * KS) = R##a1;                                    \
    *reinterpret_cast<uint4*>(la + 128 * KS) = R##a2;                                   \
    *reinterpret_cast<uint4*>(la + 192 * KS) = R##a3;                                   \
    *reinterpret_cast<uint4*>(lb) = R##b0;                                              \
    *reinterpret_cast<uint4*>(lb + 64 * KS) = R##b1;                                    \
    *reinterpret_cast<uint4*>(lb + 128 * KS) = R##b2;                                   \
    *reinterpret_cast<uint4*>(lb + 192 * KS) = R##b3;                                   \
  } while (0)

  f32x16 acc[4][2];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[m][n][v] = 0.f;

  const int lr = lane & 31, lh = lane >> 5;
#define G2_MMA(buf)                                                                     \
  do {                                                                                  \
    const uint16_t* As = Ls[(buf)][0];                                                  \
    const uint16_t* Bs = Ls[(buf)][1];                                                  \
    _Pragma("unroll") for (int ks = 0; ks < KS / 16; ++ks) {                            \
      const int c = ks * 2 + lh;                                                        \
      bf16x8 av[4], bv[2];                                                              \
      _Pragma("unroll") for (int m = 0; m < 4; ++m) {                                   \
        const int row = wm * 128 + m * 32 + lr;                                         \
        av[m] = *reinterpret_cast<const bf16x8*>(As + row * KS + ((c ^ swz(row)) << 3)); \
      }                                                                                 \
      _Pragma("unroll") for (int n = 0; n < 2; ++n) {                                   \
        const int row = wn * 64 + n * 32 + lr;                                          \
        bv[n] = *reinterpret_cast<const bf16x8*>(Bs + row * KS + ((c ^ swz(row)) << 3)); \
      }                                                                                 \
      _Pragma("unroll") for (int m = 0; m < 4; ++m)                                     \
      _Pragma("unroll") for (int n = 0; n < 2; ++n)                                     \
        acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[m], bv[n], acc[m][n], 0, 0, 0); \
    }                                                                                   \
  } while (0)

  // nk is even (the host pads every split to an even number of stages).
  // Loads past the last stage re-read the last stage and are never used.
  // Main loop, two stages per trip.  Stage kt is multiplied out of LDS buffer
  // kt&1 while, interleaved with its MFMAs, the registers holding stage kt+1
  // are written to the other buffer and refilled with stage kt+3; one barrier
  // per stage.  The sched_group_barrier pattern spreads the 8 LDS writes and 8
  // global loads of a stage over its 32 MFMAs (1 of each per 4 MFMAs), so the
  // vector-memory and LDS-write traffic overlaps the matrix cores instead of
  // stalling them around the barrier.
#define G2_PATTERN()                                                                    \
  do {                                                                                  \
    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0); /* DS read  */                   \
    _Pragma("unroll") for (int r_ = 0; r_ < 8; ++r_) {                                  \
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0); /* MFMA */                     \
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0); /* DS write */                 \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                \
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); /* VMEM read */                \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                \
      if (r_ < 6) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);                    \
    }                                                                                   \
  } while (0)
  G2_LOAD(x, 0);
  G2_STORE(x, 0);
  G2_LOAD(x, 1);
  G2_LOAD(y, 2);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    __builtin_amdgcn_sched_barrier(0);
    G2_MMA(0);           // stage kt
    G2_STORE(x, 1);      // stage kt+1
    G2_LOAD(x, kt + 3);
    G2_PATTERN();
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    G2_MMA(1);           // stage kt+1
    G2_STORE(y, 0);      // stage kt+2
    G2_LOAD(y, kt + 4);
    G2_PATTERN();
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
  }
  __builtin_amdgcn_sched_barrier(0);
#undef G2_PATTERN
#undef G2_LOAD
#undef G2_STORE
#undef G2_MMA

  // 32×32 MFMA output: lane holds rows 8*(v/4) + 4*(lane/32) + v%4, column lane%32.
  // Mirror stores: the four rows v..v+3 of one lane are four consecutive
  // columns of the transposed element row, stored as one 16-byte vector.
  // With beta != 0 the 32 H values of one m-slice are loaded together before
  // any of them is stored (the compiler cannot prove that stores to H do not
  // alias later loads, so interleaved read-modify-writes would serialise one
  // memory round trip per element).
  if (a.S == 1) {
    const int64_t i0 = I * TT, j0 = J * TT;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      float hv[2][16];
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t i = i0 + wm * 128 + m * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
          const int64_t j = j0 + wn * 64 + n * 32 + lr;
          hv[n][v] = (HAS_BETA && i < a.C && j < a.C) ? a.H[i * a.ldh + j] : 0.f;
        }
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) {
          const int64_t ib = i0 + wm * 128 + m * 32 + 8 * vq + 4 * lh;  // rows ib..ib+3
          const int64_t j = j0 + wn * 64 + n * 32 + lr;
          float val[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int64_t i = ib + u;
            val[u] = (HAS_BETA ? a.beta * hv[n][4 * vq + u] : 0.f) + a.alpha * acc[m][n][4 * vq + u];
            if (i >= a.C || j >= a.C || (diag && i > j)) continue;
            a.H[i * a.ldh + j] = val[u];
          }
          if (j >= a.C) continue;
          if (!diag && ib + 3 < a.C && (a.ldh & 3) == 0) {
            *reinterpret_cast<float4*>(a.H + j * a.ldh + ib) =
                make_float4(val[0], val[1], val[2], val[3]);
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int64_t i = ib + u;
              if (i < a.C && i < j) a.H[j * a.ldh + i] = val[u];
            }
          }
        }
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

// H[I,J] = beta·H + alpha·Σ_s partial_s (fixed order), mirrored.  One
// workgroup reduces a 64×64 block of a tile: rows are read and written as
// 16-byte vectors, and the mirror goes through an LDS transpose so that it is
// written in rows as well.
__global__ __launch_bounds__(256) void gram_reduce_kernel(G2Args a) {
  __shared__ float tr[64][65];
  const int64_t tile = blockIdx.y;
  int64_t I, J;
  tri_tile(tile, a.nt, I, J);
  const bool diag = (I == J);
  const int bi = blockIdx.x >> 2, bj = blockIdx.x & 3;  // 64×64 block within the tile
  if (diag && bi > bj) return;                          // strictly below the diagonal
  const bool full = !diag || bi < bj;                    // no element on or below the diagonal
  const float* __restrict__ P = a.P + tile * a.S * (int64_t)(TT * TT);
  float* __restrict__ Hm = a.H;
  const int tid = threadIdx.x;
  const int cq = tid & 15, r0 = tid >> 4;
  const int64_t ti = I * TT + bi * 64, tj = J * TT + bj * 64;  // global block origin
  const bool vec = (a.ldh & 3) == 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = r0 + 16 * k;  // row within the block
    const int il = bi * 64 + r, jl = bj * 64 + cq * 4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int sp = 0; sp < a.S; ++sp) {
      const float4 p = *reinterpret_cast<const float4*>(P + sp * (int64_t)(TT * TT) + il * TT + jl);
      s.x += p.x; s.y += p.y; s.z += p.z; s.w += p.w;
    }
    const int64_t i = ti + r, j = tj + cq * 4;
    float out[4] = {s.x, s.y, s.z, s.w};
    if (i < a.C) {
      float* ph = Hm + i * a.ldh + j;
      if (full && vec && j + 3 < a.C) {
        float4 h = a.beta != 0.f ? *reinterpret_cast<const float4*>(ph) : make_float4(0.f, 0.f, 0.f, 0.f);
        out[0] = a.beta * h.x + a.alpha * out[0];
        out[1] = a.beta * h.y + a.alpha * out[1];
        out[2] = a.beta * h.z + a.alpha * out[2];
        out[3] = a.beta * h.w + a.alpha * out[3];
        *reinterpret_cast<float4*>(ph) = make_float4(out[0], out[1], out[2], out[3]);
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (j + u >= a.C || (diag && i > j + u)) continue;
          out[u] = (a.beta != 0.f ? a.beta * ph[u] : 0.f) + a.alpha * out[u];
          ph[u] = out[u];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) tr[r][cq * 4 + u] = out[u];
  }
  __syncthreads();
  // Mirror: element (i, j) of the block goes to H[j][i]; thread writes row j.
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = r0 + 16 * k;  // column of the block = row of the mirror
    const int64_t j = tj + c, ib = ti + cq * 4;
    if (j >= a.C) continue;
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = tr[cq * 4 + u][c];
    float* pm = Hm + j * a.ldh + ib;
    if (full && vec && ib + 3 < a.C) {
      *reinterpret_cast<float4*>(pm) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (ib + u < a.C && ib + u < j) pm[u] = v[u];
    }
  }
}

// Split count: the smallest power of two that gives at least 4096 workgroups
// (16 waves of one 256×256 tile per CU), at most 16 splits and at least 16
// KS-token stages per split.  Powers of two keep every split on whole XCDs
// (the workgroup order is split-major and XCD-contiguous), so the
// workgroups of one XCD read one K range; measured on MI355X with random
// bf16 operands (C=4096: S=16; C=14336: S=4).
int choose_splits(int64_t tiles, int64_t K) {
  const int64_t smax = std::max<int64_t>(1, std::min<int64_t>(16, K / (KS * 16)));
  int S = 1;
  while (S * 2 <= smax && tiles * S < 4096) S *= 2;
  return S;
}

// Token width a split grid of S splits needs for K tokens: every split gets an
// even number of KS-token stages.
int64_t padded_tokens(int64_t K, int S) {
  const int64_t step = (int64_t)2 * KS * S;
  return cdiv(std::max<int64_t>(K, 1), step) * step;
}

}  // namespace

int64_t gram_padded_features(int64_t C) { return cdiv(C, TT) * TT; }

size_t gram_ws_bytes(int64_t K, int64_t C) {
  const int64_t nt = cdiv(C, TT);
  const int64_t tiles = nt * (nt + 1) / 2;
  const int S = choose_splits(tiles, std::max<int64_t>(K, 1));
  if (S == 1) return 256;
  return (size_t)tiles * S * TT * TT * sizeof(float);
}

int gram_stage(hipStream_t st, const uint16_t* X, int64_t T, int64_t C, int64_t ldx, uint16_t* XT,
               int64_t ldt, int64_t t_off) {
  if (T <= 0) return G2PTQ_OK;
  const int64_t Cp = gram_padded_features(C);
  const int64_t T64 = cdiv(T, KS) * KS;
  const int vec = (ldx % 8 == 0) && ((reinterpret_cast<uintptr_t>(X) & 15) == 0);
  G2PTQ_CHECK(ldt % 8 == 0 && t_off % 8 == 0 && (reinterpret_cast<uintptr_t>(XT) & 15) == 0,
              "hessian stage: XT must be 16-byte aligned with ldt and t_off multiples of 8");
  dim3 grid((unsigned)cdiv(T, (int64_t)ST_T), (unsigned)(Cp / ST_C));
  hipLaunchKernelGGL(stage_kernel, grid, dim3(256), 0, st, X, T, C, ldx, XT, ldt, t_off, T64, vec);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

int gram_accumulate(hipStream_t st, uint16_t* XT, int64_t ldt, int64_t K, int64_t C, float alpha,
                    float beta, float* H, int64_t ldh, void* ws, size_t ws_bytes) {
  const int64_t nt = cdiv(C, TT);
  const int64_t Cp = nt * TT;
  const int64_t tiles = nt * (nt + 1) / 2;
  const int S = choose_splits(tiles, std::max<int64_t>(K, 1));
  const int64_t Kp = padded_tokens(K, S);
  G2PTQ_CHECK(Kp <= ldt, "hessian gram: staged operand too narrow (%lld < %lld)",
              (long long)ldt, (long long)Kp);
  G2PTQ_CHECK((reinterpret_cast<uintptr_t>(XT) & 15) == 0 && ldt % 8 == 0,
              "hessian gram: XT must be 16-byte aligned with ldt a multiple of 8");
  const int64_t K64 = cdiv(std::max<int64_t>(K, 0), KS) * KS;
  if (Kp > K64) {
    const int64_t n = Cp * (Kp - K64);
    hipLaunchKernelGGL(zero_cols_bf16_kernel, dim3((unsigned)std::min<int64_t>(cdiv(n, 256), 4096)),
                       dim3(256), 0, st, XT, ldt, Cp, K64, Kp);
    G2PTQ_LAUNCHED();
  }
  G2Args a{};
  a.XT = XT; a.ldt = ldt; a.kc = Kp / S; a.nt = nt; a.tiles = tiles; a.C = C; a.S = S;
  a.alpha = alpha; a.beta = beta; a.H = H; a.ldh = ldh;
  if (S > 1) {
    const size_t need = (size_t)tiles * S * TT * TT * sizeof(float);
    G2PTQ_CHECK(ws != nullptr && ws_bytes >= need, "hessian gram: workspace %zu < %zu", ws_bytes,
                need);
    a.P = static_cast<float*>(ws);
  }
  G2PTQ_CHECK(tiles * S < (1ll << 31), "hessian gram: grid too large");
  if (S == 1 && beta != 0.f)
    hipLaunchKernelGGL(gram256_kernel<true>, dim3((unsigned)(tiles * S)), dim3(NTH), 0, st, a);
  else
    hipLaunchKernelGGL(gram256_kernel<false>, dim3((unsigned)(tiles * S)), dim3(NTH), 0, st, a);
  G2PTQ_LAUNCHED();
  if (S > 1) {
    hipLaunchKernelGGL(gram_reduce_kernel, dim3(16, (unsigned)tiles), dim3(256), 0, st, a);
    G2PTQ_LAUNCHED();
  }
  return G2PTQ_OK;
}

// One-shot update (stage + accumulate) through a caller workspace laid out as
// [staged Xᵀ: Cp × ldt bf16][split partials].
static int64_t update_ldt(int64_t T, int64_t C) {
  const int64_t nt = cdiv(C, TT);
  const int64_t tiles = nt * (nt + 1) / 2;
  return padded_tokens(T, choose_splits(tiles, std::max<int64_t>(T, 1)));
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
