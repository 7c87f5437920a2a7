// Hessian Gram products on CDNA4 bf16 matrix cores:
//
//   H  = beta·H  + alpha·XᵀX                     (GPTQ, gptq_utils.py:115-126)
//   Dx = beta·Dx + alpha·(X_fp − X)ᵀX            (GPTAQ, gptaq_utils.py:130-148)
//   H[g] = beta·H[g] + alpha·Σ_t s[t,g]·x_t x_tᵀ (G2PTQ / GuidedQuant,
//                                                  g2ptq_utils.py:182-201,
//                                                  gptq_guided_utils.py:59-81)
//
// Operands are staged feature-major: a stage kernel transposes each token-major
// batch into planes of (Cp × ldt) bf16 (features × tokens, zero padded: Cp a
// multiple of 256, staged token counts multiples of 64), so both MFMA operands
// of an output tile read K-contiguous rows.  Plane 0 is Xᵀ.  Operands that are
// not bf16-exact are split into two bf16 parts, hi = bf16(v) and
// lo = bf16(v − hi), which carry 16 significant bits (the residual is below
// 2⁻¹⁶·|v|): GPTAQ stages v = x_fp − x (exact in fp32) as two planes; the
// weighted Hessians stage one fp32 weight per (group, token) and
// wgram_kernel forms v = x·s[t,g]·s_scale and its split on the way into LDS
// (fp16/fp32 activations stage the split as planes).  A product v·x is then
// the two exact bf16 products hi·x + lo·x, accumulated in fp32.
//
// Kernel shape (gram256_kernel):
//   * one workgroup = 8 wave64s = one 256×256 output tile; wave (wm, wn) in a
//     2×4 grid owns 128×64 = 4×2 tiles of v_mfma_f32_32x32x16_bf16 (fp32
//     accumulators in AGPRs).  Symmetric products compute the upper
//     triangle of tiles (I <= J) and store every tile to both triangles, so
//     H stays exactly symmetric; the GPTAQ cross term computes all tiles;
//   * K advances 64 tokens per stage through two LDS buffers (2 × 64 KiB);
//     the next stage's 16-byte global loads are issued before the current
//     stage's MFMAs and written to the other buffer after them, so each stage
//     needs one barrier;
//   * LDS rows are 128 bytes (64 tokens) with the eight 16-byte chunks of
//     row r stored at chunk position c ^ f(r), f(r) = (r & 7) ^ ((r >> 3) & 1),
//     which makes the ds_read_b128 operand fetches of 16 consecutive rows
//     bank-conflict free on 32- and 64-bank LDS.
// K is split S ways when the tile grid alone would not fill the GPU: each
// split writes its raw fp32 tile to a workspace and gram_reduce_kernel sums
// the splits in a fixed order (deterministic) into the output.  A two-plane
// (hi, lo) operand runs as a product over twice the tokens: the first half of
// the splits multiplies hi against Xᵀ, the second half lo against Xᵀ.
#include <algorithm>

#include "common.hpp"

namespace g2ptq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int TT = 256;   // output tile edge
constexpr int KS = 64;    // tokens per LDS stage
constexpr int NTH = 512;  // threads per workgroup (8 waves)

__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Staging: X (T × C, ld ldx) → plane[c][t_off + t] for t < roundup(T, 64),
// zero padded in both directions up to the 64-token / Cp-feature grid.  No
// LDS: each thread loads an 8-token × 8-feature block (eight 16-byte row
// pieces), transposes it in registers with byte permutes, and stores eight
// 16-byte pieces of feature rows.  A wave covers 64 tokens × 64 features; the
// 8 lanes sharing a token row (or a feature row) touch one contiguous
// 128-byte segment.
constexpr int ST_T = 64, ST_C = 256;  // tokens × features per workgroup (4 waves)

// Low / high 16-bit halves of two words → one word (v_perm_b32 selectors).
__device__ __forceinline__ uint32_t lo_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t hi_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // NaN stays NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// v (two fp32 values) → packed bf16 hi word and lo word, v ≈ hi + lo.
__device__ __forceinline__ void split2(float v0, float v1, uint32_t& hw, uint32_t& lw) {
  const uint32_t h0 = f32_to_bf16_rne(v0), h1 = f32_to_bf16_rne(v1);
  const uint32_t l0 = f32_to_bf16_rne(v0 - __uint_as_float(h0 << 16));
  const uint32_t l1 = f32_to_bf16_rne(v1 - __uint_as_float(h1 << 16));
  hw = h0 | (h1 << 16);
  lw = l0 | (l1 << 16);
}

struct StageArgs {
  const uint16_t* X;   // T × C bf16, ld ldx
  const uint16_t* F;   // GPTAQ: X_fp, ld ldf
  const float* S;      // weighted: T × G saliencies, ld lds
  int64_t T, C, ldx, ldf, lds;
  int G;
  float s_scale;
  uint16_t* XT;        // planes of Cp × ldt, plane stride `plane` elements
  int64_t ldt, plane, t_off, t_end;
  int vec;             // X (and F) rows 16-byte aligned
};

// r[i] = features f0..f0+7 of token t0+i (4 words, 2 bf16 each), zeros outside.
__device__ __forceinline__ void load_block(const uint16_t* __restrict__ X, int64_t ldx, int64_t T,
                                           int64_t C, int64_t t0, int64_t f0, int vec,
                                           uint32_t (&r)[8][4]) {
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
}

// Output row f0 + 2w (+1), tokens t0..t0+7 = low (high) halves of r[0..7][w].
__device__ __forceinline__ void store_block(uint16_t* __restrict__ P, int64_t ldt, int64_t f0,
                                            int64_t col, const uint32_t (&r)[8][4]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint4 even = make_uint4(lo_lo(r[0][w], r[1][w]), lo_lo(r[2][w], r[3][w]),
                                  lo_lo(r[4][w], r[5][w]), lo_lo(r[6][w], r[7][w]));
    const uint4 odd = make_uint4(hi_hi(r[0][w], r[1][w]), hi_hi(r[2][w], r[3][w]),
                                 hi_hi(r[4][w], r[5][w]), hi_hi(r[6][w], r[7][w]));
    *reinterpret_cast<uint4*>(P + (f0 + 2 * w) * ldt + col) = even;
    *reinterpret_cast<uint4*>(P + (f0 + 2 * w + 1) * ldt + col) = odd;
  }
}

// KIND 0: plane 0 = Xᵀ.  KIND 1 (GPTAQ): planes 0..2 = Xᵀ, hi and lo of
// (X_fp − X)ᵀ.  KIND 2 (weighted): plane 0 = Xᵀ, then G rows of ldt fp32
// token weights w[g][t] = S[t,g]·s_scale (wgram_kernel forms x·w itself).
template <int KIND>
__global__ __launch_bounds__(256) void stage_kernel(StageArgs s) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tb = lane >> 3, fb = lane & 7;
  const int64_t t0 = (int64_t)blockIdx.x * ST_T + tb * 8;
  const int64_t f0 = (int64_t)blockIdx.y * ST_C + wave * 64 + fb * 8;
  uint32_t r[8][4];
  load_block(s.X, s.ldx, s.T, s.C, t0, f0, s.vec, r);
  if (t0 >= s.t_end) return;  // t_end is a multiple of 8
  const int64_t col = s.t_off + t0;
  store_block(s.XT, s.ldt, f0, col, r);
  if (KIND == 1) {
    uint32_t f[8][4], h[8][4];
    load_block(s.F, s.ldf, s.T, s.C, t0, f0, s.vec, f);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        uint32_t hw, lw;
        split2(lo_f32(f[i][w]) - lo_f32(r[i][w]), hi_f32(f[i][w]) - hi_f32(r[i][w]), hw, lw);
        h[i][w] = hw;
        f[i][w] = lw;
      }
    store_block(s.XT + s.plane, s.ldt, f0, col, h);
    store_block(s.XT + 2 * s.plane, s.ldt, f0, col, f);
  }
  if (KIND == 2 && blockIdx.y == 0 && wave == 0) {
    // the weights w[g][t] = S[t,g]·s_scale of this wave's 64 tokens, fp32 rows
    // of ldt after plane 0 (lane: tokens t0..t0+7, groups fb, fb + 8, …)
    float* W = reinterpret_cast<float*>(s.XT + s.plane);
    for (int g = fb; g < s.G; g += 8) {
      float wv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        wv[i] = (t0 + i < s.T) ? s.S[(t0 + i) * s.lds + g] * s.s_scale : 0.f;
      float4* dst = reinterpret_cast<float4*>(W + g * s.ldt + col);
      dst[0] = make_float4(wv[0], wv[1], wv[2], wv[3]);
      dst[1] = make_float4(wv[4], wv[5], wv[6], wv[7]);
    }
  }
}

// Activations that are not bf16 (fp16: P = 2, fp32: P = 3) are staged as P
// bf16 planes whose sum is the value exactly: plane q holds bf16(r_q) with
// r_0 = x and r_{q+1} = r_q − bf16(r_q), each difference exact in fp32 (x and
// its nearest bf16 are within a factor of two).  An fp16 value (11
// significant bits) leaves at most 3 bits after its first plane; an fp32
// value (24) leaves at most 16, then 8.  Planes 0..P−1 then play the part of
// the bf16 path's Xᵀ, and the GPTAQ / weighted planes follow at P, P + 1, ….
template <typename TIN>
__device__ __forceinline__ void load_block_f32(const TIN* __restrict__ X, int64_t ldx, int64_t T,
                                               int64_t C, int64_t t0, int64_t f0, int vec,
                                               float (&v)[8][8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t t = t0 + i;
    if (t < T && vec && f0 + 8 <= C) {
      const TIN* row = X + t * ldx + f0;
      if constexpr (sizeof(TIN) == 2) {
        const uint4 u = *reinterpret_cast<const uint4*>(row);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          v[i][2 * k] = (float)__builtin_bit_cast(_Float16, (unsigned short)(w[k] & 0xffffu));
          v[i][2 * k + 1] = (float)__builtin_bit_cast(_Float16, (unsigned short)(w[k] >> 16));
        }
      } else {
        const float4 a = *reinterpret_cast<const float4*>(row);
        const float4 b = *reinterpret_cast<const float4*>(row + 4);
        v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w;
        v[i][4] = b.x; v[i][5] = b.y; v[i][6] = b.z; v[i][7] = b.w;
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        v[i][k] = (t < T && f0 + k < C) ? (float)X[t * ldx + f0 + k] : 0.f;
    }
  }
}

template <typename TIN, int KIND>
__global__ __launch_bounds__(256) void stage_split_kernel(StageArgs s) {
  constexpr int P = sizeof(TIN) == 2 ? 2 : 3;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tb = lane >> 3, fb = lane & 7;
  const int64_t t0 = (int64_t)blockIdx.x * ST_T + tb * 8;
  const int64_t f0 = (int64_t)blockIdx.y * ST_C + wave * 64 + fb * 8;
  float v[8][8];
  load_block_f32(reinterpret_cast<const TIN*>(s.X), s.ldx, s.T, s.C, t0, f0, s.vec, v);
  if (t0 >= s.t_end) return;  // t_end is a multiple of 8
  const int64_t col = s.t_off + t0;
  {
    float r[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int k = 0; k < 8; ++k) r[i][k] = v[i][k];
#pragma unroll
    for (int q = 0; q < P; ++q) {
      uint32_t w[8][4];
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t h0 = f32_to_bf16_rne(r[i][2 * k]);
          const uint32_t h1 = f32_to_bf16_rne(r[i][2 * k + 1]);
          w[i][k] = h0 | (h1 << 16);
          r[i][2 * k] -= __uint_as_float(h0 << 16);
          r[i][2 * k + 1] -= __uint_as_float(h1 << 16);
        }
      store_block(s.XT + q * s.plane, s.ldt, f0, col, w);
    }
  }
  if (KIND == 1) {
    float f[8][8];
    load_block_f32(reinterpret_cast<const TIN*>(s.F), s.ldf, s.T, s.C, t0, f0, s.vec, f);
    uint32_t h[8][4], l[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k)
        split2(f[i][2 * k] - v[i][2 * k], f[i][2 * k + 1] - v[i][2 * k + 1], h[i][k], l[i][k]);
    store_block(s.XT + P * s.plane, s.ldt, f0, col, h);
    store_block(s.XT + (P + 1) * s.plane, s.ldt, f0, col, l);
  }
  if (KIND == 2) {
    for (int g = 0; g < s.G; ++g) {
      float sv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        sv[i] = (t0 + i < s.T) ? s.S[(t0 + i) * s.lds + g] * s.s_scale : 0.f;
      uint32_t h[8][4], l[8][4];
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k)
          split2(v[i][2 * k] * sv[i], v[i][2 * k + 1] * sv[i], h[i][k], l[i][k]);
      store_block(s.XT + (P + 2 * g) * s.plane, s.ldt, f0, col, h);
      store_block(s.XT + (P + 2 * g + 1) * s.plane, s.ldt, f0, col, l);
    }
  }
}

// act = act_beta·act + act_alpha·Σ_t x[t,c]² over tokens [t0, t0 + len) of
// the staged Xᵀ (one wave per feature, 16-byte loads; len a multiple of 8);
// x is the sum of the P staged planes (exact, see stage_split_kernel).
__global__ __launch_bounds__(256) void act_square_kernel(const uint16_t* __restrict__ XT,
                                                         int64_t ldt, int64_t t0, int64_t len,
                                                         int64_t C, float* act, float act_alpha,
                                                         float act_beta, int P, int64_t plane) {
  const int64_t c = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (c >= C) return;
  const uint16_t* row = XT + c * ldt + t0;
  float s = 0.f;
  for (int64_t t = (int64_t)lane * 8; t < len; t += 512) {
    const uint4 v = *reinterpret_cast<const uint4*>(row + t);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float x[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = lo_f32(w[k]);
      x[2 * k + 1] = hi_f32(w[k]);
    }
    for (int q = 1; q < P; ++q) {
      const uint4 u = *reinterpret_cast<const uint4*>(row + q * plane + t);
      const uint32_t wq[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        x[2 * k] += lo_f32(wq[k]);
        x[2 * k + 1] += hi_f32(wq[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      s += x[2 * k] * x[2 * k];
      s += x[2 * k + 1] * x[2 * k + 1];
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) act[c] = act_beta * act[c] + act_alpha * s;
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
  const uint16_t* A1;  // row operand planes (Cp × ldt): A2 feeds the second and
  const uint16_t* A2;  // A3 the third part of the splits when halves is 2 or 3
  const uint16_t* A3;
  const uint16_t* B;   // column operand plane
  int64_t ldt;
  int64_t kc;      // tokens per split (an even number of KS stages)
  int64_t nt;      // tiles per dimension
  int64_t tiles;   // upper triangle nt (nt + 1) / 2, or nt² for full products
  int64_t C;
  int S;           // splits (halves × splits per half)
  int halves;
  float alpha, beta;
  float* H; int64_t ldh;
  float* P;        // split partials: (tile * S + s) * TT*TT
  // weighted products (wgram_kernel): per-group token weights and outputs
  const float* W;  // G rows of ldw fp32 weights, one per staged token
  int64_t ldw;
  int64_t G;       // groups (1 for the other products)
  int64_t sH;      // stride between the groups' outputs
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

// Full-grid tile number idx → (I, J): bands of GB tile-rows walked column by
// column.
__device__ __forceinline__ void grid_tile(int64_t idx, int64_t nt, int64_t& I, int64_t& J) {
  const int64_t per = GB * nt;
  const int64_t band = idx / per, r = idx - band * per;
  const int64_t g0 = band * GB;
  const int64_t h = nt - g0 < GB ? nt - g0 : GB;
  I = g0 + r % h;
  J = r / h;
}

// Epilogue of a 256×256 tile of 8 waves (2 × 4 wave grid, 128×64 per wave):
// H (one output matrix) = beta·H + alpha·acc, mirrored for symmetric products
// (diagonal tiles store their upper triangle both ways), or the raw tile to
// the split partials Pt when K is split (a.S > 1).
template <bool HAS_BETA, bool FULL>
__device__ __forceinline__ void store_tile(const G2Args& a, float* H, float* Pt,
                                           f32x16 (&acc)[4][2], int64_t I, int64_t J, bool diag,
                                           int wm, int wn, int lh, int lr) {
  // 32×32 MFMA output: lane holds rows 8*(v/4) + 4*(lane/32) + v%4, column lane%32.
  // Mirror stores: the four rows v..v+3 of one lane are four consecutive
  // columns of the transposed element row, stored as one 16-byte vector.
  // With beta != 0 the 32 H values of one m-slice are loaded together before
  // any of them is stored (the compiler cannot prove that stores to H do not
  // alias later loads, so interleaved read-modify-writes would serialise one
  // memory round trip per element).
  if (FULL && a.S == 1) {
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
          hv[n][v] = (HAS_BETA && i < a.C && j < a.C) ? H[i * a.ldh + j] : 0.f;
        }
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t i = i0 + wm * 128 + m * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
          const int64_t j = j0 + wn * 64 + n * 32 + lr;
          if (i < a.C && j < a.C)
            H[i * a.ldh + j] = (HAS_BETA ? a.beta * hv[n][v] : 0.f) + a.alpha * acc[m][n][v];
        }
    }
  } else if (a.S == 1) {
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
          hv[n][v] = (HAS_BETA && i < a.C && j < a.C) ? H[i * a.ldh + j] : 0.f;
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
            H[i * a.ldh + j] = val[u];
          }
          if (j >= a.C) continue;
          if (!diag && ib + 3 < a.C && (a.ldh & 3) == 0) {
            *reinterpret_cast<float4*>(H + j * a.ldh + ib) =
                make_float4(val[0], val[1], val[2], val[3]);
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int64_t i = ib + u;
              if (i < a.C && i < j) H[j * a.ldh + i] = val[u];
            }
          }
        }
    }
  } else {
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int il = wm * 128 + m * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
          const int jl = wn * 64 + n * 32 + lr;
          Pt[il * TT + jl] = acc[m][n][v];
        }
  }
}

template <bool HAS_BETA, bool FULL>
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
  int64_t tile;  // row-major tile number (partials layout)
  if (FULL) {
    grid_tile(tile_ord, a.nt, I, J);
    tile = I * a.nt + J;
  } else {
    band_tile(tile_ord, a.nt, I, J);
    tile = I * a.nt - I * (I - 1) / 2 + (J - I);
  }
  const bool diag = !FULL && (I == J);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;

  // Split → operand plane and token range.
  const int per_half = a.S / a.halves;
  const int half = split / per_half, sp = split - half * per_half;
  const uint16_t* Aop = half == 0 ? a.A1 : (half == 1 ? a.A2 : a.A3);
  const uint16_t* Ag = Aop + (I * TT) * a.ldt + (int64_t)sp * a.kc;
  const uint16_t* Bg = a.B + (J * TT) * a.ldt + (int64_t)sp * a.kc;

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

  store_tile<HAS_BETA, FULL>(a, a.H, a.S == 1 ? nullptr : a.P + (tile * a.S + split) * (int64_t)(TT * TT),
                             acc, I, J, diag, wm, wn, lh, lr);
}

// Weighted Hessians of bf16 activations, the split formed on the way into LDS:
//   H[g] = beta·H[g] + alpha·Σ_t x_t·(x_t·w[g][t])ᵀ,   w[g][t] = S[t,g]·s_scale,
// over the upper tiles of every group g, one launch for all groups.  The row
// operand is Xᵀ (panel I).  The column operand v = x·w (panel J) is formed per
// stage from Xᵀ and the staged weights, split in registers into bf16
// hi = bf16(v) and lo = bf16(v − hi) (split_chunk), written to LDS as two
// tiles, and both are multiplied into the same accumulator.  One workgroup = one (tile, group,
// split); a tile's groups are consecutive in the work list, so they run
// together on one XCD and read the same two panels through its L2.
//   * 8 waves in a 2 × 4 grid, 128×64 per wave (the gram256 epilogue);
//   * a stage is WKS = 32 tokens: three 256 × 32 bf16 tiles (Xᵀ_I, hi, lo),
//     48 KiB, double buffered; LDS rows are 64 bytes (four 16-byte chunks),
//     chunk c of row r at c ^ swz4(r), conflict free for the fragment reads
//     (16 consecutive rows, one chunk) and the stage writes (4 rows × 4
//     chunks) on 32- and 64-bank LDS;
//   * per 16-token k-step a wave reads 4 row and 2 + 2 column fragments for
//     16 MFMAs (the plane-staged path reads 6 for 8).
constexpr int WKS = 32;

__device__ __forceinline__ int swz4(int r) { return ((r >> 1) & 3) ^ ((r >> 3) & 1); }

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 values → packed bf16 (round to nearest even, v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// Eight bf16 x (tokens t..t+7 of one feature) times their weights → the hi
// and lo chunks of v = x·w: hi = bf16(fl(x·w)), lo = bf16(x·w − hi) with the
// residual formed by one fused multiply-add from the exact product, so
// hi + lo carries x·w to 16 significant bits.
__device__ __forceinline__ void split_chunk(const uint4& x, const float4& w0, const float4& w1,
                                            uint4& h, uint4& l) {
  const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
  const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  uint32_t hw[4], lw[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float x0 = lo_f32(xw[k]), x1 = hi_f32(xw[k]);
    hw[k] = pk_bf16(x0 * wv[2 * k], x1 * wv[2 * k + 1]);
    lw[k] = pk_bf16(__builtin_fmaf(x0, wv[2 * k], -lo_f32(hw[k])),
                    __builtin_fmaf(x1, wv[2 * k + 1], -hi_f32(hw[k])));
  }
  h = make_uint4(hw[0], hw[1], hw[2], hw[3]);
  l = make_uint4(lw[0], lw[1], lw[2], lw[3]);
}

template <bool HAS_BETA>
__global__ __launch_bounds__(NTH) void wgram_kernel(G2Args a) {
  __shared__ __attribute__((aligned(16))) uint16_t Lw[2][3][TT * WKS];  // [buf][Xᵀ_I / hi / lo]

  // XCD-contiguous renumbering as in gram256_kernel; the work list is
  // split-major, then band-ordered tiles, then groups.
  const int64_t nwg = gridDim.x, bid = blockIdx.x;
  const int64_t q8 = nwg >> 3, r8 = nwg & 7, xcd = bid & 7;
  const int64_t id = xcd * q8 + (xcd < r8 ? xcd : r8) + (bid >> 3);
  const int64_t grp = id % a.G, rest = id / a.G;
  const int split = (int)(rest / a.tiles);
  const int64_t tile_ord = rest - (int64_t)split * a.tiles;
  int64_t I, J;
  band_tile(tile_ord, a.nt, I, J);
  const int64_t tile = I * a.nt - I * (I - 1) / 2 + (J - I);
  const bool diag = I == J;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;

  const uint16_t* Ag = a.B + (I * TT) * a.ldt + (int64_t)split * a.kc;
  const uint16_t* Bg = a.B + (J * TT) * a.ldt + (int64_t)split * a.kc;
  // Chunk q = tid + i*512 of a stage tile: row q >> 2, 16-byte chunk q & 3.
  const int qrow = tid >> 2, qc = tid & 3;  // chunk i adds 128 rows
  const float* Wg = a.W + grp * a.ldw + (int64_t)split * a.kc + qc * 8;
  const int64_t goff = (int64_t)qrow * a.ldt + qc * 8;
  const int64_t gstep = (int64_t)128 * a.ldt;
  const int nk = (int)(a.kc / WKS);
  uint4 xa0, xa1, xb0, xb1, ya0, ya1, yb0, yb1;
  float4 xw0, xw1, yw0, yw1;
#define W_LOAD(R, st)                                                                   \
  do {                                                                                  \
    const int64_t k0_ = (int64_t)((st) < nk ? (st) : nk - 1) * WKS;                     \
    R##a0 = *reinterpret_cast<const uint4*>(Ag + goff + k0_);                           \
    R##a1 = *reinterpret_cast<const uint4*>(Ag + goff + gstep + k0_);                   \
    R##b0 = *reinterpret_cast<const uint4*>(Bg + goff + k0_);                           \
    R##b1 = *reinterpret_cast<const uint4*>(Bg + goff + gstep + k0_);                   \
    R##w0 = *reinterpret_cast<const float4*>(Wg + k0_);                                 \
    R##w1 = *reinterpret_cast<const float4*>(Wg + k0_ + 4);                             \
  } while (0)
  // rows qrow and qrow + 128 share swz4 (bits 1..3 of the row)
  const int lpos = qrow * WKS + ((qc ^ swz4(qrow)) << 3);
#define W_STORE(R, buf)                                                                 \
  do {                                                                                  \
    uint4 h0_, l0_, h1_, l1_;                                                           \
    split_chunk(R##b0, R##w0, R##w1, h0_, l0_);                                         \
    split_chunk(R##b1, R##w0, R##w1, h1_, l1_);                                         \
    uint16_t* la = &Lw[(buf)][0][lpos];                                                 \
    uint16_t* lh_ = &Lw[(buf)][1][lpos];                                                \
    uint16_t* ll_ = &Lw[(buf)][2][lpos];                                                \
    *reinterpret_cast<uint4*>(la) = R##a0;                                              \
    *reinterpret_cast<uint4*>(la + 128 * WKS) = R##a1;                                  \
    *reinterpret_cast<uint4*>(lh_) = h0_;                                               \
    *reinterpret_cast<uint4*>(lh_ + 128 * WKS) = h1_;                                   \
    *reinterpret_cast<uint4*>(ll_) = l0_;                                               \
    *reinterpret_cast<uint4*>(ll_ + 128 * WKS) = l1_;                                   \
  } while (0)

  f32x16 acc[4][2];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[m][n][v] = 0.f;

  const int lr = lane & 31, lh = lane >> 5;
#define W_MMA(buf)                                                                      \
  do {                                                                                  \
    const uint16_t* As = Lw[(buf)][0];                                                  \
    const uint16_t* Bh = Lw[(buf)][1];                                                  \
    const uint16_t* Bl = Lw[(buf)][2];                                                  \
    _Pragma("unroll") for (int ks = 0; ks < WKS / 16; ++ks) {                           \
      const int c = ks * 2 + lh;                                                        \
      bf16x8 av[4], bh[2], bl[2];                                                       \
      _Pragma("unroll") for (int m = 0; m < 4; ++m) {                                   \
        const int row = wm * 128 + m * 32 + lr;                                         \
        av[m] = *reinterpret_cast<const bf16x8*>(As + row * WKS + ((c ^ swz4(row)) << 3)); \
      }                                                                                 \
      _Pragma("unroll") for (int n = 0; n < 2; ++n) {                                   \
        const int row = wn * 64 + n * 32 + lr;                                          \
        const int off = row * WKS + ((c ^ swz4(row)) << 3);                             \
        bh[n] = *reinterpret_cast<const bf16x8*>(Bh + off);                             \
        bl[n] = *reinterpret_cast<const bf16x8*>(Bl + off);                             \
      }                                                                                 \
      _Pragma("unroll") for (int m = 0; m < 4; ++m)                                     \
      _Pragma("unroll") for (int n = 0; n < 2; ++n)                                     \
        acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[m], bh[n], acc[m][n], 0, 0, 0); \
      _Pragma("unroll") for (int m = 0; m < 4; ++m)                                     \
      _Pragma("unroll") for (int n = 0; n < 2; ++n)                                     \
        acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[m], bl[n], acc[m][n], 0, 0, 0); \
    }                                                                                   \
  } while (0)

  // nk is a multiple of 4 (the host pads every split to an even number of
  // 64-token stages); loads past the last stage re-read it and go unused.
  // Stage kt is multiplied out of buffer kt&1 while the registers holding
  // stage kt+1 are split and written to the other buffer and refilled with
  // stage kt+3; one barrier per stage.
  // Per stage: 16 fragment reads, 32 MFMAs, the split's VALU work, 6 LDS
  // writes and 6 global loads, spread so that every group of four MFMAs
  // carries a share of the other work.
#define W_PATTERN()                                                                     \
  do {                                                                                  \
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0); /* DS read  */                   \
    _Pragma("unroll") for (int r_ = 0; r_ < 8; ++r_) {                                  \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); /* MFMA */                     \
      __builtin_amdgcn_sched_group_barrier(0x002, 10, 0); /* VALU */                    \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                \
      if (r_ < 6) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0); /* DS write */     \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                \
      if (r_ < 6) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); /* VMEM read */    \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                \
      if (r_ < 4) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);                    \
    }                                                                                   \
  } while (0)
  W_LOAD(x, 0);
  W_STORE(x, 0);
  W_LOAD(x, 1);
  W_LOAD(y, 2);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    __builtin_amdgcn_sched_barrier(0);
    W_MMA(0);
    W_STORE(x, 1);
    W_LOAD(x, kt + 3);
    W_PATTERN();
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    W_MMA(1);
    W_STORE(y, 0);
    W_LOAD(y, kt + 4);
    W_PATTERN();
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
  }
#undef W_PATTERN
  __builtin_amdgcn_sched_barrier(0);
#undef W_LOAD
#undef W_STORE
#undef W_MMA

  store_tile<HAS_BETA, false>(
      a, a.H + grp * a.sH,
      a.S == 1 ? nullptr : a.P + ((grp * a.tiles + tile) * a.S + split) * (int64_t)(TT * TT), acc,
      I, J, diag, wm, wn, lh, lr);
}

// H[I,J] = beta·H + alpha·Σ_s partial_s (fixed order), mirrored for symmetric
// products.  One workgroup reduces a 64×64 block of a tile: rows are read and
// written as 16-byte vectors, and the mirror goes through an LDS transpose so
// that it is written in rows as well.
template <bool FULL>
__global__ __launch_bounds__(256) void gram_reduce_kernel(G2Args a) {
  __shared__ float tr[64][65];
  const int64_t tile = blockIdx.y, grp = blockIdx.z;  // grp: weighted products' group
  int64_t I, J;
  if (FULL) {
    I = tile / a.nt;
    J = tile - I * a.nt;
  } else {
    tri_tile(tile, a.nt, I, J);
  }
  const bool diag = !FULL && (I == J);
  const int bi = blockIdx.x >> 2, bj = blockIdx.x & 3;  // 64×64 block within the tile
  if (diag && bi > bj) return;                          // strictly below the diagonal
  const bool full = !diag || bi < bj;                    // no element on or below the diagonal
  const float* __restrict__ P = a.P + (grp * a.tiles + tile) * a.S * (int64_t)(TT * TT);
  float* __restrict__ Hm = a.H + grp * a.sH;
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
    if (!FULL) {
#pragma unroll
      for (int u = 0; u < 4; ++u) tr[r][cq * 4 + u] = out[u];
    }
  }
  if (FULL) return;
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

// Split plan.  Splits per operand half: the smallest power of two that gives
// at least 4096 workgroups (16 waves of one 256×256 tile per CU), at most 16
// splits in all and at least 16 KS-token stages per split; then, among the
// counts down to three quarters of it, the one whose grid fills its last wave
// of workgroups best (one workgroup per CU, kCUs of them): C=4096 has 136
// tiles, 2176 workgroups (8.5 waves) at 16 splits and 2040 (7.97) at 15, and
// its Gram takes 4.25 instead of 4.49 ms; C=14336 keeps 4 splits (6384
// workgroups, 24.9 waves).  Measured on MI355X with random bf16 operands.
// Every split gets an even number of stages, so the staged width is K padded
// to a multiple of 2·KS·(splits per half), at most 2048.
struct GramPlan {
  int S;        // total splits
  int64_t Kp;   // padded tokens per half
  int64_t kc;   // tokens per split
};

constexpr int64_t kCUs = 256;  // MI355X

// Share of the workgroup slots that a grid of n workgroups keeps busy over its waves.
double wave_fill(int64_t n) { return (double)n / (double)(cdiv(n, kCUs) * kCUs); }

GramPlan gram_plan(int64_t tiles, int64_t K, int halves, int64_t max_chain = 0,
                   int64_t max_s = 16) {
  const int64_t K1 = std::max<int64_t>(K, 1);
  const int64_t smax =
      std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(16 / halves, max_s), K1 / (KS * 16)));
  int s = 1;
  while (s * 2 <= smax && tiles * halves * s < 4096) s *= 2;
  {
    int best = s;
    for (int c = s - 1; c >= 1 && 4 * c >= 3 * s; --c)
      if (wave_fill(tiles * halves * c) > wave_fill(tiles * halves * best) + 1e-9) best = c;
    s = best;
  }
  while (max_chain > 0 && s * 2 <= smax && cdiv(K1, s) > max_chain) s *= 2;
  const int64_t step = (int64_t)2 * KS * s;
  GramPlan p;
  p.S = s * halves;
  p.Kp = cdiv(K1, step) * step;
  p.kc = p.Kp / s;
  return p;
}

int64_t n_tiles(int64_t C, bool full) {
  const int64_t nt = cdiv(C, TT);
  return full ? nt * nt : nt * (nt + 1) / 2;
}

size_t plan_ws_bytes(int64_t tiles, const GramPlan& p) {
  return p.S == 1 ? 256 : (size_t)tiles * p.S * TT * TT * sizeof(float);
}

// The products, as (full, halves).
struct Product {
  bool full;
  int halves;
};
constexpr Product SYM1{false, 1};  // H from Xᵀ
constexpr Product SYM2{false, 2};  // weighted H[g] from (hi_g, lo_g) against Xᵀ
constexpr Product FULL2{true, 2};  // GPTAQ Dx from (hi, lo) against Xᵀ

// Staged bf16 planes of one activation: 1 for bf16, 2 for fp16, 3 for fp32
// (dtype codes 0, 1, 2).  With P > 1 every product runs once per plane q of
// the column operand (Σ_q planes = X), accumulating into the output, and the
// plain Hessian's row operand is all P planes (halves = P): H = Σ_q XᵀX_q.
// Each run computes upper tiles only, which is exact for the symmetric sum.
int dtype_planes(int dtype) { return dtype == 0 ? 1 : dtype == 1 ? 2 : 3; }
Product x_product(int P) { return Product{false, P}; }

size_t product_ws(int64_t K, int64_t C, Product pr) {
  const int64_t tiles = n_tiles(C, pr.full);
  return plan_ws_bytes(tiles, gram_plan(tiles, K, pr.halves));
}

int64_t product_width(int64_t K, int64_t C, Product pr) {
  return gram_plan(n_tiles(C, pr.full), K, pr.halves).Kp;
}

// The weighted kind of bf16 activations runs all G groups in one
// wgram_kernel launch over tiles·G work items (no operand halves); with P > 1
// activation planes it stages the hi/lo planes of x·w and runs SYM2 products.
bool fused_weighted(int kind, int P) { return kind == 2 && P == 1; }
// Each split of a weighted product is also cut to at most kWChain tokens: its
// fp32 accumulators take two MFMA updates (hi, lo) per 16 tokens, and the
// rounding error grows with the chain (measured on MI355X at C = 14336 over
// 65536 tokens: 6.8e-6 of fp64 for one 65536-token chain; 32768-token
// chains keep it at the plane-staged path's level).  The split partials of
// one flush stay within kWBudget (config 3's C = 14336 flush: 8 splits,
// 13.4 GB): a wider product (many groups at a large C) takes fewer, longer
// splits, down to one with no partials at all.
constexpr int64_t kWChain = 32768;
constexpr int64_t kWBudget = int64_t(16) << 30;
GramPlan wplan(int64_t K, int64_t C, int64_t G) {
  const int64_t items = n_tiles(C, false) * G;
  const int64_t max_s = std::max<int64_t>(1, kWBudget / (items * TT * TT * 4));
  return gram_plan(items, K, 1, kWChain, max_s);
}

// Feature planes (Cp rows) staged per kind (0 Hessian, 1 GPTAQ, 2 weighted
// with G groups) for an activation of P planes.
int64_t kind_planes(int kind, int64_t G, int P = 1) {
  if (fused_weighted(kind, P)) return 1;
  return P + (kind == 1 ? 2 : kind == 2 ? 2 * G : 0);
}

int64_t padded_features(int64_t C) { return cdiv(C, TT) * TT; }

// Rows of ldt bf16 elements a kind's staged buffer holds: its planes, and for
// the fused weighted kind the G fp32 weight rows (2G bf16 rows) after them.
int64_t kind_height(int kind, int64_t C, int64_t G, int P = 1) {
  return kind_planes(kind, G, P) * padded_features(C) + (fused_weighted(kind, P) ? 2 * G : 0);
}

// Staged token width and Gram workspace a kind needs for K tokens.
int64_t kind_width(int kind, int64_t K, int64_t C, int P = 1, int64_t G = 1) {
  if (kind == 0) return product_width(K, C, x_product(P));
  if (kind == 1) return std::max(product_width(K, C, x_product(P)), product_width(K, C, FULL2));
  if (fused_weighted(kind, P)) return wplan(K, C, G).Kp;
  return product_width(K, C, SYM2);
}
size_t kind_gram_ws(int kind, int64_t K, int64_t C, int P = 1, int64_t G = 1) {
  if (kind == 0) return product_ws(K, C, x_product(P));
  if (kind == 1) return std::max(product_ws(K, C, x_product(P)), product_ws(K, C, FULL2));
  if (fused_weighted(kind, P)) return plan_ws_bytes(n_tiles(C, false) * G, wplan(K, C, G));
  return product_ws(K, C, SYM2);
}

// Zero token columns [roundup(K, 64), width) of `rows` staged rows.
int zero_pad(hipStream_t st, uint16_t* XT, int64_t ldt, int64_t rows, int64_t K, int64_t width) {
  const int64_t K64 = cdiv(std::max<int64_t>(K, 0), KS) * KS;
  if (width <= K64) return G2PTQ_OK;
  const int64_t n = rows * (width - K64);
  hipLaunchKernelGGL(zero_cols_bf16_kernel, dim3((unsigned)std::min<int64_t>(cdiv(n, 256), 4096)),
                     dim3(256), 0, st, XT, ldt, rows, K64, width);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

// out = beta·out + alpha·(product over K staged tokens).  The staged planes
// must be zero from token roundup(K, 64) up to product_width(K, C, pr).
int run_product(hipStream_t st, Product pr, const uint16_t* A1, const uint16_t* A2,
                const uint16_t* A3, const uint16_t* B, int64_t ldt, int64_t K, int64_t C,
                float alpha, float beta, float* out, int64_t ldo, void* ws, size_t ws_bytes) {
  const int64_t nt = cdiv(C, TT);
  const int64_t tiles = n_tiles(C, pr.full);
  const GramPlan p = gram_plan(tiles, K, pr.halves);
  G2PTQ_CHECK(p.Kp <= ldt, "hessian gram: staged operand too narrow (%lld < %lld)",
              (long long)ldt, (long long)p.Kp);
  G2PTQ_CHECK(tiles * p.S < (1ll << 31) && tiles < 65536, "hessian gram: grid too large");
  G2Args a{};
  a.A1 = A1; a.A2 = A2; a.A3 = A3; a.B = B; a.ldt = ldt; a.kc = p.kc; a.nt = nt; a.tiles = tiles; a.C = C;
  a.S = p.S; a.halves = pr.halves; a.alpha = alpha; a.beta = beta; a.H = out; a.ldh = ldo;
  a.G = 1;
  if (p.S > 1) {
    const size_t need = plan_ws_bytes(tiles, p);
    G2PTQ_CHECK(ws != nullptr && ws_bytes >= need, "hessian gram: workspace %zu < %zu", ws_bytes,
                need);
    a.P = static_cast<float*>(ws);
  }
  const dim3 grid((unsigned)(tiles * p.S));
  const bool direct_beta = p.S == 1 && beta != 0.f;
  if (pr.full) {
    if (direct_beta) hipLaunchKernelGGL((gram256_kernel<true, true>), grid, dim3(NTH), 0, st, a);
    else hipLaunchKernelGGL((gram256_kernel<false, true>), grid, dim3(NTH), 0, st, a);
  } else {
    if (direct_beta) hipLaunchKernelGGL((gram256_kernel<true, false>), grid, dim3(NTH), 0, st, a);
    else hipLaunchKernelGGL((gram256_kernel<false, false>), grid, dim3(NTH), 0, st, a);
  }
  G2PTQ_LAUNCHED();
  if (p.S > 1) {
    if (pr.full)
      hipLaunchKernelGGL(gram_reduce_kernel<true>, dim3(16, (unsigned)tiles), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL(gram_reduce_kernel<false>, dim3(16, (unsigned)tiles), dim3(256), 0, st, a);
    G2PTQ_LAUNCHED();
  }
  return G2PTQ_OK;
}

// H[g] = beta·H[g] + alpha·Σ_t x_t·(x_t·w[g][t])ᵀ for the G groups, from
// Xᵀ and the weight rows W (G × ldw fp32); both zero from token
// roundup(K, 64) up to wplan(K, C, G).Kp.
int run_wproduct(hipStream_t st, const uint16_t* XT, const float* W, int64_t ldw, int64_t ldt,
                 int64_t K, int64_t C, int64_t G, float alpha, float beta, float* H, int64_t ldh,
                 int64_t sH, void* ws, size_t ws_bytes) {
  const int64_t nt = cdiv(C, TT);
  const int64_t tiles = n_tiles(C, false);
  const GramPlan p = wplan(K, C, G);
  G2PTQ_CHECK(p.Kp <= ldt && p.Kp <= ldw, "hessian gram: staged operand too narrow (%lld < %lld)",
              (long long)std::min(ldt, ldw), (long long)p.Kp);
  G2PTQ_CHECK(tiles * G * p.S < (1ll << 31) && tiles < 65536 && G <= 65535,
              "hessian gram: grid too large");
  G2PTQ_CHECK((reinterpret_cast<uintptr_t>(W) & 15) == 0 && ldw % 4 == 0,
              "hessian gram: weights must be 16-byte aligned with ldw a multiple of 4");
  G2Args a{};
  a.B = XT; a.ldt = ldt; a.kc = p.kc; a.nt = nt; a.tiles = tiles; a.C = C;
  a.S = p.S; a.halves = 1; a.alpha = alpha; a.beta = beta; a.H = H; a.ldh = ldh;
  a.W = W; a.ldw = ldw; a.G = G; a.sH = sH;
  if (p.S > 1) {
    const size_t need = plan_ws_bytes(tiles * G, p);
    G2PTQ_CHECK(ws != nullptr && ws_bytes >= need, "hessian gram: workspace %zu < %zu", ws_bytes,
                need);
    a.P = static_cast<float*>(ws);
  }
  const dim3 grid((unsigned)(tiles * G * p.S));
  if (p.S == 1 && beta != 0.f) hipLaunchKernelGGL(wgram_kernel<true>, grid, dim3(NTH), 0, st, a);
  else hipLaunchKernelGGL(wgram_kernel<false>, grid, dim3(NTH), 0, st, a);
  G2PTQ_LAUNCHED();
  if (p.S > 1) {
    hipLaunchKernelGGL(gram_reduce_kernel<false>, dim3(16, (unsigned)tiles, (unsigned)G), dim3(256),
                       0, st, a);
    G2PTQ_LAUNCHED();
  }
  return G2PTQ_OK;
}

int stage(hipStream_t st, int kind, const uint16_t* X, const uint16_t* F, const float* S,
          int64_t T, int64_t C, int64_t ldx, int64_t ldf, int64_t G, int64_t lds, float s_scale,
          uint16_t* XT, int64_t ldt, int64_t t_off, int dtype = 0) {
  if (T <= 0) return G2PTQ_OK;
  G2PTQ_CHECK(C > 0 && C <= (1ll << 20), "hessian stage: bad feature count %lld", (long long)C);
  G2PTQ_CHECK(ldt % 8 == 0 && t_off % 64 == 0 && (reinterpret_cast<uintptr_t>(XT) & 15) == 0,
              "hessian stage: XT must be 16-byte aligned, ldt a multiple of 8 and t_off of 64");
  G2PTQ_CHECK(t_off + cdiv(T, KS) * KS <= ldt,
              "hessian stage: token offset %lld (+%lld) outside the staged width %lld",
              (long long)t_off, (long long)T, (long long)ldt);
  const int64_t Cp = padded_features(C);
  auto aligned = [](const void* p, int64_t ld) {
    return ld % 8 == 0 && (reinterpret_cast<uintptr_t>(p) & 15) == 0;
  };
  G2PTQ_CHECK(dtype >= 0 && dtype <= 2, "hessian stage: dtype code %d unsupported", dtype);
  StageArgs s{};
  s.X = X; s.F = F; s.S = S; s.T = T; s.C = C; s.ldx = ldx; s.ldf = ldf; s.lds = lds;
  s.G = (int)G; s.s_scale = s_scale; s.XT = XT; s.ldt = ldt; s.plane = Cp * ldt; s.t_off = t_off;
  s.t_end = cdiv(T, KS) * KS;
  s.vec = aligned(X, ldx) && (kind != 1 || aligned(F, ldf));
  const dim3 grid((unsigned)cdiv(T, (int64_t)ST_T), (unsigned)(Cp / ST_C));
  if (dtype == 0) {
    if (kind == 0) hipLaunchKernelGGL(stage_kernel<0>, grid, dim3(256), 0, st, s);
    else if (kind == 1) hipLaunchKernelGGL(stage_kernel<1>, grid, dim3(256), 0, st, s);
    else hipLaunchKernelGGL(stage_kernel<2>, grid, dim3(256), 0, st, s);
  } else if (dtype == 1) {
    if (kind == 0) hipLaunchKernelGGL((stage_split_kernel<_Float16, 0>), grid, dim3(256), 0, st, s);
    else if (kind == 1) hipLaunchKernelGGL((stage_split_kernel<_Float16, 1>), grid, dim3(256), 0, st, s);
    else hipLaunchKernelGGL((stage_split_kernel<_Float16, 2>), grid, dim3(256), 0, st, s);
  } else {
    if (kind == 0) hipLaunchKernelGGL((stage_split_kernel<float, 0>), grid, dim3(256), 0, st, s);
    else if (kind == 1) hipLaunchKernelGGL((stage_split_kernel<float, 1>), grid, dim3(256), 0, st, s);
    else hipLaunchKernelGGL((stage_split_kernel<float, 2>), grid, dim3(256), 0, st, s);
  }
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

int act_square(hipStream_t st, const uint16_t* XT, int64_t ldt, int64_t t_off, int64_t T, int64_t C,
               float* act, float act_alpha, float act_beta, int P = 1) {
  if (!act) return G2PTQ_OK;
  const int64_t len = cdiv(std::max<int64_t>(T, 0), KS) * KS;
  hipLaunchKernelGGL(act_square_kernel, dim3((unsigned)cdiv(C, 4)), dim3(256), 0, st, XT, ldt,
                     t_off, len, C, act, act_alpha, act_beta, P, padded_features(C) * ldt);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

int check_gram_args(const uint16_t* XT, int64_t ldt, int64_t K, int64_t C) {
  G2PTQ_CHECK(XT && C > 0 && C <= (1ll << 20) && K >= 0, "hessian gram: bad arguments");
  G2PTQ_CHECK((reinterpret_cast<uintptr_t>(XT) & 15) == 0 && ldt % 8 == 0,
              "hessian gram: XT must be 16-byte aligned with ldt a multiple of 8");
  return G2PTQ_OK;
}

// The Gram products of each kind over K tokens staged in XT (planes of Cp × ldt).
int gram_kind(hipStream_t st, int kind, uint16_t* XT, int64_t ldt, int64_t K, int64_t C, int64_t G,
              float alpha, float beta, float* H, int64_t ldh, int64_t sH, float* Dx, int64_t ldd,
              void* ws, size_t ws_bytes, int P = 1) {
  G2PTQ_TRY(check_gram_args(XT, ldt, K, C));
  const int64_t Cp = padded_features(C);
  const int64_t plane = Cp * ldt;
  const int64_t width = kind_width(kind, K, C, P, G);
  G2PTQ_CHECK(width <= ldt, "hessian gram: staged operand too narrow (%lld < %lld)",
              (long long)ldt, (long long)width);
  G2PTQ_TRY(zero_pad(st, XT, ldt, kind_planes(kind, G, P) * Cp, K, width));
  if (fused_weighted(kind, P)) {
    // the weight rows, as 2G rows of 2·ldt bf16 elements
    G2PTQ_TRY(zero_pad(st, XT + plane, 2 * ldt, G, 2 * K, 2 * width));
    return run_wproduct(st, XT, reinterpret_cast<const float*>(XT + plane), ldt, ldt, K, C, G,
                        alpha, beta, H, ldh, sH, ws, ws_bytes);
  }
  const uint16_t* Xq[3] = {XT, XT + plane, XT + 2 * plane};
  // every product over the column planes q = 0..P−1: the first applies beta,
  // the others add to it
  for (int q = 0; q < P; ++q) {
    const float b = q == 0 ? beta : 1.f;
    if (kind != 2)
      G2PTQ_TRY(run_product(st, x_product(P), Xq[0], P > 1 ? Xq[1] : nullptr,
                            P > 2 ? Xq[2] : nullptr, Xq[q], ldt, K, C, alpha, b, H, ldh, ws,
                            ws_bytes));
    if (kind == 1)
      G2PTQ_TRY(run_product(st, FULL2, XT + P * plane, XT + (P + 1) * plane, nullptr, Xq[q], ldt,
                            K, C, alpha, b, Dx, ldd, ws, ws_bytes));
    if (kind == 2)
      for (int64_t g = 0; g < G; ++g)
        G2PTQ_TRY(run_product(st, SYM2, XT + (P + 2 * g) * plane, XT + (P + 2 * g + 1) * plane,
                              nullptr, Xq[q], ldt, K, C, alpha, b, H + g * sH, ldh, ws,
                              ws_bytes));
  }
  return G2PTQ_OK;
}

// One-shot updates (stage + Gram) through a caller workspace laid out as
// [staged planes: planes × Cp × width bf16][split partials].
size_t staged_bytes(int kind, int64_t T, int64_t C, int64_t G, int P = 1) {
  return ((size_t)kind_height(kind, C, G, P) * kind_width(kind, T, C, P, G) * 2 + 255) / 256 * 256;
}
size_t update_ws_bytes(int kind, int64_t T, int64_t C, int64_t G) {
  return staged_bytes(kind, T, C, G) + kind_gram_ws(kind, T, C, 1, G);
}

}  // namespace
}  // namespace g2ptq

using namespace g2ptq;

extern "C" int g2ptq_hessian_workspace(int64_t T, int64_t C, int kind, int64_t G, size_t* bytes) {
  G2PTQ_CHECK(bytes != nullptr && C > 0 && T >= 0 && kind >= 0 && kind <= 2,
              "hessian_workspace: bad arguments");
  G2PTQ_CHECK(kind != 2 || (G >= 1 && G <= 64), "hessian_workspace: G=%lld unsupported",
              (long long)G);
  *bytes = update_ws_bytes(kind, T, C, G);
  return G2PTQ_OK;
}

extern "C" int g2ptq_hessian_update(void* stream, const uint16_t* X, int64_t T, int64_t C,
                                    int64_t ldx, float alpha, float beta, float* H, int64_t ldh,
                                    void* ws, size_t ws_bytes) {
  G2PTQ_CHECK(H != nullptr && (X != nullptr || T == 0) && C > 0 && T >= 0,
              "hessian_update: bad arguments");
  const size_t need = update_ws_bytes(0, T, C, 0);
  G2PTQ_CHECK(ws != nullptr && ws_bytes >= need, "hessian_update: workspace %zu < %zu", ws_bytes,
              need);
  hipStream_t st = as_stream(stream);
  const int64_t ldt = kind_width(0, T, C);
  uint16_t* XT = static_cast<uint16_t*>(ws);
  const size_t xt = staged_bytes(0, T, C, 0);
  G2PTQ_TRY(stage(st, 0, X, nullptr, nullptr, T, C, ldx, 0, 0, 0, 1.f, XT, ldt, 0));
  return gram_kind(st, 0, XT, ldt, T, C, 0, alpha, beta, H, ldh, 0, nullptr, 0,
                   static_cast<char*>(ws) + xt, ws_bytes - xt);
}

extern "C" int g2ptq_gptaq_update(void* stream, const uint16_t* X, const uint16_t* Xfp, int64_t T,
                                  int64_t C, int64_t ldx, int64_t ldxf, float alpha, float beta,
                                  float* H, float* Dx, int64_t ld, void* ws, size_t ws_bytes) {
  G2PTQ_CHECK(H && Dx && ((X && Xfp) || T == 0) && C > 0 && T >= 0,
              "gptaq_update: bad arguments");
  const size_t need = update_ws_bytes(1, T, C, 0);
  G2PTQ_CHECK(ws != nullptr && ws_bytes >= need, "gptaq_update: workspace %zu < %zu", ws_bytes,
              need);
  hipStream_t st = as_stream(stream);
  const int64_t ldt = kind_width(1, T, C);
  uint16_t* XT = static_cast<uint16_t*>(ws);
  const size_t xt = staged_bytes(1, T, C, 0);
  G2PTQ_TRY(stage(st, 1, X, Xfp, nullptr, T, C, ldx, ldxf, 0, 0, 1.f, XT, ldt, 0));
  return gram_kind(st, 1, XT, ldt, T, C, 0, alpha, beta, H, ld, 0, Dx, ld,
                   static_cast<char*>(ws) + xt, ws_bytes - xt);
}

extern "C" int g2ptq_weighted_hessian_update(void* stream, const uint16_t* X, int64_t T,
                                             int64_t C, int64_t ldx, const float* S, int64_t G,
                                             int64_t lds, float alpha, float beta, float* H,
                                             int64_t ldh, int64_t sH, float* act,
                                             float act_alpha, float act_beta, void* ws,
                                             size_t ws_bytes) {
  G2PTQ_CHECK(G >= 1 && G <= 64, "weighted_hessian_update: G=%lld unsupported", (long long)G);
  G2PTQ_CHECK(H && ((X && S) || T == 0) && C > 0 && T >= 0,
              "weighted_hessian_update: bad arguments");
  const size_t need = update_ws_bytes(2, T, C, G);
  G2PTQ_CHECK(ws != nullptr && ws_bytes >= need, "weighted_hessian_update: workspace %zu < %zu",
              ws_bytes, need);
  hipStream_t st = as_stream(stream);
  const int64_t ldt = kind_width(2, T, C, 1, G);
  uint16_t* XT = static_cast<uint16_t*>(ws);
  const size_t xt = staged_bytes(2, T, C, G);
  G2PTQ_TRY(stage(st, 2, X, nullptr, S, T, C, ldx, 0, G, lds, 1.f, XT, ldt, 0));
  G2PTQ_TRY(act_square(st, XT, ldt, 0, T, C, act, act_alpha, act_beta));
  return gram_kind(st, 2, XT, ldt, T, C, G, alpha, beta, H, ldh, sH, nullptr, 0,
                   static_cast<char*>(ws) + xt, ws_bytes - xt);
}

extern "C" int g2ptq_hessian_stage_rows(int64_t C, int64_t* rows) {
  G2PTQ_CHECK(rows != nullptr && C > 0, "hessian_stage_rows: bad arguments");
  *rows = padded_features(C);
  return G2PTQ_OK;
}

extern "C" int g2ptq_hessian_stage(void* stream, const uint16_t* X, int64_t T, int64_t C,
                                   int64_t ldx, uint16_t* XT, int64_t ldt, int64_t t_off) {
  G2PTQ_CHECK(XT && (X || T == 0) && C > 0 && T >= 0, "hessian_stage: bad arguments");
  return stage(as_stream(stream), 0, X, nullptr, nullptr, T, C, ldx, 0, 0, 0, 1.f, XT, ldt,
               t_off);
}

extern "C" int g2ptq_hessian_gram_workspace(int64_t K, int64_t C, size_t* bytes) {
  G2PTQ_CHECK(bytes != nullptr && C > 0 && K >= 0, "hessian_gram_workspace: bad arguments");
  *bytes = kind_gram_ws(0, K, C);
  return G2PTQ_OK;
}

extern "C" int g2ptq_hessian_gram(void* stream, uint16_t* XT, int64_t ldt, int64_t K, int64_t C,
                                  float alpha, float beta, float* H, int64_t ldh, void* ws,
                                  size_t ws_bytes) {
  G2PTQ_CHECK(H != nullptr, "hessian_gram: null H");
  return gram_kind(as_stream(stream), 0, XT, ldt, K, C, 0, alpha, beta, H, ldh, 0, nullptr, 0, ws,
                   ws_bytes);
}

// *equal = 0 where rows × cols of two staged buffers differ anywhere: the
// check before a stager copies the Gram another stager computed from what
// should be the same tokens (16-byte chunks; rows grid-strided).
__global__ __launch_bounds__(256) void staged_equal_kernel(const uint16_t* __restrict__ A,
                                                           int64_t lda,
                                                           const uint16_t* __restrict__ B,
                                                           int64_t ldb, int64_t rows,
                                                           int64_t chunks, int* equal) {
  int diff = 0;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const uint4* a = reinterpret_cast<const uint4*>(A + r * lda);
    const uint4* b = reinterpret_cast<const uint4*>(B + r * ldb);
#pragma unroll 4
    for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < chunks;
         c += (int64_t)gridDim.x * 256) {
      const uint4 x = a[c], y = b[c];
      diff |= (x.x != y.x) | (x.y != y.y) | (x.z != y.z) | (x.w != y.w);
    }
  }
  if (diff) *equal = 0;
}

extern "C" int g2ptq_staged_equal(void* stream, const uint16_t* A, int64_t lda, const uint16_t* B,
                                  int64_t ldb, int64_t rows, int64_t cols, int* equal) {
  G2PTQ_CHECK(A && B && equal, "staged_equal: null pointer");
  G2PTQ_CHECK(rows >= 0 && cols >= 0 && cols % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 &&
                  cols <= lda && cols <= ldb && (reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(B) & 15) == 0,
              "staged_equal: columns and pitches must be multiples of 8 (16-byte aligned rows)");
  if (rows == 0 || cols == 0) return G2PTQ_OK;
  const int64_t chunks = cols / 8;
  const dim3 grid((unsigned)std::min<int64_t>(cdiv(chunks, (int64_t)256 * 8), 64),
                  (unsigned)std::min<int64_t>(rows, 8192));
  hipLaunchKernelGGL(staged_equal_kernel, grid, dim3(256), 0, as_stream(stream), A, lda, B, ldb,
                     rows, chunks, equal);
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

extern "C" int g2ptq_gptaq_stage(void* stream, const uint16_t* X, const uint16_t* Xfp, int64_t T,
                                 int64_t C, int64_t ldx, int64_t ldxf, uint16_t* XT, int64_t ldt,
                                 int64_t t_off) {
  G2PTQ_CHECK(XT && ((X && Xfp) || T == 0) && C > 0 && T >= 0, "gptaq_stage: bad arguments");
  return stage(as_stream(stream), 1, X, Xfp, nullptr, T, C, ldx, ldxf, 0, 0, 1.f, XT, ldt, t_off);
}

extern "C" int g2ptq_gptaq_gram_workspace(int64_t K, int64_t C, size_t* bytes) {
  G2PTQ_CHECK(bytes != nullptr && C > 0 && K >= 0, "gptaq_gram_workspace: bad arguments");
  *bytes = kind_gram_ws(1, K, C);
  return G2PTQ_OK;
}

extern "C" int g2ptq_gptaq_gram(void* stream, uint16_t* XT, int64_t ldt, int64_t K, int64_t C,
                                float alpha, float beta, float* H, float* Dx, int64_t ld, void* ws,
                                size_t ws_bytes) {
  G2PTQ_CHECK(H && Dx, "gptaq_gram: null output");
  return gram_kind(as_stream(stream), 1, XT, ldt, K, C, 0, alpha, beta, H, ld, 0, Dx, ld, ws,
                   ws_bytes);
}

extern "C" int g2ptq_weighted_stage(void* stream, const uint16_t* X, int64_t T, int64_t C,
                                    int64_t ldx, const float* S, int64_t G, int64_t lds,
                                    float s_scale, uint16_t* XT, int64_t ldt, int64_t t_off,
                                    float* act, float act_alpha, float act_beta) {
  G2PTQ_CHECK(G >= 1 && G <= 64, "weighted_stage: G=%lld unsupported", (long long)G);
  G2PTQ_CHECK(XT && ((X && S) || T == 0) && C > 0 && T >= 0, "weighted_stage: bad arguments");
  hipStream_t st = as_stream(stream);
  G2PTQ_TRY(stage(st, 2, X, nullptr, S, T, C, ldx, 0, G, lds, s_scale, XT, ldt, t_off));
  return act_square(st, XT, ldt, t_off, T, C, act, act_alpha, act_beta);
}

extern "C" int g2ptq_weighted_gram_workspace(int64_t K, int64_t C, int64_t G, size_t* bytes) {
  G2PTQ_CHECK(bytes != nullptr && C > 0 && K >= 0 && G >= 1 && G <= 64,
              "weighted_gram_workspace: bad arguments");
  *bytes = kind_gram_ws(2, K, C, 1, G);
  return G2PTQ_OK;
}

extern "C" int g2ptq_weighted_gram(void* stream, uint16_t* XT, int64_t ldt, int64_t K, int64_t C,
                                   int64_t G, float alpha, float beta, float* H, int64_t ldh,
                                   int64_t sH, void* ws, size_t ws_bytes) {
  G2PTQ_CHECK(G >= 1 && G <= 64 && H, "weighted_gram: bad arguments");
  return gram_kind(as_stream(stream), 2, XT, ldt, K, C, G, alpha, beta, H, ldh, sH, nullptr, 0, ws,
                   ws_bytes);
}

// Any-dtype staging (bf16, fp16, fp32 activations; dtype codes 0, 1, 2): the
// staged planes of a kind, the stage, the Gram products and their workspace.
extern "C" int g2ptq_hessian_stage_planes(int kind, int dtype, int64_t G, int64_t* planes) {
  G2PTQ_CHECK(planes != nullptr && kind >= 0 && kind <= 2 && dtype >= 0 && dtype <= 2 &&
                  (kind != 2 || (G >= 1 && G <= 64)),
              "hessian_stage_planes: bad arguments");
  *planes = kind_planes(kind, G, dtype_planes(dtype));
  return G2PTQ_OK;
}

extern "C" int g2ptq_hessian_stage_height(int kind, int dtype, int64_t C, int64_t G,
                                          int64_t* rows) {
  G2PTQ_CHECK(rows != nullptr && kind >= 0 && kind <= 2 && dtype >= 0 && dtype <= 2 && C > 0 &&
                  C <= (1ll << 20) && (kind != 2 || (G >= 1 && G <= 64)),
              "hessian_stage_height: bad arguments");
  *rows = kind_height(kind, C, G, dtype_planes(dtype));
  return G2PTQ_OK;
}

extern "C" int g2ptq_hessian_stage_ex(void* stream, int kind, int dtype, const void* X,
                                      const void* Xfp, int64_t T, int64_t C, int64_t ldx,
                                      int64_t ldxf, const float* S, int64_t G, int64_t lds,
                                      float s_scale, uint16_t* XT, int64_t ldt, int64_t t_off,
                                      float* act, float act_alpha, float act_beta) {
  G2PTQ_CHECK(kind >= 0 && kind <= 2 && dtype >= 0 && dtype <= 2,
              "hessian_stage_ex: kind %d / dtype %d unsupported", kind, dtype);
  G2PTQ_CHECK(kind != 2 || (G >= 1 && G <= 64), "hessian_stage_ex: G=%lld unsupported",
              (long long)G);
  G2PTQ_CHECK(XT && (T == 0 || (X && (kind != 1 || Xfp) && (kind != 2 || S))) && C > 0 && T >= 0,
              "hessian_stage_ex: bad arguments");
  hipStream_t st = as_stream(stream);
  G2PTQ_TRY(stage(st, kind, static_cast<const uint16_t*>(X), static_cast<const uint16_t*>(Xfp), S,
                  T, C, ldx, ldxf, G, lds, s_scale, XT, ldt, t_off, dtype));
  if (kind == 2)
    return act_square(st, XT, ldt, t_off, T, C, act, act_alpha, act_beta, dtype_planes(dtype));
  return G2PTQ_OK;
}

extern "C" int g2ptq_hessian_gram_ex_workspace(int kind, int dtype, int64_t K, int64_t C,
                                               int64_t G, size_t* bytes) {
  G2PTQ_CHECK(bytes != nullptr && kind >= 0 && kind <= 2 && dtype >= 0 && dtype <= 2 && C > 0 &&
                  K >= 0 && (kind != 2 || (G >= 1 && G <= 64)),
              "hessian_gram_ex_workspace: bad arguments");
  *bytes = kind_gram_ws(kind, K, C, dtype_planes(dtype), G);
  return G2PTQ_OK;
}

extern "C" int g2ptq_hessian_gram_ex(void* stream, int kind, int dtype, uint16_t* XT, int64_t ldt,
                                     int64_t K, int64_t C, int64_t G, float alpha, float beta,
                                     float* H, int64_t ldh, int64_t sH, float* Dx, int64_t ldd,
                                     void* ws, size_t ws_bytes) {
  G2PTQ_CHECK(kind >= 0 && kind <= 2 && dtype >= 0 && dtype <= 2 && H &&
                  (kind != 1 || Dx) && (kind != 2 || (G >= 1 && G <= 64)),
              "hessian_gram_ex: bad arguments");
  return gram_kind(as_stream(stream), kind, XT, ldt, K, C, G, alpha, beta, H, ldh, sH, Dx, ldd, ws,
                   ws_bytes, dtype_planes(dtype));
}
