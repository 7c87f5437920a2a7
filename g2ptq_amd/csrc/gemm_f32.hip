// Batched fp32 GEMM on CDNA4 matrix cores.
//
//   D = alpha·A·B + beta·C + gamma·X     (optionally one triangle of D only)
//
// Two product paths share the staging: v_mfma_f32_32x32x2_f32 on the fp32
// operands (K < 128: the latency-bound panel updates of the factor), and for
// K >= 128 v_mfma_f32_32x32x16_bf16 on a three-way bf16 split of each operand
// fragment (a = a_h + a_m + a_l exactly), summing the six cross products above
// 2⁻²³·|a·b|: six bf16 MFMAs per 16 k instead of eight fp32 ones, each a
// quarter of the cycles (8192³: 158–165 TFLOP/s against 125 on fp32 MFMAs).
// Its error is below the fp32 MFMA path's (measured max |err| / (|A|·|B|)
// 2.8e-7 vs 3.6e-7 at K = 1536, both against fp64).  With B given N×K both
// operands are k-contiguous and each element is split once per workgroup, as
// its 16-k slab is stored to LDS as three bf16 planes; with B given K×N the
// fp32 slab is staged and each wave splits the fragments it reads (a split at
// store time would have to transpose B into 2-byte LDS writes).  Both orders
// sum the same six products in the same order, so the results are identical.
//
// A is M×K row-major; B is K×N row-major, or N×K row-major (b_kcontig).  The
// same kernel serves every fp32 product of the path: block-tail updates of the
// compensation sweep, the Cholesky TRSM/SYRK steps, the triangular-inverse
// levels, GPTAQ's P and the G2PTQ trust-region products.
//
// Shape: a workgroup (4 wave64s, two per CU) computes a 128×128 tile (64×64
// for small grids); each wave a quadrant made of 32×32 MFMA blocks.  K advances
// in slabs of 32 through double-buffered LDS with 16-byte global loads for
// two slabs in flight, interleaved with the MFMAs of the current slab.  Large
// split products with B given N×K (a grid of at least 256 tiles of 256×256,
// K >= 384) take an 8-wave 256×256 workgroup instead, which halves the LDS
// reads and barriers per MFMA and sums the same products in the same order.
//
// Operand layout: a 32x32x2 MFMA takes one k per lane half, so a slab's k
// order is permuted: for k-octet o, lane half h holds k = 8o + 4h + j in the
// j-th of four consecutive MFMAs.  Both operands use the same permutation,
// so one 16-byte LDS read (4 consecutive k of one row) feeds four MFMAs.
// A (and B given N×K) sit in LDS as [row][k] with a 36-float pitch: the
// 16-byte reads of 16 consecutive rows hit distinct bank quads.  B given K×N
// sits as [k][n] with a 136-float pitch and is read 4 bytes per lane (the
// two lane halves land 32 banks apart).
#include "common.hpp"

namespace g2ptq {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// f = h + m + l for eight fp32 values: h = bf16(f), m = bf16(f − h),
// l = bf16(f − h − m), each rounded to nearest, the remainders exact.  The
// pieces carry 8 significant bits each and |m| ≤ 2⁻⁸|f|, |l| ≤ 2⁻¹⁶|f|.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
// Two values at a time, so each conversion is one packed v_cvt_pk_bf16_f32.
__device__ __forceinline__ void split3_2(f32x2 f, bf16x2& h, bf16x2& m, bf16x2& l) {
  h = __builtin_convertvector(f, bf16x2);
  const f32x2 r1 = f - __builtin_convertvector(h, f32x2);
  m = __builtin_convertvector(r1, bf16x2);
  const f32x2 r2 = r1 - __builtin_convertvector(m, f32x2);
  l = __builtin_convertvector(r2, bf16x2);
}
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void split4(float4 u, bf16x4& h, bf16x4& m, bf16x4& l) {
  bf16x2 h0, h1, m0, m1, l0, l1;
  split3_2(f32x2{u.x, u.y}, h0, m0, l0);
  split3_2(f32x2{u.z, u.w}, h1, m1, l1);
  h = __builtin_shufflevector(h0, h1, 0, 1, 2, 3);
  m = __builtin_shufflevector(m0, m1, 0, 1, 2, 3);
  l = __builtin_shufflevector(l0, l1, 0, 1, 2, 3);
}
__device__ __forceinline__ void split3(float4 u0, float4 u1, bf16x8& h, bf16x8& m, bf16x8& l) {
  bf16x2 h0, h1, h2, h3, m0, m1, m2, m3, l0, l1, l2, l3;
  split3_2(f32x2{u0.x, u0.y}, h0, m0, l0);
  split3_2(f32x2{u0.z, u0.w}, h1, m1, l1);
  split3_2(f32x2{u1.x, u1.y}, h2, m2, l2);
  split3_2(f32x2{u1.z, u1.w}, h3, m3, l3);
  h = __builtin_shufflevector(__builtin_shufflevector(h0, h1, 0, 1, 2, 3),
                              __builtin_shufflevector(h2, h3, 0, 1, 2, 3), 0, 1, 2, 3, 4, 5, 6, 7);
  m = __builtin_shufflevector(__builtin_shufflevector(m0, m1, 0, 1, 2, 3),
                              __builtin_shufflevector(m2, m3, 0, 1, 2, 3), 0, 1, 2, 3, 4, 5, 6, 7);
  l = __builtin_shufflevector(__builtin_shufflevector(l0, l1, 0, 1, 2, 3),
                              __builtin_shufflevector(l2, l3, 0, 1, 2, 3), 0, 1, 2, 3, 4, 5, 6, 7);
}

constexpr int BK = 32;
constexpr int PK = 36;   // [row][k] pitch (floats)
// Split path: 16-k slabs, each operand staged in LDS as three bf16 planes
// (h, m, l) split once per workgroup as the slab is stored.  A plane is
// [row][k] (B's [n][k]) with a 24-element (48-byte) pitch: the 16-byte reads
// of 8 consecutive rows start 12 banks apart and hit distinct bank quads.
constexpr int SK = 16;
constexpr int SP = 24;
constexpr int GH = 8;    // tile-rows per group of the tile order

// Tile id → (tm, tn): groups of GH tile-rows walked column by column.
__device__ __forceinline__ void tile_of(int64_t id, int64_t tm, int64_t tn, int64_t& im,
                                        int64_t& in) {
  const int64_t per_group = GH * tn;
  const int64_t grp = id / per_group, r = id - grp * per_group;
  const int64_t first = grp * GH;
  const int64_t h = (tm - first) < GH ? (tm - first) : GH;
  im = first + r % h;
  in = r / h;
}

// TILE × TILE output per workgroup (4 waves in 2×2, each TILE/2 square made
// of 32×32 MFMA blocks): 128 for large products, 64 when a 128 grid would
// leave most CUs idle (the factor's TRSM / panel updates, short tails).
template <int TILE, bool B_KCONTIG, bool VEC, bool SPLIT>
__global__ __launch_bounds__(256, 2) void gemm_f32_kernel(GemmF32 g, int64_t tm, int64_t tn) {
  constexpr int BM = TILE, BN = TILE;
  constexpr int PN = BN + 8;                       // [k][n] pitch (floats)
  constexpr int LDS_A = BM * PK;
  constexpr int LDS_B = (BN * PK > BK * PN) ? BN * PK : BK * PN;
  constexpr int WT = TILE / 2, NBLK = WT / 32;     // wave tile, 32×32 blocks per side
  constexpr int RA = BM / 32;                      // float4 per thread per slab (A)
  constexpr int KQ = BN / 4, RB_ROWS = 256 / KQ;   // B as K×N: n-quads per k row, k rows per pass
  constexpr int RB = BN / 32;                      // float4 per thread per slab (B)
  __shared__ __attribute__((aligned(16))) float As[2][LDS_A];
  __shared__ __attribute__((aligned(16))) float Bs[2][LDS_B];

  const int z = blockIdx.z;
  const int64_t b1 = z / g.batch2, b2 = z % g.batch2;
  if (g.skip && g.skip[b1]) return;
  const int64_t nwg = gridDim.x, bid = blockIdx.x;
  int64_t im, in;
  if (g.tri == 0) {
    // XCD-aware renumbering (workgroups go round-robin over 8 XCDs): every
    // XCD gets a contiguous range of the grouped tile order.
    const int64_t q8 = nwg >> 3, r8 = nwg & 7, xcd = bid & 7;
    const int64_t id = xcd * q8 + (xcd < r8 ? xcd : r8) + (bid >> 3);
    tile_of(id, tm, tn, im, in);
  } else if (g.tri & 8) {
    // Triangular upper B: tile (im, in) multiplies at most n0 + BN columns
    // (fewer still when A is upper too), so the work grows to the right.
    // Longest first: bands of GH tile-columns from the right, each walked
    // row by row from the top, in dispatch order.
    const int64_t per = GH * tm;
    const int64_t band = bid / per, r = bid - band * per;
    const int64_t c0 = band * GH;
    const int64_t h = tn - c0 < GH ? tn - c0 : GH;
    in = tn - 1 - (c0 + r % h);
    im = r / h;
  } else if (g.tri & 2) {
    // Triangular B: tile (im, in) multiplies K − n0 columns, so the work falls
    // from left to right.  Longest first: bands of GH tile-columns from the
    // left, each walked row by row, in dispatch order (no renumbering, so the
    // 8 XCDs share every band evenly; consecutive tiles of a row land on
    // different XCDs, each XCD keeping to one column of the band).
    const int64_t per = GH * tm;
    const int64_t band = bid / per, r = bid - band * per;
    const int64_t c0 = band * GH;
    const int64_t h = tn - c0 < GH ? tn - c0 : GH;
    in = c0 + r % h;
    im = r / h;
  } else {
    // Triangular A: tile (im, in) multiplies m0 + BM columns, so the work
    // grows downwards.  Longest first: the grouped order from the bottom
    // group up, in dispatch order (each XCD keeps to one row of a group).
    tile_of(bid, tm, tn, im, in);
    im = tm - 1 - im;
  }
  const int64_t m0 = im * BM, n0 = in * BN;
  if (g.uplo == 1 && n0 > m0 + BM - 1) return;
  if (g.uplo == 2 && m0 > n0 + BN - 1) return;

  const float* __restrict__ A = g.A + b1 * g.sA + b2 * g.sA2;
  const float* __restrict__ B = g.B + b1 * g.sB + b2 * g.sB2;
  const int64_t M = g.M, N = g.N;
  // K range of this tile: triangular operands contribute nothing outside it.
  int64_t klo = 0, K = g.K;
  if (g.tri & 1) K = K < m0 + BM ? K : m0 + BM;
  if (g.tri & 2) klo = n0 / BK * BK;
  if ((g.tri & 4) && m0 / BK * BK > klo) klo = m0 / BK * BK;
  if (g.tri & 8) K = K < n0 + BN ? K : n0 + BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Global → register mapping.
  //   [row][k] operands: row = tid/8 + 32 i, k-quad = tid % 8.
  //   B as K×N:          k = tid/KQ + RB_ROWS i, n-quad = tid % KQ.
  const int ra_row = tid >> 3, ra_kq = (tid & 7) * 4;
  const int rb_k = tid / KQ, rb_nq = (tid % KQ) * 4;

  auto ld4 = [&](const float* base, int64_t ld, int64_t r, int64_t c, int64_t R, int64_t Ccols) {
    if (VEC) {
      // Rows of a multiple of 4 columns (c is one): a 16-byte chunk is wholly
      // inside or outside, so one load from a clamped address and a select
      // replace per-element tests (no branches).
      const bool ok = r < R && c < Ccols;
      const uint4 w = *reinterpret_cast<const uint4*>(base + (ok ? r * ld + c : 0));
      const uint32_t m = ok ? 0xffffffffu : 0u;  // a mask, not a branch around the load
      return make_float4(__uint_as_float(w.x & m), __uint_as_float(w.y & m),
                         __uint_as_float(w.z & m), __uint_as_float(w.w & m));
    }
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r < R) {
      const float* p = base + r * ld + c;
      if (c < Ccols) v.x = p[0];
      if (c + 1 < Ccols) v.y = p[1];
      if (c + 2 < Ccols) v.z = p[2];
      if (c + 3 < Ccols) v.w = p[3];
    }
    return v;
  };

  // Register sets x / y hold one slab each (indices are compile-time constants).
  float4 xa[RA], xb[RB], ya[RA], yb[RB];
#define GF_LOAD(RAr, RBr, slab)                                                                \
  do {                                                                                         \
    const int64_t k0_ = klo + (int64_t)(slab) * BK;                                            \
    _Pragma("unroll") for (int i_ = 0; i_ < RA; ++i_)                                          \
      RAr[i_] = ld4(A, g.lda, m0 + ra_row + 32 * i_, k0_ + ra_kq, M, K);                       \
    _Pragma("unroll") for (int i_ = 0; i_ < RB; ++i_) {                                        \
      if (B_KCONTIG) RBr[i_] = ld4(B, g.ldb, n0 + ra_row + 32 * i_, k0_ + ra_kq, N, K);         \
      else RBr[i_] = ld4(B, g.ldb, k0_ + rb_k + RB_ROWS * i_, n0 + rb_nq, K, N);                \
    }                                                                                          \
  } while (0)
#define GF_STORE(RAr, RBr, buf)                                                                \
  do {                                                                                         \
    _Pragma("unroll") for (int i_ = 0; i_ < RA; ++i_)                                          \
      *reinterpret_cast<float4*>(&As[(buf)][(ra_row + 32 * i_) * PK + ra_kq]) = RAr[i_];       \
    _Pragma("unroll") for (int i_ = 0; i_ < RB; ++i_) {                                        \
      if (B_KCONTIG)                                                                           \
        *reinterpret_cast<float4*>(&Bs[(buf)][(ra_row + 32 * i_) * PK + ra_kq]) = RBr[i_];     \
      else                                                                                     \
        *reinterpret_cast<float4*>(&Bs[(buf)][(rb_k + RB_ROWS * i_) * PN + rb_nq]) = RBr[i_];  \
    }                                                                                          \
  } while (0)

  f32x16 acc[NBLK][NBLK];
#pragma unroll
  for (int i = 0; i < NBLK; ++i)
#pragma unroll
    for (int j = 0; j < NBLK; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int lr = lane & 31, lh = lane >> 5;
  // One slab: 4 k-octets × (NBLK×NBLK blocks × 4 MFMAs).
#define GF_MMA(buf)                                                                            \
  do {                                                                                         \
    const float* as_ = As[(buf)];                                                              \
    const float* bs_ = Bs[(buf)];                                                              \
    _Pragma("unroll") for (int o = 0; o < BK / 8; ++o) {                                       \
      float4 av[NBLK], bv[NBLK];                                                               \
      _Pragma("unroll") for (int i = 0; i < NBLK; ++i)                                         \
        av[i] = *reinterpret_cast<const float4*>(as_ + (wm * WT + i * 32 + lr) * PK + o * 8 + lh * 4); \
      _Pragma("unroll") for (int j = 0; j < NBLK; ++j) {                                       \
        if (B_KCONTIG) {                                                                       \
          bv[j] = *reinterpret_cast<const float4*>(bs_ + (wn * WT + j * 32 + lr) * PK + o * 8 + lh * 4); \
        } else {                                                                               \
          const float* pb_ = bs_ + (o * 8 + lh * 4) * PN + wn * WT + j * 32 + lr;            \
          bv[j] = make_float4(pb_[0], pb_[PN], pb_[2 * PN], pb_[3 * PN]);                      \
        }                                                                                      \
      }                                                                                        \
      _Pragma("unroll") for (int i = 0; i < NBLK; ++i)                                         \
      _Pragma("unroll") for (int j = 0; j < NBLK; ++j) {                                       \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].x, bv[j].x, acc[i][j], 0, 0, 0); \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].y, bv[j].y, acc[i][j], 0, 0, 0); \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].z, bv[j].z, acc[i][j], 0, 0, 0); \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i].w, bv[j].w, acc[i][j], 0, 0, 0); \
      }                                                                                        \
    }                                                                                          \
  } while (0)

  // Split products: per 16-k step each lane's 8 consecutive k of a row (A) or
  // column (B) are split into three bf16 fragments, and the six products
  // whose pieces sum to at most 2⁻¹⁶ relative go through the bf16 matrix
  // cores (the three dropped ones are below 2⁻²³ of |a·b|).
#define GF_MMA_SPLIT(buf)                                                                      \
  do {                                                                                         \
    const float* as_ = As[(buf)];                                                              \
    const float* bs_ = Bs[(buf)];                                                              \
    _Pragma("unroll") for (int s_ = 0; s_ < BK / 16; ++s_) {                                   \
      bf16x8 ah[NBLK], am[NBLK], al[NBLK], bh[NBLK], bm[NBLK], bl[NBLK];                       \
      _Pragma("unroll") for (int i = 0; i < NBLK; ++i) {                                       \
        const float* p_ = as_ + (wm * WT + i * 32 + lr) * PK + s_ * 16 + lh * 8;               \
        split3(*reinterpret_cast<const float4*>(p_), *reinterpret_cast<const float4*>(p_ + 4), \
               ah[i], am[i], al[i]);                                                           \
      }                                                                                        \
      _Pragma("unroll") for (int j = 0; j < NBLK; ++j) {                                       \
        float4 u0_, u1_;                                                                       \
        if (B_KCONTIG) {                                                                       \
          const float* p_ = bs_ + (wn * WT + j * 32 + lr) * PK + s_ * 16 + lh * 8;             \
          u0_ = *reinterpret_cast<const float4*>(p_);                                          \
          u1_ = *reinterpret_cast<const float4*>(p_ + 4);                                      \
        } else {                                                                               \
          const float* p_ = bs_ + (s_ * 16 + lh * 8) * PN + wn * WT + j * 32 + lr;             \
          u0_ = make_float4(p_[0], p_[PN], p_[2 * PN], p_[3 * PN]);                            \
          u1_ = make_float4(p_[4 * PN], p_[5 * PN], p_[6 * PN], p_[7 * PN]);                   \
        }                                                                                      \
        split3(u0_, u1_, bh[j], bm[j], bl[j]);                                                 \
      }                                                                                        \
      _Pragma("unroll") for (int i = 0; i < NBLK; ++i)                                         \
      _Pragma("unroll") for (int j = 0; j < NBLK; ++j) {                                       \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bh[j], acc[i][j], 0, 0, 0); \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bl[j], acc[i][j], 0, 0, 0); \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am[i], bm[j], acc[i][j], 0, 0, 0); \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am[i], bh[j], acc[i][j], 0, 0, 0); \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bm[j], acc[i][j], 0, 0, 0); \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bh[j], acc[i][j], 0, 0, 0); \
      }                                                                                        \
    }                                                                                          \
  } while (0)

  if constexpr (SPLIT && B_KCONTIG) {
    // 16-k slabs through three bf16 planes per operand, four slabs of global
    // loads in flight (register sets s0..s3 hold the slabs ≡ 0..3 mod 4).
    constexpr int PL = TILE * SP;                          // bf16 per plane
    static_assert(2 * 3 * PL * 2 <= (int)sizeof(As) && 2 * 3 * PL * 2 <= (int)sizeof(Bs),
                  "split planes exceed the operand buffers");
    __bf16* const Ap = reinterpret_cast<__bf16*>(&As[0][0]);  // [buf][plane][row][SP]
    __bf16* const Bp = reinterpret_cast<__bf16*>(&Bs[0][0]);
    constexpr int RS = TILE / 64;                          // float4 per thread ([row][k])
    constexpr int KPT = SK * TILE / 256;                   // B as K×N: k per thread (8 or 4)
    const int sa_row = tid >> 2, sa_kq = (tid & 3) * 4;
    const int sb_n = tid % TILE, sb_k = (tid / TILE) * KPT;
    const uint32_t b_off = B_KCONTIG ? 0u : (uint32_t)(sb_k * g.ldb + sb_n);
    float4 ra0[RS], ra1[RS], ra2[RS], ra3[RS];
    float4 rb0[RS], rb1[RS], rb2[RS], rb3[RS];
    float bs0[KPT], bs1[KPT], bs2[KPT], bs3[KPT];
#define GS_LOAD(RA_, RB_, BS_, slab)                                                           \
  do {                                                                                         \
    const int64_t k0_ = klo + (int64_t)(slab) * SK;                                            \
    _Pragma("unroll") for (int i_ = 0; i_ < RS; ++i_)                                          \
      RA_[i_] = ld4(A, g.lda, m0 + sa_row + 64 * i_, k0_ + sa_kq, M, K);                       \
    if (B_KCONTIG) {                                                                           \
      _Pragma("unroll") for (int i_ = 0; i_ < RS; ++i_)                                        \
        RB_[i_] = ld4(B, g.ldb, n0 + sa_row + 64 * i_, k0_ + sa_kq, N, K);                     \
    } else {                                                                                   \
      /* uniform row base + a 32-bit per-thread offset */                                      \
      const bool n_ok_ = n0 + sb_n < N;                                                        \
      _Pragma("unroll") for (int c_ = 0; c_ < KPT; ++c_) {                                     \
        const float* row_ = B + (k0_ + c_) * g.ldb + n0;                                       \
        BS_[c_] = (n_ok_ && k0_ + sb_k + c_ < K) ? row_[b_off] : 0.f;                          \
      }                                                                                        \
    }                                                                                          \
  } while (0)
#define GS_STORE(RA_, RB_, BS_, buf)                                                           \
  do {                                                                                         \
    _Pragma("unroll") for (int i_ = 0; i_ < RS; ++i_) {                                        \
      bf16x4 h_, m_, l_;                                                                       \
      split4(RA_[i_], h_, m_, l_);                                                             \
      __bf16* p_ = Ap + (buf) * 3 * PL + (sa_row + 64 * i_) * SP + sa_kq;                      \
      *reinterpret_cast<bf16x4*>(p_) = h_;                                                     \
      *reinterpret_cast<bf16x4*>(p_ + PL) = m_;                                                \
      *reinterpret_cast<bf16x4*>(p_ + 2 * PL) = l_;                                            \
    }                                                                                          \
    if (B_KCONTIG) {                                                                           \
      _Pragma("unroll") for (int i_ = 0; i_ < RS; ++i_) {                                      \
        bf16x4 h_, m_, l_;                                                                     \
        split4(RB_[i_], h_, m_, l_);                                                           \
        __bf16* p_ = Bp + (buf) * 3 * PL + (sa_row + 64 * i_) * SP + sa_kq;                    \
        *reinterpret_cast<bf16x4*>(p_) = h_;                                                   \
        *reinterpret_cast<bf16x4*>(p_ + PL) = m_;                                              \
        *reinterpret_cast<bf16x4*>(p_ + 2 * PL) = l_;                                          \
      }                                                                                        \
    } else {                                                                                   \
      _Pragma("unroll") for (int q_ = 0; q_ < KPT / 4; ++q_) {                                 \
        bf16x4 h_, m_, l_;                                                                     \
        split4(make_float4(BS_[4 * q_], BS_[4 * q_ + 1], BS_[4 * q_ + 2], BS_[4 * q_ + 3]),    \
               h_, m_, l_);                                                                    \
        __bf16* p_ = Bp + (buf) * 3 * PL + sb_n * SP + sb_k + 4 * q_;                          \
        *reinterpret_cast<bf16x4*>(p_) = h_;                                                   \
        *reinterpret_cast<bf16x4*>(p_ + PL) = m_;                                              \
        *reinterpret_cast<bf16x4*>(p_ + 2 * PL) = l_;                                          \
      }                                                                                        \
    }                                                                                          \
  } while (0)
    // The six cross products whose pieces sum to at most 2⁻¹⁶ relative (the
    // three dropped ones are below 2⁻²³ of |a·b|), smallest first.
#define GS_MMA(buf)                                                                            \
  do {                                                                                         \
    const __bf16* a_ = Ap + (buf) * 3 * PL;                                                    \
    const __bf16* b_ = Bp + (buf) * 3 * PL;                                                    \
    bf16x8 ah[NBLK], am[NBLK], al[NBLK], bh[NBLK], bm[NBLK], bl[NBLK];                         \
    _Pragma("unroll") for (int i = 0; i < NBLK; ++i) {                                         \
      const int o_ = (wm * WT + i * 32 + lr) * SP + lh * 8;                                    \
      ah[i] = *reinterpret_cast<const bf16x8*>(a_ + o_);                                       \
      am[i] = *reinterpret_cast<const bf16x8*>(a_ + PL + o_);                                  \
      al[i] = *reinterpret_cast<const bf16x8*>(a_ + 2 * PL + o_);                              \
    }                                                                                          \
    _Pragma("unroll") for (int j = 0; j < NBLK; ++j) {                                         \
      const int o_ = (wn * WT + j * 32 + lr) * SP + lh * 8;                                    \
      bh[j] = *reinterpret_cast<const bf16x8*>(b_ + o_);                                       \
      bm[j] = *reinterpret_cast<const bf16x8*>(b_ + PL + o_);                                  \
      bl[j] = *reinterpret_cast<const bf16x8*>(b_ + 2 * PL + o_);                              \
    }                                                                                          \
    _Pragma("unroll") for (int i = 0; i < NBLK; ++i)                                           \
    _Pragma("unroll") for (int j = 0; j < NBLK; ++j) {                                         \
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bh[j], acc[i][j], 0, 0, 0);   \
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bl[j], acc[i][j], 0, 0, 0);   \
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am[i], bm[j], acc[i][j], 0, 0, 0);   \
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am[i], bh[j], acc[i][j], 0, 0, 0);   \
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bm[j], acc[i][j], 0, 0, 0);   \
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bh[j], acc[i][j], 0, 0, 0);   \
    }                                                                                          \
  } while (0)
    // Step t: the MMAs of slab t (buffer t % 2), then slab t+1 goes from its
    // register set into the other buffer and that set loads slab t+5.  Slabs
    // past the end load zeros and skip their MMAs.
    // Interleave the step's MFMAs with the next slab's split (VALU), LDS
    // stores and global loads, so one wave's conversions overlap its own
    // matrix-core work instead of waiting behind the whole MFMA burst.
    constexpr int NMF = 6 * NBLK * NBLK;                   // MFMAs per step
#define GS_PATTERN()                                                                           \
  do {                                                                                         \
    __builtin_amdgcn_sched_group_barrier(0x100, 6 * NBLK, 0); /* DS read */                    \
    __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);        /* VALU */                       \
    _Pragma("unroll") for (int r_ = 0; r_ < NMF; ++r_) {                                       \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);      /* MFMA */                       \
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);                                       \
      if (r_ % 2 == 1) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0); /* DS write */       \
      if (r_ % 4 == 3) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); /* VMEM read */      \
    }                                                                                          \
  } while (0)
#define GS_STEP(t, RA_, RB_, BS_)                                                              \
  do {                                                                                         \
    __builtin_amdgcn_sched_barrier(0);                                                         \
    if ((t) < nk) GS_MMA((t) & 1);                                                             \
    GS_STORE(RA_, RB_, BS_, ((t) + 1) & 1);                                                    \
    GS_LOAD(RA_, RB_, BS_, (t) + 5);                                                           \
    __builtin_amdgcn_sched_barrier(0);                                                         \
    __syncthreads();                                                                           \
  } while (0)
    // A step known to be inside the K range: one basic block, interleaved.
#define GS_STEP_IN(t, RA_, RB_, BS_)                                                           \
  do {                                                                                         \
    __builtin_amdgcn_sched_barrier(0);                                                         \
    GS_MMA((t) & 1);                                                                           \
    GS_STORE(RA_, RB_, BS_, ((t) + 1) & 1);                                                    \
    GS_LOAD(RA_, RB_, BS_, (t) + 5);                                                           \
    GS_PATTERN();                                                                              \
    __builtin_amdgcn_sched_barrier(0);                                                         \
    __syncthreads();                                                                           \
  } while (0)
    const int nk = K > klo ? (int)cdiv(K - klo, (int64_t)SK) : 0;
    if (nk > 0) {
      GS_LOAD(ra0, rb0, bs0, 0);
      GS_STORE(ra0, rb0, bs0, 0);
      GS_LOAD(ra1, rb1, bs1, 1);
      GS_LOAD(ra2, rb2, bs2, 2);
      GS_LOAD(ra3, rb3, bs3, 3);
      GS_LOAD(ra0, rb0, bs0, 4);
    }
    __syncthreads();
    int kt = 0;
    for (; kt + 4 <= nk; kt += 4) {
      GS_STEP_IN(kt, ra1, rb1, bs1);
      GS_STEP_IN(kt + 1, ra2, rb2, bs2);
      GS_STEP_IN(kt + 2, ra3, rb3, bs3);
      GS_STEP_IN(kt + 3, ra0, rb0, bs0);
    }
    if (kt < nk) {
      GS_STEP(kt, ra1, rb1, bs1);
      GS_STEP(kt + 1, ra2, rb2, bs2);
      GS_STEP(kt + 2, ra3, rb3, bs3);
      GS_STEP(kt + 3, ra0, rb0, bs0);
    }
    __builtin_amdgcn_sched_barrier(0);
#undef GS_LOAD
#undef GS_STORE
#undef GS_MMA
#undef GS_STEP
#undef GS_STEP_IN
#undef GS_PATTERN
  } else {
    // Slabs are processed in pairs; a trailing odd slab and the prefetches
    // past the end load zeros (k >= K is masked), which add nothing.
    const int nk = K > klo ? (int)cdiv(K - klo, (int64_t)BK) : 0;
    const int nk2 = (nk + 1) & ~1;
    if (nk2 > 0) {
      GF_LOAD(xa, xb, 0);
      GF_STORE(xa, xb, 0);
      GF_LOAD(xa, xb, 1);
      GF_LOAD(ya, yb, 2);
    }
    __syncthreads();
    for (int kt = 0; kt < nk2; kt += 2) {
      __builtin_amdgcn_sched_barrier(0);
      if (SPLIT) GF_MMA_SPLIT(0); else GF_MMA(0);  // slab kt
      GF_STORE(xa, xb, 1);    // slab kt+1
      GF_LOAD(xa, xb, kt + 3);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      if (SPLIT) GF_MMA_SPLIT(1); else GF_MMA(1);  // slab kt+1
      GF_STORE(ya, yb, 0);    // slab kt+2
      GF_LOAD(ya, yb, kt + 4);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#undef GF_LOAD
#undef GF_STORE
#undef GF_MMA
#undef GF_MMA_SPLIT

  // Epilogue.  32×32 MFMA output: lane holds rows 8*(v/4) + 4*(lane/32) + v%4,
  // column lane%32.  C / X may alias D (in-place updates), so the inputs of a
  // row of blocks (16·NBLK per lane) are loaded before any of its outputs is
  // stored: NBLK memory round trips per lane instead of one per element.
  const float* C = g.C ? g.C + b1 * g.sC + b2 * g.sC2 : nullptr;
  const float* X = g.X ? g.X + b1 * g.sX + b2 * g.sX2 : nullptr;
  float* D = g.D + b1 * g.sD + b2 * g.sD2;
  const bool use_c = g.beta != 0.f, use_x = g.gamma != 0.f;
#pragma unroll
  for (int i = 0; i < NBLK; ++i) {
    float cv[NBLK][16];
#pragma unroll
    for (int j = 0; j < NBLK; ++j) {
      const int64_t n = n0 + wn * WT + j * 32 + lr;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + wm * WT + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
        const bool in = m < M && n < N;
        cv[j][v] = (use_c && in) ? C[m * g.ldc + n] : 0.f;
      }
    }
    if (use_x) {
#pragma unroll
      for (int j = 0; j < NBLK; ++j) {
        const int64_t n = n0 + wn * WT + j * 32 + lr;
        float xv[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t m = m0 + wm * WT + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
          xv[v] = (m < M && n < N) ? X[m * g.ldx + n] : 0.f;
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) cv[j][v] = g.beta * cv[j][v] + g.gamma * xv[v];
      }
    } else {
#pragma unroll
      for (int j = 0; j < NBLK; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) cv[j][v] = g.beta * cv[j][v];
    }
#pragma unroll
    for (int j = 0; j < NBLK; ++j) {
      const int64_t n = n0 + wn * WT + j * 32 + lr;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + wm * WT + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
        const float val = g.alpha * acc[i][j][v] + cv[j][v];
        if (m >= M || n >= N) continue;
        if (g.uplo == 1 && n > m) continue;
        if (g.uplo == 2 && m > n) continue;
        D[m * g.ldd + n] = val;
      }
    }
  }
}

// Large split products (K >= 384, B given N×K, no triangular skipping, a grid
// of at least a wave of 256×256 tiles): one workgroup of 8 waves computes a
// 256×256 tile, each wave 128×64 (4×2 blocks of 32×32), from 16-k stages of
// both operands split into three bf16 planes as they are stored to LDS.  Per
// stage a wave reads 12 row and 6 column fragments for 48 MFMAs (the 128×128
// kernel: 12 for 24) and a workgroup splits 16 elements per thread for twice
// the MFMAs per barrier.  Each accumulator receives the same six products in
// the same order, stage by stage, as gemm_f32_kernel's split path, so the
// results equal it bit for bit.
constexpr int S2T = 256;  // tile edge
template <bool VEC>
__global__ __launch_bounds__(512) void gemm_s256_kernel(GemmF32 g, int64_t tm, int64_t tn) {
  constexpr int PL = S2T * SP;  // bf16 per plane
  __shared__ __attribute__((aligned(16))) __bf16 Ap[2][3][PL];
  __shared__ __attribute__((aligned(16))) __bf16 Bp[2][3][PL];

  const int z = blockIdx.z;
  const int64_t b1 = z / g.batch2, b2 = z % g.batch2;
  if (g.skip && g.skip[b1]) return;
  const int64_t nwg = gridDim.x, bid = blockIdx.x;
  const int64_t q8 = nwg >> 3, r8 = nwg & 7, xcd = bid & 7;
  const int64_t id = xcd * q8 + (xcd < r8 ? xcd : r8) + (bid >> 3);
  int64_t im, in;
  tile_of(id, tm, tn, im, in);
  const int64_t m0 = im * S2T, n0 = in * S2T;
  if (g.uplo == 1 && n0 > m0 + S2T - 1) return;
  if (g.uplo == 2 && m0 > n0 + S2T - 1) return;

  const float* __restrict__ A = g.A + b1 * g.sA + b2 * g.sA2;
  const float* __restrict__ B = g.B + b1 * g.sB + b2 * g.sB2;
  const int64_t M = g.M, N = g.N, K = g.K;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;

  auto ld4 = [&](const float* base, int64_t ld, int64_t r, int64_t c, int64_t R, int64_t Ccols) {
    if (VEC) {
      const bool ok = r < R && c < Ccols;
      const uint4 w = *reinterpret_cast<const uint4*>(base + (ok ? r * ld + c : 0));
      const uint32_t m = ok ? 0xffffffffu : 0u;
      return make_float4(__uint_as_float(w.x & m), __uint_as_float(w.y & m),
                         __uint_as_float(w.z & m), __uint_as_float(w.w & m));
    }
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r < R) {
      const float* p = base + r * ld + c;
      if (c < Ccols) v.x = p[0];
      if (c + 1 < Ccols) v.y = p[1];
      if (c + 2 < Ccols) v.z = p[2];
      if (c + 3 < Ccols) v.w = p[3];
    }
    return v;
  };

  // Stage = 16 k: row r of a tile as four 4-k quads; thread tid holds quads
  // (tid >> 2) + 128 i of both operands.
  const int sa_row = tid >> 2, sa_kq = (tid & 3) * 4;
  float4 xa0, xa1, xb0, xb1, ya0, ya1, yb0, yb1;
#define S2_LOAD(R, st)                                                                         \
  do {                                                                                         \
    const int64_t k0_ = (int64_t)(st) * SK;                                                    \
    R##a0 = ld4(A, g.lda, m0 + sa_row, k0_ + sa_kq, M, K);                                     \
    R##a1 = ld4(A, g.lda, m0 + sa_row + 128, k0_ + sa_kq, M, K);                               \
    R##b0 = ld4(B, g.ldb, n0 + sa_row, k0_ + sa_kq, N, K);                                     \
    R##b1 = ld4(B, g.ldb, n0 + sa_row + 128, k0_ + sa_kq, N, K);                               \
  } while (0)
#define S2_PUT(P, buf, row, v)                                                                 \
  do {                                                                                         \
    bf16x4 h_, m_, l_;                                                                         \
    split4((v), h_, m_, l_);                                                                   \
    const int o_ = (row) * SP + sa_kq;                                                         \
    *reinterpret_cast<bf16x4*>(&P[(buf)][0][o_]) = h_;                                         \
    *reinterpret_cast<bf16x4*>(&P[(buf)][1][o_]) = m_;                                         \
    *reinterpret_cast<bf16x4*>(&P[(buf)][2][o_]) = l_;                                         \
  } while (0)
#define S2_STORE(R, buf)                                                                       \
  do {                                                                                         \
    S2_PUT(Ap, buf, sa_row, R##a0);                                                            \
    S2_PUT(Ap, buf, sa_row + 128, R##a1);                                                      \
    S2_PUT(Bp, buf, sa_row, R##b0);                                                            \
    S2_PUT(Bp, buf, sa_row + 128, R##b1);                                                      \
  } while (0)

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int lr = lane & 31, lh = lane >> 5;
  // The six cross products in gemm_f32_kernel's order, per accumulator.
#define S2_MMA(buf)                                                                            \
  do {                                                                                         \
    bf16x8 bh[2], bm[2], bl[2];                                                                \
    _Pragma("unroll") for (int j = 0; j < 2; ++j) {                                            \
      const int o_ = (wn * 64 + j * 32 + lr) * SP + lh * 8;                                    \
      bh[j] = *reinterpret_cast<const bf16x8*>(&Bp[(buf)][0][o_]);                             \
      bm[j] = *reinterpret_cast<const bf16x8*>(&Bp[(buf)][1][o_]);                             \
      bl[j] = *reinterpret_cast<const bf16x8*>(&Bp[(buf)][2][o_]);                             \
    }                                                                                          \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                            \
      const int o_ = (wm * 128 + i * 32 + lr) * SP + lh * 8;                                   \
      const bf16x8 ah = *reinterpret_cast<const bf16x8*>(&Ap[(buf)][0][o_]);                   \
      const bf16x8 am = *reinterpret_cast<const bf16x8*>(&Ap[(buf)][1][o_]);                   \
      const bf16x8 al = *reinterpret_cast<const bf16x8*>(&Ap[(buf)][2][o_]);                   \
      _Pragma("unroll") for (int j = 0; j < 2; ++j) {                                          \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh[j], acc[i][j], 0, 0, 0);     \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl[j], acc[i][j], 0, 0, 0);     \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bm[j], acc[i][j], 0, 0, 0);     \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bh[j], acc[i][j], 0, 0, 0);     \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bm[j], acc[i][j], 0, 0, 0);     \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh[j], acc[i][j], 0, 0, 0);     \
      }                                                                                        \
    }                                                                                          \
  } while (0)

  // Stage t is multiplied out of buffer t&1 while stage t+1 goes from its
  // register set to the other buffer and that set loads stage t+3; stages
  // past K load zeros and skip their MFMAs.  One barrier per stage.
  const int nk = (int)cdiv(K, (int64_t)SK);
  S2_LOAD(x, 0);
  S2_STORE(x, 0);
  S2_LOAD(x, 1);
  S2_LOAD(y, 2);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    __builtin_amdgcn_sched_barrier(0);
    S2_MMA(0);
    S2_STORE(x, 1);
    S2_LOAD(x, kt + 3);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    if (kt + 1 < nk) {
      __builtin_amdgcn_sched_barrier(0);
      S2_MMA(1);
      S2_STORE(y, 0);
      S2_LOAD(y, kt + 4);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
    }
  }
  __builtin_amdgcn_sched_barrier(0);
#undef S2_LOAD
#undef S2_PUT
#undef S2_STORE
#undef S2_MMA

  // Epilogue as gemm_f32_kernel's: the inputs of a row of blocks are loaded
  // before any of its outputs is stored (C / X may alias D).
  const float* C = g.C ? g.C + b1 * g.sC + b2 * g.sC2 : nullptr;
  const float* X = g.X ? g.X + b1 * g.sX + b2 * g.sX2 : nullptr;
  float* D = g.D + b1 * g.sD + b2 * g.sD2;
  const bool use_c = g.beta != 0.f, use_x = g.gamma != 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float cv[2][16];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n0 + wn * 64 + j * 32 + lr;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + wm * 128 + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
        const bool ok = m < M && n < N;
        cv[j][v] = (use_c && ok) ? C[m * g.ldc + n] : 0.f;
      }
    }
    if (use_x) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t n = n0 + wn * 64 + j * 32 + lr;
        float xv[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t m = m0 + wm * 128 + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
          xv[v] = (m < M && n < N) ? X[m * g.ldx + n] : 0.f;
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) cv[j][v] = g.beta * cv[j][v] + g.gamma * xv[v];
      }
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) cv[j][v] = g.beta * cv[j][v];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n0 + wn * 64 + j * 32 + lr;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + wm * 128 + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
        const float val = g.alpha * acc[i][j][v] + cv[j][v];
        if (m >= M || n >= N) continue;
        if (g.uplo == 1 && n > m) continue;
        if (g.uplo == 2 && m > n) continue;
        D[m * g.ldd + n] = val;
      }
    }
  }
}

template <int TILE, bool SPLIT>
void launch_variant(hipStream_t stream, const GemmF32& g, bool vec, dim3 grid, int64_t tm,
                    int64_t tn) {
  if (g.b_kcontig) {
    if (vec)
      hipLaunchKernelGGL((gemm_f32_kernel<TILE, true, true, SPLIT>), grid, dim3(256), 0, stream, g, tm, tn);
    else
      hipLaunchKernelGGL((gemm_f32_kernel<TILE, true, false, SPLIT>), grid, dim3(256), 0, stream, g, tm, tn);
  } else {
    if (vec)
      hipLaunchKernelGGL((gemm_f32_kernel<TILE, false, true, SPLIT>), grid, dim3(256), 0, stream, g, tm, tn);
    else
      hipLaunchKernelGGL((gemm_f32_kernel<TILE, false, false, SPLIT>), grid, dim3(256), 0, stream, g, tm, tn);
  }
}

template <int TILE>
void launch_gemm(hipStream_t stream, const GemmF32& g, bool vec, int64_t nz, bool split) {
  const int64_t tm = cdiv(g.M, (int64_t)TILE), tn = cdiv(g.N, (int64_t)TILE);
  dim3 grid((unsigned)(tm * tn), 1, (unsigned)nz);
  if (split) {
    launch_variant<TILE, true>(stream, g, vec, grid, tm, tn);
  } else {
    launch_variant<TILE, false>(stream, g, vec, grid, tm, tn);
  }
}

}  // namespace

int gemm_f32(hipStream_t stream, const GemmF32& g) {
  if (g.M <= 0 || g.N <= 0 || g.batch <= 0 || g.batch2 <= 0) return G2PTQ_OK;
  G2PTQ_CHECK(g.K >= 0, "gemm_f32: negative K");
  G2PTQ_CHECK(g.A != nullptr || g.K == 0, "gemm_f32: null A");
  G2PTQ_CHECK(g.B != nullptr || g.K == 0, "gemm_f32: null B");
  G2PTQ_CHECK(g.D != nullptr, "gemm_f32: null D");
  G2PTQ_CHECK(g.beta == 0.f || g.C != nullptr, "gemm_f32: beta != 0 needs C");
  G2PTQ_CHECK(g.gamma == 0.f || g.X != nullptr, "gemm_f32: gamma != 0 needs X");
  const int64_t nz = g.batch * g.batch2;
  const int64_t t128 = cdiv(g.M, (int64_t)128) * cdiv(g.N, (int64_t)128);
  G2PTQ_CHECK(cdiv(g.M, (int64_t)64) * cdiv(g.N, (int64_t)64) < (1ll << 31) && nz < 65536,
              "gemm_f32: grid too large");
  // 16-byte operand loads need 16-byte aligned rows (every batch entry too).
  auto al = [](const void* p, int64_t ld, int64_t s1, int64_t s2) {
    return p == nullptr || ((reinterpret_cast<uintptr_t>(p) & 15) == 0 && ld % 4 == 0 &&
                            s1 % 4 == 0 && s2 % 4 == 0);
  };
  // ... and whole 16-byte chunks along k (and along n for B given K×N).
  const bool vec = al(g.A, g.lda, g.sA, g.sA2) && al(g.B, g.ldb, g.sB, g.sB2) && g.K % 4 == 0 &&
                   (g.b_kcontig || g.N % 4 == 0);
  // 128×128 tiles unless that grid would leave most of the 256 CUs (two
  // workgroups each) idle.
  // Products with K >= 128 run on the bf16 matrix cores from split operands
  // (about 1.3x the fp32 MFMA rate, and no less accurate); the short-K updates
  // of the factor's panels are latency-bound and keep the fp32 MFMAs.
  const bool split = g.K >= 128;
  G2PTQ_CHECK(!split || g.b_kcontig || g.ldb < (1ll << 27),
              "gemm_f32: ldb %lld too large for the split path's 32-bit row offsets",
              (long long)g.ldb);
  const int64_t t256 = cdiv(g.M, (int64_t)S2T) * cdiv(g.N, (int64_t)S2T);
  if (split && g.b_kcontig && g.tri == 0 && g.K >= 384 && t256 * nz >= 256) {
    const int64_t tm = cdiv(g.M, (int64_t)S2T), tn = cdiv(g.N, (int64_t)S2T);
    const dim3 grid((unsigned)(tm * tn), 1, (unsigned)nz);
    if (vec) hipLaunchKernelGGL(gemm_s256_kernel<true>, grid, dim3(512), 0, stream, g, tm, tn);
    else hipLaunchKernelGGL(gemm_s256_kernel<false>, grid, dim3(512), 0, stream, g, tm, tn);
  } else if (t128 * nz >= 512) {
    launch_gemm<128>(stream, g, vec, nz, split);
  } else {
    launch_gemm<64>(stream, g, vec, nz, split);
  }
  G2PTQ_LAUNCHED();
  return G2PTQ_OK;
}

}  // namespace g2ptq

extern "C" int g2ptq_gemm_f32(void* stream, int64_t M, int64_t N, int64_t K, int64_t batch,
                              const float* A, int64_t lda, int64_t sA, const float* B, int64_t ldb,
                              int64_t sB, int b_trans, const float* C, int64_t ldc, int64_t sC,
                              float* D, int64_t ldd, int64_t sD, float alpha, float beta) {
  g2ptq::GemmF32 g;
  g.M = M; g.N = N; g.K = K; g.batch = batch;
  g.A = A; g.lda = lda; g.sA = sA;
  g.B = B; g.ldb = ldb; g.sB = sB; g.b_kcontig = b_trans;
  g.C = C; g.ldc = ldc; g.sC = sC;
  g.D = D; g.ldd = ldd; g.sD = sD;
  g.alpha = alpha; g.beta = beta;
  return g2ptq::gemm_f32(g2ptq::as_stream(stream), g);
}
