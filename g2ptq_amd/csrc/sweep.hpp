// Block-sweep argument block shared by the run_eager entry point and the
// per-layer compensation driver.
#pragma once
#include "common.hpp"

namespace g2ptq {

constexpr int kMaxBlock = 128;  // largest supported lazy-batch block width

// Element (b, r, c) of a strided 3-D operand lives at p + b*sb + r*sr + c*sc.
struct SweepArgs {
  int64_t R;     // rows per layer
  int n;         // block width (columns), 1..kMaxBlock
  int maxq;
  const float* W; int64_t wb, wr, wc;          // block input values
  const float* U; int64_t ub, uj;              // U(b, j, k) = U[b*ub + j*uj + k]
  const float* P;                              // GPTAQ, same strides as U
  const float* Zg; int64_t zb, zr, zc;         // G2PTQ z
  const float* GH; int64_t gb, gr, gc;         // G2PTQ ghinv (block input)
  float* GHout;                                // block ghinv written back (nullable; same strides)
  // Quantizer parameters: scale of (b, r, column j) = S[b*sb + r*sr + group(j)*sg]
  // with group(j) = colgroup[j] if colgroup, else (col0 + j) / gsize (gsize <= 0: 0).
  const float* S; const float* Z0; int64_t sb, sr, sg;
  const int* colgroup; int64_t col0; int64_t gsize;
  // Fused dynamic-group parameters (fuse > 0): the min/max parameters of each
  // fuse-wide column group of the block are fitted from the block's input
  // values at the start of the sweep, written to FS/FZ (the S/Z0 table
  // layout) and used in place of S/Z0.  Requires fuse % 32 == 0, the block
  // starting on a group boundary and n % 32 == 0 (the 32-column panel path).
  int64_t fuse; int sym;
  float* FS; float* FZ;
  float* Q; int64_t qb, qr, qc;                // dequantized output
  float* I; int64_t ib, ir, ic;                // integer codes (nullable)
  float* E; int64_t eb, er, ec;                // scaled errors (nullable)
  float* Sc; int64_t cb, cr, cc;               // per-column scale (nullable)
  float* CW; int64_t cwb, cwr;                 // GPTAQ last pre-quant column (nullable)
  float* E2; int64_t e2b, e2r, e2c;            // G2PTQ: err - z*(dist0 - j) (nullable)
  int64_t dist0;                               // G2PTQ: blocksize - 1
  // G2PTQ, super-block far tail: err - z*(dist3 - j) (nullable; same strides
  // as E2); dist3 = dist0 + the columns of the super-block after this block.
  float* E3; int64_t e3b, e3r; int64_t dist3;
  // Super-block mode (GPTQ, 16 lanes per row, full 128-column blocks,
  // column-contiguous rows; nblk > 1): the launch sweeps nblk consecutive
  // blocks, W, U and the outputs pointing at the first, and applies each
  // block's errors to its rows' columns of the later blocks in Wsb (the
  // writable W the block inputs come from) before sweeping the next.
  int nblk;
  float* Wsb;
  int* flags;
};

int launch_sweep(hipStream_t stream, int variant, const SweepArgs& a, int64_t B);
// Whether a GPTQ block (a.nblk unset) can run as the first of a super-block
// launch: 16 lanes per row, a full 128-column block, 16-byte aligned rows.
bool sweep_superblock_ok(const SweepArgs& a, int64_t B);
int launch_find_params(hipStream_t stream, const float* x, int64_t rows, int64_t cols,
                       int64_t ldx, int maxq, int sym, float* scale, float* zero, int64_t ldp,
                       int* flags);
// Hessian-diagonal weights of the clip search (WeightQuantizer with hclip,
// utils/quant_utils.py:393-397 and _quant_err :84-105): the searched rows
// split into `nblocks` equal consecutive shares, share b weighted by row b of
// h (nblocks × gpr·cols, pitch ld).  With gpr > 1 each original row was
// split into gpr column groups of `cols` (weight_groupsize > 0): searched row
// r is group r % gpr of original row r / gpr.  h == nullptr: no weights.
struct HDiag {
  const float* h = nullptr;
  int64_t ld = 0;
  int64_t nblocks = 0;
  int64_t gpr = 1;
};

int launch_find_params_mse(hipStream_t stream, const float* x, int64_t rows, int64_t cols,
                           int64_t ldx, int maxq, int sym, float norm, int grid, float maxshrink,
                           const HDiag& hd, float* scale, float* zero, int64_t ldp, int* flags);

}  // namespace g2ptq
