// Shared helpers for the g2ptq HIP library (gfx950 / CDNA4 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/g2ptq_hip.h"

namespace g2ptq {

// Thread-local detail string for the last failing call on this host thread.
void set_error(const char* fmt, ...);

#define G2PTQ_HIP(call)                                                        \
  do {                                                                         \
    hipError_t _e = (call);                                                    \
    if (_e != hipSuccess) {                                                    \
      ::g2ptq::set_error("%s failed: %s (%s:%d)", #call, hipGetErrorString(_e), \
                         __FILE__, __LINE__);                                  \
      return G2PTQ_ERR_HIP;                                                    \
    }                                                                          \
  } while (0)

#define G2PTQ_LAUNCHED()                                                       \
  do {                                                                         \
    hipError_t _e = hipGetLastError();                                         \
    if (_e != hipSuccess) {                                                    \
      ::g2ptq::set_error("kernel launch failed: %s (%s:%d)",                   \
                         hipGetErrorString(_e), __FILE__, __LINE__);           \
      return G2PTQ_ERR_HIP;                                                    \
    }                                                                          \
  } while (0)

#define G2PTQ_CHECK(cond, ...)                                                 \
  do {                                                                         \
    if (!(cond)) {                                                             \
      ::g2ptq::set_error(__VA_ARGS__);                                         \
      return G2PTQ_ERR_ARG;                                                    \
    }                                                                          \
  } while (0)

#define G2PTQ_TRY(call)                                                        \
  do {                                                                         \
    int _s = (call);                                                           \
    if (_s != G2PTQ_OK) return _s;                                             \
  } while (0)

static inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Error-flag bits written by kernels into a caller-owned int32 (vector atomics).
enum : int {
  FLAG_BAD_SCALE = 1,   // a quantization scale was <= 0 or NaN
  FLAG_NAN_OUTPUT = 2,  // NaN in dequantized weights
};

// ---------------------------------------------------------------------------
// Generic batched fp32 GEMM on MFMA (gemm_f32.hip).
//
//   D[b](m, n) = alpha * sum_k A[b](m, k) * B[b](k, n) + beta * C[b](m, n)
//                + gamma * X[b](m, n)
//
// A is row-major M x K (k contiguous, leading dimension lda).  B is either
// row-major K x N (b_kcontig = 0, ldb) or given as its transpose, row-major
// N x K (b_kcontig = 1).  C, D and X are row-major with their own leading
// dimensions; C and D may alias.  uplo: 0 full output, 1 only tiles touching
// the lower triangle (m >= n) are computed and only m >= n is stored, 2 the
// same for the upper triangle.
// ---------------------------------------------------------------------------
struct GemmF32 {
  int64_t M = 0, N = 0, K = 0;
  // Two batch levels: entry z = b1 * batch2 + b2 lives at base + b1*s? + b2*s?2.
  int64_t batch = 1, batch2 = 1;
  const float* A = nullptr; int64_t lda = 0, sA = 0, sA2 = 0;
  const float* B = nullptr; int64_t ldb = 0, sB = 0, sB2 = 0; int b_kcontig = 0;
  const float* C = nullptr; int64_t ldc = 0, sC = 0, sC2 = 0;
  float* D = nullptr; int64_t ldd = 0, sD = 0, sD2 = 0;
  const float* X = nullptr; int64_t ldx = 0, sX = 0, sX2 = 0;
  float alpha = 1.f, beta = 0.f, gamma = 0.f;
  int uplo = 0;
  // Structural zeros the kernel may skip (optimisation only; the skipped
  // products must be zero): bit 1 = A lower triangular (A[m][k] = 0 for
  // k > m), bit 2 = B lower triangular (B[k][n] = 0 for k < n), bit 4 = A
  // upper triangular (A[m][k] = 0 for k < m), bit 8 = B upper triangular
  // (B[k][n] = 0 for k > n).
  int tri = 0;
  const int* skip = nullptr;  // optional per-b1 flag: nonzero => skip that entry
};

int gemm_f32(hipStream_t stream, const GemmF32& g);

// Two more streams (default priority) and events per (device, caller stream),
// created on first use and kept, for the lookahead of the factor (the
// trailing updates on `stream`, the triangular inverse's block rows on
// `stream2`) and of the compensation loop (the far block tails on `stream`).
// Calls on different caller streams get different side streams and events, so
// they can overlap; calls from several host threads on one caller stream
// interleave their launches and must not overlap (nor share a workspace).
struct SideStream {
  hipStream_t stream = nullptr;
  hipStream_t stream2 = nullptr;
  hipEvent_t factored = nullptr;                // factor: panel done, on the main stream
  hipEvent_t done[2] = {nullptr, nullptr};      // factor: trailing updates done, on the side
  hipEvent_t inverted = nullptr;                // factor: inverse block rows done (stream2)
  hipEvent_t swept = nullptr;                   // compensation: a super-block swept (main)
  hipEvent_t tailed = nullptr;                  // compensation: its far tail applied (side)
};
int side_stream(hipStream_t caller, SideStream& out);

// p[0..n) = v with a kernel (graph-capture safe, unlike hipMemsetAsync).
int fill_f32(hipStream_t stream, float* p, int64_t n, float v);

}  // namespace g2ptq
