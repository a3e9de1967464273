// Small fp32 GEMM entry shared by the GEMM dispatcher (gemm.hip) and the
// gradient-group kernel (smallstep.hip): C[M,N] = act(A[M,K] . B[K,N] + bias)
// for problems with few output tiles, where a wave computes one 16 x 16 tile
// straight from global memory (no LDS staging) and the waves of a workgroup
// split K.  A and B are logical views given by element strides, so every
// transposition of a row-major operand is read in place.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "registry.hpp"

namespace aicf::hip {

struct SmallGemm {
  const float* A;     // A[m, k] at A[m * a_m + k * a_k]
  const float* B;     // B[k, n] at B[k * b_k + n * b_n]
  float* C;           // C[m, n] at C[m * c_m + n]
  const float* bias;  // bias[n * bias_s], nullptr = none
  int64_t a_m, a_k, b_k, b_n, c_m, bias_s;
  int64_t M, N, K;
  int relu;           // relu(acc + bias)
  // nullptr, or a copy of B written at B's element offsets (B[k * b_k +
  // n * b_n] -> bcopy[k * b_k + n * b_n]) from the loads of B the tiles make
  // anyway, shared out over the rows of tiles; needs K-contiguous B (b_k ==
  // 1, 16-byte aligned rows)
  float* bcopy;
};

// The GEMM dispatcher sends an fp32 problem with fewer than this many
// 64 x 64 output tiles to small_gemm_f32 (at most 127 such tiles, i.e. 2032
// tiles of 16 x 16); the lowering's gradient-group jobs use the same bound
// (SMALL_GEMM_MAX_TILES64 in python/aicf_hip/lower.py).
constexpr int64_t kSmallGemmMaxTiles64 = 128;

// True when small_gemm_f32 takes the problem (sizes within int range, unit
// column stride of C).
bool small_gemm_ok(const SmallGemm& g);
Status small_gemm_f32(const SmallGemm& g, hipStream_t s);

}  // namespace aicf::hip
