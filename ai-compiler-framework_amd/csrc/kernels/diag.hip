// Measurement aid (no reference counterpart): the sustained bf16 MFMA rate of
// a loop that touches no memory, on random operands.  Under the board's power
// limit the MFMA rate depends on how many operand bits switch, so this loop
// is the practical ceiling a GEMM on the same part can approach; bench.py
// reports it beside the GEMM roofline, measured in the same run.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../common/hip_util.hpp"

namespace aicf::hip {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Integer hash -> uniform value in [-2, 2): operands with random mantissas
// and signs, as a GEMM on real data presents them.
__device__ __forceinline__ float hash_uniform(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return ((float)(x & 0xffffff) / 16777216.0f - 0.5f) * 4.0f;
}

// Each wave: 8 independent 32x32 fp32 accumulators (128 registers) updated
// by v_mfma_f32_32x32x16_bf16 from 4 operand sets, `iters` rounds of 8
// MFMAs; 2 * 32 * 32 * 16 flop per MFMA.  The accumulators feed one
// conditional store so that the loop is kept.
__global__ __launch_bounds__(256) void mfma_loop_kernel(float* out, int iters, uint32_t seed) {
  bf16x8 a[4], b[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[q][i] = (__bf16)hash_uniform(threadIdx.x * 131u + q * 17u + i + seed * 7919u);
      b[q][i] = (__bf16)hash_uniform(threadIdx.x * 977u + q * 29u + i * 3u + seed * 104729u);
    }
  floatx16 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[j & 3], b[(j >> 1) & 3], acc[j], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  if (s == 1234.5f) out[0] = s;
}

}  // namespace
}  // namespace aicf::hip

extern "C" int32_t aicf_diag_mfma_loop(float* out, int32_t blocks, int32_t iters, uint32_t seed, void* stream) {
  using namespace aicf::hip;
  if (!out || blocks < 1 || iters < 1) return static_cast<int32_t>(Status::InvalidArgument);
  mfma_loop_kernel<<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(out, iters, seed);
  return static_cast<int32_t>(launch_status("aicf_diag_mfma_loop"));
}
