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
typedef float floatx4 __attribute__((ext_vector_type(4)));
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

// Each wave: `iters` rounds of 2^18 flop on accumulators that touch no
// memory.  FORM 32: 8 independent 32x32 fp32 accumulators (128 registers)
// updated by v_mfma_f32_32x32x16_bf16 (2 * 32 * 32 * 16 flop each); FORM 16:
// 16 independent 16x16 accumulators (64 registers) updated by
// v_mfma_f32_16x16x32_bf16 (2 * 16 * 16 * 32 flop each), the form the GEMM
// kernels issue.  Both read the same 4 random operand sets.  The
// accumulators feed one conditional store so that the loop is kept.
template <int FORM>
__global__ __launch_bounds__(256) void mfma_loop_kernel(float* out, int iters, uint32_t seed) {
  bf16x8 a[4], b[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[q][i] = (__bf16)hash_uniform(threadIdx.x * 131u + q * 17u + i + seed * 7919u);
      b[q][i] = (__bf16)hash_uniform(threadIdx.x * 977u + q * 29u + i * 3u + seed * 104729u);
    }
  float s = 0.0f;
  if constexpr (FORM == 32) {
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
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += acc[j][r];
  } else {
    floatx4 acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[j][r] = 0.0f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 16; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j & 3], b[(j >> 2) & 3], acc[j], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) s += acc[j][r];
  }
  if (s == 1234.5f) out[0] = s;
}

}  // namespace
}  // namespace aicf::hip

extern "C" int32_t aicf_diag_mfma_loop_form(float* out, int32_t blocks, int32_t iters, uint32_t seed,
                                            int32_t form, void* stream) {
  using namespace aicf::hip;
  if (!out || blocks < 1 || iters < 1 || (form != 16 && form != 32))
    return static_cast<int32_t>(Status::InvalidArgument);
  if (form == 32)
    mfma_loop_kernel<32><<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(out, iters, seed);
  else
    mfma_loop_kernel<16><<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(out, iters, seed);
  return static_cast<int32_t>(launch_status("aicf_diag_mfma_loop"));
}

extern "C" int32_t aicf_diag_mfma_loop(float* out, int32_t blocks, int32_t iters, uint32_t seed, void* stream) {
  return aicf_diag_mfma_loop_form(out, blocks, iters, seed, 32, stream);
}
