// HIP helpers shared by the gfx950 kernels: launch-status mapping, 16-bit
// float conversions, vector types and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "host_util.hpp"

namespace aicf::hip {

// Maps the launch-error state to Status (reference pattern: cudaGetLastError
// after every launch, e.g. gemm/launcher.cu:28-33).
inline Status launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) return Status::Ok;
  set_last_error(what, hipGetErrorString(e));
  return Status::Internal;
}

inline Status hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return Status::Ok;
  set_last_error(what, hipGetErrorString(e));
  return Status::Internal;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// out[col] = sum over p < P of partial[p * N + col], fixed order (reduce.hip;
// the second pass of the column sums, shared with the GEMM epilogue that
// writes one partial row per 256-row tile).
Status colsum_finish(const float* partial, float* out, int64_t P, int64_t N, void* stream);

// Grid size for a 1-D launch: enough blocks to cover n items, at most cap.
inline unsigned grid_1d(int64_t n, int threads, int64_t cap) {
  int64_t b = (n + threads - 1) / threads;
  if (b < 1) b = 1;
  if (b > cap) b = cap;
  return static_cast<unsigned>(b);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

// ---- 16-bit float storage (raw bits) <-> fp32 -----------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// fp32 -> bf16, round-to-nearest-even, NaN -> quiet NaN (top payload bits
// kept, quiet bit set): gfx950's v_cvt_pk_bf16_f32, two values per
// instruction.  Its results equal the integer formulation
// (u + 0x7fff + ((u >> 16) & 1)) >> 16, with (u >> 16) | 0x40 for NaN, on
// every rounding tie, denormal, infinity and NaN pattern; that formulation
// written with a NaN branch compiled to divergent code in unrolled loops.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return static_cast<uint16_t>(f32x2_to_bf16x2(f, 0.0f));
}
// binary16 <-> fp32 with integer operations only.  The reference converts
// with __half2float (exact) and __float2half_rn (one RNE rounding of the
// fp32 value); doing the same here keeps hipcc from fusing a convert-fma-
// convert chain into v_fma_mix*, which rounds the exact result straight to
// f16 and can differ from the reference in the last bit.
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    // zero / subnormal: m * 2^-24 is exact in fp32
    const float v = (float)m * 5.9604644775390625e-8f;
    return __uint_as_float(__float_as_uint(v) | sign);
  }
  if (e == 31) return __uint_as_float(sign | 0x7f800000u | (m << 13));
  return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  uint32_t x = __float_as_uint(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  x &= 0x7fffffffu;
  if (x >= 0x7f800000u) return sign | (x > 0x7f800000u ? 0x7e00u : 0x7c00u);  // NaN / inf
  if (x >= 0x477ff000u) return sign | 0x7c00u;  // >= 65520 rounds to inf
  if (x >= 0x38800000u) {                       // normal binary16 range
    x += 0xc8000fffu + ((x >> 13) & 1u);        // rebias exponent, round half to even
    return sign | (uint16_t)(x >> 13);
  }
  // subnormal / zero: adding 0.5 aligns the 2^-24 quantum to the fp32 ulp,
  // so the fp32 addition performs the RNE rounding
  const float r = __uint_as_float(x) + 0.5f;
  return sign | (uint16_t)(__float_as_uint(r) - 0x3f000000u);
}

// ---- wave64 reductions (butterfly over all 64 lanes) ----------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// ---- GELU (tanh approximation) ---------------------------------------------
// gelu(x) = 0.5 x (1 + tanh(u)),  u = sqrt(2/pi) (x + 0.044715 x^3)
// Since 0.5 (1 + tanh(u)) = sigmoid(2u) = s:
//   gelu(x)  = x s,            s = 1 / (1 + 2^{x (a + b x^2)})
//   gelu'(x) = s + s (1 - s) x (2 k0 + 6 k0 k1 x^2)
// with a = -2 k0 log2(e), b = -2 k0 k1 log2(e).  One v_exp_f32 and one
// v_rcp_f32 (each ~1 ulp), no IEEE divide: relative error a few 1e-7.
// Limits: 2^(..) overflowing to +inf gives s = 0 (gelu -> -0, gelu' -> 0);
// underflowing to 0 gives s = 1 (gelu -> x, gelu' -> 1).
__device__ __forceinline__ float gelu_sigmoid_arg(float x) {
  const float a = -2.302208198144325f, b = -0.1029432395800235f;  // -2k0/ln2, -2k0k1/ln2
  return 1.0f + __builtin_amdgcn_exp2f(x * fmaf(b, x * x, a));
}
__device__ __forceinline__ float gelu_tanh_f(float x) {
  return x * __builtin_amdgcn_rcpf(gelu_sigmoid_arg(x));
}
__device__ __forceinline__ float gelu_tanh_grad_f(float x) {
  const float c2 = 1.5957691216057308f, c3 = 0.21406444881780076f;  // 2k0, 6k0k1
  const float s = __builtin_amdgcn_rcpf(gelu_sigmoid_arg(x));
  return fmaf(s * (1.0f - s), x * fmaf(c3, x * x, c2), s);
}

// ---- mean of a vector in a fixed order (one 256-lane workgroup) -----------
// Lane t accumulates v[t], v[t + 256], ... in fp64; the lanes of each wave
// combine by butterfly, the four waves as ((w0 + w1) + (w2 + w3)); the
// result is rounded to fp32 once.  `red` is 4 doubles of LDS.  The loss
// means of softmax cross-entropy use it wherever they are taken, so a fused
// and an unfused step produce the same bits.
__device__ __forceinline__ void block_mean_f64(const float* __restrict__ v, int64_t n,
                                               float* __restrict__ out, double* red) {
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += 256) acc += (double)v[i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) out[0] = (float)(((red[0] + red[1]) + (red[2] + red[3])) / (double)n);
}

}  // namespace aicf::hip
