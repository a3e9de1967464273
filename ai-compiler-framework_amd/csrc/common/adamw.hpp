// AdamW element update shared by the streaming optimizer kernel (optim.hip)
// and the GEMM epilogue that applies it to a weight-gradient tile (gemm.hip),
// so that both produce the same bits.  No reference counterpart (the
// reference's Adam divides by host-computed bias corrections).  Per element:
//   p  <- p * (1 - lr*wd)                        (decoupled weight decay)
//   m' <- fma(b1, m, (1-b1) g);  v' <- fma(b2, v, (1-b2) g^2)
//   p  <- p - step * m' / (sqrt(v' * ibc2) + eps)
// with bc_k = 1 - b_k^t computed in double from the device step counter,
// step = lr / bc1 and ibc2 = 1 / bc2 (both rounded to fp32 once).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace aicf::hip {

struct AdamWArgs {
  float lr, beta1, beta2, eps, wd, omb1, omb2, decay;  // decay = 1 - lr*wd
};

struct AdamWScalars {
  float step, ibc2;
};

__device__ __forceinline__ AdamWScalars adamw_scalars_at(int t, const AdamWArgs& a) {
  if (t < 1) t = 1;
  const float bc1 = (float)(1.0 - pow((double)a.beta1, (double)t));
  const float bc2 = (float)(1.0 - pow((double)a.beta2, (double)t));
  AdamWScalars s;
  s.step = a.lr / bc1;
  s.ibc2 = 1.0f / bc2;
  return s;
}

__device__ __forceinline__ AdamWScalars adamw_scalars(const int32_t* stepp, const AdamWArgs& a) {
  return adamw_scalars_at(stepp[0], a);
}

__device__ __forceinline__ void adamw_elem(float& p, float g, float& m, float& v,
                                           const AdamWScalars& s, const AdamWArgs& a) {
  p = p * a.decay;
  const float m_new = fmaf(a.beta1, m, a.omb1 * g);
  const float v_new = fmaf(a.beta2, v, a.omb2 * (g * g));
  const float denom = sqrtf(v_new * s.ibc2) + a.eps;
  p = fmaf(-s.step, m_new / denom, p);
  m = m_new;
  v = v_new;
}

}  // namespace aicf::hip
