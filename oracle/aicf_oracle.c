/*
 * aicf_oracle.c — CPU restatement of the reference's op arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the gfx950
 * backend and the CPU baseline timed by bench.py.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product path never does.
 *
 * Two kinds of function:
 *   *_ref_*  reference-exact fp32: the same operations in the same order as
 *            the reference kernel cited, including the FMA contractions nvcc
 *            applies by default (written as explicit fmaf), so a faithful
 *            GPU kernel matches bit for bit;
 *   *_f64    accuracy mode: fp64 arithmetic on the stored (already rounded)
 *            inputs, used with the normwise tolerances.
 * Reference paths are relative to ai-compiler-framework/ in the reference.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int orc_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void orc_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------------------------ */
/* 16-bit float formats                                                      */
/* ------------------------------------------------------------------------ */

/* IEEE binary16 from double, round to nearest even (one rounding). */
uint16_t orc_f16_from_f64(double x) {
  uint64_t u;
  memcpy(&u, &x, 8);
  const uint16_t sign = (uint16_t)((u >> 48) & 0x8000u);
  if (isnan(x)) return (uint16_t)(sign | 0x7e00u);
  const double a = fabs(x);
  if (isinf(x) || a >= 65520.0) return (uint16_t)(sign | 0x7c00u); /* overflow rounds to inf */
  if (a < ldexp(1.0, -14)) {
    /* subnormal range: quantum 2^-24 */
    const double q = a * 16777216.0; /* a / 2^-24 */
    double r = nearbyint(q);         /* default rounding mode: nearest even */
    return (uint16_t)(sign | (uint16_t)r);
  }
  int e;
  const double m = frexp(a, &e); /* a = m * 2^e, m in [0.5, 1) */
  /* 11 significant bits: scale mantissa to [1024, 2048) */
  double s = nearbyint(m * 2048.0);
  int ee = e - 1;
  if (s >= 2048.0) {
    s = 1024.0;
    ee += 1;
  }
  if (ee > 15) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | (uint16_t)((ee + 15) << 10) | (uint16_t)((int)s - 1024));
}

double orc_f16_to_f64(uint16_t h) {
  const int s = (h >> 15) & 1, e = (h >> 10) & 0x1f, f = h & 0x3ff;
  double v;
  if (e == 0)
    v = ldexp((double)f, -24);
  else if (e == 31)
    v = f ? NAN : INFINITY;
  else
    v = ldexp((double)(f + 1024), e - 25);
  return s ? -v : v;
}

/* bfloat16 from fp32, round to nearest even; NaN stays quiet NaN. */
uint16_t orc_bf16_from_f32(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void orc_f32_to_bf16_array(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_bf16_from_f32(x[i]);
}
void orc_bf16_to_f32_array(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_bf16_to_f32(x[i]);
}
void orc_f64_to_f16_array(const double* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_f16_from_f64(x[i]);
}

/* ------------------------------------------------------------------------ */
/* Optimizer ops                                                             */
/* ------------------------------------------------------------------------ */

/* adam_step/launcher.cu:276-291 (adam_step_f32_kernel_v2), one element per
 * i; bc1/bc2 are divisors (the probe passes 1 - beta^t).  Out-of-place
 * reads P and writes Pout (the launcher copies P to Pout first,
 * :220-224, which is the same). */
void orc_adam_ref_f32(const float* P, const float* G, const float* M, const float* V, float* Pout,
                      float* Mout, float* Vout, int64_t n, float lr, float beta1, float beta2,
                      float eps, float bc1, float bc2) {
  const float omb1 = 1.0f - beta1, omb2 = 1.0f - beta2;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const float g = G[i];
    const float m_new = fmaf(beta1, M[i], omb1 * g);
    const float v_new = fmaf(beta2, V[i], omb2 * (g * g));
    const float m_hat = m_new / bc1;
    const float v_hat = v_new / bc2;
    const float denom = sqrtf(v_hat) + eps;
    const float p = fmaf(-lr, m_hat / denom, P[i]);
    Mout[i] = m_new;
    Vout[i] = v_new;
    Pout[i] = p;
  }
}

/* Adam in fp64 on the same inputs (accuracy mode for the reference op). */
void orc_adam_f64(const float* P, const float* G, const float* M, const float* V, double* Pout,
                  double* Mout, double* Vout, int64_t n, double lr, double beta1, double beta2,
                  double eps, double bc1, double bc2) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const double g = G[i];
    const double m = beta1 * M[i] + (1.0 - beta1) * g;
    const double v = beta2 * V[i] + (1.0 - beta2) * g * g;
    Pout[i] = P[i] - lr * (m / bc1) / (sqrt(v / bc2) + eps);
    Mout[i] = m;
    Vout[i] = v;
  }
}

/* AdamW with in-kernel bias correction (appended op adamw_step_f32_v1):
 *   t = max(step,1); bc_k = (float)(1 - b_k^t) computed in double;
 *   step_size = lr / bc1; ibc2 = 1 / bc2;
 *   p *= (1 - lr*wd); m' = fma(b1, m, (1-b1) g); v' = fma(b2, v, (1-b2) g^2);
 *   p = fma(-step_size, m' / (sqrt(v' * ibc2) + eps), p);
 * Optional bf16 shadow of p (Wb may be NULL). */
void orc_adamw_f32(const float* P, const float* G, const float* M, const float* V, float* Pout,
                   float* Mout, float* Vout, uint16_t* Wb, int64_t n, float lr, float beta1,
                   float beta2, float eps, float wd, int32_t step) {
  int t = step < 1 ? 1 : step;
  const float bc1 = (float)(1.0 - pow((double)beta1, (double)t));
  const float bc2 = (float)(1.0 - pow((double)beta2, (double)t));
  const float ss = lr / bc1, ibc2 = 1.0f / bc2;
  const float omb1 = 1.0f - beta1, omb2 = 1.0f - beta2, decay = 1.0f - lr * wd;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const float g = G[i];
    float p = P[i] * decay;
    const float m_new = fmaf(beta1, M[i], omb1 * g);
    const float v_new = fmaf(beta2, V[i], omb2 * (g * g));
    const float denom = sqrtf(v_new * ibc2) + eps;
    p = fmaf(-ss, m_new / denom, p);
    Pout[i] = p;
    Mout[i] = m_new;
    Vout[i] = v_new;
    if (Wb) Wb[i] = orc_bf16_from_f32(p);
  }
}

/* biascorr/launcher.cu:86-99: t = max(step,1), d = 1 - beta^t (clamped to
 * 1e-20 when |d| < 1e-20), outputs 1/d. */
void orc_bias_corr(int32_t step, float beta1, float beta2, float* o1, float* o2) {
  int t = step < 1 ? 1 : step;
  float d1 = 1.0f - powf(beta1, (float)t);
  float d2 = 1.0f - powf(beta2, (float)t);
  if (fabsf(d1) < 1e-20f) d1 = 1e-20f;
  if (fabsf(d2) < 1e-20f) d2 = 1e-20f;
  *o1 = 1.0f / d1;
  *o2 = 1.0f / d2;
}

/* sgd_step/launcher.cu:118-120: O = P - lr*G (contracted to one fma). */
void orc_sgd_f32(const float* P, const float* G, float* O, int64_t n, float lr) {
  for (int64_t i = 0; i < n; ++i) O[i] = fmaf(-lr, G[i], P[i]);
}
/* sgd_step/launcher.cu:122-149: fp32 math on f16 inputs, RNE store. */
void orc_sgd_f16(const uint16_t* P, const uint16_t* G, uint16_t* O, int64_t n, float lr) {
  for (int64_t i = 0; i < n; ++i) {
    const float p = (float)orc_f16_to_f64(P[i]), g = (float)orc_f16_to_f64(G[i]);
    O[i] = orc_f16_from_f64((double)fmaf(-lr, g, p));
  }
}

/* ------------------------------------------------------------------------ */
/* Elementwise ops                                                           */
/* ------------------------------------------------------------------------ */

/* add/launcher.cu:52-58: __hadd rounds the exact sum once; the exact sum
 * of two f16 values fits in a double. */
void orc_add_f16(const uint16_t* a, const uint16_t* b, uint16_t* o, int64_t n) {
  for (int64_t i = 0; i < n; ++i) o[i] = orc_f16_from_f64(orc_f16_to_f64(a[i]) + orc_f16_to_f64(b[i]));
}
void orc_add_f32(const float* a, const float* b, float* o, int64_t n) {
  for (int64_t i = 0; i < n; ++i) o[i] = a[i] + b[i];
}

/* relu/launcher.cu:49-50 and :58-60: x > 0 ? x : +0 (NaN and -0 give +0). */
void orc_relu_f32(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = x[i] > 0.0f ? x[i] : 0.0f;
}
void orc_relu_f16(const uint16_t* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_f16_to_f64(x[i]) > 0.0 ? x[i] : (uint16_t)0;
}
/* relu_bwd/launcher.cu:37-77: dY = (Y > 0) ? dOut : 0. */
void orc_relu_bwd_f32(const float* dout, const float* y, float* dy, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dy[i] = y[i] > 0.0f ? dout[i] : 0.0f;
}
void orc_relu_bwd_f16(const uint16_t* dout, const uint16_t* y, uint16_t* dy, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dy[i] = orc_f16_to_f64(y[i]) > 0.0 ? dout[i] : (uint16_t)0;
}

/* bias_add/launcher.cu:36-62: Out[r, c] = Y[r, c] + b[c]. */
void orc_bias_add_f32(const float* y, const float* b, float* o, int64_t M, int64_t N) {
  for (int64_t r = 0; r < M; ++r)
    for (int64_t c = 0; c < N; ++c) o[r * N + c] = y[r * N + c] + b[c];
}
void orc_bias_add_f16(const uint16_t* y, const uint16_t* b, uint16_t* o, int64_t M, int64_t N) {
  for (int64_t r = 0; r < M; ++r)
    for (int64_t c = 0; c < N; ++c)
      o[r * N + c] = orc_f16_from_f64(orc_f16_to_f64(y[r * N + c]) + orc_f16_to_f64(b[c]));
}

/* mse_grad/launcher.cu:61-71: d = (p - t) * scale. */
void orc_mse_grad_f32(const float* p, const float* t, float* d, int64_t n, float scale) {
  for (int64_t i = 0; i < n; ++i) d[i] = (p[i] - t[i]) * scale;
}
/* mse_grad/launcher.cu:73-85: fp32 math, RNE store (scalar f16 path). */
void orc_mse_grad_f16_scalar(const uint16_t* p, const uint16_t* t, uint16_t* d, int64_t n,
                             float scale) {
  for (int64_t i = 0; i < n; ++i) {
    const float e = (float)orc_f16_to_f64(p[i]) - (float)orc_f16_to_f64(t[i]);
    d[i] = orc_f16_from_f64((double)(e * scale));
  }
}
/* mse_grad/launcher.cu:87-98: half math, each op rounded to f16, scale
 * rounded to f16 first (__float2half2_rn). */
void orc_mse_grad_f16_half(const uint16_t* p, const uint16_t* t, uint16_t* d, int64_t n,
                           float scale) {
  const double s = orc_f16_to_f64(orc_f16_from_f64((double)scale));
  for (int64_t i = 0; i < n; ++i) {
    const double e = orc_f16_to_f64(orc_f16_from_f64(orc_f16_to_f64(p[i]) - orc_f16_to_f64(t[i])));
    d[i] = orc_f16_from_f64(e * s);
  }
}

/* Fused MSE loss + grad (appended op): loss = mean((p - t)^2) in fp64. */
double orc_mse_loss_f64(const float* p, const float* t, int64_t n) {
  double acc = 0.0;
#pragma omp parallel for reduction(+ : acc) schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const double e = (double)p[i] - (double)t[i];
    acc += e * e;
  }
  return acc / (double)n;
}

/* GELU, tanh approximation, and its derivative (closed forms, fp64). */
void orc_gelu_f64(const double* x, double* y, int64_t n) {
  const double k0 = 0.7978845608028654, k1 = 0.044715;
  for (int64_t i = 0; i < n; ++i) {
    const double v = x[i];
    y[i] = 0.5 * v * (1.0 + tanh(k0 * (v + k1 * v * v * v)));
  }
}
void orc_gelu_grad_f64(const double* x, double* y, int64_t n) {
  const double k0 = 0.7978845608028654, k1 = 0.044715;
  for (int64_t i = 0; i < n; ++i) {
    const double v = x[i];
    const double t = tanh(k0 * (v + k1 * v * v * v));
    y[i] = 0.5 * (1.0 + t) + 0.5 * v * (1.0 - t * t) * k0 * (1.0 + 3.0 * k1 * v * v);
  }
}

/* ------------------------------------------------------------------------ */
/* Reductions                                                                */
/* ------------------------------------------------------------------------ */

/* reduce_sum/launcher.cu:140-155: out[c] = sum_r x[r, c] (fp64 accumulate). */
void orc_colsum_f64(const float* x, double* out, int64_t M, int64_t N) {
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < N; ++c) {
    double s = 0.0;
    for (int64_t r = 0; r < M; ++r) s += x[r * N + c];
    out[c] = s;
  }
}

/* Row softmax / row max / row sum (appended ops), fp64 on fp32 inputs.
 * Any output pointer may be NULL. */
void orc_softmax_rows_f64(const float* x, double* y, double* rmax, double* rsum, int64_t R,
                          int64_t C) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < R; ++r) {
    const float* xr = x + r * C;
    double mx = xr[0], sx = 0.0, se = 0.0;
    for (int64_t c = 0; c < C; ++c) {
      if (xr[c] > mx) mx = xr[c];
      sx += xr[c];
    }
    for (int64_t c = 0; c < C; ++c) se += exp((double)xr[c] - mx);
    if (y)
      for (int64_t c = 0; c < C; ++c) y[r * C + c] = exp((double)xr[c] - mx) / se;
    if (rmax) rmax[r] = mx;
    if (rsum) rsum[r] = sx;
  }
}

/* Softmax cross-entropy, mean over rows (appended op):
 *   loss_i = log(sum_j exp(z_ij - m_i)) + m_i - z_i[y_i]
 *   dz = (softmax(z) - onehot(y)) / B,  argmax = first index of the max. */
double orc_softmax_xent_f64(const float* z, const int32_t* labels, double* dz, int32_t* argmax,
                            double* row_loss, int64_t B, int64_t C) {
  double total = 0.0;
  for (int64_t r = 0; r < B; ++r) {
    const float* zr = z + r * C;
    double mx = zr[0];
    int32_t am = 0;
    for (int64_t c = 1; c < C; ++c)
      if (zr[c] > mx) {
        mx = zr[c];
        am = (int32_t)c;
      }
    double se = 0.0;
    for (int64_t c = 0; c < C; ++c) se += exp((double)zr[c] - mx);
    const int32_t lab = labels[r];
    const double l = log(se) + mx - (double)zr[lab];
    if (row_loss) row_loss[r] = l;
    if (argmax) argmax[r] = am;
    total += l;
    if (dz)
      for (int64_t c = 0; c < C; ++c)
        dz[r * C + c] = (exp((double)zr[c] - mx) / se - (c == lab ? 1.0 : 0.0)) / (double)B;
  }
  return total / (double)B;
}

/* ------------------------------------------------------------------------ */
/* GEMM                                                                      */
/* ------------------------------------------------------------------------ */

/* C[m, n] = sum_k A(m, k) B(k, n) in fp64; A(m,k) = A[m*ars + k*acs],
 * B(k,n) = B[k*brs + n*bcs]; inputs are fp32 values (bf16/f16 inputs are
 * passed already widened). */
void orc_gemm_f64(const float* A, int64_t ars, int64_t acs, const float* B, int64_t brs,
                  int64_t bcs, double* C, int64_t M, int64_t N, int64_t K) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) C[m * N + n] = 0.0;
    for (int64_t k = 0; k < K; ++k) {
      const double a = A[m * ars + k * acs];
      if (a == 0.0) continue;
      for (int64_t n = 0; n < N; ++n) C[m * N + n] += a * (double)B[k * brs + n * bcs];
    }
  }
}

/* gemm/launcher.cu:155-172 (gemm_f32_naive_strided_kernel): one output at a
 * time, sequential-k fp32 accumulation acc = fma(a, b, acc) (nvcc contracts
 * `acc += a * b`).  This is the reference's own algorithm and serves as the
 * CPU baseline; rows [m_begin, m_end) only. */
void orc_gemm_ref_f32(const float* A, int64_t ars, int64_t acs, const float* B, int64_t brs,
                      int64_t bcs, float* C, int64_t ldc, int64_t m_begin, int64_t m_end,
                      int64_t N, int64_t K) {
#pragma omp parallel for schedule(static)
  for (int64_t m = m_begin; m < m_end; ++m)
    for (int64_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) acc = fmaf(A[m * ars + k * acs], B[k * brs + n * bcs], acc);
      C[m * ldc + n] = acc;
    }
}
