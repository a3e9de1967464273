// Normalisation kernels for gfx950: LayerNorm forward/backward (f32, f16)
// and BatchNorm forward/backward (f16 NCHW).
//
// Reference contracts:
//   LayerNorm  src/backends/cuda/ops/layernorm/launcher.cu:1-10 (I/O),
//              :41-58 (LNEP eps, default 1e-5), :399-429 (fwd checks),
//              :538-573 (bwd checks); 2-D contiguous row-major x[M,N],
//              normalised over N; mean/rstd f32 [M]; dgamma/dbeta f32 [N].
//   BatchNorm  src/backends/cuda/ops/batchnorm/launcher.cu:1-20 (I/O),
//              :51-84 (BNEP eps + flags), :295-345 (fwd checks),
//              :364-366 (training requires batch statistics), :483-526 (bwd
//              checks, affine only); f16 NCHW contiguous, statistics f32 [C].
//
// Design: LayerNorm runs a wave per row (4 rows per 256-thread workgroup),
// with the row held in registers up to 2048 columns (one HBM read), else
// re-read.  BatchNorm runs a workgroup per channel.  Every reduction is a
// fixed-order wave64 butterfly plus an LDS combine: no atomics and no memsets,
// so results are reproducible and the ops are safe under graph capture.
// Variances are centred (sum of squared deviations from the mean), which is
// the accurate form of the reference's E[x^2] - mean^2.
#include "../common/hip_util.hpp"

namespace aicf::hip {

namespace {

size_t no_workspace(const TensorDesc*, int, const void*) { return 0; }

KernelVariant make(const char* name, LaunchFn l, SupportedFn s, uint32_t schema = 0) {
  KernelVariant v;
  v.name = name;
  v.launch = l;
  v.supported = s;
  v.query_workspace = no_workspace;
  v.expected_attr_schema_id = schema;
  return v;
}

template <typename T>
__device__ __forceinline__ float ld_as_f32(const T* p, int64_t i) {
  if constexpr (sizeof(T) == 4) {
    return p[i];
  } else {
    return f16_to_f32(p[i]);
  }
}
template <typename T>
__device__ __forceinline__ void st_from_f32(T* p, int64_t i, float v) {
  if constexpr (sizeof(T) == 4) {
    p[i] = v;
  } else {
    p[i] = f32_to_f16(v);
  }
}

// Sum over the 256 threads of a workgroup (4 waves), every thread gets it.
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();  // red is reused across calls
  if (lane == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// ===========================================================================
// LayerNorm
// ===========================================================================
// Forward.  VPT > 0: the lane keeps columns lane + 64 i (i < VPT) in
// registers; VPT == 0: any N, the row is read three times.
template <typename T, int VPT>
__global__ __launch_bounds__(256) void ln_fwd_kernel(const T* __restrict__ x, const T* __restrict__ gamma,
                                                     const T* __restrict__ beta, T* __restrict__ y,
                                                     float* __restrict__ mean, float* __restrict__ rstd,
                                                     int M, int N, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;  // whole wave
  const T* xr = x + (int64_t)row * N;
  T* yr = y + (int64_t)row * N;
  const float invN = 1.0f / (float)N;
  float mu, rs;
  if constexpr (VPT > 0) {
    float v[VPT];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = lane + 64 * i;
      v[i] = c < N ? ld_as_f32(xr, c) : 0.0f;
      s += v[i];
    }
    mu = wave_sum(s) * invN;
    float d = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = lane + 64 * i;
      const float t = c < N ? v[i] - mu : 0.0f;
      d = fmaf(t, t, d);
    }
    rs = 1.0f / sqrtf(wave_sum(d) * invN + eps);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = lane + 64 * i;
      if (c < N) {
        float o = (v[i] - mu) * rs;
        if (gamma) o = fmaf(o, ld_as_f32(gamma, c), ld_as_f32(beta, c));
        st_from_f32(yr, c, o);
      }
    }
  } else {
    float s = 0.0f;
    for (int c = lane; c < N; c += 64) s += ld_as_f32(xr, c);
    mu = wave_sum(s) * invN;
    float d = 0.0f;
    for (int c = lane; c < N; c += 64) {
      const float t = ld_as_f32(xr, c) - mu;
      d = fmaf(t, t, d);
    }
    rs = 1.0f / sqrtf(wave_sum(d) * invN + eps);
    for (int c = lane; c < N; c += 64) {
      float o = (ld_as_f32(xr, c) - mu) * rs;
      if (gamma) o = fmaf(o, ld_as_f32(gamma, c), ld_as_f32(beta, c));
      st_from_f32(yr, c, o);
    }
  }
  if (lane == 0) {
    mean[row] = mu;
    rstd[row] = rs;
  }
}

// Backward dx: dyh = dy * gamma (gamma null => 1), xhat = (x - mean) rstd,
// dx = (N dyh - sum(dyh) - xhat sum(dyh xhat)) * rstd / N.
template <typename T, int VPT>
__global__ __launch_bounds__(256) void ln_bwd_dx_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                        const T* __restrict__ gamma,
                                                        const float* __restrict__ mean,
                                                        const float* __restrict__ rstd, T* __restrict__ dx,
                                                        int M, int N) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const T* xr = x + (int64_t)row * N;
  const T* dyr = dy + (int64_t)row * N;
  T* dxr = dx + (int64_t)row * N;
  const float mu = mean[row], rs = rstd[row];
  const float fN = (float)N, scale = rs / fN;
  if constexpr (VPT > 0) {
    float xh[VPT], g[VPT];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = lane + 64 * i;
      xh[i] = 0.0f;
      g[i] = 0.0f;
      if (c < N) {
        xh[i] = (ld_as_f32(xr, c) - mu) * rs;
        g[i] = ld_as_f32(dyr, c);
        if (gamma) g[i] *= ld_as_f32(gamma, c);
      }
      s1 += g[i];
      s2 = fmaf(g[i], xh[i], s2);
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = lane + 64 * i;
      if (c < N) st_from_f32(dxr, c, (fN * g[i] - s1 - xh[i] * s2) * scale);
    }
  } else {
    float s1 = 0.0f, s2 = 0.0f;
    for (int c = lane; c < N; c += 64) {
      const float xh = (ld_as_f32(xr, c) - mu) * rs;
      float g = ld_as_f32(dyr, c);
      if (gamma) g *= ld_as_f32(gamma, c);
      s1 += g;
      s2 = fmaf(g, xh, s2);
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    for (int c = lane; c < N; c += 64) {
      const float xh = (ld_as_f32(xr, c) - mu) * rs;
      float g = ld_as_f32(dyr, c);
      if (gamma) g *= ld_as_f32(gamma, c);
      st_from_f32(dxr, c, (fN * g - s1 - xh * s2) * scale);
    }
  }
}

// Backward dgamma[c] = sum_m dy xhat, dbeta[c] = sum_m dy: lane per column,
// the 4 waves take every fourth row, combined in LDS in a fixed order.
template <typename T>
__global__ __launch_bounds__(256) void ln_bwd_dgdb_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                          const float* __restrict__ mean,
                                                          const float* __restrict__ rstd,
                                                          float* __restrict__ dgamma, float* __restrict__ dbeta,
                                                          int M, int N) {
  __shared__ float red[2][4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  float sg = 0.0f, sb = 0.0f;
  if (c < N) {
    for (int r = w; r < M; r += 4) {
      const float xh = (ld_as_f32(x, (int64_t)r * N + c) - mean[r]) * rstd[r];
      const float d = ld_as_f32(dy, (int64_t)r * N + c);
      sb += d;
      sg = fmaf(d, xh, sg);
    }
  }
  red[0][w][lane] = sg;
  red[1][w][lane] = sb;
  __syncthreads();
  if (w == 0 && c < N) {
    dgamma[c] = (red[0][0][lane] + red[0][1][lane]) + (red[0][2][lane] + red[0][3][lane]);
    dbeta[c] = (red[1][0][lane] + red[1][1][lane]) + (red[1][2][lane] + red[1][3][lane]);
  }
}

// LNEP <f> eps; schema 0 (or anything else, or a short payload) => 1e-5
// (layernorm/launcher.cu:49-58).
float read_ln_eps(const void* attr) {
  const AttrBlob& a = blob(attr);
  if (!attr || a.schema_id != AICF_SCHEMA_LNEP || !payload_ok(a, 4)) return 1e-5f;
  return field<float>(a, 0);
}

bool vec1_len(const TensorDesc& t, DType d, int64_t n) {
  return dt(t) == d && t.rank == 1 && t.contiguous && t.shape[0] == n;
}

// layernorm/launcher.cu:399-429: inputs (X) or (X, G, B); outputs (Y, Mean, Rstd)
bool ln_fwd_check(const TensorDesc* in, int ni, const TensorDesc* out, int no, DType d) {
  if (!in || !out || !(ni == 1 || ni == 3) || no != 3) return false;
  const TensorDesc &X = in[0], &Y = out[0];
  if (dt(X) != d || dt(Y) != d || !is_contig_2d_rowmajor(X) || !is_contig_2d_rowmajor(Y)) return false;
  if (!same_shape(X, Y)) return false;
  const int64_t M = X.shape[0], N = X.shape[1];
  if (M > INT32_MAX || N > INT32_MAX || N < 1) return false;
  if (!vec1_len(out[1], DType::kF32, M) || !vec1_len(out[2], DType::kF32, M)) return false;
  if (ni == 3 && (!vec1_len(in[1], d, N) || !vec1_len(in[2], d, N))) return false;
  return true;
}

// layernorm/launcher.cu:538-573: (X, dY, Mean, Rstd) -> (dX) or
// (X, dY, G, Mean, Rstd) -> (dX, dG, dB)
bool ln_bwd_check(const TensorDesc* in, int ni, const TensorDesc* out, int no, DType d) {
  if (!in || !out) return false;
  const bool affine = ni == 5 && no == 3, noaff = ni == 4 && no == 1;
  if (!affine && !noaff) return false;
  const TensorDesc &X = in[0], &dY = in[1], &dX = out[0];
  for (const TensorDesc* t : {&X, &dY, &dX})
    if (dt(*t) != d || !is_contig_2d_rowmajor(*t)) return false;
  if (!same_shape(X, dY) || !same_shape(X, dX)) return false;
  const int64_t M = X.shape[0], N = X.shape[1];
  if (M > INT32_MAX || N > INT32_MAX || N < 1) return false;
  if (!vec1_len(in[affine ? 3 : 2], DType::kF32, M) || !vec1_len(in[affine ? 4 : 3], DType::kF32, M)) return false;
  if (affine && (!vec1_len(in[2], d, N) || !vec1_len(out[1], DType::kF32, N) || !vec1_len(out[2], DType::kF32, N)))
    return false;
  return true;
}

template <typename T>
Status ln_fwd_run(const T* x, const T* g, const T* b, T* y, float* mean, float* rstd, int M, int N, float eps,
                  hipStream_t s) {
  const unsigned blocks = (unsigned)((M + 3) / 4);
#define LN_FWD(V) ln_fwd_kernel<T, V><<<blocks, 256, 0, s>>>(x, g, b, y, mean, rstd, M, N, eps)
  if (N <= 64) LN_FWD(1);
  else if (N <= 256) LN_FWD(4);
  else if (N <= 1024) LN_FWD(16);
  else if (N <= 2048) LN_FWD(32);
  else LN_FWD(0);
#undef LN_FWD
  return launch_status("layernorm_fwd");
}

template <typename T>
Status ln_bwd_run(const T* x, const T* dy, const T* g, const float* mean, const float* rstd, T* dx,
                  float* dgamma, float* dbeta, int M, int N, hipStream_t s) {
  const unsigned blocks = (unsigned)((M + 3) / 4);
#define LN_BWD(V) ln_bwd_dx_kernel<T, V><<<blocks, 256, 0, s>>>(x, dy, g, mean, rstd, dx, M, N)
  if (N <= 64) LN_BWD(1);
  else if (N <= 256) LN_BWD(4);
  else if (N <= 1024) LN_BWD(16);
  else if (N <= 2048) LN_BWD(32);
  else LN_BWD(0);
#undef LN_BWD
  if (dgamma) {
    const Status st = launch_status("layernorm_bwd_dx");
    if (st != Status::Ok) return st;
    ln_bwd_dgdb_kernel<T><<<(unsigned)((N + 63) / 64), 256, 0, s>>>(x, dy, mean, rstd, dgamma, dbeta, M, N);
  }
  return launch_status("layernorm_bwd");
}

#define LN_VARIANTS(SFX, T, D)                                                                          \
  bool ln_fwd_##SFX##_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {    \
    return ln_fwd_check(i, ni, o, no, D);                                                              \
  }                                                                                                    \
  Status ln_fwd_##SFX##_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a,      \
                               void*, size_t, void* s) {                                               \
    if (!ln_fwd_check(i, ni, o, no, D)) return Status::InvalidArgument;                               \
    const T* g = ni == 3 ? (const T*)i[1].data : nullptr;                                              \
    const T* b = ni == 3 ? (const T*)i[2].data : nullptr;                                              \
    return ln_fwd_run<T>((const T*)i[0].data, g, b, (T*)o[0].data, (float*)o[1].data,                 \
                         (float*)o[2].data, (int)i[0].shape[0], (int)i[0].shape[1], read_ln_eps(a),   \
                         as_stream(s));                                                               \
  }                                                                                                    \
  bool ln_bwd_##SFX##_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {    \
    return ln_bwd_check(i, ni, o, no, D);                                                              \
  }                                                                                                    \
  Status ln_bwd_##SFX##_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void*,        \
                               void*, size_t, void* s) {                                               \
    if (!ln_bwd_check(i, ni, o, no, D)) return Status::InvalidArgument;                               \
    const bool aff = ni == 5;                                                                          \
    return ln_bwd_run<T>((const T*)i[0].data, (const T*)i[1].data, aff ? (const T*)i[2].data : nullptr,\
                         (const float*)i[aff ? 3 : 2].data, (const float*)i[aff ? 4 : 3].data,        \
                         (T*)o[0].data, aff ? (float*)o[1].data : nullptr,                            \
                         aff ? (float*)o[2].data : nullptr, (int)i[0].shape[0], (int)i[0].shape[1],   \
                         as_stream(s));                                                               \
  }

LN_VARIANTS(f32, float, DType::kF32)
LN_VARIANTS(f16, uint16_t, DType::kF16)

// ===========================================================================
// BatchNorm (f16, NCHW)
// ===========================================================================
// Element (n, c, hw) of channel c sits at n*C*HW + c*HW + hw; a workgroup
// owns one channel and walks its N slabs of HW contiguous elements.
struct BNShape {
  int N, C, HW;
};

__device__ __forceinline__ int64_t bn_index(const BNShape& s, int c, int64_t k) {
  const int64_t n = k / s.HW, hw = k - n * s.HW;
  return (n * s.C + c) * (int64_t)s.HW + hw;
}

// Training forward: batch mean, centred variance, rstd = 1/sqrt(var + eps),
// then y = (x - mean) rstd gamma + beta (gamma/beta null => 1/0).
__global__ __launch_bounds__(256) void bn_fwd_train_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ gamma,
                                                           const uint16_t* __restrict__ beta,
                                                           uint16_t* __restrict__ y,
                                                           float* __restrict__ save_mean,
                                                           float* __restrict__ save_rstd, BNShape sh, float eps) {
  __shared__ float red[4];
  const int c = blockIdx.x;
  const int64_t cnt = (int64_t)sh.N * sh.HW;
  float s = 0.0f;
  for (int64_t k = threadIdx.x; k < cnt; k += 256) s += f16_to_f32(x[bn_index(sh, c, k)]);
  const float mu = block_sum256(s, red) / (float)cnt;
  float d = 0.0f;
  for (int64_t k = threadIdx.x; k < cnt; k += 256) {
    const float t = f16_to_f32(x[bn_index(sh, c, k)]) - mu;
    d = fmaf(t, t, d);
  }
  const float rs = 1.0f / sqrtf(block_sum256(d, red) / (float)cnt + eps);
  const float g = gamma ? f16_to_f32(gamma[c]) : 1.0f, b = beta ? f16_to_f32(beta[c]) : 0.0f;
  for (int64_t k = threadIdx.x; k < cnt; k += 256) {
    const int64_t i = bn_index(sh, c, k);
    y[i] = f32_to_f16(fmaf((f16_to_f32(x[i]) - mu) * rs, g, b));
  }
  if (threadIdx.x == 0) {
    save_mean[c] = mu;
    save_rstd[c] = rs;
  }
}

// Inference forward with running statistics: elementwise.
__global__ __launch_bounds__(256) void bn_fwd_infer_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ gamma,
                                                           const uint16_t* __restrict__ beta,
                                                           const float* __restrict__ rmean,
                                                           const float* __restrict__ rvar, uint16_t* __restrict__ y,
                                                           BNShape sh, float eps, int64_t total) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int c = (int)((i / sh.HW) % sh.C);
    const float rs = 1.0f / sqrtf(rvar[c] + eps);
    const float g = gamma ? f16_to_f32(gamma[c]) : 1.0f, b = beta ? f16_to_f32(beta[c]) : 0.0f;
    y[i] = f32_to_f16(fmaf((f16_to_f32(x[i]) - rmean[c]) * rs, g, b));
  }
}

// Backward (affine): dbeta = sum(dy), dgamma = sum(dy xhat),
// dx = (NHW dy - dbeta - xhat dgamma) gamma rstd / NHW.
__global__ __launch_bounds__(256) void bn_bwd_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ dy,
                                                     const uint16_t* __restrict__ gamma,
                                                     const float* __restrict__ mean,
                                                     const float* __restrict__ rstd, uint16_t* __restrict__ dx,
                                                     float* __restrict__ dgamma, float* __restrict__ dbeta,
                                                     BNShape sh) {
  __shared__ float red[4];
  const int c = blockIdx.x;
  const int64_t cnt = (int64_t)sh.N * sh.HW;
  const float mu = mean[c], rs = rstd[c];
  float s1 = 0.0f, s2 = 0.0f;
  for (int64_t k = threadIdx.x; k < cnt; k += 256) {
    const int64_t i = bn_index(sh, c, k);
    const float d = f16_to_f32(dy[i]);
    s1 += d;
    s2 = fmaf(d, (f16_to_f32(x[i]) - mu) * rs, s2);
  }
  s1 = block_sum256(s1, red);
  s2 = block_sum256(s2, red);
  const float fcnt = (float)cnt, scale = f16_to_f32(gamma[c]) * rs / fcnt;
  for (int64_t k = threadIdx.x; k < cnt; k += 256) {
    const int64_t i = bn_index(sh, c, k);
    const float xh = (f16_to_f32(x[i]) - mu) * rs;
    dx[i] = f32_to_f16((fcnt * f16_to_f32(dy[i]) - s1 - xh * s2) * scale);
  }
  if (threadIdx.x == 0) {
    dgamma[c] = s2;
    dbeta[c] = s1;
  }
}

struct BNAttr {
  float eps = 1e-5f;
  bool use_running_stats = true;
};
// batchnorm/launcher.cu:69-84: BNEP <fI> with >= 8 bytes, else defaults.
BNAttr read_bn_attr(const void* attr) {
  BNAttr r;
  const AttrBlob& a = blob(attr);
  if (!attr || a.schema_id != AICF_SCHEMA_BNEP || !payload_ok(a, 8)) return r;
  r.eps = field<float>(a, 0);
  r.use_running_stats = (field<uint32_t>(a, 4) & 1u) != 0;
  return r;
}

bool nchw_f16(const TensorDesc& t) {
  if (dt(t) != DType::kF16 || t.rank != 4) return false;
  for (int i = 0; i < 4; ++i)
    if (t.stride[i] <= 0 || t.shape[i] <= 0) return false;
  return t.stride[3] == 1 && t.stride[2] == t.shape[3] && t.stride[1] == t.shape[2] * t.shape[3] &&
         t.stride[0] == t.shape[1] * t.shape[2] * t.shape[3];
}
bool vec_c(const TensorDesc& t, DType d, int64_t C) { return dt(t) == d && t.rank == 1 && t.shape[0] == C; }

// batchnorm/launcher.cu:295-345: inference (X,G,B,RM,RV)->(Y) or (X,RM,RV)->(Y);
// training (X,G,B)->(Y,SM,SR) or (X)->(Y,SM,SR).
bool bn_fwd_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void*) {
  if (!in || !out) return false;
  const bool inf_aff = ni == 5 && no == 1, inf_no = ni == 3 && no == 1;
  const bool tr_aff = ni == 3 && no == 3, tr_no = ni == 1 && no == 3;
  if (!(inf_aff || inf_no || tr_aff || tr_no)) return false;
  const TensorDesc &X = in[0], &Y = out[0];
  if (!nchw_f16(X) || !nchw_f16(Y) || !same_shape(X, Y)) return false;
  const int64_t C = X.shape[1];
  if (X.shape[0] * X.shape[2] * X.shape[3] > INT32_MAX) return false;
  if ((inf_aff || tr_aff) && (!vec_c(in[1], DType::kF16, C) || !vec_c(in[2], DType::kF16, C))) return false;
  if (inf_aff || inf_no) return vec_c(in[inf_aff ? 3 : 1], DType::kF32, C) && vec_c(in[inf_aff ? 4 : 2], DType::kF32, C);
  return vec_c(out[1], DType::kF32, C) && vec_c(out[2], DType::kF32, C);
}

Status bn_fwd_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* attr, void*, size_t,
                     void* stream) {
  if (!bn_fwd_sup(in, ni, out, no, attr)) return Status::InvalidArgument;
  const BNAttr A = read_bn_attr(attr);
  const bool training = no == 3;
  if (training && A.use_running_stats) return Status::InvalidArgument;  // launcher.cu:364-366
  const TensorDesc& X = in[0];
  const BNShape sh{(int)X.shape[0], (int)X.shape[1], (int)(X.shape[2] * X.shape[3])};
  hipStream_t s = as_stream(stream);
  const uint16_t* x = (const uint16_t*)X.data;
  uint16_t* y = (uint16_t*)out[0].data;
  if (training) {
    const uint16_t* g = ni == 3 ? (const uint16_t*)in[1].data : nullptr;
    const uint16_t* b = ni == 3 ? (const uint16_t*)in[2].data : nullptr;
    bn_fwd_train_kernel<<<(unsigned)sh.C, 256, 0, s>>>(x, g, b, y, (float*)out[1].data, (float*)out[2].data, sh,
                                                       A.eps);
  } else {
    const bool aff = ni == 5;
    const uint16_t* g = aff ? (const uint16_t*)in[1].data : nullptr;
    const uint16_t* b = aff ? (const uint16_t*)in[2].data : nullptr;
    const int64_t total = numel_of(X);
    bn_fwd_infer_kernel<<<grid_1d(total, 256, 4096), 256, 0, s>>>(
        x, g, b, (const float*)in[aff ? 3 : 1].data, (const float*)in[aff ? 4 : 2].data, y, sh, A.eps, total);
  }
  return launch_status("batchnorm_fwd");
}

// batchnorm/launcher.cu:483-526: (X, dY, G, SM, SR) -> (dX, dG, dB); the
// non-affine form (X, dY, SM, SR) -> (dX) is accepted by supported() and
// answered with NotImplemented at launch, as in the reference.
bool bn_bwd_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void*) {
  if (!in || !out) return false;
  const bool affine = ni == 5 && no == 3, noaff = ni == 4 && no == 1;
  if (!affine && !noaff) return false;
  const TensorDesc &X = in[0], &dY = in[1], &dX = out[0];
  if (!nchw_f16(X) || !nchw_f16(dY) || !nchw_f16(dX) || !same_shape(X, dY) || !same_shape(X, dX)) return false;
  const int64_t C = X.shape[1];
  if (X.shape[0] * X.shape[2] * X.shape[3] > INT32_MAX) return false;
  if (!vec_c(in[affine ? 3 : 2], DType::kF32, C) || !vec_c(in[affine ? 4 : 3], DType::kF32, C)) return false;
  if (affine && (!vec_c(in[2], DType::kF16, C) || !vec_c(out[1], DType::kF32, C) || !vec_c(out[2], DType::kF32, C)))
    return false;
  return true;
}

Status bn_bwd_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* attr, void*, size_t,
                     void* stream) {
  if (!bn_bwd_sup(in, ni, out, no, attr)) return Status::InvalidArgument;
  if (ni != 5) return Status::NotImplemented;
  const TensorDesc& X = in[0];
  const BNShape sh{(int)X.shape[0], (int)X.shape[1], (int)(X.shape[2] * X.shape[3])};
  bn_bwd_kernel<<<(unsigned)sh.C, 256, 0, as_stream(stream)>>>(
      (const uint16_t*)X.data, (const uint16_t*)in[1].data, (const uint16_t*)in[2].data, (const float*)in[3].data,
      (const float*)in[4].data, (uint16_t*)out[0].data, (float*)out[1].data, (float*)out[2].data, sh);
  return launch_status("batchnorm_bwd");
}

}  // namespace

KernelVariant make_layernorm_fwd_f32_variant() {
  return make("layernorm_fwd_f32_contig2d", ln_fwd_f32_launch, ln_fwd_f32_sup, AICF_SCHEMA_LNEP);
}
KernelVariant make_layernorm_fwd_f16_variant() {
  return make("layernorm_fwd_f16_contig2d", ln_fwd_f16_launch, ln_fwd_f16_sup, AICF_SCHEMA_LNEP);
}
KernelVariant make_layernorm_bwd_f32_variant() {
  return make("layernorm_bwd_f32_contig2d", ln_bwd_f32_launch, ln_bwd_f32_sup);
}
KernelVariant make_layernorm_bwd_f16_variant() {
  return make("layernorm_bwd_f16_contig2d", ln_bwd_f16_launch, ln_bwd_f16_sup);
}
KernelVariant make_batchnorm_fwd_f16_variant() {
  return make("batchnorm_fwd_f16_nchw", bn_fwd_launch, bn_fwd_sup, AICF_SCHEMA_BNEP);
}
KernelVariant make_batchnorm_bwd_f16_variant() {
  return make("batchnorm_bwd_f16_nchw_affine", bn_bwd_launch, bn_bwd_sup);
}

}  // namespace aicf::hip
