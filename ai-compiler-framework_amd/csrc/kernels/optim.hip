// Optimizer-side kernels for gfx950: fused Adam (reference contract and the
// AdamW variant with in-kernel bias correction and bf16 shadow refresh),
// bias correction, step counter increment and SGD.
//
// Reference contracts:
//   adam_step  src/backends/cuda/ops/adam_step/launcher.cu:32-60 (attrs),
//              :95-128 (alias policy), :143-176 (checks), :257-293 (math)
//   bias_corr  src/backends/cuda/ops/biascorr/launcher.cu:31-50,82-131
//   step_inc   src/backends/cuda/ops/step_inc/launcher.cu:34-38,93-157
//   sgd_step   src/backends/cuda/ops/sgd_step/launcher.cu:31-45,111-385
//
// Design: every streaming kernel moves 16-byte vectors (global_load_dwordx4)
// with UNROLL independent vectors per thread in flight and no grid-stride
// loop, so the whole array is covered by one wave of workgroups that the
// dispatcher spreads over all 8 XCDs.  Out-of-place Adam reads P and writes
// Pout in the same pass instead of copying P first.
#include "../common/adamw.hpp"
#include "../common/hip_util.hpp"

namespace aicf::hip {

namespace {

// ---------------------------------------------------------------------------
// Adam, reference arithmetic (adam_step/launcher.cu:276-291).  The two
// moment updates are written as explicit fmaf so that the CPU oracle can
// reproduce them bit for bit (nvcc contracts the same expressions to FMA).
// ---------------------------------------------------------------------------
struct AdamRefArgs {
  float lr, beta1, beta2, eps, omb1, omb2;
};

__device__ __forceinline__ void adam_ref_elem(float& p, float g, float& m, float& v, float bc1,
                                              float bc2, const AdamRefArgs& a) {
  const float m_new = fmaf(a.beta1, m, a.omb1 * g);
  const float v_new = fmaf(a.beta2, v, a.omb2 * (g * g));
  const float m_hat = m_new / bc1;
  const float v_hat = v_new / bc2;
  const float denom = sqrtf(v_hat) + a.eps;
  p = fmaf(-a.lr, m_hat / denom, p);
  m = m_new;
  v = v_new;
}

template <int UNROLL>
__global__ __launch_bounds__(256) void adam_ref_vec4_kernel(
    const float* __restrict__ P, const float* __restrict__ G, const float* __restrict__ M,
    const float* __restrict__ V, float* __restrict__ Pout, float* __restrict__ Mout,
    float* __restrict__ Vout, int64_t n4, AdamRefArgs a, const float* __restrict__ bc1p,
    const float* __restrict__ bc2p) {
  const float bc1 = bc1p[0], bc2 = bc2p[0];
  const int64_t base = (int64_t)blockIdx.x * (256 * UNROLL) + threadIdx.x;
  f32x4 p[UNROLL], g[UNROLL], m[UNROLL], v[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t i = base + (int64_t)u * 256;
    if (i < n4) {
      p[u] = reinterpret_cast<const f32x4*>(P)[i];
      g[u] = reinterpret_cast<const f32x4*>(G)[i];
      m[u] = reinterpret_cast<const f32x4*>(M)[i];
      v[u] = reinterpret_cast<const f32x4*>(V)[i];
    }
  }
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t i = base + (int64_t)u * 256;
    if (i < n4) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float pp = p[u][c], mm = m[u][c], vv = v[u][c];
        adam_ref_elem(pp, g[u][c], mm, vv, bc1, bc2, a);
        p[u][c] = pp;
        m[u][c] = mm;
        v[u][c] = vv;
      }
      reinterpret_cast<f32x4*>(Pout)[i] = p[u];
      reinterpret_cast<f32x4*>(Mout)[i] = m[u];
      reinterpret_cast<f32x4*>(Vout)[i] = v[u];
    }
  }
}

__global__ __launch_bounds__(256) void adam_ref_scalar_kernel(
    const float* __restrict__ P, const float* __restrict__ G, const float* __restrict__ M,
    const float* __restrict__ V, float* __restrict__ Pout, float* __restrict__ Mout,
    float* __restrict__ Vout, int64_t begin, int64_t n, AdamRefArgs a,
    const float* __restrict__ bc1p, const float* __restrict__ bc2p) {
  const int64_t i = begin + (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float p = P[i], m = M[i], v = V[i];
  adam_ref_elem(p, G[i], m, v, bc1p[0], bc2p[0], a);
  Pout[i] = p;
  Mout[i] = m;
  Vout[i] = v;
}

// ---------------------------------------------------------------------------
// AdamW with in-kernel bias correction (no reference counterpart; the
// reference feeds host-computed divisors).  Per element:
//   p  <- p * (1 - lr*wd)                        (decoupled weight decay)
//   m' <- fma(b1, m, (1-b1) g);  v' <- fma(b2, v, (1-b2) g^2)
//   p  <- p - step * m' / (sqrt(v' * ibc2) + eps)
// with bc_k = 1 - b_k^t computed in double from the device step counter,
// step = lr / bc1 and ibc2 = 1 / bc2 (both rounded to fp32 once per thread).
// Optionally writes bf16(p) into a shadow copy used by bf16 GEMMs.
// ---------------------------------------------------------------------------
template <int UNROLL, bool SHADOW>
__global__ __launch_bounds__(256) void adamw_vec4_kernel(
    const float* __restrict__ P, const float* __restrict__ G, const float* __restrict__ M,
    const float* __restrict__ V, float* __restrict__ Pout, float* __restrict__ Mout,
    float* __restrict__ Vout, uint16_t* __restrict__ Wb, int64_t n, AdamWArgs a,
    const int32_t* __restrict__ stepp) {
  // vectors 0 .. n4-1; the thread that would take vector n4 updates the
  // n % 4 remaining elements one by one (the same expression), so one launch
  // covers any length
  const int64_t n4 = n / 4;
  // The element loads go out first: they do not depend on the step counter,
  // whose read and the bias corrections (two fp64 pow, one wave per block)
  // then overlap them (2^28 parameters: 6.17 -> 6.27 TB/s against the
  // counter read before the loads; the same bits; a per-wave computation
  // without the barrier, and two vectors per thread, measured slower).
  const int64_t base = (int64_t)blockIdx.x * (256 * UNROLL) + threadIdx.x;
  f32x4 p[UNROLL], g[UNROLL], m[UNROLL], v[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t i = base + (int64_t)u * 256;
    if (i < n4) {
      p[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(P) + i);
      g[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(G) + i);
      m[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(M) + i);
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(V) + i);
    }
  }
  __shared__ float sh[2];
  if (threadIdx.x < 64) {
    const AdamWScalars t = adamw_scalars(stepp, a);
    if (threadIdx.x == 0) {
      sh[0] = t.step;
      sh[1] = t.ibc2;
    }
  }
  __syncthreads();
  const AdamWScalars s{sh[0], sh[1]};
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t i = base + (int64_t)u * 256;
    if (i < n4) {
      u16x4 w;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float pp = p[u][c], mm = m[u][c], vv = v[u][c];
        adamw_elem(pp, g[u][c], mm, vv, s, a);
        p[u][c] = pp;
        m[u][c] = mm;
        v[u][c] = vv;
        if (SHADOW) w[c] = f32_to_bf16(pp);
      }
      __builtin_nontemporal_store(p[u], reinterpret_cast<f32x4*>(Pout) + i);
      __builtin_nontemporal_store(m[u], reinterpret_cast<f32x4*>(Mout) + i);
      __builtin_nontemporal_store(v[u], reinterpret_cast<f32x4*>(Vout) + i);
      if (SHADOW) __builtin_nontemporal_store(w, reinterpret_cast<u16x4*>(Wb) + i);
    } else if (i == n4) {
      for (int64_t e = 4 * n4; e < n; ++e) {
        float pp = P[e], mm = M[e], vv = V[e];
        adamw_elem(pp, G[e], mm, vv, s, a);
        Pout[e] = pp;
        Mout[e] = mm;
        Vout[e] = vv;
        if (SHADOW) Wb[e] = f32_to_bf16(pp);
      }
    }
  }
}

__global__ __launch_bounds__(256) void adamw_scalar_kernel(
    const float* __restrict__ P, const float* __restrict__ G, const float* __restrict__ M,
    const float* __restrict__ V, float* __restrict__ Pout, float* __restrict__ Mout,
    float* __restrict__ Vout, uint16_t* __restrict__ Wb, int64_t begin, int64_t n, AdamWArgs a,
    const int32_t* __restrict__ stepp) {
  const int64_t i = begin + (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const AdamWScalars s = adamw_scalars(stepp, a);
  float p = P[i], m = M[i], v = V[i];
  adamw_elem(p, G[i], m, v, s, a);
  Pout[i] = p;
  Mout[i] = m;
  Vout[i] = v;
  if (Wb) Wb[i] = f32_to_bf16(p);
}

constexpr int kAdamUnroll = 1;  // measured best on MI355X (more blocks in flight)

// ---------------------------------------------------------------------------
// Host glue: Adam
// ---------------------------------------------------------------------------
struct AdamAttrs {
  float lr = 1e-3f, beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f, wd = 0.0f;
};

// adam_step/launcher.cu:47-60: defaults unless schema ADAM with >= 16 bytes.
// The appended 5th field (weight decay) is read only by the AdamW variant.
AdamAttrs read_adam_attrs(const void* attr) {
  AdamAttrs out;
  const AttrBlob& a = blob(attr);
  if (a.schema_id != AICF_SCHEMA_ADAM || !payload_ok(a, 16)) return out;
  out.lr = field<float>(a, 0);
  out.beta1 = field<float>(a, 4);
  out.beta2 = field<float>(a, 8);
  out.eps = field<float>(a, 12);
  if (payload_ok(a, 20)) out.wd = field<float>(a, 16);
  return out;
}

bool f32_contig_anyrank(const TensorDesc& d) {
  return dt(d) == DType::kF32 && d.contiguous && d.rank >= 1;
}
bool f32_scalar0d_contig(const TensorDesc& d) {
  return dt(d) == DType::kF32 && d.rank == 0 && d.contiguous;
}
bool i32_scalar_contig(const TensorDesc& d) {
  return dt(d) == DType::kI32 && (d.rank == 0 || (d.rank == 1 && d.shape[0] == 1)) && d.contiguous;
}
bool peq(const TensorDesc& a, const TensorDesc& b) { return a.data == b.data; }

// adam_step/launcher.cu:98-128: in-place per buffer allowed, any other alias rejected.
bool adam_bad_alias(const TensorDesc& P, const TensorDesc& G, const TensorDesc& M,
                    const TensorDesc& V, const TensorDesc& Po, const TensorDesc& Mo,
                    const TensorDesc& Vo) {
  if (peq(G, P) || peq(G, M) || peq(G, V) || peq(G, Po) || peq(G, Mo) || peq(G, Vo)) return true;
  if (!peq(Po, P) && (peq(Po, M) || peq(Po, V) || peq(Po, Mo) || peq(Po, Vo))) return true;
  if (!peq(Mo, M) && (peq(Mo, P) || peq(Mo, V) || peq(Mo, Po) || peq(Mo, Vo))) return true;
  if (!peq(Vo, V) && (peq(Vo, P) || peq(Vo, M) || peq(Vo, Po) || peq(Vo, Mo))) return true;
  if (peq(M, V) || peq(P, M) || peq(P, V)) return true;
  return false;
}

// adam_step/launcher.cu:143-176
bool adam_ref_check(const TensorDesc* in, int ni, const TensorDesc* out, int no) {
  if (!in || !out || ni != 6 || no != 3) return false;
  const TensorDesc &P = in[0], &G = in[1], &M = in[2], &V = in[3];
  const TensorDesc &Po = out[0], &Mo = out[1], &Vo = out[2];
  for (const TensorDesc* t : {&P, &G, &M, &V, &Po, &Mo, &Vo})
    if (!f32_contig_anyrank(*t)) return false;
  if (!f32_scalar0d_contig(in[4]) || !f32_scalar0d_contig(in[5])) return false;
  if (!same_shape(P, G) || !same_shape(P, M) || !same_shape(P, V)) return false;
  if (!same_shape(P, Po) || !same_shape(M, Mo) || !same_shape(V, Vo)) return false;
  return !adam_bad_alias(P, G, M, V, Po, Mo, Vo);
}

bool all_aligned16(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (p && !aligned(p, 16)) return false;
  return true;
}

bool adam_ref_supported(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void*) {
  return adam_ref_check(in, ni, out, no);
}

Status adam_ref_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* attr,
                       void*, size_t, void* stream) {
  if (!adam_ref_check(in, ni, out, no) || !attr) return Status::InvalidArgument;
  const int64_t n = numel_of(in[0]);
  if (n <= 0) return Status::Ok;
  const AdamAttrs at = read_adam_attrs(attr);
  AdamRefArgs a{at.lr, at.beta1, at.beta2, at.eps, 1.0f - at.beta1, 1.0f - at.beta2};
  const float *P = (const float*)in[0].data, *G = (const float*)in[1].data,
              *M = (const float*)in[2].data, *V = (const float*)in[3].data;
  float *Po = (float*)out[0].data, *Mo = (float*)out[1].data, *Vo = (float*)out[2].data;
  const float *b1 = (const float*)in[4].data, *b2 = (const float*)in[5].data;
  hipStream_t s = as_stream(stream);
  int64_t done = 0;
  if (all_aligned16({P, G, M, V, Po, Mo, Vo})) {
    const int64_t n4 = n / 4;
    if (n4 > 0) {
      const unsigned blocks = (unsigned)((n4 + 256 * kAdamUnroll - 1) / (256 * kAdamUnroll));
      adam_ref_vec4_kernel<kAdamUnroll><<<blocks, 256, 0, s>>>(P, G, M, V, Po, Mo, Vo, n4, a, b1, b2);
    }
    done = n4 * 4;
  }
  if (done < n) {
    const unsigned blocks = (unsigned)((n - done + 255) / 256);
    adam_ref_scalar_kernel<<<blocks, 256, 0, s>>>(P, G, M, V, Po, Mo, Vo, done, n, a, b1, b2);
  }
  return launch_status("adam_step_f32_v0");
}

// AdamW variant: inputs (P, G, M, V, step:i32 scalar), outputs
// (Pout, Mout, Vout[, Wb:bf16 same shape]).
bool adamw_check(const TensorDesc* in, int ni, const TensorDesc* out, int no) {
  if (!in || !out || ni != 5 || (no != 3 && no != 4)) return false;
  const TensorDesc &P = in[0], &G = in[1], &M = in[2], &V = in[3];
  const TensorDesc &Po = out[0], &Mo = out[1], &Vo = out[2];
  for (const TensorDesc* t : {&P, &G, &M, &V, &Po, &Mo, &Vo})
    if (!f32_contig_anyrank(*t)) return false;
  if (!i32_scalar_contig(in[4])) return false;
  if (!same_shape(P, G) || !same_shape(P, M) || !same_shape(P, V)) return false;
  if (!same_shape(P, Po) || !same_shape(M, Mo) || !same_shape(V, Vo)) return false;
  if (adam_bad_alias(P, G, M, V, Po, Mo, Vo)) return false;
  if (no == 4) {
    const TensorDesc& W = out[3];
    if (dt(W) != DType::kBF16 || !W.contiguous || numel_of(W) != numel_of(P)) return false;
  }
  return true;
}

bool adamw_supported(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void*) {
  return adamw_check(in, ni, out, no);
}

Status adamw_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* attr,
                    void*, size_t, void* stream) {
  if (!adamw_check(in, ni, out, no)) return Status::InvalidArgument;
  const int64_t n = numel_of(in[0]);
  if (n <= 0) return Status::Ok;
  const AdamAttrs at = read_adam_attrs(attr);
  AdamWArgs a{at.lr, at.beta1, at.beta2, at.eps, at.wd, 1.0f - at.beta1, 1.0f - at.beta2,
              1.0f - at.lr * at.wd};
  const float *P = (const float*)in[0].data, *G = (const float*)in[1].data,
              *M = (const float*)in[2].data, *V = (const float*)in[3].data;
  float *Po = (float*)out[0].data, *Mo = (float*)out[1].data, *Vo = (float*)out[2].data;
  uint16_t* Wb = no == 4 ? (uint16_t*)out[3].data : nullptr;
  const int32_t* step = (const int32_t*)in[4].data;
  hipStream_t s = as_stream(stream);
  int64_t done = 0;
  if (all_aligned16({P, G, M, V, Po, Mo, Vo}) && (!Wb || aligned(Wb, 8))) {
    const int64_t slots = n / 4 + (n % 4 ? 1 : 0);  // vectors, plus the tail's thread
    const unsigned blocks = (unsigned)((slots + 256 * kAdamUnroll - 1) / (256 * kAdamUnroll));
    if (Wb)
      adamw_vec4_kernel<kAdamUnroll, true><<<blocks, 256, 0, s>>>(P, G, M, V, Po, Mo, Vo, Wb, n, a,
                                                                   step);
    else
      adamw_vec4_kernel<kAdamUnroll, false><<<blocks, 256, 0, s>>>(P, G, M, V, Po, Mo, Vo, nullptr,
                                                                    n, a, step);
    done = n;
  }
  if (done < n) {
    const unsigned blocks = (unsigned)((n - done + 255) / 256);
    adamw_scalar_kernel<<<blocks, 256, 0, s>>>(P, G, M, V, Po, Mo, Vo, Wb, done, n, a, step);
  }
  return launch_status("adamw_step_f32_v1");
}

size_t no_workspace(const TensorDesc*, int, const void*) { return 0; }

// ---------------------------------------------------------------------------
// Bias correction (biascorr/launcher.cu:82-101): t = max(step, 1),
// d = 1 - beta^t clamped away from 0, outputs 1/d.  beta^t uses ocml powf.
// ---------------------------------------------------------------------------
__global__ void bias_corr_kernel(const int32_t* __restrict__ step, float beta1, float beta2,
                                 float* __restrict__ o1, float* __restrict__ o2) {
  if (threadIdx.x != 0) return;
  int t = step[0];
  if (t < 1) t = 1;
  float d1 = 1.0f - powf(beta1, (float)t);
  float d2 = 1.0f - powf(beta2, (float)t);
  if (fabsf(d1) < 1e-20f) d1 = 1e-20f;
  if (fabsf(d2) < 1e-20f) d2 = 1e-20f;
  o1[0] = 1.0f / d1;
  o2[0] = 1.0f / d2;
}

bool read_betas(const void* attr, float* b1, float* b2) {
  const AttrBlob& a = blob(attr);
  if (!attr || a.schema_id != AICF_SCHEMA_BCOR || !payload_ok(a, 8)) return false;
  *b1 = field<float>(a, 0);
  *b2 = field<float>(a, 4);
  return *b1 == *b1 && *b2 == *b2;  // NaN rejected
}

bool f32_scalar_contig(const TensorDesc& d) {
  return dt(d) == DType::kF32 && (d.rank == 0 || (d.rank == 1 && d.shape[0] == 1)) && d.contiguous;
}

bool bias_corr_supported(const TensorDesc* in, int ni, const TensorDesc* out, int no,
                         const void* attr) {
  if (!in || !out || ni != 1 || no != 2) return false;
  if (!i32_scalar_contig(in[0]) || !f32_scalar_contig(out[0]) || !f32_scalar_contig(out[1]))
    return false;
  float b1, b2;
  return read_betas(attr, &b1, &b2);
}

Status bias_corr_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* attr,
                        void*, size_t, void* stream) {
  if (!bias_corr_supported(in, ni, out, no, attr)) return Status::InvalidArgument;
  float b1 = 0.f, b2 = 0.f;
  read_betas(attr, &b1, &b2);
  bias_corr_kernel<<<1, 64, 0, as_stream(stream)>>>((const int32_t*)in[0].data, b1, b2,
                                                    (float*)out[0].data, (float*)out[1].data);
  return launch_status("bias_corr_v0");
}

// ---------------------------------------------------------------------------
// Step increment (step_inc/launcher.cu:34-38,140-141): SO[i] += 1 on the
// output buffer; the input only fixes the shape.
// ---------------------------------------------------------------------------
__global__ void step_inc_kernel(int32_t* __restrict__ s, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) s[i] += 1;
}

bool i32_ok_scalar0d(const TensorDesc& t) {
  return dt(t) == DType::kI32 && (t.rank == 0 || t.contiguous);
}

bool step_inc_supported(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void*) {
  if (!in || !out || ni != 1 || no != 1) return false;
  if (!i32_ok_scalar0d(in[0]) || !i32_ok_scalar0d(out[0])) return false;
  if (in[0].rank != out[0].rank) return false;
  if (in[0].rank == 0) return true;
  if (!same_shape(in[0], out[0])) return false;
  int64_t n;
  return numel_pos(in[0], &n);
}

Status step_inc_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void*, void*,
                       size_t, void* stream) {
  if (!step_inc_supported(in, ni, out, no, nullptr)) return Status::InvalidArgument;
  const int64_t n = in[0].rank == 0 ? 1 : numel_of(in[0]);
  step_inc_kernel<<<grid_1d(n, 256, INT32_MAX), 256, 0, as_stream(stream)>>>(
      (int32_t*)out[0].data, n);
  return launch_status("step_inc_v0");
}

// ---------------------------------------------------------------------------
// SGD (sgd_step/launcher.cu:111-151): O = P - lr*G in fp32 as one fma (the
// contraction nvcc applies to that expression), f16 stored RNE.
// lr from schema SGDS <f>, default 1e-3 (:40-45,210).  O must not alias G.
// ---------------------------------------------------------------------------
float read_sgd_lr(const void* attr) {
  const AttrBlob& a = blob(attr);
  if (a.schema_id != AICF_SCHEMA_SGDS || !payload_ok(a, 4)) return 1e-3f;
  return field<float>(a, 0);
}

__global__ __launch_bounds__(256) void sgd_f32_kernel(const float* __restrict__ P,
                                                      const float* __restrict__ G,
                                                      float* __restrict__ O, int64_t n, float lr) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) O[i] = fmaf(-lr, G[i], P[i]);
}

template <int VEC>
__global__ __launch_bounds__(256) void sgd_f16_kernel(const uint16_t* __restrict__ P,
                                                      const uint16_t* __restrict__ G,
                                                      uint16_t* __restrict__ O, int64_t n,
                                                      float lr) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * VEC;
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    if (i + c < n) {
      const float p = f16_to_f32(P[i + c]), g = f16_to_f32(G[i + c]);
      O[i + c] = f32_to_f16(fmaf(-lr, g, p));
    }
  }
}

bool sgd_check(const TensorDesc* in, int ni, const TensorDesc* out, int no, DType d) {
  if (!in || !out || ni != 2 || no != 1) return false;
  for (int i = 0; i < 2; ++i)
    if (dt(in[i]) != d || !in[i].contiguous || in[i].rank < 1) return false;
  if (dt(out[0]) != d || !out[0].contiguous || out[0].rank < 1) return false;
  if (!same_shape(in[0], in[1]) || !same_shape(in[0], out[0])) return false;
  int64_t n;
  return numel_pos(in[0], &n);
}

bool sgd_f32_supported(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void*) {
  return sgd_check(in, ni, out, no, DType::kF32);
}
bool sgd_f16_supported(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void*) {
  return sgd_check(in, ni, out, no, DType::kF16);
}
bool sgd_f16_half2_supported(const TensorDesc* in, int ni, const TensorDesc* out, int no,
                             const void*) {
  if (!sgd_check(in, ni, out, no, DType::kF16)) return false;
  return (numel_of(in[0]) & 1) == 0 && aligned(in[0].data, 4) && aligned(in[1].data, 4) &&
         aligned(out[0].data, 4);
}

Status sgd_f32_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* attr,
                      void*, size_t, void* stream) {
  if (!sgd_f32_supported(in, ni, out, no, attr) || out[0].data == in[1].data)
    return Status::InvalidArgument;
  const int64_t n = numel_of(in[0]);
  sgd_f32_kernel<<<grid_1d(n, 256, INT32_MAX), 256, 0, as_stream(stream)>>>(
      (const float*)in[0].data, (const float*)in[1].data, (float*)out[0].data, n,
      read_sgd_lr(attr));
  return launch_status("sgd_step_f32_v0");
}

template <int VEC>
Status sgd_f16_launch_impl(const TensorDesc* in, TensorDesc* out, const void* attr, void* stream) {
  const int64_t n = numel_of(in[0]);
  sgd_f16_kernel<VEC><<<grid_1d((n + VEC - 1) / VEC, 256, INT32_MAX), 256, 0, as_stream(stream)>>>(
      (const uint16_t*)in[0].data, (const uint16_t*)in[1].data, (uint16_t*)out[0].data, n,
      read_sgd_lr(attr));
  return launch_status("sgd_step_f16");
}

Status sgd_f16_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* attr,
                      void*, size_t, void* stream) {
  if (!sgd_f16_supported(in, ni, out, no, attr) || out[0].data == in[1].data)
    return Status::InvalidArgument;
  return sgd_f16_launch_impl<1>(in, out, attr, stream);
}

Status sgd_f16_half2_launch(const TensorDesc* in, int ni, TensorDesc* out, int no,
                            const void* attr, void*, size_t, void* stream) {
  if (!sgd_f16_half2_supported(in, ni, out, no, attr) || out[0].data == in[1].data)
    return Status::InvalidArgument;
  return sgd_f16_launch_impl<2>(in, out, attr, stream);
}

KernelVariant make(const char* name, LaunchFn l, SupportedFn s, uint32_t schema = 0) {
  KernelVariant v;
  v.name = name;
  v.launch = l;
  v.supported = s;
  v.query_workspace = no_workspace;
  v.expected_attr_schema_id = schema;
  return v;
}

// ---------------------------------------------------------------------------
// colsum_adamw (no reference counterpart): the bias tail of the MLP step.
// inputs (C_0 .. C_{T-1} column partials f32 [R_t, N_t], P, M, V f32 [n],
// step i32), outputs (G f32 [n], P, M, V in place, Wb bf16 [n]) with
// n = sum N_t.  Element j of tensor t's range (offset o_t = N_0 + .. +
// N_{t-1}) gets g = the sum over r of C_t[r][j - o_t], taken in the order of
// the column-sum finish kernel (four row strides of 4, combined
// (s0 + s1) + (s2 + s3)), so g equals that kernel's output bit for bit; g
// is stored in G and AdamW (adamw.hpp) is applied to P[j], M[j], V[j] with
// it, bf16(P[j]) stored in Wb.  Attr CADW <i fffff>: T, lr, b1, b2, eps, wd.
// ---------------------------------------------------------------------------
constexpr int kColsumAdamMax = 8;

struct ColsumAdamWParams {
  const float* part[kColsumAdamMax];
  int64_t rows[kColsumAdamMax];
  int64_t cols[kColsumAdamMax];
  int64_t off[kColsumAdamMax + 1];
  int T;
  int64_t n;
  float* G;
  float* P;
  float* M;
  float* V;
  uint16_t* Wb;
  const int32_t* step;
  AdamWArgs a;
};

// 64 elements per workgroup: wave w sums rows w, w + 4, .. of the element's
// partials (16 rows at a time as (a0 + a1) + (a2 + a3)), the four sums are
// combined (s0 + s1) + (s2 + s3) in LDS -- the finish kernel's layout and
// order -- and wave 0 applies AdamW.  A workgroup's 64 elements may span two
// tensors.
__global__ __launch_bounds__(256) void colsum_adamw_kernel(ColsumAdamWParams q) {
  __shared__ float red[4][64];
  __shared__ float sh[2];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (threadIdx.x < 64) {
    const AdamWScalars t = adamw_scalars(q.step, q.a);
    if (threadIdx.x == 0) {
      sh[0] = t.step;
      sh[1] = t.ibc2;
    }
  }
  const int64_t j = (int64_t)blockIdx.x * 64 + lane;
  float s = 0.0f;
  if (j < q.n) {
    int t = 0;
    while (t + 1 < q.T && j >= q.off[t + 1]) ++t;
    const int64_t N = q.cols[t], R = q.rows[t];
    const float* c = q.part[t] + (j - q.off[t]);
    int64_t r = w;
    for (; r + 12 < R; r += 16) {
      const float a0 = c[r * N], a1 = c[(r + 4) * N], a2 = c[(r + 8) * N], a3 = c[(r + 12) * N];
      s += (a0 + a1) + (a2 + a3);
    }
    for (; r < R; r += 4) s += c[r * N];
  }
  red[w][lane] = s;
  __syncthreads();
  if (w != 0 || j >= q.n) return;
  const AdamWScalars sc{sh[0], sh[1]};
  const float g = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
  q.G[j] = g;
  float p = q.P[j], m = q.M[j], v = q.V[j];
  adamw_elem(p, g, m, v, sc, q.a);
  q.P[j] = p;
  q.M[j] = m;
  q.V[j] = v;
  q.Wb[j] = f32_to_bf16(p);
}

struct CadwAttr {
  int T = 0;
  AdamWArgs a{};
  bool ok = false;
};
CadwAttr read_cadw(const void* attr) {
  CadwAttr c;
  const AttrBlob& b = blob(attr);
  if (!attr || b.schema_id != AICF_SCHEMA_CADW || !payload_ok(b, 24)) return c;
  c.T = field<int32_t>(b, 0);
  const float lr = field<float>(b, 4), b1 = field<float>(b, 8), b2 = field<float>(b, 12);
  const float eps = field<float>(b, 16), wd = field<float>(b, 20);
  if (c.T < 1 || c.T > kColsumAdamMax || lr != lr || b1 != b1 || b2 != b2 || eps != eps || wd != wd) return c;
  c.a = AdamWArgs{lr, b1, b2, eps, wd, 1.0f - b1, 1.0f - b2, 1.0f - lr * wd};
  c.ok = true;
  return c;
}

bool colsum_adamw_fill(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr,
                       ColsumAdamWParams* qp) {
  const CadwAttr c = read_cadw(attr);
  if (!c.ok || !in || !out || ni != c.T + 4 || no != 5) return false;
  ColsumAdamWParams q{};
  q.T = c.T;
  q.a = c.a;
  int64_t n = 0;
  for (int t = 0; t < c.T; ++t) {
    const TensorDesc& C = in[t];
    if (dt(C) != DType::kF32 || !C.contiguous || C.rank != 2 || C.shape[0] < 1 || C.shape[1] < 1) return false;
    q.part[t] = (const float*)C.data;
    q.rows[t] = C.shape[0];
    q.cols[t] = C.shape[1];
    q.off[t] = n;
    n += C.shape[1];
  }
  q.off[c.T] = n;
  const TensorDesc &P = in[c.T], &M = in[c.T + 1], &V = in[c.T + 2], &S = in[c.T + 3];
  const TensorDesc &G = out[0], &Po = out[1], &Mo = out[2], &Vo = out[3], &W = out[4];
  for (const TensorDesc* x : {&P, &M, &V, &G})
    if (dt(*x) != DType::kF32 || !x->contiguous || numel_of(*x) != n) return false;
  if (dt(W) != DType::kBF16 || !W.contiguous || numel_of(W) != n) return false;
  if (!i32_scalar_contig(S)) return false;
  if (Po.data != P.data || Mo.data != M.data || Vo.data != V.data) return false;  // in place
  if (!same_shape(Po, P) || !same_shape(Mo, M) || !same_shape(Vo, V)) return false;
  // the outputs are written where nothing else is read or written
  const TensorDesc* w[5] = {&G, &P, &M, &V, &W};
  for (int x = 0; x < 5; ++x) {
    for (int y = x + 1; y < 5; ++y)
      if (views_overlap(*w[x], *w[y])) return false;
    for (int t = 0; t < c.T; ++t)
      if (views_overlap(*w[x], in[t])) return false;
    if (views_overlap(*w[x], S)) return false;
  }
  q.n = n;
  q.G = (float*)G.data;
  q.P = (float*)P.data;
  q.M = (float*)M.data;
  q.V = (float*)V.data;
  q.Wb = (uint16_t*)W.data;
  q.step = (const int32_t*)S.data;
  if (qp) *qp = q;
  return true;
}
bool colsum_adamw_supported(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* a) {
  return colsum_adamw_fill(in, ni, out, no, a, nullptr);
}
Status colsum_adamw_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* attr, void*,
                           size_t, void* stream) {
  ColsumAdamWParams q{};
  if (!colsum_adamw_fill(in, ni, out, no, attr, &q)) return Status::InvalidArgument;
  const unsigned blocks = (unsigned)((q.n + 63) / 64);
  colsum_adamw_kernel<<<blocks, 256, 0, as_stream(stream)>>>(q);
  return launch_status("colsum_adamw_f32_v0");
}

}  // namespace

KernelVariant make_adam_step_f32_variant() {
  return make("adam_step_f32_vec4", adam_ref_launch, adam_ref_supported, AICF_SCHEMA_ADAM);
}
KernelVariant make_adamw_step_f32_variant() {
  return make("adamw_step_f32_vec4", adamw_launch, adamw_supported, AICF_SCHEMA_ADAM);
}
KernelVariant make_colsum_adamw_f32_variant() {
  return make("colsum_adamw_f32", colsum_adamw_launch, colsum_adamw_supported, AICF_SCHEMA_CADW);
}
KernelVariant make_biascorr_variant() {
  return make("bias_corr_f32", bias_corr_launch, bias_corr_supported, AICF_SCHEMA_BCOR);
}
KernelVariant make_step_inc_variant() {
  return make("step_inc_i32", step_inc_launch, step_inc_supported);
}
KernelVariant make_sgd_step_f32_variant() {
  return make("sgd_step_f32", sgd_f32_launch, sgd_f32_supported);
}
KernelVariant make_sgd_step_f16_variant() {
  return make("sgd_step_f16", sgd_f16_launch, sgd_f16_supported);
}
KernelVariant make_sgd_step_f16_half2_variant() {
  return make("sgd_step_f16_half2", sgd_f16_half2_launch, sgd_f16_half2_supported);
}

}  // namespace aicf::hip
