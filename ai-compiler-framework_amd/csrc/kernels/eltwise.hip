// Elementwise kernels for gfx950: add, relu, relu_bwd, bias_add, copy,
// grad_zero, mse_grad (+ fused MSE loss value), gelu and gelu_bwd.
//
// Reference contracts (src/backends/cuda/ops/...):
//   add       add/launcher.cu:44-66 (math), :118-140 (checks)
//   relu      relu/launcher.cu:44-74 (math), :83-133 (checks)
//   relu_bwd  relu_bwd/launcher.cu:37-77 (math), :119-164 (checks)
//   bias_add  bias_add/launcher.cu:36-76 (math), :96-189 (attrs, checks)
//   copy      copy/kernels.cuh:8-18, copy/launcher.cu:66-181
//   grad_zero grad_zero/launcher.cu:45-119
//   mse_grad  mse_grad/launcher.cu:36-98 (attrs, math), :140-298 (checks, variants)
//
// All kernels are one pass over 16-byte vectors where the contract allows
// (contiguous buffers, vector-aligned) with a scalar path for the rest.
// f16 arithmetic uses native v_*_f16 instructions, which round once, as the
// reference's __hadd/__hmul2/__hsub2 do.  grad_zero writes zeros with a
// kernel, not a memset, so it is safe inside captured graphs.
#include <mutex>

#include "../common/hip_util.hpp"

namespace aicf::hip {

namespace {

size_t no_workspace(const TensorDesc*, int, const void*) { return 0; }

KernelVariant make(const char* name, LaunchFn l, SupportedFn s) {
  KernelVariant v;
  v.name = name;
  v.launch = l;
  v.supported = s;
  v.query_workspace = no_workspace;
  return v;
}

__device__ __forceinline__ _Float16 h_of(uint16_t u) {
  _Float16 h;
  __builtin_memcpy(&h, &u, 2);
  return h;
}
__device__ __forceinline__ uint16_t u_of(_Float16 h) {
  uint16_t u;
  __builtin_memcpy(&u, &h, 2);
  return u;
}

// ---------------------------------------------------------------------------
// Generic unary / binary elementwise launch over n elements of 4-byte or
// 2-byte storage: each thread handles one 16-byte vector (4 or 8 elements),
// with a guarded scalar tail.  Nontemporal 16-byte loads and stores, one
// 4 KB block per workgroup: the access pattern of this part's best measured
// copy rate.
// ---------------------------------------------------------------------------
template <typename T, int V, typename F>
__global__ __launch_bounds__(256) void map1_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                   int64_t n, F f) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
  if (i + V <= n) {
    typedef T vec __attribute__((ext_vector_type(V)));
    const vec a = __builtin_nontemporal_load(reinterpret_cast<const vec*>(x + i));
    vec r;
#pragma unroll
    for (int c = 0; c < V; ++c) r[c] = f(a[c]);
    __builtin_nontemporal_store(r, reinterpret_cast<vec*>(y + i));
  } else {
    for (int64_t j = i; j < n; ++j) y[j] = f(x[j]);
  }
}

template <typename T, int V, typename F>
__global__ __launch_bounds__(256) void map2_kernel(const T* __restrict__ x0, const T* __restrict__ x1,
                                                   T* __restrict__ y, int64_t n, F f) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
  if (i + V <= n) {
    typedef T vec __attribute__((ext_vector_type(V)));
    const vec a = __builtin_nontemporal_load(reinterpret_cast<const vec*>(x0 + i));
    const vec b = __builtin_nontemporal_load(reinterpret_cast<const vec*>(x1 + i));
    vec r;
#pragma unroll
    for (int c = 0; c < V; ++c) r[c] = f(a[c], b[c]);
    __builtin_nontemporal_store(r, reinterpret_cast<vec*>(y + i));
  } else {
    for (int64_t j = i; j < n; ++j) y[j] = f(x0[j], x1[j]);
  }
}

template <typename T>
constexpr int vec_of() {
  return 16 / (int)sizeof(T);
}

template <typename T, typename F>
Status launch_map1(const void* x, void* y, int64_t n, F f, void* stream, const char* what) {
  if (n <= 0) return Status::Ok;
  constexpr int V = vec_of<T>();
  const bool vec_ok = aligned(x, 16) && aligned(y, 16);
  if (vec_ok) {
    map1_kernel<T, V, F><<<grid_1d((n + V - 1) / V, 256, INT32_MAX), 256, 0, as_stream(stream)>>>(
        (const T*)x, (T*)y, n, f);
  } else {
    map1_kernel<T, 1, F><<<grid_1d(n, 256, INT32_MAX), 256, 0, as_stream(stream)>>>((const T*)x,
                                                                                  (T*)y, n, f);
  }
  return launch_status(what);
}

template <typename T, typename F>
Status launch_map2(const void* x0, const void* x1, void* y, int64_t n, F f, void* stream,
                   const char* what) {
  if (n <= 0) return Status::Ok;
  constexpr int V = vec_of<T>();
  const bool vec_ok = aligned(x0, 16) && aligned(x1, 16) && aligned(y, 16);
  if (vec_ok) {
    map2_kernel<T, V, F><<<grid_1d((n + V - 1) / V, 256, INT32_MAX), 256, 0, as_stream(stream)>>>(
        (const T*)x0, (const T*)x1, (T*)y, n, f);
  } else {
    map2_kernel<T, 1, F><<<grid_1d(n, 256, INT32_MAX), 256, 0, as_stream(stream)>>>(
        (const T*)x0, (const T*)x1, (T*)y, n, f);
  }
  return launch_status(what);
}

// ---- functors ---------------------------------------------------------------
struct AddF32 {
  __device__ float operator()(float a, float b) const { return a + b; }
};
struct AddF16 {
  __device__ uint16_t operator()(uint16_t a, uint16_t b) const { return u_of(h_of(a) + h_of(b)); }
};
// relu: x > 0 ? x : +0  (NaN -> 0, -0 -> +0), compared in the storage type.
struct ReluF32 {
  __device__ float operator()(float x) const { return x > 0.0f ? x : 0.0f; }
};
struct ReluF16 {
  __device__ uint16_t operator()(uint16_t x) const {
    return h_of(x) > (_Float16)0.0f ? x : (uint16_t)0;
  }
};
// relu_bwd: (Y > 0) ? dOut : 0, inputs (dOut, Y).
struct ReluBwdF32 {
  __device__ float operator()(float d, float y) const { return y > 0.0f ? d : 0.0f; }
};
struct ReluBwdF16 {
  __device__ uint16_t operator()(uint16_t d, uint16_t y) const {
    return h_of(y) > (_Float16)0.0f ? d : (uint16_t)0;
  }
};
struct IdentityF32 {
  __device__ float operator()(float x) const { return x; }
};
struct IdentityU16 {
  __device__ uint16_t operator()(uint16_t x) const { return x; }
};
struct ZeroF32 {
  __device__ float operator()(float) const { return 0.0f; }
};
struct ZeroU16 {
  __device__ uint16_t operator()(uint16_t) const { return 0; }
};
struct GeluF32 {
  __device__ float operator()(float x) const { return gelu_tanh_f(x); }
};
struct GeluBF16 {
  __device__ uint16_t operator()(uint16_t x) const { return f32_to_bf16(gelu_tanh_f(bf16_to_f32(x))); }
};
struct GeluBwdF32 {
  __device__ float operator()(float d, float z) const { return d * gelu_tanh_grad_f(z); }
};
struct GeluBwdBF16 {
  __device__ uint16_t operator()(uint16_t d, uint16_t z) const {
    return f32_to_bf16(bf16_to_f32(d) * gelu_tanh_grad_f(bf16_to_f32(z)));
  }
};
struct MseF32 {
  float s;
  __device__ float operator()(float p, float t) const { return (p - t) * s; }
};
struct MseF16Scalar {  // fp32 math, RNE store (mse_grad/launcher.cu:73-85)
  float s;
  __device__ uint16_t operator()(uint16_t p, uint16_t t) const {
    return f32_to_f16((f16_to_f32(p) - f16_to_f32(t)) * s);
  }
};
struct MseF16Half {  // half math (mse_grad/launcher.cu:87-98)
  _Float16 s;
  __device__ uint16_t operator()(uint16_t p, uint16_t t) const {
    return u_of((_Float16)(h_of(p) - h_of(t)) * s);
  }
};

// ---- shared checks ------------------------------------------------------------
bool same3(const TensorDesc& a, const TensorDesc& b, const TensorDesc& c) {
  return same_shape(a, b) && same_shape(a, c);
}

// ---------------------------------------------------------------------------
// add: inputs (A, B) -> O, same dtype/shape, contiguous flag, numel > 0.
// ---------------------------------------------------------------------------
bool add_check(const TensorDesc* in, int ni, const TensorDesc* out, int no, DType d) {
  if (!in || !out || ni != 2 || no != 1) return false;
  const TensorDesc &A = in[0], &B = in[1], &O = out[0];
  if (dt(A) != d || dt(B) != d || dt(O) != d) return false;
  if (!A.contiguous || !B.contiguous || !O.contiguous) return false;
  if (!same3(A, B, O)) return false;
  return numel_of(O) > 0;
}
bool vec2_ok(const TensorDesc* in, int ni, const TensorDesc* out) {
  if ((numel_of(out[0]) & 1) != 0) return false;
  for (int i = 0; i < ni; ++i)
    if (!aligned(in[i].data, 4)) return false;
  return aligned(out[0].data, 4);
}
bool add_f32_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return add_check(i, ni, o, no, DType::kF32);
}
bool add_f16_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return add_check(i, ni, o, no, DType::kF16);
}
bool add_f16v2_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return add_check(i, ni, o, no, DType::kF16) && vec2_ok(i, 2, o);
}
Status add_f32_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                      size_t, void* s) {
  if (!add_f32_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map2<float>(i[0].data, i[1].data, o[0].data, numel_of(o[0]), AddF32{}, s, "add_f32");
}
Status add_f16_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                      size_t, void* s) {
  if (!add_f16_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map2<uint16_t>(i[0].data, i[1].data, o[0].data, numel_of(o[0]), AddF16{}, s,
                               "add_f16");
}
Status add_f16v2_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                        size_t, void* s) {
  if (!add_f16v2_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map2<uint16_t>(i[0].data, i[1].data, o[0].data, numel_of(o[0]), AddF16{}, s,
                               "add_f16_vec2");
}

// ---------------------------------------------------------------------------
// relu: X -> O, same shape, row-major strides, 0 < numel <= INT_MAX.
// ---------------------------------------------------------------------------
bool relu_check(const TensorDesc* in, int ni, const TensorDesc* out, int no, DType d) {
  if (!in || !out || ni != 1 || no != 1) return false;
  if (dt(in[0]) != d || dt(out[0]) != d) return false;
  if (!same_shape(in[0], out[0])) return false;
  if (!strides_rowmajor(in[0]) || !strides_rowmajor(out[0])) return false;
  const int64_t n = numel_of(out[0]);
  return n > 0 && n <= (int64_t)INT32_MAX;
}
bool relu_f32_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return relu_check(i, ni, o, no, DType::kF32);
}
bool relu_f16_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return relu_check(i, ni, o, no, DType::kF16);
}
bool relu_f16v2_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return relu_check(i, ni, o, no, DType::kF16) && vec2_ok(i, 1, o);
}
Status relu_f32_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                       size_t, void* s) {
  if (!relu_f32_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map1<float>(i[0].data, o[0].data, numel_of(o[0]), ReluF32{}, s, "relu_f32");
}
Status relu_f16_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                       size_t, void* s) {
  if (!relu_f16_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map1<uint16_t>(i[0].data, o[0].data, numel_of(o[0]), ReluF16{}, s, "relu_f16");
}
Status relu_f16v2_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                         size_t, void* s) {
  if (!relu_f16v2_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map1<uint16_t>(i[0].data, o[0].data, numel_of(o[0]), ReluF16{}, s, "relu_f16_vec2");
}

// ---------------------------------------------------------------------------
// relu_bwd: inputs (dOut, Y) -> dY, contiguous flag, same shape, numel > 0.
// Covers every element (the reference's grid cap skips indices >= 16,776,960).
// ---------------------------------------------------------------------------
bool relu_bwd_check(const TensorDesc* in, int ni, const TensorDesc* out, int no, DType d) {
  if (!in || !out || ni != 2 || no != 1) return false;
  const TensorDesc &dO = in[0], &Y = in[1], &dY = out[0];
  for (const TensorDesc* t : {&dO, &Y, &dY})
    if (dt(*t) != d || !t->contiguous) return false;
  if (Y.rank < 1 || !same_shape(Y, dO) || !same_shape(Y, dY)) return false;
  int64_t n;
  return numel_pos(Y, &n);
}
bool relu_bwd_f32_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return relu_bwd_check(i, ni, o, no, DType::kF32);
}
bool relu_bwd_f16_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return relu_bwd_check(i, ni, o, no, DType::kF16);
}
bool relu_bwd_f16v2_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return relu_bwd_check(i, ni, o, no, DType::kF16) && vec2_ok(i, 2, o);
}
Status relu_bwd_f32_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a,
                           void*, size_t, void* s) {
  if (!relu_bwd_f32_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map2<float>(i[0].data, i[1].data, o[0].data, numel_of(o[0]), ReluBwdF32{}, s,
                            "relu_bwd_f32");
}
Status relu_bwd_f16_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a,
                           void*, size_t, void* s) {
  if (!relu_bwd_f16_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map2<uint16_t>(i[0].data, i[1].data, o[0].data, numel_of(o[0]), ReluBwdF16{}, s,
                               "relu_bwd_f16");
}
Status relu_bwd_f16v2_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a,
                             void*, size_t, void* s) {
  if (!relu_bwd_f16v2_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map2<uint16_t>(i[0].data, i[1].data, o[0].data, numel_of(o[0]), ReluBwdF16{}, s,
                               "relu_bwd_f16_vec2");
}

// ---------------------------------------------------------------------------
// bias_add: inputs (Y [...,N], b [N]) -> O, last dim only.  Axis from schema
// BADD <q> or schema 0 with a payload; default -1 (bias_add/launcher.cu:104-124).
// 2-D grid: blockIdx.y walks row tiles, threads walk columns, so no per-element
// integer modulo is needed.
// ---------------------------------------------------------------------------
int64_t read_bias_axis(const void* attr) {
  const AttrBlob& a = blob(attr);
  if (a.schema_id != 0 && a.schema_id != AICF_SCHEMA_BADD) return -1;
  if (!payload_ok(a, 8)) return -1;
  return field<int64_t>(a, 0);
}

bool bias_add_check(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr,
                    DType d) {
  if (!in || !out || ni != 2 || no != 1) return false;
  const TensorDesc &Y = in[0], &B = in[1], &O = out[0];
  if (dt(Y) != d || !Y.contiguous || Y.rank < 2) return false;
  if (dt(O) != d || !O.contiguous || O.rank < 2) return false;
  if (!(B.contiguous && B.rank == 1 && dt(B) == d)) return false;
  const int64_t axis = read_bias_axis(attr);
  if (!(axis == -1 || axis == Y.rank - 1)) return false;
  if (!same_shape(Y, O)) return false;
  int64_t M, N;
  if (!rows_cols(Y, &M, &N)) return false;
  return B.shape[0] == N;
}

template <typename T, bool F16>
__global__ __launch_bounds__(256) void bias_add_kernel(const T* __restrict__ Y, const T* __restrict__ b,
                                                       T* __restrict__ O, int64_t M, int64_t N,
                                                       int rows_per_block) {
  const int64_t col = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (col >= N) return;
  const T bv = b[col];
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < M ? r0 + rows_per_block : M;
  for (int64_t r = r0; r < r1; ++r) {
    const int64_t i = r * N + col;
    if constexpr (F16) {
      O[i] = u_of(h_of(Y[i]) + h_of(bv));
    } else {
      O[i] = Y[i] + bv;
    }
  }
}

template <typename T, bool F16>
Status bias_add_run(const TensorDesc* in, TensorDesc* out, void* stream, const char* what) {
  int64_t M, N;
  rows_cols(in[0], &M, &N);
  const int rpb = 16;
  const unsigned gx = (unsigned)((N + 255) / 256);
  const int64_t gy = (M + rpb - 1) / rpb;
  if (gy > 65535 * 64) return Status::InvalidArgument;
  // rows beyond the y-grid limit are folded into more rows per block
  int rows = rpb;
  int64_t gyy = gy;
  while (gyy > 65535) {
    rows *= 2;
    gyy = (M + rows - 1) / rows;
  }
  dim3 grid(gx, (unsigned)gyy);
  bias_add_kernel<T, F16><<<grid, 256, 0, as_stream(stream)>>>((const T*)in[0].data,
                                                               (const T*)in[1].data, (T*)out[0].data,
                                                               M, N, rows);
  return launch_status(what);
}

bool bias_add_f32_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void* a) {
  return bias_add_check(i, ni, o, no, a, DType::kF32);
}
bool bias_add_f16_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void* a) {
  return bias_add_check(i, ni, o, no, a, DType::kF16);
}
bool bias_add_f16v2_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void* a) {
  if (!bias_add_check(i, ni, o, no, a, DType::kF16)) return false;
  return (i[0].shape[i[0].rank - 1] & 1) == 0 && aligned(i[0].data, 4) && aligned(i[1].data, 4) &&
         aligned(o[0].data, 4);
}
Status bias_add_f32_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a,
                           void*, size_t, void* s) {
  if (!bias_add_f32_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return bias_add_run<float, false>(i, o, s, "bias_add_f32");
}
Status bias_add_f16_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a,
                           void*, size_t, void* s) {
  if (!bias_add_f16_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return bias_add_run<uint16_t, true>(i, o, s, "bias_add_f16");
}
Status bias_add_f16v2_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a,
                             void*, size_t, void* s) {
  if (!bias_add_f16v2_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return bias_add_run<uint16_t, true>(i, o, s, "bias_add_f16_vec2");
}

// ---------------------------------------------------------------------------
// copy: X -> Y, same dtype/shape, contiguous flag.
// ---------------------------------------------------------------------------
bool copy_check(const TensorDesc* in, int ni, const TensorDesc* out, int no, DType d) {
  if (!in || !out || ni != 1 || no != 1) return false;
  if (dt(in[0]) != d || dt(out[0]) != d) return false;
  if (!in[0].contiguous || !out[0].contiguous) return false;
  return same_shape(in[0], out[0]);
}
bool copy_f32_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return copy_check(i, ni, o, no, DType::kF32);
}
bool copy_f16_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return copy_check(i, ni, o, no, DType::kF16);
}
bool copy_bf16_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return copy_check(i, ni, o, no, DType::kBF16);
}
Status copy_f32_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                       size_t, void* s) {
  if (!copy_f32_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map1<float>(i[0].data, o[0].data, numel_of(i[0]), IdentityF32{}, s, "copy_f32");
}
Status copy_u16_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                       size_t, void* s) {
  if (!copy_check(i, ni, o, no, dt(i[0])) || (dt(i[0]) != DType::kF16 && dt(i[0]) != DType::kBF16))
    return Status::InvalidArgument;
  return launch_map1<uint16_t>(i[0].data, o[0].data, numel_of(i[0]), IdentityU16{}, s, "copy_u16");
}

// ---------------------------------------------------------------------------
// grad_zero: X -> Y (zeros), same dtype/shape, contiguous, f32/f16 (+bf16).
// ---------------------------------------------------------------------------
bool grad_zero_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void*) {
  if (!in || !out || ni != 1 || no != 1) return false;
  if (dt(in[0]) != dt(out[0])) return false;
  if (!same_shape(in[0], out[0])) return false;
  if (!in[0].contiguous || !out[0].contiguous) return false;
  const DType d = dt(in[0]);
  return d == DType::kF32 || d == DType::kF16 || d == DType::kBF16;
}
Status grad_zero_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                        size_t, void* s) {
  if (!grad_zero_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  const int64_t n = numel_of(o[0]);
  if (dt(o[0]) == DType::kF32)
    return launch_map1<float>(o[0].data, o[0].data, n, ZeroF32{}, s, "grad_zero");
  return launch_map1<uint16_t>(o[0].data, o[0].data, n, ZeroU16{}, s, "grad_zero");
}

// ---------------------------------------------------------------------------
// mse_grad: inputs (pred, target) -> dPred = (pred - target) * scale.
// scale from schema MSEG <f>, else 2/numel computed in fp32 on the host.
// ---------------------------------------------------------------------------
bool read_mse_scale(const void* attr, float* s) {
  const AttrBlob& a = blob(attr);
  if (!attr || a.schema_id != AICF_SCHEMA_MSEG || !payload_ok(a, 4)) return false;
  *s = field<float>(a, 0);
  return true;
}

bool mse_check(const TensorDesc* in, int ni, const TensorDesc* out, int no, DType d) {
  if (!in || !out || ni != 2 || no != 1) return false;
  const TensorDesc &P = in[0], &T = in[1], &G = out[0];
  for (const TensorDesc* t : {&P, &T, &G})
    if (dt(*t) != d || !t->contiguous) return false;
  if (P.rank < 1 || !same_shape(P, T) || !same_shape(P, G)) return false;
  int64_t n;
  return numel_pos(P, &n);
}
bool mse_f32_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return mse_check(i, ni, o, no, DType::kF32);
}
bool mse_f16_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return mse_check(i, ni, o, no, DType::kF16);
}
float mse_scale(const void* attr, int64_t n) {
  float s;
  if (read_mse_scale(attr, &s)) return s;
  return 2.0f / (float)n;
}
Status mse_f32_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                      size_t, void* s) {
  if (!mse_f32_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  const int64_t n = numel_of(i[0]);
  return launch_map2<float>(i[0].data, i[1].data, o[0].data, n, MseF32{mse_scale(a, n)}, s,
                            "mse_grad_f32");
}
// The f16 variant picks the half2 math path when numel is even and all
// pointers are 4-byte aligned, like mse_grad/launcher.cu:272-283.
Status mse_f16_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                      size_t, void* s) {
  if (!mse_f16_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  const int64_t n = numel_of(i[0]);
  const float sc = mse_scale(a, n);
  if (vec2_ok(i, 2, o))
    return launch_map2<uint16_t>(i[0].data, i[1].data, o[0].data, n, MseF16Half{(_Float16)sc}, s,
                                 "mse_grad_f16x2");
  return launch_map2<uint16_t>(i[0].data, i[1].data, o[0].data, n, MseF16Scalar{sc}, s,
                               "mse_grad_f16");
}

// ---------------------------------------------------------------------------
// Fused MSE loss + gradient (no reference counterpart: the reference emits
// only the gradient).  inputs (pred f32|bf16, target f32), outputs
// (dPred same dtype as pred, loss f32 scalar, partials f32 [>= kMseBlocks]).
//   dPred = (pred - target) * scale          (scale as mse_grad)
//   loss  = mean((pred - target)^2)
// Pass 1: when the partials buffer holds one value per 2048 elements and n
// is a multiple of 8, one workgroup per 2048 elements, 8 per lane with
// 16-byte nontemporal accesses and no loop (streams at ~79% of HBM peak at
// 8192 x 4096, against ~69% for a grid-stride loop); otherwise kMseBlocks
// workgroups stride over the data.  Each workgroup writes its partial sum of
// squares to partials[b].  Pass 2: one workgroup sums the partials in a
// fixed order.  The result is deterministic for a given size.
// ---------------------------------------------------------------------------
constexpr int kMseBlocks = 1024;
constexpr int64_t kMseElemsPerBlock = 2048;  // one-shot pass 1: 256 lanes x 8

template <bool BF16>
__global__ __launch_bounds__(256) void mse_loss_grad_oneshot(const void* __restrict__ pred,
                                                             const float* __restrict__ tgt,
                                                             void* __restrict__ dpred,
                                                             float* __restrict__ partial, int64_t n8,
                                                             float scale) {
  __shared__ float red[4];
  float acc = 0.0f;
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;  // group of 8 elements
  if (v < n8) {
    const f32x4 t0 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(tgt) + 2 * v);
    const f32x4 t1 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(tgt) + 2 * v + 1);
    float pv[8], tv[8];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      tv[c] = t0[c];
      tv[c + 4] = t1[c];
    }
    if constexpr (BF16) {
      const u16x8 pb = __builtin_nontemporal_load(reinterpret_cast<const u16x8*>(pred) + v);
#pragma unroll
      for (int c = 0; c < 8; ++c) pv[c] = bf16_to_f32(pb[c]);
    } else {
      const f32x4 p0 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(pred) + 2 * v);
      const f32x4 p1 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(pred) + 2 * v + 1);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        pv[c] = p0[c];
        pv[c + 4] = p1[c];
      }
    }
    float d[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float e = pv[c] - tv[c];
      acc = fmaf(e, e, acc);
      d[c] = e * scale;
    }
    if constexpr (BF16) {
      u16x8 db;
#pragma unroll
      for (int c = 0; c < 8; ++c) db[c] = f32_to_bf16(d[c]);
      __builtin_nontemporal_store(db, reinterpret_cast<u16x8*>(dpred) + v);
    } else {
      __builtin_nontemporal_store(f32x4{d[0], d[1], d[2], d[3]}, reinterpret_cast<f32x4*>(dpred) + 2 * v);
      __builtin_nontemporal_store(f32x4{d[4], d[5], d[6], d[7]}, reinterpret_cast<f32x4*>(dpred) + 2 * v + 1);
    }
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

template <bool BF16>
__global__ __launch_bounds__(256) void mse_loss_grad_pass1(const void* __restrict__ pred,
                                                           const float* __restrict__ tgt,
                                                           void* __restrict__ dpred,
                                                           float* __restrict__ partial, int64_t n,
                                                           float scale) {
  __shared__ float red[4];
  float acc = 0.0f;
  const int64_t nv = n / 4;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < nv; v += stride) {
    const f32x4 t = reinterpret_cast<const f32x4*>(tgt)[v];
    f32x4 p;
    if constexpr (BF16) {
      const u16x4 pb = reinterpret_cast<const u16x4*>(pred)[v];
#pragma unroll
      for (int c = 0; c < 4; ++c) p[c] = bf16_to_f32(pb[c]);
    } else {
      p = reinterpret_cast<const f32x4*>(pred)[v];
    }
    f32x4 d;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float e = p[c] - t[c];
      acc = fmaf(e, e, acc);
      d[c] = e * scale;
    }
    if constexpr (BF16) {
      u16x4 db;
#pragma unroll
      for (int c = 0; c < 4; ++c) db[c] = f32_to_bf16(d[c]);
      reinterpret_cast<u16x4*>(dpred)[v] = db;
    } else {
      reinterpret_cast<f32x4*>(dpred)[v] = d;
    }
  }
  // tail (n % 4) handled by block 0
  if (blockIdx.x == 0) {
    for (int64_t i = nv * 4 + threadIdx.x; i < n; i += 256) {
      const float p = BF16 ? bf16_to_f32(((const uint16_t*)pred)[i]) : ((const float*)pred)[i];
      const float e = p - tgt[i];
      acc = fmaf(e, e, acc);
      if (BF16)
        ((uint16_t*)dpred)[i] = f32_to_bf16(e * scale);
      else
        ((float*)dpred)[i] = e * scale;
    }
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// One workgroup of 1024 lanes; each lane loads 8 partials at a time (all in
// flight together) and adds them in a fixed order, then lanes and waves are
// combined in a fixed order.
__global__ __launch_bounds__(1024) void mse_loss_grad_pass2(const float* __restrict__ partial,
                                                            int nparts, float* __restrict__ loss,
                                                            double inv_n) {
  constexpr int T = 1024, U = 8;
  __shared__ double red[T / 64];
  double acc = 0.0;
  for (int base = 0; base < nparts; base += T * U) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + u * T + (int)threadIdx.x;
      v[u] = i < nparts ? partial[i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc += (double)v[u];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < T / 64; ++w) tot += red[w];
    loss[0] = (float)(tot * inv_n);
  }
}

bool mse_loss_check(const TensorDesc* in, int ni, const TensorDesc* out, int no) {
  if (!in || !out || ni != 2 || no != 3) return false;
  const TensorDesc &P = in[0], &T = in[1], &G = out[0], &L = out[1], &W = out[2];
  if (dt(P) != DType::kF32 && dt(P) != DType::kBF16) return false;
  if (dt(T) != DType::kF32 || dt(G) != dt(P)) return false;
  if (!P.contiguous || !T.contiguous || !G.contiguous) return false;
  if (P.rank < 1 || !same_shape(P, T) || !same_shape(P, G)) return false;
  if (dt(L) != DType::kF32 || numel_of(L) != 1) return false;
  if (dt(W) != DType::kF32 || !W.contiguous || numel_of(W) < kMseBlocks) return false;
  int64_t n;
  if (!numel_pos(P, &n)) return false;
  const int psz = dt(P) == DType::kF32 ? 16 : 8;
  return aligned(P.data, psz) && aligned(G.data, psz) && aligned(T.data, 16);
}
bool mse_loss_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return mse_loss_check(i, ni, o, no);
}
// Both passes over n elements with `partial` (room for `cap` >= kMseBlocks
// floats) holding the per-workgroup sums; every slot pass 2 reads is written
// by pass 1 first, so the buffer needs no clearing.
Status mse_loss_run(const void* pred, const float* tgt, void* dpred, float* loss, float* partial,
                    int64_t cap, int64_t n, bool bf, float sc, hipStream_t s) {
  const int64_t oneshot_blocks = (n + kMseElemsPerBlock - 1) / kMseElemsPerBlock;
  const bool oneshot = n % 8 == 0 && aligned(pred, 16) && aligned(dpred, 16) && oneshot_blocks <= cap &&
                       oneshot_blocks <= INT32_MAX;
  int nparts = kMseBlocks;
  if (oneshot) {
    nparts = (int)oneshot_blocks;
    if (bf)
      mse_loss_grad_oneshot<true><<<(unsigned)nparts, 256, 0, s>>>(pred, tgt, dpred, partial, n / 8, sc);
    else
      mse_loss_grad_oneshot<false><<<(unsigned)nparts, 256, 0, s>>>(pred, tgt, dpred, partial, n / 8, sc);
  } else if (bf) {
    mse_loss_grad_pass1<true><<<kMseBlocks, 256, 0, s>>>(pred, tgt, dpred, partial, n, sc);
  } else {
    mse_loss_grad_pass1<false><<<kMseBlocks, 256, 0, s>>>(pred, tgt, dpred, partial, n, sc);
  }
  mse_loss_grad_pass2<<<1, 1024, 0, s>>>(partial, nparts, loss, 1.0 / (double)n);
  return launch_status("mse_loss_grad_v0");
}

Status mse_loss_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* a, void*,
                       size_t, void* stream) {
  if (!mse_loss_check(in, ni, out, no)) return Status::InvalidArgument;
  const int64_t n = numel_of(in[0]);
  return mse_loss_run(in[0].data, (const float*)in[1].data, out[0].data, (float*)out[1].data,
                      (float*)out[2].data, numel_of(out[2]), n, dt(in[0]) == DType::kBF16,
                      mse_scale(a, n), as_stream(stream));
}

// ---------------------------------------------------------------------------
// MSE loss + gradient + the gradient's column partial sums + the step
// counter in one pass (no reference counterpart: the loss tail of the MLP
// step, where the reference runs mse_grad, reduce_sum(axis 0) over the
// gradient for the last bias and step_inc).  inputs (pred [M, N] f32|bf16,
// target f32, step i32), outputs (dPred, loss f32, loss partials f32
// [>= blocks], column partials f32 [P, N], step (in place)).  Attr MSCS
// <f scale, i inc>: dPred = (pred - target) * scale (scale <= 0 or no attr:
// 2/n), step += inc (0 or 1; default 1).
// Rows go in P blocks of M / P; within a block the four waves stride the
// rows, each lane holds 16 bytes of pred columns, and the waves are combined
// (w0 + w1) + (w2 + w3): the column sums the two-pass column-sum kernel
// takes of the stored gradient with the same [P, N] workspace, bit for bit.
// The loss partials (one per workgroup) are summed by the second pass of
// the MSE loss.
// ---------------------------------------------------------------------------
constexpr int kMseColsumVecBf16 = 8;
constexpr int kMseColsumUnroll = 2;

template <bool BF16, int VEC, int UNROLL>
__global__ __launch_bounds__(256) void mse_colsum_kernel(const void* __restrict__ pred,
                                                         const float* __restrict__ tgt,
                                                         void* __restrict__ dpred, float* __restrict__ lpart,
                                                         float* __restrict__ cpart, int32_t* __restrict__ step,
                                                         int inc, int64_t M, int64_t N, int64_t rpp,
                                                         float scale) {
  // VEC columns per lane, CB per workgroup, UNROLL rows in flight per lane
  static_assert(VEC == 4 || (BF16 && VEC == 8), "4 or 8 columns per lane");
  constexpr int CB = 64 * VEC;
  __shared__ float red[4][CB];
  __shared__ float lred[4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * CB + lane * VEC;
  const int64_t r0 = (int64_t)blockIdx.y * rpp;
  const int64_t r1 = r0 + rpp < M ? r0 + rpp : M;
  if (inc && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) step[0] += 1;
  float acc[VEC], sq = 0.0f;
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
  // one row: gradient stored, its stored value added to the column sums
  auto row = [&](int64_t r, const float (&pv)[VEC], const float (&tv)[VEC]) {
    float d[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float x = pv[e] - tv[e];
      sq = fmaf(x, x, sq);
      d[e] = x * scale;
    }
    if constexpr (BF16) {
      using V = std::conditional_t<VEC == 8, u16x8, u16x4>;
      V o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        o[e] = f32_to_bf16(d[e]);
        acc[e] += bf16_to_f32(o[e]);
      }
      __builtin_nontemporal_store(o, reinterpret_cast<V*>((uint16_t*)dpred + r * N + c0));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += d[e];
      __builtin_nontemporal_store(f32x4{d[0], d[1], d[2], d[3]},
                                  reinterpret_cast<f32x4*>((float*)dpred + r * N + c0));
    }
  };
  auto load = [&](int64_t r, float (&pv)[VEC], float (&tv)[VEC]) {
    const float* t = tgt + r * N + c0;
    if constexpr (BF16) {
      using V = std::conditional_t<VEC == 8, u16x8, u16x4>;
      const V pb = __builtin_nontemporal_load(reinterpret_cast<const V*>((const uint16_t*)pred + r * N + c0));
#pragma unroll
      for (int e = 0; e < VEC; ++e) pv[e] = bf16_to_f32(pb[e]);
#pragma unroll
      for (int h = 0; h < VEC / 4; ++h) {
        const f32x4 tt = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(t) + h);
#pragma unroll
        for (int e = 0; e < 4; ++e) tv[4 * h + e] = tt[e];
      }
    } else {
      const f32x4 p0 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>((const float*)pred + r * N + c0));
      const f32x4 t0 = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(t));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pv[e] = p0[e];
        tv[e] = t0[e];
      }
    }
  };
  if (c0 < N) {  // N % VEC == 0: the lane's columns are all in range
    int64_t r = r0 + w;
    for (; r + (UNROLL - 1) * 4 < r1; r += UNROLL * 4) {
      float pv[UNROLL][VEC], tv[UNROLL][VEC];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) load(r + u * 4, pv[u], tv[u]);
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) row(r + u * 4, pv[u], tv[u]);
    }
    for (; r < r1; r += 4) {
      float pv[VEC], tv[VEC];
      load(r, pv, tv);
      row(r, pv, tv);
    }
  }
#pragma unroll
  for (int e = 0; e < VEC; ++e) red[w][lane * VEC + e] = acc[e];
  sq = wave_sum(sq);
  if (lane == 0) lred[w] = sq;
  __syncthreads();
  for (int cc = threadIdx.x; cc < CB; cc += 256) {
    const int64_t col = (int64_t)blockIdx.x * CB + cc;
    if (col < N) cpart[(int64_t)blockIdx.y * N + col] = (red[0][cc] + red[1][cc]) + (red[2][cc] + red[3][cc]);
  }
  if (threadIdx.x == 0)
    lpart[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = (lred[0] + lred[1]) + (lred[2] + lred[3]);
}

struct MscsAttr {
  float scale = 0.0f;  // <= 0: 2/n
  int inc = 1;
  bool ok = true;
};
MscsAttr read_mscs(const void* attr) {
  MscsAttr m;
  if (!attr) return m;
  const AttrBlob& a = blob(attr);
  if (a.schema_id == 0 && a.bytes == 0) return m;
  if (a.schema_id != AICF_SCHEMA_MSCS || !payload_ok(a, 8)) {
    m.ok = false;
    return m;
  }
  m.scale = field<float>(a, 0);
  m.inc = field<int32_t>(a, 4);
  if (m.scale != m.scale || (m.inc != 0 && m.inc != 1)) m.ok = false;
  return m;
}

bool mse_colsum_check(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr) {
  if (!in || !out || ni != 3 || no != 5) return false;
  if (!read_mscs(attr).ok) return false;
  const TensorDesc &P = in[0], &T = in[1], &S = in[2];
  const TensorDesc &G = out[0], &L = out[1], &LP = out[2], &CP = out[3], &S2 = out[4];
  if (dt(P) != DType::kF32 && dt(P) != DType::kBF16) return false;
  const bool bf = dt(P) == DType::kBF16;
  if (dt(T) != DType::kF32 || dt(G) != dt(P)) return false;
  for (const TensorDesc* t : {&P, &T, &G})
    if (!t->contiguous || t->rank != 2) return false;
  if (!same_shape(P, T) || !same_shape(P, G)) return false;
  const int64_t M = P.shape[0], N = P.shape[1];
  const int VEC = bf ? kMseColsumVecBf16 : 4;
  if (M < 1 || N < 1 || N % VEC) return false;
  if (dt(S) != DType::kI32 || numel_of(S) != 1 || S2.data != S.data || dt(S2) != DType::kI32) return false;
  if (dt(L) != DType::kF32 || numel_of(L) != 1) return false;
  if (dt(CP) != DType::kF32 || !CP.contiguous || CP.rank != 2 || CP.shape[1] != N) return false;
  const int64_t parts = CP.shape[0];
  if (parts < 1 || M % parts) return false;  // every partial row covers M / P rows
  const int64_t gx = (N + 64 * VEC - 1) / (64 * VEC);
  if (gx * parts > INT32_MAX || parts > 65535) return false;
  if (dt(LP) != DType::kF32 || !LP.contiguous || numel_of(LP) < gx * parts) return false;
  // the written buffers (the step counter aside, updated in place) touch
  // nothing the kernel reads and not each other
  const TensorDesc* w[4] = {&G, &L, &LP, &CP};
  for (int x = 0; x < 4; ++x) {
    for (int y = x + 1; y < 4; ++y)
      if (views_overlap(*w[x], *w[y])) return false;
    for (const TensorDesc* r : {&P, &T, &S})
      if (views_overlap(*w[x], *r)) return false;
  }
  return aligned(P.data, 16) && aligned(G.data, 16) && aligned(T.data, 16);
}
bool mse_colsum_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void* a) {
  return mse_colsum_check(i, ni, o, no, a);
}
Status mse_colsum_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* a, void*,
                         size_t, void* stream) {
  if (!mse_colsum_check(in, ni, out, no, a)) return Status::InvalidArgument;
  const MscsAttr m = read_mscs(a);
  hipStream_t s = as_stream(stream);
  const bool bf = dt(in[0]) == DType::kBF16;
  const int64_t M = in[0].shape[0], N = in[0].shape[1], n = M * N;
  const int64_t parts = out[3].shape[0], rpp = M / parts;
  const float sc = m.scale > 0.0f ? m.scale : 2.0f / (float)n;
  constexpr int VB = kMseColsumVecBf16;  // bf16 columns per lane
  const int vec = bf ? VB : 4;
  const unsigned gx = (unsigned)((N + 64 * vec - 1) / (64 * vec));
  const dim3 grid(gx, (unsigned)parts);
  float* lp = (float*)out[2].data;
  if (bf)
    mse_colsum_kernel<true, VB, kMseColsumUnroll><<<grid, 256, 0, s>>>(
        in[0].data, (const float*)in[1].data, out[0].data, lp, (float*)out[3].data, (int32_t*)in[2].data, m.inc,
        M, N, rpp, sc);
  else
    mse_colsum_kernel<false, 4, kMseColsumUnroll><<<grid, 256, 0, s>>>(
        in[0].data, (const float*)in[1].data, out[0].data, lp, (float*)out[3].data, (int32_t*)in[2].data, m.inc,
        M, N, rpp, sc);
  mse_loss_grad_pass2<<<1, 1024, 0, s>>>(lp, (int)(gx * parts), (float*)out[1].data, 1.0 / (double)n);
  return launch_status("mse_colsum_v0");
}

// ---------------------------------------------------------------------------
// gelu (tanh) forward and backward, f32 and bf16 storage, fp32 math.
//   gelu:     X -> Y
//   gelu_bwd: (dOut, Z) -> dZ = dOut * gelu'(Z)
// ---------------------------------------------------------------------------
bool unary_same(const TensorDesc* in, int ni, const TensorDesc* out, int no, DType d) {
  if (!in || !out || ni != 1 || no != 1) return false;
  if (dt(in[0]) != d || dt(out[0]) != d || !in[0].contiguous || !out[0].contiguous) return false;
  int64_t n;
  return same_shape(in[0], out[0]) && numel_pos(in[0], &n);
}
bool binary_same(const TensorDesc* in, int ni, const TensorDesc* out, int no, DType d) {
  if (!in || !out || ni != 2 || no != 1) return false;
  for (const TensorDesc* t : {&in[0], &in[1], &out[0]})
    if (dt(*t) != d || !t->contiguous) return false;
  int64_t n;
  return same3(in[0], in[1], out[0]) && numel_pos(in[0], &n);
}
bool gelu_f32_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return unary_same(i, ni, o, no, DType::kF32);
}
bool gelu_bf16_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return unary_same(i, ni, o, no, DType::kBF16);
}
bool gelu_bwd_f32_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return binary_same(i, ni, o, no, DType::kF32);
}
bool gelu_bwd_bf16_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void*) {
  return binary_same(i, ni, o, no, DType::kBF16);
}
Status gelu_f32_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                       size_t, void* s) {
  if (!gelu_f32_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map1<float>(i[0].data, o[0].data, numel_of(o[0]), GeluF32{}, s, "gelu_f32");
}
Status gelu_bf16_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,
                        size_t, void* s) {
  if (!gelu_bf16_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map1<uint16_t>(i[0].data, o[0].data, numel_of(o[0]), GeluBF16{}, s, "gelu_bf16");
}
Status gelu_bwd_f32_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a,
                           void*, size_t, void* s) {
  if (!gelu_bwd_f32_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map2<float>(i[0].data, i[1].data, o[0].data, numel_of(o[0]), GeluBwdF32{}, s,
                            "gelu_bwd_f32");
}
Status gelu_bwd_bf16_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a,
                            void*, size_t, void* s) {
  if (!gelu_bwd_bf16_sup(i, ni, o, no, a)) return Status::InvalidArgument;
  return launch_map2<uint16_t>(i[0].data, i[1].data, o[0].data, numel_of(o[0]), GeluBwdBF16{}, s,
                               "gelu_bwd_bf16");
}

// ---------------------------------------------------------------------------
// 2-D transpose (appended op): X [R, C] -> Y [C, R], both row-major with
// arbitrary row strides, 2- or 4-byte elements.  64 x 64 tiles through LDS:
// each thread reads two 16-byte chunks along a row of X and writes two
// 16-byte chunks along a row of Y; the LDS row pitch is padded by 16 bytes.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T* __restrict__ X, T* __restrict__ Y,
                                                        int64_t R, int64_t C, int64_t ldx,
                                                        int64_t ldy) {
  constexpr int TILE = 64;
  constexpr int V = 16 / (int)sizeof(T);        // elements per 16-byte chunk
  constexpr int CPR = TILE / V;                 // chunks per tile row
  constexpr int PITCH = TILE + V;               // padded LDS row (elements)
  __shared__ __attribute__((aligned(16))) T tile[TILE * PITCH];
  typedef T vec __attribute__((ext_vector_type(V)));
  const int64_t r0 = (int64_t)blockIdx.y * TILE, c0 = (int64_t)blockIdx.x * TILE;
  const bool full = r0 + TILE <= R && c0 + TILE <= C;
  const bool vx = full && ((uintptr_t)X % 16 == 0) && ((ldx * (int64_t)sizeof(T)) % 16 == 0);
  const bool vy = full && ((uintptr_t)Y % 16 == 0) && ((ldy * (int64_t)sizeof(T)) % 16 == 0);
  for (int q = threadIdx.x; q < TILE * CPR; q += 256) {
    const int r = q / CPR, c = (q % CPR) * V;
    vec v;
    if (vx) {
      v = *reinterpret_cast<const vec*>(X + (r0 + r) * ldx + c0 + c);
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = (r0 + r < R && c0 + c + e < C) ? X[(r0 + r) * ldx + c0 + c + e] : T(0);
    }
    *reinterpret_cast<vec*>(tile + r * PITCH + c) = v;
  }
  __syncthreads();
  for (int q = threadIdx.x; q < TILE * CPR; q += 256) {
    const int c = q / CPR, r = (q % CPR) * V;  // output row c (= input column), columns r..r+V
    vec v;
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = tile[(r + e) * PITCH + c];
    if (vy) {
      *reinterpret_cast<vec*>(Y + (c0 + c) * ldy + r0 + r) = v;
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e)
        if (c0 + c < C && r0 + r + e < R) Y[(c0 + c) * ldy + r0 + r + e] = v[e];
    }
  }
}

bool transpose_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void*) {
  if (!in || !out || ni != 1 || no != 1) return false;
  const TensorDesc &X = in[0], &Y = out[0];
  if (X.rank != 2 || Y.rank != 2 || dt(X) != dt(Y)) return false;
  const DType d = dt(X);
  if (d != DType::kF32 && d != DType::kF16 && d != DType::kBF16 && d != DType::kI32) return false;
  if (Y.shape[0] != X.shape[1] || Y.shape[1] != X.shape[0]) return false;
  if (X.shape[0] <= 0 || X.shape[1] <= 0) return false;
  if (X.stride[1] != 1 || Y.stride[1] != 1 || X.stride[0] < X.shape[1] || Y.stride[0] < Y.shape[1])
    return false;
  return X.data != Y.data;
}

Status transpose_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* a, void*,
                        size_t, void* stream) {
  if (!transpose_sup(in, ni, out, no, a)) return Status::InvalidArgument;
  const int64_t R = in[0].shape[0], C = in[0].shape[1];
  if ((C + 63) / 64 > INT32_MAX || (R + 63) / 64 > 65535) return Status::InvalidArgument;
  dim3 grid((unsigned)((C + 63) / 64), (unsigned)((R + 63) / 64));
  hipStream_t s = as_stream(stream);
  if (dt(in[0]) == DType::kF32 || dt(in[0]) == DType::kI32)
    transpose_kernel<float><<<grid, 256, 0, s>>>((const float*)in[0].data, (float*)out[0].data, R, C,
                                                 in[0].stride[0], out[0].stride[0]);
  else
    transpose_kernel<uint16_t><<<grid, 256, 0, s>>>((const uint16_t*)in[0].data,
                                                    (uint16_t*)out[0].data, R, C, in[0].stride[0],
                                                    out[0].stride[0]);
  return launch_status("transpose2d_v0");
}

}  // namespace

KernelVariant make_add_f32_variant() { return make("add_f32", add_f32_launch, add_f32_sup); }
KernelVariant make_add_f16_variant() { return make("add_f16", add_f16_launch, add_f16_sup); }
KernelVariant make_add_f16_vec2_variant() {
  return make("add_f16_vec2", add_f16v2_launch, add_f16v2_sup);
}
KernelVariant make_relu_f32_variant() { return make("relu_f32", relu_f32_launch, relu_f32_sup); }
KernelVariant make_relu_f16_variant() { return make("relu_f16", relu_f16_launch, relu_f16_sup); }
KernelVariant make_relu_f16_vec2_variant() {
  return make("relu_f16_vec2", relu_f16v2_launch, relu_f16v2_sup);
}
KernelVariant make_relu_bwd_f32_variant() {
  return make("relu_bwd_f32", relu_bwd_f32_launch, relu_bwd_f32_sup);
}
KernelVariant make_relu_bwd_f16_variant() {
  return make("relu_bwd_f16", relu_bwd_f16_launch, relu_bwd_f16_sup);
}
KernelVariant make_relu_bwd_f16_vec2_variant() {
  return make("relu_bwd_f16_vec2", relu_bwd_f16v2_launch, relu_bwd_f16v2_sup);
}
KernelVariant make_bias_add_f32_variant() {
  return make("bias_add_f32", bias_add_f32_launch, bias_add_f32_sup);
}
KernelVariant make_bias_add_f16_variant() {
  return make("bias_add_f16", bias_add_f16_launch, bias_add_f16_sup);
}
KernelVariant make_bias_add_f16_vec2_variant() {
  return make("bias_add_f16_vec2", bias_add_f16v2_launch, bias_add_f16v2_sup);
}
KernelVariant make_copy_f32_variant() { return make("copy_f32", copy_f32_launch, copy_f32_sup); }
KernelVariant make_copy_f16_variant() { return make("copy_f16", copy_u16_launch, copy_f16_sup); }
KernelVariant make_copy_bf16_variant() { return make("copy_bf16", copy_u16_launch, copy_bf16_sup); }
KernelVariant make_grad_zero_variant() {
  return make("grad_zero_fill", grad_zero_launch, grad_zero_sup);
}
KernelVariant make_mse_grad_f32_variant() {
  return make("mse_grad_f32", mse_f32_launch, mse_f32_sup);
}
KernelVariant make_mse_grad_f16_variant() {
  return make("mse_grad_f16", mse_f16_launch, mse_f16_sup);
}
KernelVariant make_mse_loss_grad_variant() {
  return make("mse_loss_grad", mse_loss_launch, mse_loss_sup);
}
KernelVariant make_mse_colsum_variant() {
  return make("mse_colsum", mse_colsum_launch, mse_colsum_sup);
}
KernelVariant make_gelu_f32_variant() { return make("gelu_f32", gelu_f32_launch, gelu_f32_sup); }
KernelVariant make_gelu_bf16_variant() {
  return make("gelu_bf16", gelu_bf16_launch, gelu_bf16_sup);
}
KernelVariant make_gelu_bwd_f32_variant() {
  return make("gelu_bwd_f32", gelu_bwd_f32_launch, gelu_bwd_f32_sup);
}
KernelVariant make_gelu_bwd_bf16_variant() {
  return make("gelu_bwd_bf16", gelu_bwd_bf16_launch, gelu_bwd_bf16_sup);
}
KernelVariant make_transpose_variant() {
  return make("transpose2d_lds64", transpose_launch, transpose_sup);
}

}  // namespace aicf::hip

// ---------------------------------------------------------------------------
// MSE loss + gradient without allocation.  The partial sums of both passes
// live in `scratch`, a library-owned device array of kMseScratchParts floats
// (256 KiB, held on every GPU the library runs on until the process ends).
// In host code `scratch` names a host-side stand-in, not device memory: its
// device address is taken once per device with hipGetSymbolAddress, with
// that device current, and only that address is handed to the kernels.
// Calls on one GPU share the array: calls that overlap on one GPU (on
// different streams, unordered) race on it.  Nothing in it needs clearing:
// pass 1 writes every slot pass 2 reads.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[65536];

namespace {
constexpr int64_t kMseScratchParts = sizeof(scratch) / sizeof(float);
constexpr int64_t kMseNoallocMaxElems = kMseScratchParts * aicf::hip::kMseElemsPerBlock;  // 2^27
constexpr int kMaxDevices = 64;
static_assert(aicf::hip::kMseBlocks <= kMseScratchParts, "strided pass 1 needs kMseBlocks partials");

std::mutex g_scratch_mu;
float* g_scratch_dev[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the
// first call per device), or nullptr with the error recorded.
float* scratch_on_current_device() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    aicf::hip::set_last_error("hipGetDevice", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    aicf::hip::set_last_error("aicf_mse_loss_grad_noalloc", "device ordinal out of range");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      aicf::hip::set_last_error("hipGetSymbolAddress", e != hipSuccess ? hipGetErrorString(e) : "null address");
      return nullptr;
    }
    g_scratch_dev[dev] = static_cast<float*>(p);
  }
  return g_scratch_dev[dev];
}
}  // namespace

extern "C" int32_t aicf_mse_loss_grad_noalloc(const void* pred, const float* target, void* dpred,
                                              float* loss, int64_t n, int32_t dtype, float scale,
                                              void* stream) {
  using aicf::hip::aligned;
  const char* what = "aicf_mse_loss_grad_noalloc";
  if (!pred || !target || !dpred || !loss || n < 1) {
    aicf::hip::set_last_error(what, "null pointer or n < 1");
    return AICF_STATUS_INVALID_ARGUMENT;
  }
  if (dtype != AICF_DTYPE_F32 && dtype != AICF_DTYPE_BF16) {
    aicf::hip::set_last_error(what, "pred/dpred dtype must be AICF_DTYPE_F32 or AICF_DTYPE_BF16");
    return AICF_STATUS_INVALID_ARGUMENT;
  }
  if (n > kMseNoallocMaxElems) {
    aicf::hip::set_last_error(what, "n exceeds 134217728 elements, the maximum of the no-allocation "
                                    "entry point (its scratch holds 65536 partial sums)");
    return AICF_STATUS_INVALID_ARGUMENT;
  }
  const uintptr_t psz = dtype == AICF_DTYPE_F32 ? 16 : 8;
  if (!aligned(pred, psz) || !aligned(dpred, psz) || !aligned(target, 16) || !aligned(loss, 4)) {
    aicf::hip::set_last_error(what, "misaligned pointer (pred/dpred 16 B for f32, 8 B for bf16; "
                                    "target 16 B)");
    return AICF_STATUS_INVALID_ARGUMENT;
  }
  float* part = scratch_on_current_device();
  if (!part) return AICF_STATUS_INTERNAL;
  return static_cast<int32_t>(aicf::hip::mse_loss_run(pred, target, dpred, loss, part, kMseScratchParts, n,
                                                      dtype == AICF_DTYPE_BF16, scale,
                                                      aicf::hip::as_stream(stream)));
}
