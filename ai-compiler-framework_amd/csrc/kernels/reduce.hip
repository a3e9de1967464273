// Reductions for gfx950: column sum (bias gradient), row max / row sum,
// row softmax with fused row statistics, and fused softmax cross-entropy.
//
// Reference contracts:
//   reduce_sum  src/backends/cuda/ops/reduce_sum/launcher.cu:33-85 (attrs, shapes),
//               :244-304 (checks), :494-503 (direct API)
//   row max/sum, softmax, softmax-xent: no reference counterpart (appended
//   OpKinds RowReduce, RowSoftmax, SoftmaxXent).
//
// Row kernels keep a whole row in registers: a row is owned by LPR lanes
// (a fraction of a wave, one wave, or several waves of one workgroup), each
// holding VPT 16-byte vectors, so X is read from HBM exactly once and every
// output is written once.  Shapes that do not match a register-resident
// configuration use a looping kernel that reads the row twice.
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

// ===========================================================================
// Column sum: dY [M, N] (leading dims flattened) -> out [N].
// Vector kernel (N a multiple of the 16-byte vector): each lane owns 16
// bytes of columns, so a wave reads 1 KB of one row per load and keeps 4
// such loads in flight; scalar kernel otherwise (one column per lane).  The
// RS row-slices (waves) of a workgroup are combined in LDS in a fixed order.
// With a partials buffer [P, N] the rows are also split over P workgroup
// rows and a second pass adds the P partials in a fixed order.
// ===========================================================================
template <typename TI, bool BF16IN>
__device__ __forceinline__ float load_elem(const TI* p, int64_t i) {
  if constexpr (sizeof(TI) == 4) {
    return p[i];
  } else if constexpr (BF16IN) {
    return bf16_to_f32(p[i]);
  } else {
    return f16_to_f32(p[i]);
  }
}

constexpr int kColRS = 4;  // row slices (waves) per workgroup

template <typename TI, bool BF16IN, bool OUT_F16>
__global__ __launch_bounds__(256) void colsum_kernel(const TI* __restrict__ x, void* __restrict__ out,
                                                     float* __restrict__ partial, int64_t M,
                                                     int64_t N, int64_t rows_per_part) {
  __shared__ float red[kColRS][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * 64 + lane;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_part;
  const int64_t r1 = r0 + rows_per_part < M ? r0 + rows_per_part : M;
  float acc = 0.0f;
  if (col < N) {
    int64_t r = r0 + w;
    // 4 independent loads in flight per lane
    for (; r + 3 * kColRS < r1; r += 4 * kColRS) {
      const float a0 = load_elem<TI, BF16IN>(x, r * N + col);
      const float a1 = load_elem<TI, BF16IN>(x, (r + kColRS) * N + col);
      const float a2 = load_elem<TI, BF16IN>(x, (r + 2 * kColRS) * N + col);
      const float a3 = load_elem<TI, BF16IN>(x, (r + 3 * kColRS) * N + col);
      acc += (a0 + a1) + (a2 + a3);
    }
    for (; r < r1; r += kColRS) acc += load_elem<TI, BF16IN>(x, r * N + col);
  }
  red[w][lane] = acc;
  __syncthreads();
  if (w == 0 && col < N) {
    const float s = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
    if (partial) {
      partial[(int64_t)blockIdx.y * N + col] = s;
    } else if constexpr (OUT_F16) {
      ((uint16_t*)out)[col] = f32_to_f16(s);
    } else {
      ((float*)out)[col] = s;
    }
  }
}

template <typename TI, bool BF16IN>
__device__ __forceinline__ void add_vec16(float* acc, const uint4& v) {
  if constexpr (sizeof(TI) == 4) {
    acc[0] += __uint_as_float(v.x);
    acc[1] += __uint_as_float(v.y);
    acc[2] += __uint_as_float(v.z);
    acc[3] += __uint_as_float(v.w);
  } else {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t lo = (uint16_t)(w[k] & 0xffffu), hi = (uint16_t)(w[k] >> 16);
      acc[2 * k] += BF16IN ? bf16_to_f32(lo) : f16_to_f32(lo);
      acc[2 * k + 1] += BF16IN ? bf16_to_f32(hi) : f16_to_f32(hi);
    }
  }
}

template <typename TI, bool BF16IN, bool OUT_F16>
__global__ __launch_bounds__(256) void colsum_vec_kernel(const TI* __restrict__ x, void* __restrict__ out,
                                                         float* __restrict__ partial, int64_t M,
                                                         int64_t N, int64_t rows_per_part) {
  constexpr int VEC = 16 / sizeof(TI);
  constexpr int CB = 64 * VEC;  // columns per workgroup
  // rows in flight per lane: with the step's [64, N] partials (two
  // workgroups per CU at 8192 x 4096 bf16) 4 streams at 4.0 TB/s against
  // 3.8 for 8 and for 2
  constexpr int UNROLL = 4;
  __shared__ float red[kColRS][CB];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * CB + lane * VEC;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_part;
  const int64_t r1 = r0 + rows_per_part < M ? r0 + rows_per_part : M;
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
  if (c0 < N) {  // N % VEC == 0: the whole vector is in range
    int64_t r = r0 + w;
    for (; r + (UNROLL - 1) * kColRS < r1; r += UNROLL * kColRS) {
      uint4 v[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u)
        v[u] = *reinterpret_cast<const uint4*>(x + (r + u * kColRS) * N + c0);
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) add_vec16<TI, BF16IN>(acc, v[u]);
    }
    for (; r < r1; r += kColRS) add_vec16<TI, BF16IN>(acc, *reinterpret_cast<const uint4*>(x + r * N + c0));
  }
#pragma unroll
  for (int e = 0; e < VEC; ++e) red[w][lane * VEC + e] = acc[e];
  __syncthreads();
  for (int cc = threadIdx.x; cc < CB; cc += 256) {
    const int64_t col = (int64_t)blockIdx.x * CB + cc;
    if (col >= N) break;
    const float s = (red[0][cc] + red[1][cc]) + (red[2][cc] + red[3][cc]);
    if (partial) {
      partial[(int64_t)blockIdx.y * N + col] = s;
    } else if constexpr (OUT_F16) {
      ((uint16_t*)out)[col] = f32_to_f16(s);
    } else {
      ((float*)out)[col] = s;
    }
  }
}

// out[col] = sum over p of partial[p][col]: 64 columns per workgroup, the
// four waves take every fourth partial row, combined in LDS in fixed order.
__global__ __launch_bounds__(256) void colsum_finish_kernel(const float* __restrict__ partial,
                                                            float* __restrict__ out, int64_t P,
                                                            int64_t N) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * 64 + lane;
  float s = 0.0f;
  if (col < N) {
    int64_t p = w;
    for (; p + 12 < P; p += 16) {
      const float a0 = partial[p * N + col], a1 = partial[(p + 4) * N + col];
      const float a2 = partial[(p + 8) * N + col], a3 = partial[(p + 12) * N + col];
      s += (a0 + a1) + (a2 + a3);
    }
    for (; p < P; p += 4) s += partial[p * N + col];
  }
  red[w][lane] = s;
  __syncthreads();
  if (w == 0 && col < N) out[col] = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
}

// One-output column sum without a partials buffer (the reference's
// signature): every workgroup owns a narrow column block for all rows, so the
// grid has N / (kNarrowLanes * VEC) workgroups instead of N / (64 * VEC).  A
// row segment of the block is kNarrowLanes 16-byte vectors (32 bytes); the 256
// threads hold 256 / kNarrowLanes row slots, each summing rows slot, slot +
// 128, ... with 4 loads in flight, and the slots are added in LDS by a
// fixed-order tree (deterministic).  Consecutive column blocks, which share
// 128-byte lines, are given to workgroups on one XCD (workgroup i runs on
// XCD i % 8), so each line is fetched into one L2.  [8192, 4096] bf16: 16.6
// us (4 lanes, 8 loads, no remap: 25.6 us; 1 lane: 23.3 us).
constexpr int kNarrowLanes = 2;
constexpr int kNarrowSlots = 256 / kNarrowLanes;

template <typename TI, bool BF16IN, bool OUT_F16>
__global__ __launch_bounds__(256) void colsum_narrow_kernel(const TI* __restrict__ x, void* __restrict__ out,
                                                            int64_t M, int64_t N) {
  constexpr int VEC = 16 / sizeof(TI);
  constexpr int CB = kNarrowLanes * VEC;  // columns per workgroup
  constexpr int UNROLL = 4;
  __shared__ float red[kNarrowSlots][CB + 1];
  const int slot = (int)threadIdx.x / kNarrowLanes, v = (int)threadIdx.x % kNarrowLanes;
  int bid = blockIdx.x;  // column block: XCD-contiguous when the grid is a multiple of 8
  if ((gridDim.x & 7) == 0) bid = (bid & 7) * (gridDim.x >> 3) + (bid >> 3);
  const int64_t c0 = (int64_t)bid * CB + v * VEC;
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
  if (c0 < N) {  // N % VEC == 0: the whole vector is in range
    int64_t r = slot;
    for (; r + (UNROLL - 1) * kNarrowSlots < M; r += UNROLL * kNarrowSlots) {
      uint4 q[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u)
        q[u] = *reinterpret_cast<const uint4*>(x + (r + u * kNarrowSlots) * N + c0);
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) add_vec16<TI, BF16IN>(acc, q[u]);
    }
    for (; r < M; r += kNarrowSlots) add_vec16<TI, BF16IN>(acc, *reinterpret_cast<const uint4*>(x + r * N + c0));
  }
#pragma unroll
  for (int e = 0; e < VEC; ++e) red[slot][v * VEC + e] = acc[e];
  __syncthreads();
  for (int half = kNarrowSlots / 2; half > 0; half >>= 1) {  // slot i += slot i + half
    for (int t = (int)threadIdx.x; t < half * CB; t += 256) {
      const int i = t / CB, c = t % CB;
      red[i][c] += red[i + half][c];
    }
    __syncthreads();
  }
  if ((int)threadIdx.x < CB) {
    const int64_t col = (int64_t)bid * CB + threadIdx.x;
    if (col < N) {
      const float sum = red[0][threadIdx.x];
      if constexpr (OUT_F16)
        ((uint16_t*)out)[col] = f32_to_f16(sum);
      else
        ((float*)out)[col] = sum;
    }
  }
}

// RSUM axis attribute (reduce_sum/launcher.cu:75-85): default 0.
int64_t read_rsum_axis(const void* attr) {
  const AttrBlob& a = blob(attr);
  if (!attr) return 0;
  if (a.schema_id != 0 && a.schema_id != AICF_SCHEMA_RSUM) return 0;
  if (!payload_ok(a, 8)) return 0;
  return field<int64_t>(a, 0);
}

bool colsum_check(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr,
                  DType din, DType dout, bool allow_partials) {
  if (!in || !out || ni != 1) return false;
  if (!(no == 1 || (allow_partials && no == 2))) return false;
  const TensorDesc &X = in[0], &O = out[0];
  if (dt(X) != din || !X.contiguous || X.rank < 2) return false;
  if (read_rsum_axis(attr) != 0) return false;
  int64_t M, N;
  if (!rows_cols(X, &M, &N)) return false;
  if (!(dt(O) == dout && O.contiguous && O.rank == 1 && O.shape[0] == N)) return false;
  if (no == 2) {
    const TensorDesc& W = out[1];
    if (dt(W) != DType::kF32 || !W.contiguous || W.rank != 2 || W.shape[1] != N || W.shape[0] < 1)
      return false;
  }
  return true;
}

template <typename TI, bool BF16IN, bool OUT_F16>
Status colsum_run(const void* x, void* out, float* partial, int64_t P, int64_t M, int64_t N,
                  void* stream, const char* what) {
  hipStream_t s = as_stream(stream);
  constexpr int VEC = 16 / sizeof(TI);
  const bool vec = N % VEC == 0 && (uintptr_t)x % 16 == 0;
  const unsigned gx = (unsigned)(vec ? (N + 64 * VEC - 1) / (64 * VEC) : (N + 63) / 64);
  int64_t rpp = M, parts = 1;
  if (partial && P > 1 && M >= 2 * P) {
    rpp = (M + P - 1) / P;
    parts = (M + rpp - 1) / rpp;
  } else {
    partial = nullptr;
  }
  const int64_t gn = (N + kNarrowLanes * VEC - 1) / (kNarrowLanes * VEC);
  if (vec && !partial && gn <= INT32_MAX) {
    // one output, no partials: narrow column blocks over all rows (a
    // [8192, 4096] bf16 sum on 8 workgroups of 512 columns took 133 us)
    colsum_narrow_kernel<TI, BF16IN, OUT_F16><<<(unsigned)gn, 256, 0, s>>>((const TI*)x, out, M, N);
    return launch_status(what);
  }
  if (vec)
    colsum_vec_kernel<TI, BF16IN, OUT_F16><<<dim3(gx, (unsigned)parts), 256, 0, s>>>(
        (const TI*)x, out, partial, M, N, rpp);
  else
    colsum_kernel<TI, BF16IN, OUT_F16><<<dim3(gx, (unsigned)parts), 256, 0, s>>>(
        (const TI*)x, out, partial, M, N, rpp);
  if (partial)
    colsum_finish_kernel<<<(unsigned)((N + 63) / 64), 256, 0, s>>>(partial, (float*)out, parts, N);
  return launch_status(what);
}

#define COLSUM_VARIANT(NAME, DIN, DOUT, TI, BF16IN, OUTF16, PARTS)                                   \
  bool NAME##_sup(const TensorDesc* i, int ni, const TensorDesc* o, int no, const void* a) {        \
    return colsum_check(i, ni, o, no, a, DIN, DOUT, PARTS);                                          \
  }                                                                                                  \
  Status NAME##_launch(const TensorDesc* i, int ni, TensorDesc* o, int no, const void* a, void*,    \
                       size_t, void* s) {                                                            \
    if (!NAME##_sup(i, ni, o, no, a)) return Status::InvalidArgument;                               \
    int64_t M, N;                                                                                    \
    rows_cols(i[0], &M, &N);                                                                         \
    float* part = no == 2 ? (float*)o[1].data : nullptr;                                            \
    const int64_t P = no == 2 ? o[1].shape[0] : 1;                                                   \
    return colsum_run<TI, BF16IN, OUTF16>(i[0].data, o[0].data, part, P, M, N, s, #NAME);           \
  }

COLSUM_VARIANT(colsum_f32, DType::kF32, DType::kF32, float, false, false, true)
COLSUM_VARIANT(colsum_f16_f32, DType::kF16, DType::kF32, uint16_t, false, false, false)
COLSUM_VARIANT(colsum_f16_f16, DType::kF16, DType::kF16, uint16_t, false, true, false)
COLSUM_VARIANT(colsum_bf16_f32, DType::kBF16, DType::kF32, uint16_t, true, false, true)

// ===========================================================================
// Row kernels.
// MODE_SOFTMAX: outputs y = softmax(x) per row, optional rowmax, rowsum(x).
// MODE_SUM / MODE_MAX: one value per row.
// MODE_XENT: logits + labels -> dlogits, argmax, row loss.
// ===========================================================================
enum RowMode { MODE_SOFTMAX = 0, MODE_SUM = 1, MODE_MAX = 2, MODE_XENT = 3 };

struct RowArgs {
  const float* x;
  float* y;           // softmax / dlogits
  float* rmax;        // row max (softmax, max)
  float* rsum;        // row sum of x (softmax, sum)
  const int32_t* labels;
  int32_t* argmax;
  float* row_loss;
  int64_t R, C;
  float inv_batch;    // 1/B for xent gradients
};

// Combine (value, index) pairs: larger value wins, ties go to smaller index.
__device__ __forceinline__ void amax_combine(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// Reduce over the LPR lanes that own one row.  LPR <= 64: butterfly within
// the lane group.  LPR > 64: per-wave butterfly, then LDS across the
// LPR/64 waves of the row (all waves of a workgroup belong to one row).
template <int LPR>
struct RowReducer {
  static constexpr int NW = LPR > 64 ? LPR / 64 : 1;
  float* lds;  // NW floats
  __device__ float sum(float v) const {
#pragma unroll
    for (int off = (LPR < 64 ? LPR : 64) / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if constexpr (NW > 1) {
      const int w = threadIdx.x >> 6;
      __syncthreads();
      if ((threadIdx.x & 63) == 0) lds[w] = v;
      __syncthreads();
      v = 0.0f;
#pragma unroll
      for (int k = 0; k < NW; ++k) v += lds[k];
    }
    return v;
  }
  __device__ float max(float v) const {
#pragma unroll
    for (int off = (LPR < 64 ? LPR : 64) / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    if constexpr (NW > 1) {
      const int w = threadIdx.x >> 6;
      __syncthreads();
      if ((threadIdx.x & 63) == 0) lds[w] = v;
      __syncthreads();
      v = lds[0];
#pragma unroll
      for (int k = 1; k < NW; ++k) v = fmaxf(v, lds[k]);
    }
    return v;
  }
  __device__ void argmax(float& v, int& idx, int* ilds) const {
#pragma unroll
    for (int off = (LPR < 64 ? LPR : 64) / 2; off > 0; off >>= 1) {
      const float v2 = __shfl_xor(v, off, 64);
      const int i2 = __shfl_xor(idx, off, 64);
      amax_combine(v, idx, v2, i2);
    }
    if constexpr (NW > 1) {
      const int w = threadIdx.x >> 6;
      __syncthreads();
      if ((threadIdx.x & 63) == 0) {
        lds[w] = v;
        ilds[w] = idx;
      }
      __syncthreads();
      v = lds[0];
      idx = ilds[0];
#pragma unroll
      for (int k = 1; k < NW; ++k) amax_combine(v, idx, lds[k], ilds[k]);
    }
  }
};

// Statistics of a row segment, combined in one reduction round:
//   m  maximum (and i, the first column holding it, for cross-entropy),
//   s  sum of exp(x - m) over the segment (rescaled when segments merge),
//   sx sum of x; for cross-entropy, z[label] (held by the one lane that owns
//      the label's column, zero elsewhere, so the sum is exact).
// Merging is symmetric in its two arguments (max, tie-aware argmax, and
// sums), so every lane of a butterfly ends with bit-identical statistics.
struct RowStat {
  float m, s, sx;
  int i;
};
template <int MODE>
__device__ __forceinline__ void stat_merge(RowStat& a, const RowStat& b) {
  if constexpr (MODE == MODE_SUM) {
    a.sx += b.sx;
  } else if constexpr (MODE == MODE_MAX) {
    a.m = fmaxf(a.m, b.m);
  } else {
    const float M = fmaxf(a.m, b.m);
    const float x = a.m == M ? a.s : a.s * __expf(a.m - M);  // exact when this side holds the max
    const float y = b.m == M ? b.s : b.s * __expf(b.m - M);
    if constexpr (MODE == MODE_XENT) {
      if (b.m > a.m || (b.m == a.m && b.i < a.i)) a.i = b.i;
    }
    a.sx += b.sx;
    a.m = M;
    a.s = x + y;
  }
}
template <int MODE>
__device__ __forceinline__ RowStat stat_shfl(const RowStat& v, int off) {
  RowStat r;
  r.m = __shfl_xor(v.m, off, 64);
  r.s = __shfl_xor(v.s, off, 64);
  r.sx = __shfl_xor(v.sx, off, 64);
  r.i = MODE == MODE_XENT ? __shfl_xor(v.i, off, 64) : 0;
  return r;
}

// Register-resident row kernel: row = LPR lanes x VPT float4.  Element j of
// lane l, vector k sits at column (k * LPR + l) * 4 + j, so every vector load
// of a lane group is one contiguous, coalesced segment.  Each lane reduces
// its own values (exp taken against its own maximum), the lanes of a row
// merge their statistics by butterfly, and the waves of a row (LPR > 64)
// merge through LDS after one barrier, in a fixed order.  The outputs
// then scale each lane's exponentials by exp(m_lane - M) / S.  A row whose
// values are all equal gets exactly 1/C when C is a power of two (every
// exponential and scale factor is then exactly 1 and S = C).
template <int LPR, int VPT, int MODE>
__global__ __launch_bounds__(LPR >= 256 ? LPR : 256) void row_reg_kernel(RowArgs a) {
  constexpr int THREADS = LPR >= 256 ? LPR : 256;
  constexpr int RPB = THREADS / LPR;            // rows per workgroup
  constexpr int NW = LPR > 64 ? LPR / 64 : 1;   // waves per row
  constexpr int TW = THREADS / 64;              // waves per workgroup
  constexpr int BF = LPR < 64 ? LPR : 64;       // butterfly width
  __shared__ float lds_m[TW], lds_s[TW], lds_sx[TW];
  __shared__ int lds_i[TW];
  const int sub = (int)threadIdx.x / LPR;
  const int l = (int)threadIdx.x % LPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + sub;
  const bool active = row < a.R;  // uniform across the lanes of a row
  const int64_t C = a.C;
  const f32x4* xr = reinterpret_cast<const f32x4*>(a.x + (active ? row : 0) * C);
  // cross-entropy: the label is read first, so its latency hides behind the row loads
  const int lab = (MODE == MODE_XENT && active) ? a.labels[row] : -1;

  // an inactive row (past R, uniform across its lanes) reads row 0 and
  // stores nothing: the loads need no predicate
  f32x4 v[VPT];
#pragma unroll
  for (int k = 0; k < VPT; ++k) v[k] = __builtin_nontemporal_load(xr + k * LPR + l);

  // this lane's statistics
  RowStat st{v[0][0], 0.0f, 0.0f, l * 4};
  if constexpr (MODE == MODE_SUM || MODE == MODE_SOFTMAX) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) st.sx += (v[k][0] + v[k][1]) + (v[k][2] + v[k][3]);
  }
  // cross-entropy: the label's logit sits in lane lab_l, vector lab_k,
  // element lab & 3 (no lane for a label outside [0, C))
  const int lab_q = lab >> 2;
  const bool lab_here = MODE == MODE_XENT && lab >= 0 && lab_q % LPR == l;
  const int lab_k = lab_q / LPR, lab_j = lab & 3;
  if constexpr (MODE == MODE_XENT) {
    // the lane's maximum, then the first column holding it (for finite
    // values the result of a running strict-greater scan), then the
    // label's logit by a uniform pick instead of a compare per element
    float m = v[0][0];
#pragma unroll
    for (int k = 0; k < VPT; ++k) m = fmaxf(m, fmaxf(fmaxf(v[k][0], v[k][1]), fmaxf(v[k][2], v[k][3])));
    int idx = l * 4;
#pragma unroll
    for (int k = VPT - 1; k >= 0; --k)
#pragma unroll
      for (int j = 3; j >= 0; --j) idx = v[k][j] == m ? (k * LPR + l) * 4 + j : idx;
    float zl = 0.0f;
#pragma unroll
    for (int k = 0; k < VPT; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) zl = (lab_here && k == lab_k && j == lab_j) ? v[k][j] : zl;
    st.m = m;
    st.i = idx;
    st.sx = zl;
  } else if constexpr (MODE != MODE_SUM) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) st.m = fmaxf(st.m, fmaxf(fmaxf(v[k][0], v[k][1]), fmaxf(v[k][2], v[k][3])));
  }
  const float m_lane = st.m;
  if constexpr (MODE == MODE_SOFTMAX || MODE == MODE_XENT) {
    const float mref = m_lane == -INFINITY ? 0.0f : m_lane;  // an all -inf lane contributes 0
#pragma unroll
    for (int k = 0; k < VPT; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e = __expf(v[k][j] - mref);
        v[k][j] = e;
        st.s += e;
      }
  }

  // merge over the row
#pragma unroll
  for (int off = BF / 2; off > 0; off >>= 1) stat_merge<MODE>(st, stat_shfl<MODE>(st, off));
  if constexpr (NW > 1) {
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
      lds_m[w] = st.m;
      lds_s[w] = st.s;
      lds_sx[w] = st.sx;
      lds_i[w] = st.i;
    }
    __syncthreads();
    const int w0 = sub * NW;
    st = RowStat{lds_m[w0], lds_s[w0], lds_sx[w0], lds_i[w0]};
#pragma unroll
    for (int k = 1; k < NW; ++k)
      stat_merge<MODE>(st, RowStat{lds_m[w0 + k], lds_s[w0 + k], lds_sx[w0 + k], lds_i[w0 + k]});
  }
  if (!active) return;

  if constexpr (MODE == MODE_SUM) {
    if (l == 0) a.rsum[row] = st.sx;
    return;
  }
  if constexpr (MODE == MODE_MAX) {
    if (l == 0) a.rmax[row] = st.m;
    return;
  }
  const float c = (m_lane == st.m ? 1.0f : __expf(m_lane - st.m)) / st.s;
  f32x4* yr = reinterpret_cast<f32x4*>(a.y + row * C);
  if constexpr (MODE == MODE_SOFTMAX) {
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      f32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = v[k][j] * c;
      __builtin_nontemporal_store(o, yr + k * LPR + l);
    }
    if (l == 0) {
      if (a.rmax) a.rmax[row] = st.m;
      if (a.rsum) a.rsum[row] = st.sx;
    }
  } else {  // MODE_XENT
    const bool valid = lab >= 0 && (int64_t)lab < C;
    const float sc = a.inv_batch;
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
      f32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j)  // (p - onehot) / B
        o[j] = (v[k][j] * c - ((lab_here && k == lab_k && j == lab_j) ? 1.0f : 0.0f)) * sc;
      __builtin_nontemporal_store(o, yr + k * LPR + l);
    }
    if (l == 0) {
      a.argmax[row] = st.i;
      // loss_i = (m - z[label]) + log(sum exp(z - m)): m - z[label] is exact
      // for close values and >= 0, so nothing cancels after the rounding of
      // log (added first, a row of -1e4 lost ~1e-3 of log(C))
      a.row_loss[row] = valid ? ((st.m - st.sx) + logf(st.s)) : __builtin_nanf("");
    }
  }
}

// Looping row kernel for any C (one workgroup of 256 lanes per row).
// Pass 1 computes max (and argmax / sum), pass 2 the exp-sum, pass 3 writes.
template <int MODE>
__global__ __launch_bounds__(256) void row_loop_kernel(RowArgs a) {
  __shared__ float lds[4];
  __shared__ int ilds[4];
  const RowReducer<256> rr{lds};
  const int64_t row = blockIdx.x;
  const int64_t C = a.C;
  const float* xr = a.x + row * C;
  const int t = threadIdx.x;

  if constexpr (MODE == MODE_SUM) {
    float s = 0.0f;
    for (int64_t c = t; c < C; c += 256) s += xr[c];
    s = rr.sum(s);
    if (t == 0) a.rsum[row] = s;
    return;
  }
  float mx = -INFINITY;
  int bi = INT32_MAX;
  float sx = 0.0f;
  for (int64_t c = t; c < C; c += 256) {
    const float x = xr[c];
    if (MODE == MODE_SOFTMAX) sx += x;
    if (MODE == MODE_XENT) {
      if (x > mx || bi == INT32_MAX) {
        mx = x;
        bi = (int)c;
      }
    } else {
      mx = fmaxf(mx, x);
    }
  }
  if constexpr (MODE == MODE_XENT) {
    if (bi == INT32_MAX) mx = -INFINITY;
    rr.argmax(mx, bi, ilds);
  } else {
    mx = rr.max(mx);
  }
  if constexpr (MODE == MODE_MAX) {
    if (t == 0) a.rmax[row] = mx;
    return;
  }
  float se = 0.0f;
  for (int64_t c = t; c < C; c += 256) se += __expf(xr[c] - mx);
  se = rr.sum(se);
  if constexpr (MODE == MODE_SOFTMAX) {
    if (a.rsum) sx = rr.sum(sx);
  }
  const float inv = 1.0f / se;
  float* yr = a.y + row * C;
  if constexpr (MODE == MODE_SOFTMAX) {
    for (int64_t c = t; c < C; c += 256) yr[c] = __expf(xr[c] - mx) * inv;
    if (t == 0) {
      if (a.rmax) a.rmax[row] = mx;
      if (a.rsum) a.rsum[row] = sx;
    }
  } else {
    const int lab = a.labels[row];
    const bool valid = lab >= 0 && (int64_t)lab < C;
    for (int64_t c = t; c < C; c += 256)
      yr[c] = (__expf(xr[c] - mx) * inv - (c == lab ? 1.0f : 0.0f)) * a.inv_batch;
    if (t == 0) {
      a.argmax[row] = bi;
      a.row_loss[row] = valid ? ((mx - xr[lab]) + logf(se)) : __builtin_nanf("");
    }
  }
}

// Mean of the per-row losses in a fixed order (one workgroup, fp64 accumulate).
__global__ __launch_bounds__(256) void mean_kernel(const float* __restrict__ v, int64_t n,
                                                   float* __restrict__ out) {
  __shared__ double red[4];
  block_mean_f64(v, n, out, red);
}

// Picks a register-resident configuration when C is one of the row widths
// it covers, else the looping kernel.
template <int MODE>
Status launch_rows(const RowArgs& a, void* stream) {
  hipStream_t s = as_stream(stream);
  const int64_t R = a.R, C = a.C;
  const bool al = aligned(a.x, 16) && (a.y == nullptr || aligned(a.y, 16));
#define ROW_CASE(LPR, VPT)                                                                  \
  if (al && C == (int64_t)(LPR) * (VPT) * 4) {                                               \
    constexpr int RPB = (LPR) >= 256 ? 1 : 256 / (LPR);                                       \
    constexpr int THREADS = (LPR) >= 256 ? (LPR) : 256;                                       \
    static_assert(THREADS <= 1024, "row too wide");                                          \
    row_reg_kernel<LPR, VPT, MODE><<<(unsigned)((R + RPB - 1) / RPB), THREADS, 0, s>>>(a);  \
    return launch_status("row_kernel");                                                      \
  }
  if constexpr (MODE == MODE_SOFTMAX) {
    // C = 8192 softmax: one wave per row, 64 lanes x 32 vectors (6.06 ->
    // 6.11 TB/s against 128 x 16, three alternated rounds; cross-entropy,
    // with more registers live per element, drops to 5.3 TB/s this way and
    // keeps 128 x 16)
    ROW_CASE(64, 32)
  }
  if constexpr (MODE == MODE_SOFTMAX || MODE == MODE_XENT) {
    // C = 8192 with a row output: 128 lanes x 16 vectors (softmax 5.98 ->
    // 6.09 TB/s, xent 5.47 -> 5.73; the row statistics are merged over 128
    // lanes instead of 512, an fp32 reassociation); the read-only row sum
    // and max keep 512 x 4
    ROW_CASE(128, 16)
  }
  ROW_CASE(16, 1)     // C = 64
  ROW_CASE(16, 2)     // C = 128
  ROW_CASE(32, 2)     // C = 256
  ROW_CASE(64, 2)     // C = 512
  ROW_CASE(128, 2)    // C = 1024
  ROW_CASE(128, 4)    // C = 2048
  ROW_CASE(256, 4)    // C = 4096
  ROW_CASE(512, 4)    // C = 8192 (row sum, row max)
  ROW_CASE(512, 8)    // C = 16384
  ROW_CASE(512, 16)   // C = 32768
#undef ROW_CASE
  row_loop_kernel<MODE><<<(unsigned)R, 256, 0, s>>>(a);
  return launch_status("row_loop_kernel");
}

bool rows_f32(const TensorDesc& X, int64_t* R, int64_t* C) {
  if (dt(X) != DType::kF32 || !X.contiguous) return false;
  if (X.rank == 1) {
    *R = 1;
    *C = X.shape[0];
    return *C > 0;
  }
  return rows_cols(X, R, C);
}
bool vec_f32(const TensorDesc& t, int64_t n) {
  return dt(t) == DType::kF32 && t.contiguous && numel_of(t) == n && t.rank >= 1;
}

// ---- RowSoftmax: X -> Y [, rowmax [, rowsum]] -----------------------------
bool softmax_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void*) {
  if (!in || !out || ni != 1 || no < 1 || no > 3) return false;
  int64_t R, C;
  if (!rows_f32(in[0], &R, &C)) return false;
  if (dt(out[0]) != DType::kF32 || !out[0].contiguous || !same_shape(in[0], out[0])) return false;
  for (int k = 1; k < no; ++k)
    if (!vec_f32(out[k], R)) return false;
  return true;
}
Status softmax_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* at, void*,
                      size_t, void* s) {
  if (!softmax_sup(in, ni, out, no, at)) return Status::InvalidArgument;
  RowArgs a{};
  rows_f32(in[0], &a.R, &a.C);
  a.x = (const float*)in[0].data;
  a.y = (float*)out[0].data;
  a.rmax = no >= 2 ? (float*)out[1].data : nullptr;
  a.rsum = no >= 3 ? (float*)out[2].data : nullptr;
  return launch_rows<MODE_SOFTMAX>(a, s);
}

// ---- RowReduce: X -> out[R], schema RRED <i> (0 = sum, 1 = max) ------------
int read_rred(const void* attr) {
  const AttrBlob& a = blob(attr);
  if (a.schema_id != AICF_SCHEMA_RRED || !payload_ok(a, 4)) return 0;
  return field<int32_t>(a, 0);
}
bool row_reduce_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr) {
  if (!in || !out || ni != 1 || no != 1) return false;
  const int op = read_rred(attr);
  if (op != 0 && op != 1) return false;
  int64_t R, C;
  return rows_f32(in[0], &R, &C) && vec_f32(out[0], R);
}
Status row_reduce_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* at,
                         void*, size_t, void* s) {
  if (!row_reduce_sup(in, ni, out, no, at)) return Status::InvalidArgument;
  RowArgs a{};
  rows_f32(in[0], &a.R, &a.C);
  a.x = (const float*)in[0].data;
  if (read_rred(at) == 0) {
    a.rsum = (float*)out[0].data;
    return launch_rows<MODE_SUM>(a, s);
  }
  a.rmax = (float*)out[0].data;
  return launch_rows<MODE_MAX>(a, s);
}

// ---- SoftmaxXent: (logits [B,C] f32, labels [B] i32) ->
//      (loss f32 scalar, dlogits [B,C] f32, argmax [B] i32, row_loss [B] f32)
bool xent_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void*) {
  if (!in || !out || ni != 2 || no != 4) return false;
  int64_t B, C;
  if (!rows_f32(in[0], &B, &C) || in[0].rank != 2) return false;
  const TensorDesc& L = in[1];
  if (dt(L) != DType::kI32 || !L.contiguous || L.rank != 1 || L.shape[0] != B) return false;
  if (dt(out[0]) != DType::kF32 || numel_of(out[0]) != 1) return false;
  if (dt(out[1]) != DType::kF32 || !out[1].contiguous || !same_shape(out[1], in[0])) return false;
  const TensorDesc& A = out[2];
  if (dt(A) != DType::kI32 || !A.contiguous || numel_of(A) != B) return false;
  if (C > INT32_MAX) return false;
  return vec_f32(out[3], B);
}
Status xent_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* at, void*,
                   size_t, void* s) {
  if (!xent_sup(in, ni, out, no, at)) return Status::InvalidArgument;
  RowArgs a{};
  rows_f32(in[0], &a.R, &a.C);
  a.x = (const float*)in[0].data;
  a.labels = (const int32_t*)in[1].data;
  a.y = (float*)out[1].data;
  a.argmax = (int32_t*)out[2].data;
  a.row_loss = (float*)out[3].data;
  a.inv_batch = 1.0f / (float)a.R;
  Status st = launch_rows<MODE_XENT>(a, s);
  if (st != Status::Ok) return st;
  mean_kernel<<<1, 256, 0, as_stream(s)>>>(a.row_loss, a.R, (float*)out[0].data);
  return launch_status("softmax_xent_mean");
}

}  // namespace

Status colsum_finish(const float* partial, float* out, int64_t P, int64_t N, void* stream) {
  if (P < 1 || N < 1) return Status::InvalidArgument;
  colsum_finish_kernel<<<(unsigned)((N + 63) / 64), 256, 0, as_stream(stream)>>>(partial, out, P, N);
  return launch_status("colsum_finish");
}

// Direct C++ API counterpart of reduce_sum/api.hpp:6.
Status reduce_sum_lastdim_f32(const float* dY, float* dB, int M, int N, void* stream) {
  if (!dY || !dB || M <= 0 || N <= 0) return Status::InvalidArgument;
  return colsum_run<float, false, false>(dY, dB, nullptr, 1, M, N, stream,
                                         "reduce_sum_lastdim_f32");
}

KernelVariant make_reduce_sum_lastdim_f32_variant() {
  return make("reduce_sum_cols_f32", colsum_f32_launch, colsum_f32_sup);
}
KernelVariant make_reduce_sum_lastdim_f16_to_f32_variant() {
  return make("reduce_sum_cols_f16_f32", colsum_f16_f32_launch, colsum_f16_f32_sup);
}
KernelVariant make_reduce_sum_lastdim_f16_variant() {
  return make("reduce_sum_cols_f16", colsum_f16_f16_launch, colsum_f16_f16_sup);
}
KernelVariant make_reduce_sum_lastdim_bf16_to_f32_variant() {
  return make("reduce_sum_cols_bf16_f32", colsum_bf16_f32_launch, colsum_bf16_f32_sup);
}
KernelVariant make_row_softmax_f32_variant() {
  return make("row_softmax_f32", softmax_launch, softmax_sup);
}
KernelVariant make_row_reduce_f32_variant() {
  return make("row_reduce_f32", row_reduce_launch, row_reduce_sup);
}
KernelVariant make_softmax_xent_f32_variant() {
  return make("softmax_xent_f32", xent_launch, xent_sup);
}

}  // namespace aicf::hip

extern "C" int32_t aicf_reduce_sum_lastdim_f32(const float* dY, float* dB, int32_t M, int32_t N,
                                               void* stream) {
  return static_cast<int32_t>(aicf::hip::reduce_sum_lastdim_f32(dY, dB, M, N, stream));
}
