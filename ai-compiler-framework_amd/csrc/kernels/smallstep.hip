// Kernels for train steps whose tensors are too small for one launch per op
// to fill the GPU (the reference's own MLP: batch 64, 784 -> 256 -> 10).
// There every launch is a few microseconds of dispatch around well under a
// microsecond of work, so the step is built from few launches that each do
// several ops' work:
//
//  * small fp32 GEMM (also taken by the GEMM dispatcher for problems with
//    few tiles): one 16 x 16 output tile per wave, read straight from global
//    memory in whatever layout the operands have, v_mfma_f32_16x16x4f32, the
//    waves of a workgroup splitting K and summing through LDS in a fixed
//    order;
//  * xent_head: the classifier head of a ReLU MLP, forward and backward, one
//    wave per row: logits = H W^T + b, softmax cross-entropy (dlogits,
//    argmax, row loss), dH = dlogits W, dX = dH where the saved ReLU output
//    is positive;
//  * grad_group: independent small jobs in one launch: gradient GEMMs,
//    column sums (bias gradients), the fixed-order loss mean, the step
//    counter;
//  * adamw_multi: AdamW over several parameter tensors in one launch, with
//    the element update and bias corrections of adamw_step (same bits).
//
// Reference contracts restated: the gradient GEMMs and column sums of
// LinearBwd (python/aicf_fw/core_v2/lower.py:94-110), relu_bwd
// (src/backends/cuda/ops/relu_bwd/launcher.cu:37-77), reduce_sum over axis 0
// (reduce_sum/launcher.cu:140-155), step_inc (step_inc/launcher.cu:34-38).
// The fused ops themselves have no reference counterpart; they play the
// role of the reference's epilogue fusion (rewrites/stageC_fuse_epilogue.py)
// for a step whose cost is launches rather than bytes or flops.
#include "../common/adamw.hpp"
#include "../common/hip_util.hpp"
#include "../common/host_util.hpp"
#include "../common/smallstep.hpp"

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
// Small GEMM
// ===========================================================================
constexpr int kNB = 8;  // K blocks (16 K each) whose loads a wave issues before its MFMAs

struct SgJob {
  SmallGemm g;
  int tn;          // tiles along N
  int tiles;       // tiles along M times tn
  int kb;          // 16-K blocks
  int splits;      // waves per tile (K split): 1, 2, 4 or 8
  int tpb;         // tiles per workgroup: waves / splits
  int avec, bvec;  // 16-byte loads along K (K-contiguous, aligned operand)
  int a_bytes, b_bytes;  // byte ranges of A and B read through buffer loads (< 2^31)
};

// Elements k .. k + 3 of row `row` of an operand (zero past K or for a lane
// without a row), as buffer loads: a lane with nothing to read passes an
// offset past the buffer's range and the load returns zeros.  No branch and
// no select after the load: the compiler would wait for each load before the
// next one (a divergent branch around the loads, or a select of their
// results), one round trip per load instead of one per batch.
constexpr int kOutOfRange = (int)0x80000000u;  // past every buffer's range (< 2^31 bytes)
template <bool VEC>
__device__ __forceinline__ f32x4 sg_load(__amdgpu_buffer_rsrc_t rs, int64_t row, int64_t sm, int64_t sk, int64_t k,
                                         int64_t K, bool ok) {
  if constexpr (VEC) {  // K % 4 == 0: the four are in range together
    const int off = ok && k < K ? (int)((row * sm + k) * 4) : kOutOfRange;
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
  } else {
    f32x4 v;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int off = ok && k + c < K ? (int)((row * sm + (k + c) * sk) * 4) : kOutOfRange;
      v[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
    }
    return v;
  }
}

// One 16 x 16 tile over the K blocks split, split + splits, ...  Lane
// l = 16 q + r reads row m0 + r of A and column n0 + r of B; for K block kb
// it holds k = 16 kb + 4 q + c (c = 0..3) and feeds component c to the c-th
// MFMA of the block, so k slot q of that MFMA carries the same k for A and
// B.  Accumulator element i is C[m0 + 4 q + i][n0 + r].
// The K-block loop and m0, n0, split are wave-uniform, so only the row and
// K-range tests of sg_load differ between lanes.
template <bool AV, bool BV>
__device__ __forceinline__ f32x4 sg_tile(const SgJob& j, int64_t m0, int64_t n0, int split, int lane) {
  const int r = lane & 15, q = lane >> 4;
  const int64_t m = m0 + r, n = n0 + r;
  const bool mok = m < j.g.M, nok = n < j.g.N;
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)j.g.A, 0, j.a_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)j.g.B, 0, j.b_bytes, 0x00020000);
  // every row of tiles reads all of B: the copy of B is shared out, the
  // wave of row of tiles mt writing the u-th K block it reads when u % MT
  // == mt (MT rows of tiles)
  const bool snap = j.g.bcopy != nullptr && nok;
  float* bc = snap ? j.g.bcopy + n * j.g.b_n : nullptr;
  const int MT = (int)((j.g.M + 15) / 16), mt = (int)(m0 / 16);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int kb0 = split, ub = 0; kb0 < j.kb; kb0 += j.splits * kNB, ub += kNB) {
    f32x4 a[kNB], b[kNB];
#pragma unroll
    for (int u = 0; u < kNB; ++u) {
      const int kb = kb0 + u * j.splits;
      if (kb >= j.kb) break;  // uniform across the wave
      const int64_t k = (int64_t)kb * 16 + 4 * q;
      a[u] = sg_load<AV>(ra, m, j.g.a_m, j.g.a_k, k, j.g.K, mok);
      b[u] = sg_load<BV>(rb, n, j.g.b_n, j.g.b_k, k, j.g.K, nok);
    }
#pragma unroll
    for (int u = 0; u < kNB; ++u) {
      if (kb0 + u * j.splits >= j.kb) break;  // uniform across the wave
#pragma unroll
      for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u][c], b[u][c], acc, 0, 0, 0);
      if (snap && (ub + u) % MT == mt) {  // K % 4 == 0 (16-byte loads of B): the four are in range together
        const int64_t k = (int64_t)(kb0 + u * j.splits) * 16 + 4 * q;
        if (k < j.g.K) *reinterpret_cast<f32x4*>(bc + k) = b[u];
      }
    }
  }
  return acc;
}

// AdamW applied where a gradient is stored: P, M, V laid out like the stored
// gradient (element index of the output), updated in place with adamw_step's
// element update (csrc/common/adamw.hpp) and the step's bias corrections
// {lr / bc1, 1 / bc2} as adamw_step derives them, computed once per step by
// an earlier launch (the head that advances the step counter), so the bits
// are adamw_step's.  A lane loads its P, M, V elements before its tile's K
// loop.  The routines take the update by value under a compile-time flag: a
// pointer that may be null would keep the struct in scratch memory.
struct StoreAdamW {
  float* P;
  float* M;
  float* V;
  const float* scal;  // {lr / bc1, 1 / bc2} of this step
  AdamWArgs a;
};
struct AdamWLane {
  float p[4], m[4], v[4];
  AdamWScalars s;
};
__device__ __forceinline__ void adamw_load(const StoreAdamW& ad, int64_t i, int x, AdamWLane& r) {
  r.p[x] = ad.P[i];
  r.m[x] = ad.M[i];
  r.v[x] = ad.V[i];
}
__device__ __forceinline__ void adamw_store(const StoreAdamW& ad, int64_t i, int x, float g, AdamWLane& r) {
  adamw_elem(r.p[x], g, r.m[x], r.v[x], r.s, ad.a);
  ad.P[i] = r.p[x];
  ad.M[i] = r.m[x];
  ad.V[i] = r.v[x];
}

// The elements sg_store writes for this lane: C[m0 + 4 q + i][n0 + r]
// (branch-free, as sg_load; element 0 stands in for those outside C).
__device__ __forceinline__ void sg_adamw_prefetch(const SmallGemm& g, int64_t m0, int64_t n0, int lane,
                                                  const StoreAdamW& ad, AdamWLane& r) {
  const int rr = lane & 15, q = lane >> 4;
  const int64_t n = n0 + rr;
  r.s = AdamWScalars{ad.scal[0], ad.scal[1]};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + 4 * q + i;
    adamw_load(ad, (n < g.N && m < g.M) ? m * g.c_m + n : 0, i, r);
  }
}

// bv: the bias of column n0 + r, loaded before the tile's K loop.
template <bool ADAM>
__device__ __forceinline__ void sg_store(const SmallGemm& g, int64_t m0, int64_t n0, int lane, f32x4 acc, float bv,
                                         const StoreAdamW& ad, AdamWLane& ar) {
  const int r = lane & 15, q = lane >> 4;
  const int64_t n = n0 + r;
  if (n >= g.N) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + 4 * q + i;
    if (m >= g.M) break;
    float v = g.bias ? acc[i] + bv : acc[i];
    if (g.relu) v = v > 0.0f ? v : 0.0f;
    g.C[m * g.c_m + n] = v;
    if constexpr (ADAM) adamw_store(ad, m * g.c_m + n, i, v, ar);
  }
}

// Workgroup `blk` of a small GEMM: its waves = tpb tiles x splits K parts.
// The parts of a tile are summed in split order (part 0 + 1 + 2 + ...).
// `red` is 64 f32x4 of LDS per wave.  Every thread reaches the barrier.
// ADAM: apply AdamW to the parameter whose gradient the output is (the
// output is row-major contiguous, so its element index is the parameter's).
template <bool ADAM>
__device__ __forceinline__ void sg_block(const SgJob& j, int blk, f32x4* red, const StoreAdamW& ad) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int tile = blk * j.tpb + w / j.splits;
  const int split = w % j.splits;
  const bool live = tile < j.tiles;
  const int64_t m0 = live ? (int64_t)(tile / j.tn) * 16 : 0;
  const int64_t n0 = live ? (int64_t)(tile % j.tn) * 16 : 0;
  AdamWLane ar;
  const bool upd = ADAM && live && split == 0;
  if (upd) sg_adamw_prefetch(j.g, m0, n0, lane, ad, ar);
  float bv = 0.0f;
  if (j.g.bias && live && split == 0) {  // wave-uniform: no divergent branch around the load
    const int64_t n = n0 + (lane & 15);
    bv = j.g.bias[(n < j.g.N ? n : 0) * j.g.bias_s];
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (live) {
    if (j.avec)
      acc = j.bvec ? sg_tile<true, true>(j, m0, n0, split, lane) : sg_tile<true, false>(j, m0, n0, split, lane);
    else
      acc = j.bvec ? sg_tile<false, true>(j, m0, n0, split, lane) : sg_tile<false, false>(j, m0, n0, split, lane);
  }
  if (j.splits > 1) {
    red[w * 64 + lane] = acc;
    __syncthreads();
    if (!live || split != 0) return;
    for (int s = 1; s < j.splits; ++s) acc += red[(w + s) * 64 + lane];
  } else if (!live) {
    return;
  }
  sg_store<ADAM>(j.g, m0, n0, lane, acc, bv, ad, ar);
}

template <int NWAVE>
__global__ __launch_bounds__(64 * NWAVE) void gemm_small_kernel(SgJob j) {
  __shared__ f32x4 red[64 * NWAVE];
  sg_block<false>(j, blockIdx.x, red, StoreAdamW{});
}

// Bytes from an operand's first element to the end of its last one (rows x
// K with row stride sr and K stride sk, in floats).
int64_t sg_range_bytes(int64_t rows, int64_t sr, int64_t K, int64_t sk) {
  return ((rows - 1) * sr + (K - 1) * sk + 1) * 4;
}

// nwave 4, or 8 / 16 for the standalone kernel when K is long enough for 8
// splits (32 or more K blocks) / 16 splits (48 or more): each wave then has
// at most 8 blocks, one batch of loads in flight, and with 16 waves at most
// 4 (64 x 784 x 256, the MLP's first layer: 0.1 us less per launch).
SgJob sg_plan(const SmallGemm& g, int nwave = 4) {
  SgJob j{};
  j.g = g;
  j.tn = (int)((g.N + 15) / 16);
  j.tiles = (int)((g.M + 15) / 16) * j.tn;
  j.kb = (int)((g.K + 15) / 16);
  j.splits = (nwave == 16 && j.kb >= 48) ? 16 : (nwave >= 8 && j.kb >= 32) ? 8 : j.kb >= 16 ? 4 : j.kb >= 8 ? 2 : 1;
  j.tpb = nwave / j.splits;
  j.avec = g.a_k == 1 && g.K % 4 == 0 && (g.M == 1 || g.a_m % 4 == 0) && aligned(g.A, 16);
  j.bvec = g.b_k == 1 && g.K % 4 == 0 && (g.N == 1 || g.b_n % 4 == 0) && aligned(g.B, 16);
  j.a_bytes = (int)sg_range_bytes(g.M, g.a_m, g.K, g.a_k);
  j.b_bytes = (int)sg_range_bytes(g.N, g.b_n, g.K, g.b_k);
  return j;
}
int sg_blocks(const SgJob& j) { return (j.tiles + j.tpb - 1) / j.tpb; }

// ===========================================================================
// xent_head: classifier head forward + backward, one wave per row
// ===========================================================================
struct XentHeadArgs {
  const float* H;          // [B, K] head input (the ReLU output)
  const float* W;          // [C, K]
  const float* bias;       // [C]
  const int32_t* labels;   // [B]
  const float* S;          // [B, K] saved ReLU output (mask of the ReLU backward)
  float* logits;           // [B, C]
  float* dlogits;          // [B, C] (softmax - onehot) / B
  int32_t* argmax;         // [B]
  float* row_loss;         // [B]
  float* dH;               // [B, K] dlogits . W
  float* dX;               // [B, K] dH where S > 0, else 0
  int64_t B;
  int K, C;
  float inv_batch;
  // the step counter (nullptr: none), advanced by inc in place by workgroup
  // B; with scal, that workgroup also writes AdamW's bias corrections of
  // the advanced step, {lr / bc1, 1 / bc2} (adamw_scalars_at), for a later
  // launch's updates
  int32_t* step;
  int inc;
  float* scal;
  AdamWArgs aw;
};

// The value v of the exchange partner of this lane at level BIT: the lane
// with bit BIT flipped (BIT 5, 4: v_permlane32_swap / v_permlane16_swap),
// the lane mirrored in its row of 16 (BIT 3, lane ^ 15) or of 8 (BIT 2,
// lane ^ 7), or the lane with bit 1 or 0 flipped (quad_perm).  Every partner
// differs from the lane in bit BIT and agrees with it in the bits above, and
// all of them are VALU lane moves (no LDS round trip).
template <int BIT>
__device__ __forceinline__ float xpartner(float v, int lane) {
  const unsigned u = __float_as_uint(v);
  if constexpr (BIT == 5) {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(lane < 32 ? r[1] : r[0]);
  } else if constexpr (BIT == 4) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float((lane & 16) ? r[0] : r[1]);
  } else {
    constexpr int ctrl = BIT == 3 ? 0x140 : BIT == 2 ? 0x141 : BIT == 1 ? 0x4E : 0xB1;
    return __int_as_float(__builtin_amdgcn_update_dpp(0, (int)u, ctrl, 0xF, 0xF, false));
  }
}

// Sum over the wave, the same bits in every lane (each level adds a lane's
// value and its partner's, in either order the same IEEE sum).
template <int BIT = 5>
__device__ __forceinline__ float wave_sum_perm(float v, int lane) {
  if constexpr (BIT < 0) {
    return v;
  } else {
    return wave_sum_perm<BIT - 1>(v + xpartner<BIT>(v, lane), lane);
  }
}

// Sums over the wave of x[c] for every class c < N (16 or 32), in log2(N)
// levels that halve the classes a lane carries (it keeps the half its bit
// BIT selects and adds its partner's copy of that half), then the levels
// left add the partners that carry the same class.  Lane l returns the sum
// of class l >> (6 - log2 N), every class summed in one fixed order.
template <int N, int BIT = 5, int CM>
__device__ __forceinline__ float class_sums(float (&x)[CM], int lane) {
  if constexpr (N > 1) {
    const bool up = ((lane >> BIT) & 1) != 0;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const float send = up ? x[i] : x[i + N / 2];
      const float keep = up ? x[i + N / 2] : x[i];
      x[i] = keep + xpartner<BIT>(send, lane);
    }
    return class_sums<N / 2, BIT - 1>(x, lane);
  } else {
    return wave_sum_perm<BIT>(x[0], lane);
  }
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// The step counter's workgroup: advance it and write the advanced step's
// bias corrections (two fp64 powers).
__device__ __forceinline__ void head_counter(int32_t* step, int inc, float* scal, AdamWArgs aw) {
  const int t = step[0] + inc;
  step[0] = t;
  if (scal) {
    const AdamWScalars sc = adamw_scalars_at(t, aw);
    scal[0] = sc.step;
    scal[1] = sc.ibc2;
  }
}

// Q: 16-byte vectors per lane along K (K <= 256 Q); CM: classes (C <= CM,
// 16 or 32).  One wave (one row) per workgroup, so that the rows spread over
// as many CUs as there are rows.  With Q x CM <= 16 the lane's slice of W is
// loaded once, together with the row, and serves both the logits and dH.
// After class_sums, lane l carries class l >> SH: the softmax terms are
// computed once per class there, and every lane reads the ones it needs.
template <int Q, int CM>
__global__ __launch_bounds__(64) void xent_head_kernel(XentHeadArgs a) {
  static_assert(CM == 16 || CM == 32, "class_sums maps 64 lanes onto 16 or 32 classes");
  constexpr int SH = CM == 16 ? 2 : 1;
  const int lane = threadIdx.x;
  if (blockIdx.x == a.B) {  // the step counter's workgroup (launched only with a counter)
    if (lane == 0) head_counter(a.step, a.inc, a.scal, a.aw);
    return;
  }
  const int64_t row = blockIdx.x;
  const int K4 = a.K >> 2;
  constexpr bool PRE = Q * CM <= 16;
  // every load the row needs is issued here, before the first store (the
  // outputs alias nothing, but the compiler cannot know that)
  f32x4 wreg[PRE ? Q * CM : 1];
  if constexpr (PRE) {
#pragma unroll
    for (int c = 0; c < CM; ++c)
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const int idx = q * 64 + lane;
        wreg[c * Q + q] = (c < a.C && idx < K4) ? reinterpret_cast<const f32x4*>(a.W + (int64_t)c * a.K)[idx]
                                                : f32x4{0.f, 0.f, 0.f, 0.f};
      }
  }
  auto wload = [&](int c, int q, int idx) -> f32x4 {
    if constexpr (PRE)
      return wreg[c * Q + q];
    else
      return reinterpret_cast<const f32x4*>(a.W + (int64_t)c * a.K)[idx];
  };
  const f32x4* hr = reinterpret_cast<const f32x4*>(a.H + row * a.K);
  const f32x4* sr = reinterpret_cast<const f32x4*>(a.S + row * a.K);
  f32x4 h[Q], sv[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int idx = q * 64 + lane;
    h[q] = idx < K4 ? hr[idx] : f32x4{0.f, 0.f, 0.f, 0.f};
    sv[q] = idx < K4 ? sr[idx] : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const int mycls = lane >> SH;
  const bool mine = mycls < a.C;
  const float mybias = mine ? a.bias[mycls] : 0.0f;
  const int lab = a.labels[row];
  const bool valid = lab >= 0 && lab < a.C;

  // logits: each lane's partial dot products, then the class sums
  float x[CM];
#pragma unroll
  for (int c = 0; c < CM; ++c) {
    float p = 0.0f;
    if (c < a.C) {
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const int idx = q * 64 + lane;
        if (idx < K4) {
          const f32x4 w = wload(c, q, idx);
          p = fmaf(h[q][0], w[0], p);
          p = fmaf(h[q][1], w[1], p);
          p = fmaf(h[q][2], w[2], p);
          p = fmaf(h[q][3], w[3], p);
        }
      }
    }
    x[c] = p;
  }
  const float z = class_sums<CM>(x, lane) + mybias;  // logit of class mycls

  // softmax cross-entropy of the row: the maximum and its first index over
  // the classes in order, the exponentials per class, their sum over the wave
  float M = readlane_f(z, 0);
  int am = 0;
#pragma unroll
  for (int c = 1; c < CM; ++c) {
    if (c < a.C) {
      const float zc = readlane_f(z, c << SH);
      if (zc > M) {
        M = zc;
        am = c;
      }
    }
  }
  const float e = mine ? __expf(z - M) : 0.0f;
  const float S = wave_sum_perm((lane & ((1 << SH) - 1)) == 0 ? e : 0.0f, lane);
  const float invS = 1.0f / S;
  const float dz = (e * invS - (mycls == lab ? 1.0f : 0.0f)) * a.inv_batch;
  if (mine && (lane & ((1 << SH) - 1)) == 0) {
    a.logits[row * a.C + mycls] = z;
    a.dlogits[row * a.C + mycls] = dz;
  }
  if (lane == 0) {
    a.argmax[row] = am;
    const float zl = readlane_f(z, (valid ? lab : 0) << SH);
    a.row_loss[row] = valid ? ((M - zl) + logf(S)) : __builtin_nanf("");  // as softmax_xent
  }

  // dH = dlogits . W and the ReLU backward against the saved output
  float d[CM];
#pragma unroll
  for (int c = 0; c < CM; ++c) d[c] = c < a.C ? readlane_f(dz, c << SH) : 0.0f;
  f32x4* dhr = reinterpret_cast<f32x4*>(a.dH + row * a.K);
  f32x4* dxr = reinterpret_cast<f32x4*>(a.dX + row * a.K);
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int idx = q * 64 + lane;
    if (idx >= K4) break;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < CM; ++c) {
      if (c < a.C) {
        const f32x4 w = wload(c, q, idx);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(d[c], w[i], acc[i]);
      }
    }
    const f32x4 s = sv[q];
    f32x4 dx;
#pragma unroll
    for (int i = 0; i < 4; ++i) dx[i] = s[i] > 0.0f ? acc[i] : 0.0f;
    dhr[idx] = acc;
    dxr[idx] = dx;
  }
}

bool f32_rows(const TensorDesc& t, int64_t R, int64_t C) {
  return dt(t) == DType::kF32 && t.rank == 2 && t.shape[0] == R && t.shape[1] == C &&
         is_contig_2d_rowmajor(t) && aligned(t.data, 16);
}
bool f32_vec(const TensorDesc& t, int64_t n) {
  return dt(t) == DType::kF32 && t.contiguous && t.rank >= 1 && numel_of(t) == n;
}
bool i32_vec(const TensorDesc& t, int64_t n) {
  return dt(t) == DType::kI32 && t.contiguous && t.rank >= 1 && numel_of(t) == n;
}

// inputs (H [B,K], W [C,K], bias [C], labels [B] i32, S [B,K]);
// outputs (logits [B,C], dlogits [B,C], argmax [B] i32, row_loss [B], dH [B,K], dX [B,K]).
// inputs (H, W, bias, labels, S[, step]); outputs (logits, dlogits, argmax,
// row loss, dH, dX[, step[, AdamW scalars]]).  step: an int32 counter
// updated in place; scalars: 2 fp32.  extra: 0, 1 (step) or 2 (step and
// scalars).
bool xent_head_check(const TensorDesc* in, int ni, const TensorDesc* out, int no, int extra) {
  if (!in || !out || ni != (extra ? 6 : 5) || no != 6 + extra) return false;
  if (in[0].rank != 2 || in[1].rank != 2) return false;
  const int64_t B = in[0].shape[0], K = in[0].shape[1], C = in[1].shape[0];
  if (B < 1 || K < 4 || K % 4 || K > 2048 || C < 1 || C > 32) return false;
  if (!f32_rows(in[0], B, K) || !f32_rows(in[1], C, K) || !f32_vec(in[2], C) || !i32_vec(in[3], B) ||
      !f32_rows(in[4], B, K))
    return false;
  for (int o = 0; o < 2; ++o)  // logits, dlogits: scalar stores, any alignment
    if (dt(out[o]) != DType::kF32 || out[o].rank != 2 || out[o].shape[0] != B || out[o].shape[1] != C ||
        !is_contig_2d_rowmajor(out[o]))
      return false;
  if (!i32_vec(out[2], B) || !f32_vec(out[3], B) || !f32_rows(out[4], B, K) || !f32_rows(out[5], B, K))
    return false;
  if (extra) {  // an int32 scalar (any rank), updated in place
    const TensorDesc &si = in[5], &so = out[6];
    if (dt(si) != DType::kI32 || numel_of(si) != 1 || !si.contiguous || so.data != si.data ||
        dt(so) != DType::kI32 || numel_of(so) != 1)
      return false;
  }
  if (extra == 2 && (dt(out[7]) != DType::kF32 || numel_of(out[7]) != 2 || !out[7].contiguous)) return false;
  // the written tensors touch nothing the kernel reads and not each other
  // (the step counter is read and written by one lane)
  for (int o = 0; o < no; ++o) {
    for (int i = 0; i < ni; ++i)
      if (!(o == 6 && i == 5) && views_overlap(out[o], in[i])) return false;
    for (int q = o + 1; q < no; ++q)
      if (views_overlap(out[o], out[q])) return false;
  }
  return B < INT32_MAX;
}

bool xent_head_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void*) {
  return xent_head_check(in, ni, out, no, 0);
}

// Schema XHST <i inc> or <i inc, f lr, f beta1, f beta2>: the step counter
// advances by inc (1, or 0 for the AICF_WARMUP copy of step_inc); with the
// hyperparameters the launch also writes AdamW's bias corrections of the
// advanced step ({lr / bc1, 1 / bc2}, as adamw_step derives them).
struct XhstAttr {
  int inc;
  bool scal;
  AdamWArgs aw;
};
bool read_xhst(const void* attr, XhstAttr* x) {
  const AttrBlob& b = blob(attr);
  if (!attr || b.schema_id != AICF_SCHEMA_XHST || !payload_ok(b, 4)) return false;
  x->inc = field<int32_t>(b, 0);
  x->scal = payload_ok(b, 16);
  x->aw = AdamWArgs{};
  if (x->scal) {
    const float lr = field<float>(b, 4), b1 = field<float>(b, 8), b2 = field<float>(b, 12);
    if (lr != lr || b1 != b1 || b2 != b2) return false;
    x->aw = AdamWArgs{lr, b1, b2, 0.0f, 0.0f, 1.0f - b1, 1.0f - b2, 1.0f};
  }
  return x->inc == 0 || x->inc == 1;
}

bool xent_head_step_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr) {
  XhstAttr x;
  return read_xhst(attr, &x) && xent_head_check(in, ni, out, no, x.scal ? 2 : 1);
}

template <int Q>
void xent_head_go(const XentHeadArgs& a, unsigned grid, hipStream_t s) {
  if (a.C <= 16)
    xent_head_kernel<Q, 16><<<grid, 64, 0, s>>>(a);
  else
    xent_head_kernel<Q, 32><<<grid, 64, 0, s>>>(a);
}

Status xent_head_run(const TensorDesc* in, TensorDesc* out, int32_t* step, int inc, float* scal,
                     const AdamWArgs& aw, void* stream) {
  XentHeadArgs a{};
  a.step = step;
  a.inc = inc;
  a.scal = scal;
  a.aw = aw;
  a.H = (const float*)in[0].data;
  a.W = (const float*)in[1].data;
  a.bias = (const float*)in[2].data;
  a.labels = (const int32_t*)in[3].data;
  a.S = (const float*)in[4].data;
  a.logits = (float*)out[0].data;
  a.dlogits = (float*)out[1].data;
  a.argmax = (int32_t*)out[2].data;
  a.row_loss = (float*)out[3].data;
  a.dH = (float*)out[4].data;
  a.dX = (float*)out[5].data;
  a.B = in[0].shape[0];
  a.K = (int)in[0].shape[1];
  a.C = (int)in[1].shape[0];
  a.inv_batch = 1.0f / (float)a.B;
  // one row per workgroup, and one more for the step counter
  const unsigned grid = (unsigned)a.B + (step ? 1u : 0u);
  const int q = (a.K / 4 + 63) / 64;
  hipStream_t s = as_stream(stream);
  if (q <= 1)
    xent_head_go<1>(a, grid, s);
  else if (q <= 2)
    xent_head_go<2>(a, grid, s);
  else if (q <= 4)
    xent_head_go<4>(a, grid, s);
  else
    xent_head_go<8>(a, grid, s);
  return launch_status("xent_head");
}

Status xent_head_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* at, void*,
                        size_t, void* stream) {
  if (!xent_head_sup(in, ni, out, no, at)) return Status::InvalidArgument;
  return xent_head_run(in, out, nullptr, 0, nullptr, AdamWArgs{}, stream);
}

Status xent_head_step_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* at, void*,
                             size_t, void* stream) {
  XhstAttr x;
  if (!xent_head_step_sup(in, ni, out, no, at) || !read_xhst(at, &x)) return Status::InvalidArgument;
  return xent_head_run(in, out, (int32_t*)out[6].data, x.inc, x.scal ? (float*)out[7].data : nullptr, x.aw,
                       stream);
}

// ===========================================================================
// grad_group: independent small jobs in one launch
// ===========================================================================
enum GroupJobType { GJ_GEMM = 0, GJ_COLSUM = 1, GJ_MEAN = 2, GJ_STEP = 3 };
constexpr int kMaxJobs = 8;

struct GroupJob {
  int type;
  SgJob gemm;
  const float* x;  // colsum: out[n] = sum_r x[r * ld + n]; mean: mean of x[0 .. rows)
  float* out;
  int64_t rows, cols, ld;
  const int32_t* step_in;
  int32_t* step_out;
  int inc;  // step: out = in + inc (0 for the warmup copy)
  float *P, *M, *V;  // GEMM / column sum with AdamW: the parameter it updates (else nullptr)
};
struct GroupArgs {
  int n;
  int start[kMaxJobs + 1];  // first workgroup of each job
  GroupJob job[kMaxJobs];
  AdamWArgs aa;
  const float* scal;        // the step's bias corrections {lr / bc1, 1 / bc2}
};

// Column sum over 64 columns: wave w adds rows w, w + 4, ... in order, the
// four waves combine as (w0 + w1) + (w2 + w3).
// ADAM: apply AdamW to the parameter whose gradient the sums are.
template <bool ADAM>
__device__ __forceinline__ void colsum_block(const GroupJob& j, int b, float* red, const StoreAdamW& ad) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t n = (int64_t)b * 64 + lane;
  AdamWLane ar;
  if (ADAM && w == 0 && n < j.cols) {
    ar.s = AdamWScalars{ad.scal[0], ad.scal[1]};
    adamw_load(ad, n, 0, ar);
  }
  float s = 0.0f;
  if (n < j.cols) {
    const float* p = j.x + n;
#pragma unroll 8
    for (int64_t r = w; r < j.rows; r += 4) s += p[r * j.ld];
  }
  red[w * 64 + lane] = s;
  __syncthreads();
  if (w == 0 && n < j.cols) {
    const float sum = (red[lane] + red[64 + lane]) + (red[128 + lane] + red[192 + lane]);
    j.out[n] = sum;
    if constexpr (ADAM) adamw_store(ad, n, 0, sum, ar);
  }
}

__global__ __launch_bounds__(256) void grad_group_kernel(GroupArgs a) {
  __shared__ f32x4 red[256];
  const int blk = blockIdx.x;
  // the job whose workgroup range holds blk (independent compares: the
  // starts load together)
  int j = 0;
#pragma unroll
  for (int k = 1; k < kMaxJobs; ++k) j += (k < a.n && blk >= a.start[k]) ? 1 : 0;
  const GroupJob& job = a.job[j];
  const int b = blk - a.start[j];
  const StoreAdamW ad{job.P, job.M, job.V, a.scal, a.aa};
  switch (job.type) {
    case GJ_GEMM:
      if (job.P)
        sg_block<true>(job.gemm, b, red, ad);
      else
        sg_block<false>(job.gemm, b, red, ad);
      break;
    case GJ_COLSUM:
      if (job.P)
        colsum_block<true>(job, b, reinterpret_cast<float*>(red), ad);
      else
        colsum_block<false>(job, b, reinterpret_cast<float*>(red), ad);
      break;
    case GJ_MEAN:
      block_mean_f64(job.x, job.rows, job.out, reinterpret_cast<double*>(red));
      break;
    default:  // GJ_STEP
      if (threadIdx.x == 0) job.step_out[0] = job.step_in[0] + job.inc;
      break;
  }
}

// Schema GGRP: <i n> then n records <iiiiii> (type, in0, in1, out0, f0, f1):
//   GEMM    C[out0] = op(in0) . op(in1), f0 = transA, f1 = transB
//   COLSUM  out0[n] = sum over rows of in0 (2-D, unit column stride)
//   MEAN    out0 (1 element) = mean of in0, fp64 accumulation, fixed order
//   STEP    out0 = in0 + f0 (int32 scalars; f0 is 1, or 0 for the warmup copy)
struct GroupRec {
  int type, in0, in1, out0, f0, f1;
};

bool read_group(const void* attr, int ni, int no, GroupRec* recs, int* n) {
  const AttrBlob& a = blob(attr);
  if (a.schema_id != AICF_SCHEMA_GGRP || !payload_ok(a, 4)) return false;
  const int cnt = field<int32_t>(a, 0);
  if (cnt < 1 || cnt > kMaxJobs || !payload_ok(a, 4 + 24 * (uint32_t)cnt)) return false;
  for (int k = 0; k < cnt; ++k) {
    GroupRec r;
    r.type = field<int32_t>(a, 4 + 24 * k);
    r.in0 = field<int32_t>(a, 8 + 24 * k);
    r.in1 = field<int32_t>(a, 12 + 24 * k);
    r.out0 = field<int32_t>(a, 16 + 24 * k);
    r.f0 = field<int32_t>(a, 20 + 24 * k);
    r.f1 = field<int32_t>(a, 24 + 24 * k);
    if (r.type < GJ_GEMM || r.type > GJ_STEP) return false;
    if (r.in0 < 0 || r.in0 >= ni || r.out0 < 0 || r.out0 >= no) return false;
    if (r.type == GJ_GEMM && (r.in1 < 0 || r.in1 >= ni)) return false;
    recs[k] = r;
  }
  *n = cnt;
  return true;
}

// The jobs of a group from their records: shapes, the small-GEMM plans, the
// workgroup ranges, and that no job writes what another job reads or writes.
bool group_build(const TensorDesc* in, const TensorDesc* out, const GroupRec* recs, int n, GroupArgs& a) {
  a.n = n;
  int blocks = 0;
  for (int k = 0; k < n; ++k) {
    const GroupRec& r = recs[k];
    GroupJob& j = a.job[k];
    j.type = r.type;
    const TensorDesc &X = in[r.in0], &O = out[r.out0];
    int nb = 1;
    if (r.type == GJ_GEMM) {
      const TensorDesc& Y = in[r.in1];
      if (dt(X) != DType::kF32 || dt(Y) != DType::kF32 || dt(O) != DType::kF32) return false;
      if (X.rank != 2 || Y.rank != 2 || O.rank != 2 || O.stride[1] != 1 || O.stride[0] < O.shape[1])
        return false;
      for (const TensorDesc* t : {&X, &Y})
        if (t->stride[0] < 0 || t->stride[1] < 0) return false;
      const bool ta = r.f0 != 0, tb = r.f1 != 0;
      SmallGemm g{};
      g.A = (const float*)X.data;
      g.B = (const float*)Y.data;
      g.C = (float*)O.data;
      g.M = ta ? X.shape[1] : X.shape[0];
      g.K = ta ? X.shape[0] : X.shape[1];
      g.a_m = ta ? X.stride[1] : X.stride[0];
      g.a_k = ta ? X.stride[0] : X.stride[1];
      const int64_t KB = tb ? Y.shape[1] : Y.shape[0];
      g.N = tb ? Y.shape[0] : Y.shape[1];
      g.b_k = tb ? Y.stride[1] : Y.stride[0];
      g.b_n = tb ? Y.stride[0] : Y.stride[1];
      g.c_m = O.stride[0];
      if (KB != g.K || O.shape[0] != g.M || O.shape[1] != g.N) return false;
      if (!small_gemm_ok(g)) return false;
      j.gemm = sg_plan(g);
      nb = sg_blocks(j.gemm);
    } else if (r.type == GJ_COLSUM) {
      if (dt(X) != DType::kF32 || X.rank != 2 || X.stride[1] != 1 || X.stride[0] < X.shape[1]) return false;
      if (X.shape[0] < 1 || X.shape[1] < 1 || !f32_vec(O, X.shape[1])) return false;
      j.x = (const float*)X.data;
      j.out = (float*)O.data;
      j.rows = X.shape[0];
      j.cols = X.shape[1];
      j.ld = X.stride[0];
      nb = (int)((j.cols + 63) / 64);
    } else if (r.type == GJ_MEAN) {
      int64_t cnt = 0;
      if (dt(X) != DType::kF32 || !X.contiguous || !numel_pos(X, &cnt)) return false;
      if (dt(O) != DType::kF32 || numel_of(O) != 1) return false;
      j.x = (const float*)X.data;
      j.out = (float*)O.data;
      j.rows = numel_of(X);
    } else {  // GJ_STEP
      if (dt(X) != DType::kI32 || numel_of(X) != 1 || dt(O) != DType::kI32 || numel_of(O) != 1) return false;
      if (r.f0 != 0 && r.f0 != 1) return false;
      j.step_in = (const int32_t*)X.data;
      j.step_out = (int32_t*)O.data;
      j.inc = r.f0;
    }
    a.start[k] = blocks;
    if ((int64_t)blocks + nb > INT32_MAX) return false;
    blocks += nb;
  }
  a.start[n] = blocks;
  // the jobs run concurrently: what a job writes may not be read or written
  // by another job
  for (int k = 0; k < n; ++k) {
    const Span w = span_of(out[recs[k].out0]);
    for (int l = 0; l < n; ++l) {
      if (l == k) continue;
      if (overlap(w, span_of(out[recs[l].out0])) || overlap(w, span_of(in[recs[l].in0])))
        return false;
      if (recs[l].type == GJ_GEMM && overlap(w, span_of(in[recs[l].in1]))) return false;
    }
    // and a job does not read its own output (the step counter is the exception:
    // one lane reads it, then writes it)
    if (recs[k].type != GJ_STEP) {
      if (overlap(w, span_of(in[recs[k].in0]))) return false;
      if (recs[k].type == GJ_GEMM && overlap(w, span_of(in[recs[k].in1]))) return false;
    }
  }
  return true;
}

bool group_fill(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr,
                GroupArgs* ga) {
  if (!in || !out || ni < 1 || no < 1) return false;
  GroupRec recs[kMaxJobs];
  int n = 0;
  if (!read_group(attr, ni, no, recs, &n)) return false;
  GroupArgs a{};
  if (!group_build(in, out, recs, n, a)) return false;
  if (ga) *ga = a;
  return true;
}

// Schema GGRA: a gradient group whose GEMM / column-sum jobs may also apply
// AdamW to the parameter their output is the gradient of, where each
// gradient element is stored (the bits of adamw_step on that gradient).
//   <i n> <fffff lr, beta1, beta2, eps, weight_decay> <i scalars input>,
//   then n records <iiiiii iii iii>: the GGRP fields, then the P, M, V input
//   indices and the P, M, V output indices (in place; -1 for a job without
//   AdamW).  The scalars input holds the step's bias corrections {lr / bc1,
//   1 / bc2} (2 fp32, written by the launch that advanced the step counter).
// No step job: the counter is advanced by that earlier launch.
struct GroupAdamRec {
  int p_in, m_in, v_in, p_out, m_out, v_out;
};
bool group_adamw_fill(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr,
                      GroupArgs* ga) {
  if (!in || !out || ni < 1 || no < 1) return false;
  const AttrBlob& b = blob(attr);
  if (b.schema_id != AICF_SCHEMA_GGRA || !payload_ok(b, 28)) return false;
  const int cnt = field<int32_t>(b, 0);
  if (cnt < 1 || cnt > kMaxJobs || !payload_ok(b, 28 + 48 * (uint32_t)cnt)) return false;
  const float lr = field<float>(b, 4), b1 = field<float>(b, 8), b2 = field<float>(b, 12);
  const float eps = field<float>(b, 16), wd = field<float>(b, 20);
  if (lr != lr || b1 != b1 || b2 != b2 || eps != eps || wd != wd) return false;
  const int si = field<int32_t>(b, 24);
  if (si < 0 || si >= ni || dt(in[si]) != DType::kF32 || numel_of(in[si]) != 2 || !in[si].contiguous) return false;
  GroupRec recs[kMaxJobs];
  GroupAdamRec ar[kMaxJobs];
  for (int k = 0; k < cnt; ++k) {
    const int o = 28 + 48 * k;
    GroupRec r{field<int32_t>(b, o), field<int32_t>(b, o + 4), field<int32_t>(b, o + 8),
               field<int32_t>(b, o + 12), field<int32_t>(b, o + 16), field<int32_t>(b, o + 20)};
    if (r.type < GJ_GEMM || r.type > GJ_MEAN) return false;  // no step job: the updates read the counter
    if (r.in0 < 0 || r.in0 >= ni || r.out0 < 0 || r.out0 >= no) return false;
    if (r.type == GJ_GEMM && (r.in1 < 0 || r.in1 >= ni)) return false;
    recs[k] = r;
    ar[k] = GroupAdamRec{field<int32_t>(b, o + 24), field<int32_t>(b, o + 28), field<int32_t>(b, o + 32),
                         field<int32_t>(b, o + 36), field<int32_t>(b, o + 40), field<int32_t>(b, o + 44)};
  }
  GroupArgs a{};
  if (!group_build(in, out, recs, cnt, a)) return false;
  // every tensor the launch writes, to check the updated ones against
  const Span scal = span_of(in[si]);
  for (int k = 0; k < cnt; ++k) {
    if (overlap(span_of(out[recs[k].out0]), scal)) return false;
    const GroupAdamRec& r = ar[k];
    if (r.p_in < 0 && r.m_in < 0 && r.v_in < 0 && r.p_out < 0 && r.m_out < 0 && r.v_out < 0) continue;
    if (recs[k].type != GJ_GEMM && recs[k].type != GJ_COLSUM) return false;
    const int idx_in[3] = {r.p_in, r.m_in, r.v_in}, idx_out[3] = {r.p_out, r.m_out, r.v_out};
    const TensorDesc& G = out[recs[k].out0];
    // the gradient's element index is the parameter's: a row-major output
    if (recs[k].type == GJ_GEMM && G.stride[0] != G.shape[1]) return false;
    for (int x = 0; x < 3; ++x) {
      if (idx_in[x] < 0 || idx_in[x] >= ni || idx_out[x] < 0 || idx_out[x] >= no) return false;
      const TensorDesc &T = in[idx_in[x]], &To = out[idx_out[x]];
      if (dt(T) != DType::kF32 || !T.contiguous || numel_of(T) != numel_of(G)) return false;
      if (To.data != T.data || !same_shape(To, T)) return false;  // in place
      const Span w = span_of(T);
      if (overlap(w, scal)) return false;
      // nothing else of the launch reads or writes it: the jobs' operands
      // and outputs, and the other updated tensors
      for (int l = 0; l < cnt; ++l) {
        if (overlap(w, span_of(out[recs[l].out0])) || overlap(w, span_of(in[recs[l].in0]))) return false;
        if (recs[l].type == GJ_GEMM && overlap(w, span_of(in[recs[l].in1]))) return false;
        const GroupAdamRec& q = ar[l];
        const int others[3] = {q.p_in, q.m_in, q.v_in};
        for (int y = 0; y < 3; ++y) {
          if (others[y] < 0 || (l == k && y == x)) continue;
          if (others[y] >= ni || overlap(w, span_of(in[others[y]]))) return false;
        }
      }
    }
    a.job[k].P = (float*)in[r.p_in].data;
    a.job[k].M = (float*)in[r.m_in].data;
    a.job[k].V = (float*)in[r.v_in].data;
  }
  a.aa = AdamWArgs{lr, b1, b2, eps, wd, 1.0f - b1, 1.0f - b2, 1.0f - lr * wd};
  a.scal = (const float*)in[si].data;
  if (ga) *ga = a;
  return true;
}

bool grad_group_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr) {
  return group_fill(in, ni, out, no, attr, nullptr);
}

Status grad_group_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* attr, void*,
                         size_t, void* stream) {
  GroupArgs a;
  if (!group_fill(in, ni, out, no, attr, &a)) return Status::InvalidArgument;
  grad_group_kernel<<<(unsigned)a.start[a.n], 256, 0, as_stream(stream)>>>(a);
  return launch_status("grad_group");
}

bool grad_group_adamw_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr) {
  return group_adamw_fill(in, ni, out, no, attr, nullptr);
}

Status grad_group_adamw_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* attr, void*,
                               size_t, void* stream) {
  GroupArgs a;
  if (!group_adamw_fill(in, ni, out, no, attr, &a)) return Status::InvalidArgument;
  grad_group_kernel<<<(unsigned)a.start[a.n], 256, 0, as_stream(stream)>>>(a);
  return launch_status("grad_group_adamw");
}

// ===========================================================================
// adamw_multi: AdamW over several tensors in one launch
// ===========================================================================
constexpr int kMaxTensors = 8;

struct AdamWTensor {
  const float* P;
  const float* G;
  const float* M;
  const float* V;
  float* Po;
  float* Mo;
  float* Vo;
  int64_t n;
};
struct AdamWMultiArgs {
  int nt;
  int start[kMaxTensors + 1];
  AdamWTensor t[kMaxTensors];
  AdamWArgs a;
  const int32_t* step;
};

// Per tensor, the element mapping of adamw_step (one 16-byte vector per
// lane, 1024 elements per workgroup, the n % 4 tail by the lane of vector
// n / 4) and its element update: the same bits.
__global__ __launch_bounds__(256) void adamw_multi_kernel(AdamWMultiArgs args) {
  __shared__ float sh[2];
  if (threadIdx.x < 64) {
    const AdamWScalars t = adamw_scalars(args.step, args.a);
    if (threadIdx.x == 0) {
      sh[0] = t.step;
      sh[1] = t.ibc2;
    }
  }
  __syncthreads();
  const AdamWScalars s{sh[0], sh[1]};
  const int blk = blockIdx.x;
  int j = 0;
  while (j + 1 < args.nt && blk >= args.start[j + 1]) ++j;
  const AdamWTensor& T = args.t[j];
  const int64_t n = T.n, n4 = n / 4;
  const int64_t i = (int64_t)(blk - args.start[j]) * 256 + threadIdx.x;
  if (i < n4) {
    f32x4 p = reinterpret_cast<const f32x4*>(T.P)[i];
    const f32x4 g = reinterpret_cast<const f32x4*>(T.G)[i];
    f32x4 m = reinterpret_cast<const f32x4*>(T.M)[i];
    f32x4 v = reinterpret_cast<const f32x4*>(T.V)[i];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float pp = p[c], mm = m[c], vv = v[c];
      adamw_elem(pp, g[c], mm, vv, s, args.a);
      p[c] = pp;
      m[c] = mm;
      v[c] = vv;
    }
    reinterpret_cast<f32x4*>(T.Po)[i] = p;
    reinterpret_cast<f32x4*>(T.Mo)[i] = m;
    reinterpret_cast<f32x4*>(T.Vo)[i] = v;
  } else if (i == n4) {
    for (int64_t e = 4 * n4; e < n; ++e) {
      float pp = T.P[e], mm = T.M[e], vv = T.V[e];
      adamw_elem(pp, T.G[e], mm, vv, s, args.a);
      T.Po[e] = pp;
      T.Mo[e] = mm;
      T.Vo[e] = vv;
    }
  }
}

// Schema ADAM <fffff>: lr, beta1, beta2, eps, weight_decay (adamw_step's).
bool read_adamw(const void* attr, AdamWArgs* out) {
  float lr = 1e-3f, b1 = 0.9f, b2 = 0.999f, eps = 1e-8f, wd = 0.0f;
  const AttrBlob& a = blob(attr);
  if (attr && a.schema_id != 0) {
    if (a.schema_id != AICF_SCHEMA_ADAM || !payload_ok(a, 16)) return false;
    lr = field<float>(a, 0);
    b1 = field<float>(a, 4);
    b2 = field<float>(a, 8);
    eps = field<float>(a, 12);
    if (payload_ok(a, 20)) wd = field<float>(a, 16);
  }
  *out = AdamWArgs{lr, b1, b2, eps, wd, 1.0f - b1, 1.0f - b2, 1.0f - lr * wd};
  return true;
}

// inputs (P0, G0, M0, V0, ..., P_{T-1}, G, M, V, step i32); outputs (P0, M0, V0, ...).
bool adamw_multi_fill(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr,
                      AdamWMultiArgs* pa) {
  if (!in || !out || ni < 5 || (ni - 1) % 4 || no != 3 * ((ni - 1) / 4)) return false;
  const int T = (ni - 1) / 4;
  if (T > kMaxTensors) return false;
  AdamWMultiArgs a{};
  if (!read_adamw(attr, &a.a)) return false;
  const TensorDesc& st = in[ni - 1];
  if (dt(st) != DType::kI32 || !st.contiguous || numel_of(st) != 1) return false;
  a.step = (const int32_t*)st.data;
  a.nt = T;
  int blocks = 0;
  for (int k = 0; k < T; ++k) {
    const TensorDesc *P = &in[4 * k], *G = &in[4 * k + 1], *M = &in[4 * k + 2], *V = &in[4 * k + 3];
    const TensorDesc *Po = &out[3 * k], *Mo = &out[3 * k + 1], *Vo = &out[3 * k + 2];
    int64_t n = 0;
    if (!numel_pos(*P, &n)) return false;
    for (const TensorDesc* t : {P, G, M, V, Po, Mo, Vo})
      if (dt(*t) != DType::kF32 || !t->contiguous || numel_of(*t) != n || !aligned(t->data, 16))
        return false;
    // in place per buffer, nothing else shared (adam_step/launcher.cu:98-128)
    if (Po->data != P->data || Mo->data != M->data || Vo->data != V->data) return false;
    if (G->data == P->data || G->data == M->data || G->data == V->data || P->data == M->data ||
        P->data == V->data || M->data == V->data)
      return false;
    a.t[k] = AdamWTensor{(const float*)P->data, (const float*)G->data, (const float*)M->data,
                         (const float*)V->data, (float*)Po->data, (float*)Mo->data, (float*)Vo->data, n};
    a.start[k] = blocks;
    const int64_t nb = (n / 4 + 1 + 255) / 256;  // vectors plus the tail lane
    if ((int64_t)blocks + nb > INT32_MAX) return false;
    blocks += (int)nb;
  }
  a.start[T] = blocks;
  // distinct tensors do not overlap
  for (int k = 0; k < T; ++k)
    for (int l = k + 1; l < T; ++l)
      for (int x = 0; x < 4; ++x)
        for (int y = 0; y < 4; ++y)
          if (overlap(span_of(in[4 * k + x]), span_of(in[4 * l + y]))) return false;
  if (pa) *pa = a;
  return true;
}

bool adamw_multi_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr) {
  return adamw_multi_fill(in, ni, out, no, attr, nullptr);
}

Status adamw_multi_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* attr, void*,
                          size_t, void* stream) {
  AdamWMultiArgs a;
  if (!adamw_multi_fill(in, ni, out, no, attr, &a)) return Status::InvalidArgument;
  adamw_multi_kernel<<<(unsigned)a.start[a.nt], 256, 0, as_stream(stream)>>>(a);
  return launch_status("adamw_multi");
}

}  // namespace

// ===========================================================================
// Small GEMM entry for the GEMM dispatcher
// ===========================================================================
bool small_gemm_ok(const SmallGemm& g) {
  if (!g.A || !g.B || !g.C || g.M < 1 || g.N < 1 || g.K < 1) return false;
  if (g.M > INT32_MAX / 2 || g.N > INT32_MAX / 2 || g.K > INT32_MAX / 2) return false;
  if (g.a_m < 0 || g.a_k < 0 || g.b_k < 0 || g.b_n < 0 || g.c_m < g.N) return false;
  // the operands are read through buffer loads with 32-bit byte offsets
  if (g.a_m > INT32_MAX || g.a_k > INT32_MAX || g.b_k > INT32_MAX || g.b_n > INT32_MAX) return false;
  if (sg_range_bytes(g.M, g.a_m, g.K, g.a_k) > INT32_MAX || sg_range_bytes(g.N, g.b_n, g.K, g.b_k) > INT32_MAX)
    return false;
  const int64_t tiles = ((g.M + 15) / 16) * ((g.N + 15) / 16);
  return tiles <= INT32_MAX / 4;
}

Status small_gemm_f32(const SmallGemm& g, hipStream_t s) {
  if (!small_gemm_ok(g)) return Status::InvalidArgument;
  const int kb = (int)((g.K + 15) / 16);
  if (kb >= 48) {  // long K: sixteen waves split it
    const SgJob j = sg_plan(g, 16);
    gemm_small_kernel<16><<<(unsigned)sg_blocks(j), 1024, 0, s>>>(j);
  } else if (kb >= 32) {  // eight waves
    const SgJob j = sg_plan(g, 8);
    gemm_small_kernel<8><<<(unsigned)sg_blocks(j), 512, 0, s>>>(j);
  } else {
    const SgJob j = sg_plan(g);
    gemm_small_kernel<4><<<(unsigned)sg_blocks(j), 256, 0, s>>>(j);
  }
  return launch_status("gemm_small");
}

// ===========================================================================
// gemm_epilogue (bias+ReLU, bias, ReLU) on the small path with a second
// output: a copy of B, written by the tiles that read it.  A step whose
// gradient group updates B in place reads the copy instead (the input
// gradient dX = dY . W next to AdamW on W), so the copy costs one write of B
// and no read.
// ===========================================================================
namespace {

bool gemm_bcopy_fill(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr,
                     SmallGemm* pg) {
  if (!in || !out || ni != 3 || no != 2 || !attr) return false;
  const AttrBlob& b = blob(attr);
  if (b.schema_id != AICF_SCHEMA_GEPI || !payload_ok(b, 12)) return false;
  const bool ta = field<int32_t>(b, 0) != 0, tb = field<int32_t>(b, 4) != 0;
  const int kind = field<int32_t>(b, 8);
  if (kind != AICF_EPI_BIAS_RELU && kind != AICF_EPI_BIAS && kind != AICF_EPI_RELU) return false;
  const TensorDesc &X = in[0], &Y = in[1], &bias = in[2], &O = out[0], &Bc = out[1];
  for (const TensorDesc* t : {&X, &Y, &O, &Bc})
    if (dt(*t) != DType::kF32 || t->rank != 2) return false;
  for (const TensorDesc* t : {&X, &Y})
    if (t->stride[0] < 0 || t->stride[1] < 0) return false;
  if (O.stride[1] != 1 || O.stride[0] < O.shape[1]) return false;
  SmallGemm g{};
  g.A = (const float*)X.data;
  g.B = (const float*)Y.data;
  g.C = (float*)O.data;
  g.M = ta ? X.shape[1] : X.shape[0];
  g.K = ta ? X.shape[0] : X.shape[1];
  g.a_m = ta ? X.stride[1] : X.stride[0];
  g.a_k = ta ? X.stride[0] : X.stride[1];
  const int64_t KB = tb ? Y.shape[1] : Y.shape[0];
  g.N = tb ? Y.shape[0] : Y.shape[1];
  g.b_k = tb ? Y.stride[1] : Y.stride[0];
  g.b_n = tb ? Y.stride[0] : Y.stride[1];
  g.c_m = O.stride[0];
  if (KB != g.K || O.shape[0] != g.M || O.shape[1] != g.N) return false;
  if (kind != AICF_EPI_RELU) {
    if (dt(bias) != DType::kF32 || bias.rank != 1 || bias.shape[0] != g.N || bias.stride[0] <= 0) return false;
    g.bias = (const float*)bias.data;
    g.bias_s = bias.stride[0];
  }
  g.relu = kind != AICF_EPI_BIAS;
  // the copy moves B's 16-byte K vectors: K-contiguous, 16-byte aligned rows,
  // and the copy has B's layout
  if (g.b_k != 1 || g.K % 4 || (g.N > 1 && g.b_n % 4) || !aligned(Y.data, 16) || !aligned(Bc.data, 16))
    return false;
  if (!same_shape(Bc, Y) || Bc.stride[0] != Y.stride[0] || Bc.stride[1] != Y.stride[1]) return false;
  if (((g.M + 63) / 64) * ((g.N + 63) / 64) >= kSmallGemmMaxTiles64 || !small_gemm_ok(g)) return false;
  // the written tensors touch nothing the kernel reads and not each other
  for (const TensorDesc* w : {&O, &Bc}) {
    if (views_overlap(*w, X) || views_overlap(*w, Y)) return false;
    if (kind != AICF_EPI_RELU && views_overlap(*w, bias)) return false;
  }
  if (views_overlap(O, Bc)) return false;
  g.bcopy = (float*)Bc.data;
  if (pg) *pg = g;
  return true;
}

bool gemm_bcopy_sup(const TensorDesc* in, int ni, const TensorDesc* out, int no, const void* attr) {
  return gemm_bcopy_fill(in, ni, out, no, attr, nullptr);
}

Status gemm_bcopy_launch(const TensorDesc* in, int ni, TensorDesc* out, int no, const void* attr, void*, size_t,
                         void* stream) {
  SmallGemm g;
  if (!gemm_bcopy_fill(in, ni, out, no, attr, &g)) return Status::InvalidArgument;
  return small_gemm_f32(g, as_stream(stream));
}

}  // namespace

KernelVariant make_gemm_small_bcopy_f32_variant() {
  return make("gemm_small_bcopy_f32", gemm_bcopy_launch, gemm_bcopy_sup, AICF_SCHEMA_GEPI);
}
KernelVariant make_xent_head_f32_variant() { return make("xent_head_f32", xent_head_launch, xent_head_sup); }
KernelVariant make_xent_head_step_f32_variant() {
  return make("xent_head_step_f32", xent_head_step_launch, xent_head_step_sup, AICF_SCHEMA_XHST);
}
KernelVariant make_grad_group_f32_variant() {
  return make("grad_group_f32", grad_group_launch, grad_group_sup, AICF_SCHEMA_GGRP);
}
KernelVariant make_grad_group_adamw_f32_variant() {
  return make("grad_group_adamw_f32", grad_group_adamw_launch, grad_group_adamw_sup, AICF_SCHEMA_GGRA);
}
KernelVariant make_adamw_multi_f32_variant() {
  return make("adamw_multi_f32", adamw_multi_launch, adamw_multi_sup, AICF_SCHEMA_ADAM);
}

}  // namespace aicf::hip
