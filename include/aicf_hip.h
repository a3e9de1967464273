/*
 * aicf_hip.h — C-ABI of the MI355X (gfx950) op backend and plan runtime.
 *
 * This is the drop-in boundary that replaces the reference's CUDA backend
 * behind its unchanged kernel-registry / op-dispatch API and its
 * `aicf_cuda._C` Python bindings.  Only plain C types cross it: POD structs,
 * pointers, sizes and int32 status codes.  No torch or HIP types appear in
 * any signature; streams are passed as opaque `void*` (a `hipStream_t`).
 *
 * Reference paths below are relative to ai-compiler-framework/ in the
 * reference tree.
 */
#ifndef AICF_HIP_H
#define AICF_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Value types                                                               */
/* ------------------------------------------------------------------------ */

/* Replaces include/aicf/backends/cuda/registry/tensor_desc.hpp:8 (kMaxRank). */
#define AICF_MAX_RANK 4

/* Replaces tensor_desc.hpp:13-27 (enum class DType : uint8_t); same values. */
#define AICF_DTYPE_UNKNOWN 0
#define AICF_DTYPE_F32 1
#define AICF_DTYPE_F16 2
#define AICF_DTYPE_BF16 3
#define AICF_DTYPE_I32 4

/* Replaces registry/status.hpp:6-11 (enum class Status : int32_t); same values. */
#define AICF_STATUS_OK 0
#define AICF_STATUS_INVALID_ARGUMENT 1
#define AICF_STATUS_NOT_IMPLEMENTED 2
#define AICF_STATUS_INTERNAL 3

/*
 * Replaces registry/op_kind.hpp:5-31 (enum class OpKind : int).  Values 0..17
 * are identical; 18.. are appended kinds for ops the reference lacks.
 */
#define AICF_OP_ELTWISE_ADD 0
#define AICF_OP_ELTWISE_RELU 1
#define AICF_OP_GEMM 2
#define AICF_OP_BIAS_ADD 3
#define AICF_OP_REDUCE_SUM 4
#define AICF_OP_MSE_GRAD 5
#define AICF_OP_RELU_BWD 6
#define AICF_OP_SGD_STEP 7
#define AICF_OP_COPY 8
#define AICF_OP_GRAD_ZERO 9
#define AICF_OP_ADAM_STEP 10
#define AICF_OP_STEP_INC 11
#define AICF_OP_BIAS_CORR 12
#define AICF_OP_LAYERNORM_FWD 13
#define AICF_OP_LAYERNORM_BWD 14
#define AICF_OP_BATCHNORM_FWD 15
#define AICF_OP_BATCHNORM_BWD 16
#define AICF_OP_GEMM_EPILOGUE 17
/* appended kinds (no counterpart in the reference) */
#define AICF_OP_ROW_SOFTMAX 18  /* X[R,C] -> softmax Y (+ row max, row sum of X) */
#define AICF_OP_ROW_REDUCE 19   /* X[R,C] -> per-row sum or max (schema RRED) */
#define AICF_OP_SOFTMAX_XENT 20 /* logits, labels -> loss, dlogits, argmax, row loss */
#define AICF_OP_GELU_BWD 21     /* dOut, Z -> dOut * gelu_tanh'(Z) */
#define AICF_OP_ELTWISE_GELU 22 /* X -> gelu_tanh(X) */
#define AICF_OP_TRANSPOSE 23    /* X[R,C] -> X^T[C,R] (2-D, row-major) */
#define AICF_OP_GEMM_ADAMW 24   /* A, B, P, M, V, step -> P, M, V, Wb: AdamW on P with grad op(A).op(B) (schema GADW) */
#define AICF_OP_XENT_HEAD 25     /* H, W, b, labels, S -> logits, dlogits, argmax, row loss, dH, dX: the
                                    classifier head of a ReLU MLP forward and backward (softmax xent,
                                    dH = dlogits.W, dX = dH where S > 0); with schema XHST a 6th
                                    input and 7th output, the step counter, advanced in place (and
                                    an 8th output, the step's AdamW bias corrections) */
#define AICF_OP_GRAD_GROUP 26    /* independent small jobs in one launch: GEMMs, column sums, a loss
                                    mean, the step counter (schema GGRP); or GEMMs, column sums and
                                    the mean with AdamW applied where a gradient is stored (GGRA) */
#define AICF_OP_ADAMW_MULTI 27   /* (P, G, M, V) x T, step -> (P, M, V) x T: AdamW over T tensors (schema ADAM) */
#define AICF_OP_MSE_COLSUM 28    /* pred, target, step -> dPred, loss, loss partials, column partials of
                                    dPred [P, N], step (+1): MSE loss and gradient, the gradient's
                                    column sums over P row blocks, the step counter (schema MSCS) */
#define AICF_OP_COLSUM_ADAMW 29  /* T column-partial tensors [R_t, N_t], P, M, V, step -> G, P, M, V, Wb:
                                    G = the column sums (concatenated), AdamW on P with it (schema CADW) */
#define AICF_OP_COUNT 30

/*
 * Attribute schema ids (numeric ABI).  The reference mixes big-endian fourccs
 * (GEMM, GPEL, RSUM) with little-endian ones (the rest); the numbers are kept.
 */
#define AICF_SCHEMA_GEMM 0x47454D4Du /* gemm/launcher.cu:41          <ii>  transA, transB */
#define AICF_SCHEMA_GPEL 0x4750454Cu /* gemm_epilogue/launcher.cu:49 <iii> transA, transB, relu */
#define AICF_SCHEMA_GEPI 0x49504547u /* core_v2/exec.py:215-217      <iii> transA, transB, epilogue kind */
#define AICF_SCHEMA_RSUM 0x5253554Du /* reduce_sum/launcher.cu:75    <q>   axis */
#define AICF_SCHEMA_MSEG 0x4745534Du /* mse_grad/launcher.cu:36      <f>   scale */
#define AICF_SCHEMA_BADD 0x44444142u /* bias_add/launcher.cu:97      <q>   axis */
#define AICF_SCHEMA_ADAM 0x4D414441u /* adam_step/launcher.cu:32     <ffff> lr,b1,b2,eps (+<f> wd) */
#define AICF_SCHEMA_BCOR 0x524F4342u /* biascorr/launcher.cu:31      <ff>  beta1, beta2 */
#define AICF_SCHEMA_SGDS 0x53444753u /* sgd_step/launcher.cu:31      <f>   lr */
#define AICF_SCHEMA_LNEP 0x50454E4Cu /* layernorm/launcher.cu:41      <f>   eps (default 1e-5) */
#define AICF_SCHEMA_BNEP 0x50454E42u /* batchnorm/launcher.cu:51      <fI>  eps, flags (bit0 use_running_stats) */
#define AICF_SCHEMA_RRED 0x44455252u /* appended: b"RRED" little-endian, <i> 0=sum 1=max */
#define AICF_SCHEMA_GGRP 0x50524747u /* appended: b"GGRP" little-endian, <i n> + n x <iiiiii> type, in0, in1,
                                       out0, f0, f1 (type 0 GEMM f0,f1 = transA,transB; 1 column sum;
                                       2 mean; 3 step counter += f0) */
#define AICF_SCHEMA_GADW 0x57444147u /* appended: b"GADW" little-endian, <ii fffff> transA, transB, lr, b1, b2, eps, wd */
#define AICF_SCHEMA_MSCS 0x5343534Du /* appended: b"MSCS" little-endian, <f i> gradient scale (<= 0: 2/n), step += i (0 or 1) */
#define AICF_SCHEMA_CADW 0x57444143u /* appended: b"CADW" little-endian, <i fffff> T, lr, b1, b2, eps, wd */
#define AICF_SCHEMA_GGRA 0x41524747u /* appended: b"GGRA" little-endian, <i n> <fffff> lr, b1, b2, eps, wd,
                                       <i> input holding the step's bias corrections {lr/bc1, 1/bc2}
                                       (2 f32), then n x <iiiiii iii iii>: the GGRP record (types 0-2),
                                       the P, M, V input and P, M, V output indices of the parameter
                                       the job's output is the gradient of (-1: none) */
#define AICF_SCHEMA_XHST 0x54534858u /* appended: b"XHST" little-endian, <i> step += i (0 or 1), optionally
                                       <fff> lr, b1, b2: an 8th output (2 f32) receives the advanced
                                       step's AdamW bias corrections {lr/bc1, 1/bc2} */

/* GEPI epilogue kinds.  0..2 are the values core_v2/exec.py:223-252 packs;
 * 3..7 are appended (no counterpart in the reference). */
#define AICF_EPI_BIAS_RELU 0
#define AICF_EPI_BIAS 1
#define AICF_EPI_RELU 2
#define AICF_EPI_BIAS_GELU 3  /* bias then gelu_tanh; optional 2nd output keeps the pre-activation */
#define AICF_EPI_GELU 4       /* gelu_tanh, input 2 ignored */
#define AICF_EPI_DGELU 5      /* out = acc * gelu_tanh'(Z), input 2 is Z[M,N] */
#define AICF_EPI_DGELU_COLSUM 6 /* as 5, plus outputs db[N] f32 = column sums of out, and a f32
                                   workspace [P, N] with P >= M/256 (no reference counterpart) */
#define AICF_EPI_DGELU_PARTIALS 7 /* as 5, plus output [M/256, N] f32: row t of it is the column sums of
                                     out's 256-row block t (finished by a later COLSUM_ADAMW) */
/* Kinds 0..2 with a second output of B's shape and strides (fp32, small
 * problems, K-contiguous B): that output receives a copy of B (appended). */

/*
 * Replaces tensor_desc.hpp:88-158 (struct TensorDesc).  Field order, types
 * and therefore layout are identical (96 bytes on LP64): `rank` stands for
 * the reference's one-member union RankND.  shape/stride are in elements.
 */
typedef struct aicf_tensor_desc {
  void* data;
  uint8_t dtype; /* AICF_DTYPE_* */
  int32_t rank;
  int64_t shape[AICF_MAX_RANK];
  int64_t stride[AICF_MAX_RANK];
  bool contiguous;
  int32_t alignment; /* bytes; 0 = unknown */
  int32_t device;
} aicf_tensor_desc;

/* Replaces registry/attr_blob.hpp:13-17 (struct AttrBlob); same layout. */
typedef struct aicf_attr_blob {
  uint32_t schema_id;
  uint32_t bytes;
  const void* data;
} aicf_attr_blob;

/* ------------------------------------------------------------------------ */
/* Dispatch                                                                  */
/* ------------------------------------------------------------------------ */

/*
 * Replaces aicf::cuda::dispatch_v0 (registry/dispatch.hpp:12-17,
 * src/backends/cuda/registry/registry.cpp:144-215): priority-ordered variant
 * selection, first supported() wins.  `attrs` may be NULL (empty blob).
 * Returns AICF_STATUS_*: NOT_IMPLEMENTED when no variant accepts the call.
 */
int32_t aicf_dispatch_v0(int32_t kind, const aicf_tensor_desc* inputs, int32_t num_inputs,
                         aicf_tensor_desc* outputs, int32_t num_outputs,
                         const aicf_attr_blob* attrs, void* stream);

/*
 * Replaces aicf::cuda::dispatch_by_id_v0 (dispatch.hpp:20-26,
 * registry.cpp:16-64,218-236): run exactly the variant registered under
 * `kernel_id`.  INVALID_ARGUMENT for an empty id, a schema mismatch or an
 * unsupported call; NOT_IMPLEMENTED for an unknown id.
 */
int32_t aicf_dispatch_by_id_v0(int32_t kind, const char* kernel_id,
                               const aicf_tensor_desc* inputs, int32_t num_inputs,
                               aicf_tensor_desc* outputs, int32_t num_outputs,
                               const aicf_attr_blob* attrs, void* stream);

/* Replaces registry/register_all.hpp:8 (aicf_cuda_register_all_kernels).
 * Idempotent: registration happens once per process. */
void aicf_cuda_register_all_kernels(void);

/* Replaces include/aicf/backends/cuda/ops/reduce_sum/api.hpp:6
 * (reduce_sum_lastdim_f32, implemented at reduce_sum/launcher.cu:494-503):
 * dB[n] = sum_m dY[m, n] over a row-major [M, N] fp32 matrix. */
int32_t aicf_reduce_sum_lastdim_f32(const float* dY, float* dB, int32_t M, int32_t N, void* stream);

/*
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the fused MSE loss + gradient of kernel
 * mse_loss_grad_v0 (OpKind MseGrad with outputs dPred, loss, partials) with
 * no partials argument.  Its per-workgroup partial sums live in a
 * library-owned device array of 65536 floats (256 KiB on every GPU the
 * library runs on, held until the process ends); nothing is allocated.
 *   dpred[i] = (pred[i] - target[i]) * scale     (2/n is the reference's default)
 *   loss[0]  = mean((pred - target)^2)
 * pred and dpred are AICF_DTYPE_F32 or AICF_DTYPE_BF16 (`dtype`), target is
 * fp32; pred/dpred 16-byte aligned for f32 (8 for bf16), target 16-byte.
 * Limit: 1 <= n <= 134217728 (2^27); larger n, a null pointer, another dtype
 * or a misaligned pointer return INVALID_ARGUMENT with aicf_last_error() set.
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (unordered streams) race.  Results are bit-identical to mse_loss_grad_v0
 * given a partials buffer of at least ceil(n / 2048) floats.
 */
int32_t aicf_mse_loss_grad_noalloc(const void* pred, const float* target, void* dpred, float* loss,
                                   int64_t n, int32_t dtype, float scale, void* stream);

/* Measurement aid, no counterpart in the reference: launches `blocks`
 * workgroups of 4 waves, each running `iters` rounds of 8 independent
 * v_mfma_f32_32x32x16_bf16 on random register operands (no memory traffic),
 * 2 * 32 * 32 * 16 * 8 * iters flop per wave.  Its sustained rate is the
 * power-limited MFMA ceiling of the part; `out` (one float) is written only
 * to keep the loop.  Returns AICF_STATUS_*. */
int32_t aicf_diag_mfma_loop(float* out, int32_t blocks, int32_t iters, uint32_t seed, void* stream);

/* Measurement aid, no counterpart in the reference: as aicf_diag_mfma_loop
 * with the MFMA form chosen by `form`: 32 (v_mfma_f32_32x32x16_bf16, as
 * above) or 16 (16 independent v_mfma_f32_16x16x32_bf16 per round, the form
 * the bf16 GEMM kernels issue; the same 2^18 flop per wave and round).
 * AICF_STATUS_INVALID_ARGUMENT for any other form. */
int32_t aicf_diag_mfma_loop_form(float* out, int32_t blocks, int32_t iters, uint32_t seed, int32_t form,
                                 void* stream);

/* ------------------------------------------------------------------------ */
/* Registry introspection (replaces KernelRegistry::variants_snapshot and    */
/* find_by_id, registry/registry.hpp:39-42)                                  */
/* ------------------------------------------------------------------------ */

/* Number of variants registered for `kind` (in selection order). */
int32_t aicf_registry_count(int32_t kind);
/* kernel_id / priority / expected schema of the idx-th variant, or NULL / -1. */
const char* aicf_registry_kernel_id(int32_t kind, int32_t idx);
int32_t aicf_registry_priority(int32_t kind, int32_t idx);
uint32_t aicf_registry_schema(int32_t kind, int32_t idx);
/* 1 if `kernel_id` is registered under `kind`, else 0. */
int32_t aicf_registry_has(int32_t kind, const char* kernel_id);

/* Replaces registry/status.hpp:15-23 (status_to_string) and the OpKind name
 * table of src/python_bindings/bindings.cpp:196-219. */
const char* aicf_status_name(int32_t status);
const char* aicf_opkind_name(int32_t kind);

/* ------------------------------------------------------------------------ */
/* Graph capture / replay (replaces the CudaGraphState singleton and the     */
/* graph_* entry points of src/python_bindings/bindings.cpp:137-187,475-547) */
/* ------------------------------------------------------------------------ */

/* Ends any dangling capture, drops the previous graph, lazily creates the
 * dedicated non-blocking stream and begins a global-mode capture on it.
 * The stream handle is written to *out_stream.  Returns AICF_STATUS_*. */
int32_t aicf_graph_begin(uint64_t* out_stream);
/* Ends the capture and instantiates the executable graph.  INVALID_ARGUMENT
 * when no capture is in progress. */
int32_t aicf_graph_end(void);
/* Launches the instantiated graph on `caller_stream` (NULL: the null stream,
 * torch's default), so the replay is ordered after the work already queued
 * there (input copies, host-side updates of device scalars) and before the
 * work queued there afterwards (reads of its results).  The reference
 * replays on its dedicated stream instead, unordered against the caller's
 * work.  INVALID_ARGUMENT when no graph was captured. */
int32_t aicf_graph_launch(void* caller_stream);
/* Ends a dangling capture and destroys the graph objects. */
int32_t aicf_graph_reset(void);
/* The dedicated capture stream (0 before the first aicf_graph_begin). */
uint64_t aicf_graph_stream(void);
/* 1 while capturing, 2 when a graph is instantiated, 0 otherwise. */
int32_t aicf_graph_state(void);

/*
 * Graph handles.  The reference keeps exactly one graph per process (the
 * singleton above, which is handle 0 here); these entry points have no
 * counterpart there.  They let several plans stay instantiated at once and
 * let a plan be captured again with other buffers bound without building a
 * new executable.  Each created handle owns its own non-blocking stream and
 * captures in thread-local mode.  Handle 0 is accepted by every *_h call and
 * behaves like the singleton, except that aicf_graph_begin_h keeps its
 * executable for an in-place update.
 */
/* Creates an empty graph handle (never 0). */
int32_t aicf_graph_create(uint64_t* out_handle);
/* Ends a dangling capture, destroys the graph objects, stream and event of
 * `handle`.  INVALID_ARGUMENT for handle 0 or an unknown handle. */
int32_t aicf_graph_destroy(uint64_t handle);
/* Begins a capture on the handle's stream (written to *out_stream).  An
 * executable graph from an earlier capture is kept until aicf_graph_end_h
 * and is not launchable meanwhile. */
int32_t aicf_graph_begin_h(uint64_t handle, uint64_t* out_stream);
/* Ends the capture.  When the handle already holds an executable graph it is
 * updated in place (hipGraphExecUpdate) if the new capture has the same
 * topology; otherwise a new executable is instantiated. */
int32_t aicf_graph_end_h(uint64_t handle);
/* As aicf_graph_launch, for the handle's graph. */
int32_t aicf_graph_launch_h(uint64_t handle, void* caller_stream);
/* As aicf_graph_reset, for one handle (the handle stays valid). */
int32_t aicf_graph_reset_h(uint64_t handle);
/* The handle's stream (0 before its first capture or for unknown handles). */
uint64_t aicf_graph_stream_h(uint64_t handle);
/* As aicf_graph_state; -1 for an unknown handle. */
int32_t aicf_graph_state_h(uint64_t handle);
/* Number of captures applied to the handle by in-place update. */
uint64_t aicf_graph_updates_h(uint64_t handle);

/* Message of the last failing HIP runtime call made by this library on the
 * calling thread ("" if none). */
const char* aicf_last_error(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* AICF_HIP_H */
