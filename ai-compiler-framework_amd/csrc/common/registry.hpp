// Kernel registry types of the gfx950 backend (host-only C++17, no HIP types).
//
// Semantics follow the reference registry:
//   include/aicf/backends/cuda/registry/{kernel_variant,registry}.hpp
//   src/backends/cuda/registry/registry.cpp:16-236
// A variant is a {supported, launch, query_workspace} triple plus a stable
// kernel_id; variants of one OpKind are kept in priority order (higher
// first, insertion order among equals); the first kernel_id registered wins.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "aicf_hip.h"

namespace aicf::hip {

using TensorDesc = aicf_tensor_desc;
using AttrBlob = aicf_attr_blob;

enum class Status : int32_t {
  Ok = AICF_STATUS_OK,
  InvalidArgument = AICF_STATUS_INVALID_ARGUMENT,
  NotImplemented = AICF_STATUS_NOT_IMPLEMENTED,
  Internal = AICF_STATUS_INTERNAL,
};

enum class DType : uint8_t {
  kUnknown = AICF_DTYPE_UNKNOWN,
  kF32 = AICF_DTYPE_F32,
  kF16 = AICF_DTYPE_F16,
  kBF16 = AICF_DTYPE_BF16,
  kI32 = AICF_DTYPE_I32,
};

enum class OpKind : int {
  EltwiseAdd = AICF_OP_ELTWISE_ADD,
  EltwiseRelu = AICF_OP_ELTWISE_RELU,
  Gemm = AICF_OP_GEMM,
  BiasAdd = AICF_OP_BIAS_ADD,
  ReduceSum = AICF_OP_REDUCE_SUM,
  MseGrad = AICF_OP_MSE_GRAD,
  ReluBwd = AICF_OP_RELU_BWD,
  SgdStep = AICF_OP_SGD_STEP,
  Copy = AICF_OP_COPY,
  GradZero = AICF_OP_GRAD_ZERO,
  AdamStep = AICF_OP_ADAM_STEP,
  StepInc = AICF_OP_STEP_INC,
  BiasCorr = AICF_OP_BIAS_CORR,
  LayerNormFwd = AICF_OP_LAYERNORM_FWD,
  LayerNormBwd = AICF_OP_LAYERNORM_BWD,
  BatchNormFwd = AICF_OP_BATCHNORM_FWD,
  BatchNormBwd = AICF_OP_BATCHNORM_BWD,
  GemmEpilogue = AICF_OP_GEMM_EPILOGUE,
  RowSoftmax = AICF_OP_ROW_SOFTMAX,
  RowReduce = AICF_OP_ROW_REDUCE,
  SoftmaxXent = AICF_OP_SOFTMAX_XENT,
  GeluBwd = AICF_OP_GELU_BWD,
  EltwiseGelu = AICF_OP_ELTWISE_GELU,
  Transpose = AICF_OP_TRANSPOSE,
  GemmAdamW = AICF_OP_GEMM_ADAMW,
  XentHead = AICF_OP_XENT_HEAD,
  GradGroup = AICF_OP_GRAD_GROUP,
  AdamWMulti = AICF_OP_ADAMW_MULTI,
  MseColsum = AICF_OP_MSE_COLSUM,
  ColsumAdamW = AICF_OP_COLSUM_ADAMW,
  _Count = AICF_OP_COUNT,
};

using LaunchFn = Status (*)(const TensorDesc* inputs, int num_inputs, TensorDesc* outputs,
                            int num_outputs, const void* attr, void* workspace,
                            size_t workspace_bytes, void* stream);
using WorkspaceFn = size_t (*)(const TensorDesc* inputs, int num_inputs, const void* attr);
using SupportedFn = bool (*)(const TensorDesc* inputs, int num_inputs, const TensorDesc* outputs,
                             int num_outputs, const void* attr);

// Mirrors reference kernel_variant.hpp:30-62 field for field; the stream is
// an opaque hipStream_t.
struct KernelVariant {
  const char* name = nullptr;
  const char* kernel_id = nullptr;
  int priority = 0;
  uint32_t flags = 0;
  uint32_t expected_attr_schema_id = 0;  // 0 = accept any schema
  LaunchFn launch = nullptr;
  WorkspaceFn query_workspace = nullptr;
  SupportedFn supported = nullptr;
};

class KernelRegistry {
 public:
  static KernelRegistry& instance();
  static void ensure_registered();

  void register_kernel(OpKind kind, KernelVariant v);
  void variants_snapshot(OpKind kind, std::vector<const KernelVariant*>& out) const;
  const KernelVariant* find_by_id(OpKind kind, const char* kernel_id) const;

 private:
  KernelRegistry() = default;
  static constexpr int kKinds = static_cast<int>(OpKind::_Count);
  std::vector<std::unique_ptr<KernelVariant>> table_[kKinds];
  std::unordered_map<std::string, const KernelVariant*> by_id_[kKinds];
  mutable std::mutex mu_;
};

Status dispatch_v0(OpKind kind, const TensorDesc* inputs, int32_t num_inputs, TensorDesc* outputs,
                   int32_t num_outputs, const void* attrs, void* stream);
Status dispatch_by_id_v0(OpKind kind, const char* kernel_id, const TensorDesc* inputs,
                         int32_t num_inputs, TensorDesc* outputs, int32_t num_outputs,
                         const void* attrs, void* stream);

const char* status_name(Status s);
const char* opkind_name(OpKind k);

// Called by aicf_cuda_register_all_kernels (register_all.cpp).
void register_all_kernels_into(KernelRegistry& R);

}  // namespace aicf::hip
