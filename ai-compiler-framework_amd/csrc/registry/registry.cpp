// Kernel registry, runtime dispatch and by-id dispatch, plus their C-ABI.
//
// Behaviour follows src/backends/cuda/registry/registry.cpp of the reference:
//   DispatchById  :16-64   (empty id / bad schema / unsupported -> InvalidArgument,
//                           unknown id or workspace>0 -> NotImplemented)
//   register      :76-115  (kernel_id required, priority-descending stable
//                           insertion, first id wins on duplicates)
//   Dispatch      :144-195 (first supported() in priority order wins)
#include <cstdio>
#include <cstring>

#include "../common/host_util.hpp"
#include "../common/registry.hpp"

namespace aicf::hip {

namespace {
thread_local std::string g_last_error;
}  // namespace

const char* last_error_message() { return g_last_error.c_str(); }

void set_last_error(const char* what, const char* detail) {
  g_last_error = std::string(what ? what : "") + ": " + (detail ? detail : "");
}

namespace {
const AttrBlob kEmptyAttrBlob{0u, 0u, nullptr};

bool call_shape_ok(const TensorDesc* inputs, int32_t num_inputs, const TensorDesc* outputs,
                   int32_t num_outputs, OpKind kind) {
  if (num_inputs < 0 || num_outputs < 0) return false;
  if (num_inputs > 0 && !inputs) return false;
  if (num_outputs > 0 && !outputs) return false;
  const int k = static_cast<int>(kind);
  return k >= 0 && k < static_cast<int>(OpKind::_Count);
}
}  // namespace

KernelRegistry& KernelRegistry::instance() {
  static KernelRegistry inst;
  return inst;
}

void KernelRegistry::ensure_registered() {
  static std::once_flag once;
  std::call_once(once, []() { register_all_kernels_into(instance()); });
}

void KernelRegistry::register_kernel(OpKind kind, KernelVariant v) {
  const int k = static_cast<int>(kind);
  if (k < 0 || k >= kKinds) return;
  if (!v.kernel_id || v.kernel_id[0] == '\0') return;  // id is mandatory

  std::lock_guard<std::mutex> lock(mu_);
  auto entry = std::make_unique<KernelVariant>(v);
  auto& vec = table_[k];
  auto it = vec.begin();
  while (it != vec.end() && (*it)->priority >= entry->priority) ++it;
  const KernelVariant* raw = entry.get();
  vec.insert(it, std::move(entry));
  by_id_[k].emplace(std::string(raw->kernel_id), raw);  // keeps the first on collision
}

void KernelRegistry::variants_snapshot(OpKind kind, std::vector<const KernelVariant*>& out) const {
  out.clear();
  const int k = static_cast<int>(kind);
  if (k < 0 || k >= kKinds) return;
  std::lock_guard<std::mutex> lock(mu_);
  for (const auto& p : table_[k]) out.push_back(p.get());
}

const KernelVariant* KernelRegistry::find_by_id(OpKind kind, const char* kernel_id) const {
  const int k = static_cast<int>(kind);
  if (k < 0 || k >= kKinds || !kernel_id || kernel_id[0] == '\0') return nullptr;
  std::lock_guard<std::mutex> lock(mu_);
  auto it = by_id_[k].find(std::string(kernel_id));
  return it == by_id_[k].end() ? nullptr : it->second;
}

Status dispatch_v0(OpKind kind, const TensorDesc* inputs, int32_t num_inputs, TensorDesc* outputs,
                   int32_t num_outputs, const void* attrs, void* stream) {
  KernelRegistry::ensure_registered();
  if (!call_shape_ok(inputs, num_inputs, outputs, num_outputs, kind))
    return Status::InvalidArgument;
  const AttrBlob* ab = attrs ? static_cast<const AttrBlob*>(attrs) : &kEmptyAttrBlob;

  std::vector<const KernelVariant*> vars;
  KernelRegistry::instance().variants_snapshot(kind, vars);
  const KernelVariant* chosen = nullptr;
  for (const KernelVariant* v : vars) {
    if (!v->supported || !v->launch) continue;
    if (v->expected_attr_schema_id != 0 && ab->schema_id != v->expected_attr_schema_id) continue;
    if (v->supported(inputs, num_inputs, outputs, num_outputs, ab)) {
      chosen = v;
      break;
    }
  }
  if (!chosen) return Status::NotImplemented;
  if (chosen->query_workspace && chosen->query_workspace(inputs, num_inputs, ab) != 0)
    return Status::NotImplemented;
  return chosen->launch(inputs, num_inputs, outputs, num_outputs, ab, nullptr, 0, stream);
}

Status dispatch_by_id_v0(OpKind kind, const char* kernel_id, const TensorDesc* inputs,
                         int32_t num_inputs, TensorDesc* outputs, int32_t num_outputs,
                         const void* attrs, void* stream) {
  KernelRegistry::ensure_registered();
  if (!kernel_id || kernel_id[0] == '\0') return Status::InvalidArgument;
  if (!call_shape_ok(inputs, num_inputs, outputs, num_outputs, kind))
    return Status::InvalidArgument;
  const AttrBlob* ab = attrs ? static_cast<const AttrBlob*>(attrs) : &kEmptyAttrBlob;

  const KernelVariant* v = KernelRegistry::instance().find_by_id(kind, kernel_id);
  if (!v || !v->supported || !v->launch) return Status::NotImplemented;
  if (v->expected_attr_schema_id != 0 && ab->schema_id != v->expected_attr_schema_id)
    return Status::InvalidArgument;
  if (!v->supported(inputs, num_inputs, outputs, num_outputs, ab)) return Status::InvalidArgument;
  if (v->query_workspace && v->query_workspace(inputs, num_inputs, ab) != 0)
    return Status::NotImplemented;
  return v->launch(inputs, num_inputs, outputs, num_outputs, ab, nullptr, 0, stream);
}

const char* status_name(Status s) {
  switch (s) {
    case Status::Ok: return "Ok";
    case Status::InvalidArgument: return "InvalidArgument";
    case Status::NotImplemented: return "NotImplemented";
    case Status::Internal: return "Internal";
  }
  return "Unknown";
}

const char* opkind_name(OpKind k) {
  switch (k) {
    case OpKind::EltwiseAdd: return "add";
    case OpKind::EltwiseRelu: return "relu";
    case OpKind::Gemm: return "gemm";
    case OpKind::BiasAdd: return "bias_add";
    case OpKind::ReduceSum: return "reduce_sum";
    case OpKind::MseGrad: return "mse_grad";
    case OpKind::ReluBwd: return "relu_bwd";
    case OpKind::SgdStep: return "sgd_step";
    case OpKind::Copy: return "copy";
    case OpKind::GradZero: return "grad_zero";
    case OpKind::AdamStep: return "adam_step";
    case OpKind::StepInc: return "step_inc";
    case OpKind::BiasCorr: return "bias_corr";
    case OpKind::LayerNormFwd: return "layernorm_fwd";
    case OpKind::LayerNormBwd: return "layernorm_bwd";
    case OpKind::BatchNormFwd: return "batchnorm_fwd";
    case OpKind::BatchNormBwd: return "batchnorm_bwd";
    case OpKind::GemmEpilogue: return "gemm_epilogue";
    case OpKind::RowSoftmax: return "row_softmax";
    case OpKind::RowReduce: return "row_reduce";
    case OpKind::SoftmaxXent: return "softmax_xent";
    case OpKind::GeluBwd: return "gelu_bwd";
    case OpKind::EltwiseGelu: return "gelu";
    case OpKind::Transpose: return "transpose";
    case OpKind::GemmAdamW: return "gemm_adamw";
    case OpKind::XentHead: return "xent_head";
    case OpKind::GradGroup: return "grad_group";
    case OpKind::AdamWMulti: return "adamw_multi";
    case OpKind::MseColsum: return "mse_colsum";
    case OpKind::ColsumAdamW: return "colsum_adamw";
    case OpKind::_Count: break;
  }
  return "unknown";
}

}  // namespace aicf::hip

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
using namespace aicf::hip;

extern "C" {

int32_t aicf_dispatch_v0(int32_t kind, const aicf_tensor_desc* inputs, int32_t num_inputs,
                         aicf_tensor_desc* outputs, int32_t num_outputs,
                         const aicf_attr_blob* attrs, void* stream) {
  return static_cast<int32_t>(dispatch_v0(static_cast<OpKind>(kind), inputs, num_inputs, outputs,
                                          num_outputs, attrs, stream));
}

int32_t aicf_dispatch_by_id_v0(int32_t kind, const char* kernel_id,
                               const aicf_tensor_desc* inputs, int32_t num_inputs,
                               aicf_tensor_desc* outputs, int32_t num_outputs,
                               const aicf_attr_blob* attrs, void* stream) {
  return static_cast<int32_t>(dispatch_by_id_v0(static_cast<OpKind>(kind), kernel_id, inputs,
                                                num_inputs, outputs, num_outputs, attrs, stream));
}

void aicf_cuda_register_all_kernels(void) { KernelRegistry::ensure_registered(); }

int32_t aicf_registry_count(int32_t kind) {
  KernelRegistry::ensure_registered();
  if (kind < 0 || kind >= AICF_OP_COUNT) return 0;
  std::vector<const KernelVariant*> v;
  KernelRegistry::instance().variants_snapshot(static_cast<OpKind>(kind), v);
  return static_cast<int32_t>(v.size());
}

static const KernelVariant* variant_at(int32_t kind, int32_t idx) {
  KernelRegistry::ensure_registered();
  if (kind < 0 || kind >= AICF_OP_COUNT || idx < 0) return nullptr;
  std::vector<const KernelVariant*> v;
  KernelRegistry::instance().variants_snapshot(static_cast<OpKind>(kind), v);
  return idx < static_cast<int32_t>(v.size()) ? v[idx] : nullptr;
}

const char* aicf_registry_kernel_id(int32_t kind, int32_t idx) {
  const KernelVariant* v = variant_at(kind, idx);
  return v ? v->kernel_id : nullptr;
}

int32_t aicf_registry_priority(int32_t kind, int32_t idx) {
  const KernelVariant* v = variant_at(kind, idx);
  return v ? v->priority : -1;
}

uint32_t aicf_registry_schema(int32_t kind, int32_t idx) {
  const KernelVariant* v = variant_at(kind, idx);
  return v ? v->expected_attr_schema_id : 0u;
}

int32_t aicf_registry_has(int32_t kind, const char* kernel_id) {
  KernelRegistry::ensure_registered();
  if (kind < 0 || kind >= AICF_OP_COUNT) return 0;
  return KernelRegistry::instance().find_by_id(static_cast<OpKind>(kind), kernel_id) ? 1 : 0;
}

const char* aicf_status_name(int32_t status) {
  if (status < 0 || status > 3) return "Unknown";
  return status_name(static_cast<Status>(status));
}

const char* aicf_opkind_name(int32_t kind) {
  if (kind < 0 || kind >= AICF_OP_COUNT) return "unknown";
  return opkind_name(static_cast<OpKind>(kind));
}

const char* aicf_last_error(void) { return aicf::hip::last_error_message(); }

}  // extern "C"
