// aicf_cuda._C — Python bindings of the gfx950 backend.
//
// Same module name, functions, signatures, defaults and error messages as
// the reference binding (src/python_bindings/bindings.cpp:372-548):
//   OpKind enum, op_call (enum and int overloads), launch_by_id,
//   trace_enable / trace_reset / trace_get, graph_begin / graph_end /
//   graph_launch / graph_reset / graph_stream.
// Every call goes through the C-ABI of libaicf_hip (include/aicf_hip.h); this
// file holds no HIP code.  Differences: bf16 tensors are accepted
// (DType::kBF16 = 3), HIP errors read "[HIP] ...", and graph_launch replays
// on torch's current stream (ordered after the work already queued there and
// before the work queued there afterwards).
#include <c10/hip/HIPStream.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>
#include <torch/extension.h>

#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "aicf_hip.h"

namespace py = pybind11;

namespace {

// OpKind as a C++ enum so that pybind can expose it with the reference names.
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
};

std::string tensor_brief(const torch::Tensor& t) {
  std::ostringstream oss;
  oss << "defined=" << (t.defined() ? "true" : "false");
  if (!t.defined()) return oss.str();
  oss << " device=" << (t.is_cuda() ? "cuda" : "cpu") << " dtype=" << t.dtype()
      << " contig=" << (t.is_contiguous() ? "true" : "false") << " rank=" << t.dim() << " shape=[";
  for (int i = 0; i < t.dim(); ++i) oss << t.size(i) << (i + 1 < t.dim() ? "," : "");
  oss << "]";
  return oss.str();
}

uint8_t to_dtype(const torch::Tensor& t) {
  switch (t.scalar_type()) {
    case at::kHalf: return AICF_DTYPE_F16;
    case at::kFloat: return AICF_DTYPE_F32;
    case at::kInt: return AICF_DTYPE_I32;
    case at::kBFloat16: return AICF_DTYPE_BF16;
    default: break;
  }
  TORCH_CHECK(false, "unsupported dtype. got: ", tensor_brief(t));
}

// bindings.cpp:92-104 of the reference, plus bf16.
void check_tensor(const torch::Tensor& t, const char* what) {
  TORCH_CHECK(t.defined(), what, ": undefined tensor");
  TORCH_CHECK(t.is_cuda(), what, ": must be CUDA tensor. got: ", tensor_brief(t));
  const auto st = t.scalar_type();
  TORCH_CHECK(st == at::kHalf || st == at::kFloat || st == at::kInt || st == at::kBFloat16, what,
              ": dtype must be float16/bfloat16/float32/int32. got: ", tensor_brief(t));
  TORCH_CHECK(t.dim() >= 0 && t.dim() <= AICF_MAX_RANK, what, ": rank out of range. got rank=",
              t.dim(), " (kMaxRank=", AICF_MAX_RANK, ")");
}

aicf_tensor_desc to_desc(const torch::Tensor& t) {
  aicf_tensor_desc d{};
  d.data = const_cast<void*>(t.data_ptr());
  d.dtype = to_dtype(t);
  d.rank = static_cast<int32_t>(t.dim());
  for (int i = 0; i < d.rank; ++i) {
    d.shape[i] = t.size(i);
    d.stride[i] = t.stride(i);
  }
  d.contiguous = t.is_contiguous();
  d.alignment = 0;
  d.device = 0;
  return d;
}

void build_descs(const py::sequence& seq, std::vector<aicf_tensor_desc>& out, const char* what) {
  out.clear();
  out.reserve(seq.size());
  for (auto h : seq) {
    torch::Tensor t = py::cast<torch::Tensor>(h);
    check_tensor(t, what);
    out.push_back(to_desc(t));
  }
}

std::mutex g_mu;  // guards the trace (graph state is guarded inside the library)
std::vector<std::string> g_trace;
bool g_trace_enabled = true;

std::string fail_msg(int kind, int32_t st) {
  return std::string("aicf_cuda call failed: kind=") + std::to_string(kind) + " (" +
         aicf_opkind_name(kind) + ") status=" + aicf_status_name(st) + " (" + std::to_string(st) +
         ")";
}

void* current_stream() {
  return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream().stream());
}

struct Call {
  std::vector<aicf_tensor_desc> in, out;
  std::string buf;
  aicf_attr_blob blob{};
  const aicf_attr_blob* attrs = nullptr;
  void* stream = nullptr;

  Call(const py::sequence& inputs, const py::sequence& outputs, uint32_t schema_id,
       const py::bytes& attrs_bytes, uint64_t stream_u64) {
    build_descs(inputs, in, "inputs");
    build_descs(outputs, out, "outputs");
    buf = attrs_bytes;
    blob.schema_id = schema_id;
    blob.bytes = static_cast<uint32_t>(buf.size());
    blob.data = buf.empty() ? nullptr : buf.data();
    // an all-empty blob is passed as NULL, as the reference does
    attrs = (blob.bytes == 0 && blob.schema_id == 0) ? nullptr : &blob;
    stream = stream_u64 ? reinterpret_cast<void*>(stream_u64) : current_stream();
  }
};

void op_call_impl(int kind, const py::sequence& inputs, const py::sequence& outputs,
                  uint32_t schema_id, const py::bytes& attrs_bytes, uint64_t stream_u64) {
  Call c(inputs, outputs, schema_id, attrs_bytes, stream_u64);
  {
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_trace_enabled) g_trace.emplace_back(aicf_opkind_name(kind));
    if (std::getenv("AICF_TRACE_STDERR"))
      std::fprintf(stderr, "[aicf][op_call] %s (kind=%d) schema=0x%08x bytes=%u stream=0x%llx\n",
                   aicf_opkind_name(kind), kind, (unsigned)schema_id, (unsigned)c.blob.bytes,
                   (unsigned long long)stream_u64);
  }
  const int32_t st = aicf_dispatch_v0(kind, c.in.data(), (int32_t)c.in.size(), c.out.data(),
                                      (int32_t)c.out.size(), c.attrs, c.stream);
  if (st != AICF_STATUS_OK) throw std::runtime_error(fail_msg(kind, st));
}

void launch_by_id_impl(const std::string& kid, int kind, const py::sequence& inputs,
                       const py::sequence& outputs, uint32_t schema_id,
                       const py::bytes& attrs_bytes, uint64_t stream_u64) {
  Call c(inputs, outputs, schema_id, attrs_bytes, stream_u64);
  {
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_trace_enabled)
      g_trace.emplace_back(std::string("kid:") + kid + " kind:" + aicf_opkind_name(kind));
    if (std::getenv("AICF_TRACE_STDERR"))
      std::fprintf(stderr,
                   "[aicf][launch_by_id] kernel_id=%s kind=%s schema=0x%08x bytes=%u stream=0x%llx\n",
                   kid.c_str(), aicf_opkind_name(kind), (unsigned)schema_id,
                   (unsigned)c.blob.bytes, (unsigned long long)stream_u64);
  }
  const int32_t st = aicf_dispatch_by_id_v0(kind, kid.c_str(), c.in.data(), (int32_t)c.in.size(),
                                            c.out.data(), (int32_t)c.out.size(), c.attrs, c.stream);
  if (st != AICF_STATUS_OK) throw std::runtime_error(fail_msg(kind, st) + " kernel_id=" + kid);
}

void hip_check(int32_t st, const char* what) {
  if (st == AICF_STATUS_OK) return;
  const std::string detail = aicf_last_error();
  if (st == AICF_STATUS_INVALID_ARGUMENT) {
    // graph misuse (end without begin, launch before capture)
    const auto pos = detail.find(": ");
    throw std::runtime_error(pos == std::string::npos ? detail : detail.substr(pos + 2));
  }
  throw std::runtime_error(std::string("[HIP] ") + what + ": " + detail);
}

}  // namespace

PYBIND11_MODULE(_C, m) {
  m.doc() = "AICF gfx950 bindings (op_call + launch_by_id + hipGraph capture; AttrBlob ABI)";
  aicf_cuda_register_all_kernels();

  py::enum_<OpKind>(m, "OpKind")
      .value("EltwiseAdd", OpKind::EltwiseAdd)
      .value("EltwiseRelu", OpKind::EltwiseRelu)
      .value("Gemm", OpKind::Gemm)
      .value("BiasAdd", OpKind::BiasAdd)
      .value("ReduceSum", OpKind::ReduceSum)
      .value("MseGrad", OpKind::MseGrad)
      .value("ReluBwd", OpKind::ReluBwd)
      .value("SgdStep", OpKind::SgdStep)
      .value("Copy", OpKind::Copy)
      .value("GradZero", OpKind::GradZero)
      .value("AdamStep", OpKind::AdamStep)
      .value("StepInc", OpKind::StepInc)
      .value("BiasCorr", OpKind::BiasCorr)
      .value("LayerNormFwd", OpKind::LayerNormFwd)
      .value("LayerNormBwd", OpKind::LayerNormBwd)
      .value("BatchNormFwd", OpKind::BatchNormFwd)
      .value("BatchNormBwd", OpKind::BatchNormBwd)
      .value("GemmEpilogue", OpKind::GemmEpilogue)
      .value("RowSoftmax", OpKind::RowSoftmax)
      .value("RowReduce", OpKind::RowReduce)
      .value("SoftmaxXent", OpKind::SoftmaxXent)
      .value("GeluBwd", OpKind::GeluBwd)
      .value("EltwiseGelu", OpKind::EltwiseGelu)
      .value("Transpose", OpKind::Transpose)
      .value("GemmAdamW", OpKind::GemmAdamW)
      .value("XentHead", OpKind::XentHead)
      .value("GradGroup", OpKind::GradGroup)
      .value("AdamWMulti", OpKind::AdamWMulti)
      .value("MseColsum", OpKind::MseColsum)
      .value("ColsumAdamW", OpKind::ColsumAdamW)
      .export_values();

  m.def(
      "op_call",
      [](OpKind kind, const py::sequence& inputs, const py::sequence& outputs, uint32_t schema_id,
         py::bytes attrs_bytes, uint64_t stream) {
        op_call_impl(static_cast<int>(kind), inputs, outputs, schema_id, attrs_bytes, stream);
      },
      py::arg("kind"), py::arg("inputs"), py::arg("outputs"), py::arg("schema_id") = (uint32_t)0,
      py::arg("attrs_bytes") = py::bytes(), py::arg("stream") = (uint64_t)0);

  m.def(
      "op_call",
      [](int kind, const py::sequence& inputs, const py::sequence& outputs, uint32_t schema_id,
         py::bytes attrs_bytes, uint64_t stream) {
        op_call_impl(kind, inputs, outputs, schema_id, attrs_bytes, stream);
      },
      py::arg("kind"), py::arg("inputs"), py::arg("outputs"), py::arg("schema_id") = (uint32_t)0,
      py::arg("attrs_bytes") = py::bytes(), py::arg("stream") = (uint64_t)0);

  m.def(
      "launch_by_id",
      [](const std::string& kernel_id, OpKind kind, const py::sequence& inputs,
         const py::sequence& outputs, uint32_t schema_id, py::bytes attrs_bytes, uint64_t stream) {
        launch_by_id_impl(kernel_id, static_cast<int>(kind), inputs, outputs, schema_id,
                          attrs_bytes, stream);
      },
      py::arg("kernel_id"), py::arg("kind"), py::arg("inputs"), py::arg("outputs"),
      py::arg("schema_id") = (uint32_t)0, py::arg("attrs_bytes") = py::bytes(),
      py::arg("stream") = (uint64_t)0);

  m.def(
      "trace_enable",
      [](bool flag) {
        std::lock_guard<std::mutex> lock(g_mu);
        g_trace_enabled = flag;
      },
      py::arg("flag") = true);
  m.def("trace_reset", []() {
    std::lock_guard<std::mutex> lock(g_mu);
    g_trace.clear();
  });
  m.def("trace_get", []() {
    std::lock_guard<std::mutex> lock(g_mu);
    return g_trace;
  });

  m.def("graph_begin", []() -> uint64_t {
    {
      std::lock_guard<std::mutex> lock(g_mu);
      g_trace.clear();
    }
    if (std::getenv("AICF_VERBOSE")) std::fprintf(stderr, "[aicf] graph_begin (dedicated stream)\n");
    uint64_t s = 0;
    hip_check(aicf_graph_begin(&s), "hipStreamBeginCapture");
    return s;
  });
  m.def("graph_end", []() { hip_check(aicf_graph_end(), "hipGraphInstantiate"); });
  m.def("graph_launch", []() { hip_check(aicf_graph_launch(current_stream()), "hipGraphLaunch"); });
  m.def("graph_reset", []() {
    hip_check(aicf_graph_reset(), "graph_reset");
    std::lock_guard<std::mutex> lock(g_mu);
    g_trace.clear();
  });
  m.def("graph_stream", []() -> uint64_t { return aicf_graph_stream(); });

  // graph handles (not in the reference binding): several instantiated graphs
  // side by side, re-capture updating the executable in place
  m.def("graph_create", []() -> uint64_t {
    uint64_t h = 0;
    hip_check(aicf_graph_create(&h), "graph_create");
    return h;
  });
  m.def("graph_destroy", [](uint64_t h) { hip_check(aicf_graph_destroy(h), "graph_destroy"); },
        py::arg("handle"));
  m.def(
      "graph_begin_h",
      [](uint64_t h) -> uint64_t {
        {
          std::lock_guard<std::mutex> lock(g_mu);
          g_trace.clear();
        }
        uint64_t s = 0;
        hip_check(aicf_graph_begin_h(h, &s), "hipStreamBeginCapture");
        return s;
      },
      py::arg("handle"));
  m.def("graph_end_h", [](uint64_t h) { hip_check(aicf_graph_end_h(h), "hipGraphInstantiate"); },
        py::arg("handle"));
  m.def(
      "graph_launch_h",
      [](uint64_t h) { hip_check(aicf_graph_launch_h(h, current_stream()), "hipGraphLaunch"); },
      py::arg("handle"));
  // n replays in one call (not in the reference binding): for graphs of a
  // few microseconds the per-call interpreter overhead would otherwise set
  // the replay rate
  m.def(
      "graph_launch_h_n",
      [](uint64_t h, int64_t n) {
        void* s = current_stream();
        for (int64_t i = 0; i < n; ++i) hip_check(aicf_graph_launch_h(h, s), "hipGraphLaunch");
      },
      py::arg("handle"), py::arg("n"));
  m.def("graph_reset_h", [](uint64_t h) { hip_check(aicf_graph_reset_h(h), "graph_reset"); },
        py::arg("handle"));
  m.def("graph_stream_h", [](uint64_t h) -> uint64_t { return aicf_graph_stream_h(h); },
        py::arg("handle"));
  m.def("graph_state_h", [](uint64_t h) -> int { return aicf_graph_state_h(h); }, py::arg("handle"));
  m.def("graph_updates_h", [](uint64_t h) -> uint64_t { return aicf_graph_updates_h(h); },
        py::arg("handle"));

  // introspection helpers (not in the reference binding)
  m.def("registry_kernel_ids", [](int kind) {
    std::vector<std::string> ids;
    const int n = aicf_registry_count(kind);
    for (int i = 0; i < n; ++i) ids.emplace_back(aicf_registry_kernel_id(kind, i));
    return ids;
  });
}
