// Registration table: every kernel id the reference pins
// (src/backends/cuda/registry/register_all.cpp:105-290), with the same
// OpKind, priority and schema gate, mapped to the gfx950 implementations,
// plus the ids of the appended ops.
#include <cstdio>
#include <cstdlib>

#include "../common/registry.hpp"

namespace aicf::hip {

// optim.hip
KernelVariant make_adam_step_f32_variant();
KernelVariant make_adamw_step_f32_variant();
KernelVariant make_biascorr_variant();
KernelVariant make_step_inc_variant();
KernelVariant make_sgd_step_f32_variant();
KernelVariant make_sgd_step_f16_variant();
KernelVariant make_sgd_step_f16_half2_variant();
// eltwise.hip
KernelVariant make_add_f32_variant();
KernelVariant make_add_f16_variant();
KernelVariant make_add_f16_vec2_variant();
KernelVariant make_relu_f32_variant();
KernelVariant make_relu_f16_variant();
KernelVariant make_relu_f16_vec2_variant();
KernelVariant make_relu_bwd_f32_variant();
KernelVariant make_relu_bwd_f16_variant();
KernelVariant make_relu_bwd_f16_vec2_variant();
KernelVariant make_bias_add_f32_variant();
KernelVariant make_bias_add_f16_variant();
KernelVariant make_bias_add_f16_vec2_variant();
KernelVariant make_copy_f32_variant();
KernelVariant make_copy_f16_variant();
KernelVariant make_copy_bf16_variant();
KernelVariant make_grad_zero_variant();
KernelVariant make_mse_grad_f32_variant();
KernelVariant make_mse_grad_f16_variant();
KernelVariant make_mse_loss_grad_variant();
KernelVariant make_gelu_f32_variant();
KernelVariant make_gelu_bf16_variant();
KernelVariant make_gelu_bwd_f32_variant();
KernelVariant make_gelu_bwd_bf16_variant();
KernelVariant make_transpose_variant();
// reduce.hip
KernelVariant make_reduce_sum_lastdim_f32_variant();
KernelVariant make_reduce_sum_lastdim_f16_to_f32_variant();
KernelVariant make_reduce_sum_lastdim_f16_variant();
KernelVariant make_reduce_sum_lastdim_bf16_to_f32_variant();
KernelVariant make_row_softmax_f32_variant();
KernelVariant make_row_reduce_f32_variant();
KernelVariant make_softmax_xent_f32_variant();
// norm.hip
KernelVariant make_layernorm_fwd_f32_variant();
KernelVariant make_layernorm_fwd_f16_variant();
KernelVariant make_layernorm_bwd_f32_variant();
KernelVariant make_layernorm_bwd_f16_variant();
KernelVariant make_batchnorm_fwd_f16_variant();
KernelVariant make_batchnorm_bwd_f16_variant();
// gemm.hip
KernelVariant make_gemm_f32_naive_variant();
KernelVariant make_gemm_f16_tc_wmma_out_f16_variant();
KernelVariant make_gemm_bf16_variant();
KernelVariant make_gemm_bf16_f32out_variant();
KernelVariant make_gemm_bias_relu_f32_naive_variant();
KernelVariant make_gemm_bias_relu_f16_tc_wmma_out_f16_variant();
KernelVariant make_gemm_epilogue_bf16_variant();
KernelVariant make_gemm_epilogue_bf16_f32out_variant();
KernelVariant make_gemm_adamw_bf16_variant();
// smallstep.hip
KernelVariant make_xent_head_f32_variant();
KernelVariant make_xent_head_step_f32_variant();
KernelVariant make_grad_group_f32_variant();
KernelVariant make_grad_group_adamw_f32_variant();
KernelVariant make_gemm_small_bcopy_f32_variant();
KernelVariant make_adamw_multi_f32_variant();
// eltwise.hip / optim.hip (step tail)
KernelVariant make_mse_colsum_variant();
KernelVariant make_colsum_adamw_f32_variant();

void register_all_kernels_into(KernelRegistry& R) {
  if (std::getenv("AICF_VERBOSE")) std::fprintf(stderr, "[aicf] register_all: gfx950 backend\n");
  auto reg = [&R](OpKind k, KernelVariant v, int prio, const char* id) {
    v.priority = prio;
    v.kernel_id = id;
    R.register_kernel(k, v);
  };

  // ReduceSum (reference priorities 115 / 110 / 100)
  reg(OpKind::ReduceSum, make_reduce_sum_lastdim_f16_variant(), 115, "reduce_sum_keep_lastdim_f16_v0");
  reg(OpKind::ReduceSum, make_reduce_sum_lastdim_f16_to_f32_variant(), 110,
      "reduce_sum_keep_lastdim_f16_to_f32_v0");
  reg(OpKind::ReduceSum, make_reduce_sum_lastdim_bf16_to_f32_variant(), 105,
      "reduce_sum_keep_lastdim_bf16_to_f32_v0");
  reg(OpKind::ReduceSum, make_reduce_sum_lastdim_f32_variant(), 100, "reduce_sum_keep_lastdim_f32_v0");

  // Gemm (reference: f16 20, f32 0)
  reg(OpKind::Gemm, make_gemm_f16_tc_wmma_out_f16_variant(), 20, "gemm_f16_tc_wmma_out_f16_v0");
  reg(OpKind::Gemm, make_gemm_bf16_variant(), 15, "gemm_bf16_mfma_v0");
  reg(OpKind::Gemm, make_gemm_bf16_f32out_variant(), 14, "gemm_bf16_mfma_f32out_v0");
  reg(OpKind::Gemm, make_gemm_f32_naive_variant(), 0, "gemm_f32_naive_v0");
  reg(OpKind::Gemm, make_gemm_f32_naive_variant(), 0, "gemm_f32_mfma_v0");

  // GemmEpilogue (reference: f16 20, f32 0)
  reg(OpKind::GemmEpilogue, make_gemm_bias_relu_f16_tc_wmma_out_f16_variant(), 20,
      "gemm_bias_relu_f16_tc_wmma_out_f16_v0");
  reg(OpKind::GemmEpilogue, make_gemm_epilogue_bf16_variant(), 15, "gemm_epilogue_bf16_mfma_v0");
  reg(OpKind::GemmEpilogue, make_gemm_epilogue_bf16_f32out_variant(), 14,
      "gemm_epilogue_bf16_mfma_f32out_v0");
  reg(OpKind::GemmEpilogue, make_gemm_bias_relu_f32_naive_variant(), 0,
      "gemm_bias_relu_f32_naive_v0");
  reg(OpKind::GemmEpilogue, make_gemm_bias_relu_f32_naive_variant(), 0,
      "gemm_epilogue_f32_mfma_v0");
  reg(OpKind::GemmEpilogue, make_gemm_small_bcopy_f32_variant(), 0, "gemm_small_bcopy_f32_v0");

  // BiasAdd (30 / 20 / 0)
  reg(OpKind::BiasAdd, make_bias_add_f16_vec2_variant(), 30, "bias_add_f16_vec2_v0");
  reg(OpKind::BiasAdd, make_bias_add_f16_variant(), 20, "bias_add_f16_v0");
  reg(OpKind::BiasAdd, make_bias_add_f32_variant(), 0, "bias_add_f32_v0");

  // Add (30 / 20 / 0)
  reg(OpKind::EltwiseAdd, make_add_f16_vec2_variant(), 30, "add_f16_vec2_v0");
  reg(OpKind::EltwiseAdd, make_add_f16_variant(), 20, "add_f16_v0");
  reg(OpKind::EltwiseAdd, make_add_f32_variant(), 0, "add_f32_v0");

  // Relu (30 / 20 / 0)
  reg(OpKind::EltwiseRelu, make_relu_f16_vec2_variant(), 30, "relu_f16_vec2_v0");
  reg(OpKind::EltwiseRelu, make_relu_f16_variant(), 20, "relu_f16_v0");
  reg(OpKind::EltwiseRelu, make_relu_f32_variant(), 0, "relu_f32_v0");

  // MseGrad (20 / 0) + fused loss variant (3 outputs)
  reg(OpKind::MseGrad, make_mse_loss_grad_variant(), 40, "mse_loss_grad_v0");
  reg(OpKind::MseGrad, make_mse_grad_f16_variant(), 20, "mse_grad_f16_v0");
  reg(OpKind::MseGrad, make_mse_grad_f32_variant(), 0, "mse_grad_f32_v0");

  // ReluBwd (30 / 20 / 0)
  reg(OpKind::ReluBwd, make_relu_bwd_f16_vec2_variant(), 30, "relu_bwd_f16_vec2_v0");
  reg(OpKind::ReluBwd, make_relu_bwd_f16_variant(), 20, "relu_bwd_f16_v0");
  reg(OpKind::ReluBwd, make_relu_bwd_f32_variant(), 0, "relu_bwd_f32_v0");

  // SgdStep (30 / 20 / 0)
  reg(OpKind::SgdStep, make_sgd_step_f16_half2_variant(), 30, "sgd_step_f16_half2_v0");
  reg(OpKind::SgdStep, make_sgd_step_f16_variant(), 20, "sgd_step_f16_v0");
  reg(OpKind::SgdStep, make_sgd_step_f32_variant(), 0, "sgd_step_f32_v0");

  // Copy (20 / 0) + bf16
  reg(OpKind::Copy, make_copy_f16_variant(), 20, "copy_f16_v0");
  reg(OpKind::Copy, make_copy_bf16_variant(), 10, "copy_bf16_v0");
  reg(OpKind::Copy, make_copy_f32_variant(), 0, "copy_f32_v0");

  reg(OpKind::GradZero, make_grad_zero_variant(), 0, "grad_zero_v0");

  // AdamStep: reference contract (6 inputs) and the AdamW variant (5 inputs)
  reg(OpKind::AdamStep, make_adamw_step_f32_variant(), 10, "adamw_step_f32_v1");
  reg(OpKind::AdamStep, make_adam_step_f32_variant(), 0, "adam_step_f32_v0");

  reg(OpKind::StepInc, make_step_inc_variant(), 0, "step_inc_v0");
  reg(OpKind::BiasCorr, make_biascorr_variant(), 0, "bias_corr_v0");

  // LayerNorm / BatchNorm (reference: f16 10, f32 0)
  reg(OpKind::LayerNormFwd, make_layernorm_fwd_f16_variant(), 10, "layernorm_fwd_f16_v0");
  reg(OpKind::LayerNormFwd, make_layernorm_fwd_f32_variant(), 0, "layernorm_fwd_f32_v0");
  reg(OpKind::LayerNormBwd, make_layernorm_bwd_f16_variant(), 10, "layernorm_bwd_f16_v0");
  reg(OpKind::LayerNormBwd, make_layernorm_bwd_f32_variant(), 0, "layernorm_bwd_f32_v0");
  reg(OpKind::BatchNormFwd, make_batchnorm_fwd_f16_variant(), 10, "batchnorm_fwd_f16_v0");
  reg(OpKind::BatchNormBwd, make_batchnorm_bwd_f16_variant(), 10, "batchnorm_bwd_f16_v0");

  // appended kinds
  reg(OpKind::RowSoftmax, make_row_softmax_f32_variant(), 0, "row_softmax_f32_v0");
  reg(OpKind::RowReduce, make_row_reduce_f32_variant(), 0, "row_reduce_f32_v0");
  reg(OpKind::SoftmaxXent, make_softmax_xent_f32_variant(), 0, "softmax_xent_f32_v0");
  reg(OpKind::GeluBwd, make_gelu_bwd_bf16_variant(), 10, "gelu_bwd_bf16_v0");
  reg(OpKind::GeluBwd, make_gelu_bwd_f32_variant(), 0, "gelu_bwd_f32_v0");
  reg(OpKind::EltwiseGelu, make_gelu_bf16_variant(), 10, "gelu_bf16_v0");
  reg(OpKind::EltwiseGelu, make_gelu_f32_variant(), 0, "gelu_f32_v0");
  reg(OpKind::Transpose, make_transpose_variant(), 0, "transpose2d_v0");
  reg(OpKind::GemmAdamW, make_gemm_adamw_bf16_variant(), 0, "gemm_adamw_bf16_v0");
  reg(OpKind::XentHead, make_xent_head_f32_variant(), 0, "xent_head_f32_v0");
  reg(OpKind::XentHead, make_xent_head_step_f32_variant(), 0, "xent_head_step_f32_v0");
  reg(OpKind::GradGroup, make_grad_group_f32_variant(), 0, "grad_group_f32_v0");
  reg(OpKind::GradGroup, make_grad_group_adamw_f32_variant(), 0, "grad_group_adamw_f32_v0");
  reg(OpKind::AdamWMulti, make_adamw_multi_f32_variant(), 0, "adamw_multi_f32_v0");
  reg(OpKind::MseColsum, make_mse_colsum_variant(), 0, "mse_colsum_v0");
  reg(OpKind::ColsumAdamW, make_colsum_adamw_f32_variant(), 0, "colsum_adamw_f32_v0");
}

}  // namespace aicf::hip
