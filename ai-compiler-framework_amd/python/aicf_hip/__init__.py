"""aicf_hip: execution-plan runtime for the gfx950 backend.

Host-side counterpart of the reference framework's plan path
(python/aicf_fw/core_v2/{ir,lower,plan,kernel_select,exec}.py and
rewrites/stageC_fuse_epilogue.py): a small IR, lowering to the backend's
primitive ops, kernel-id pinning, a binding plan, and a planned executor
that runs the lowered list through aicf_cuda._C or captures it as one
hipGraph.
"""
from .ir import IRGraph, IRNode, IRValue  # noqa: F401
from .lower import (apply_kernel_selection, fuse_gemm_epilogue, lower_to_backend_ops,  # noqa: F401
                    lowered_to_text, compile_lowered)
from .plan import BindingPlan, allocate_static_env, build_binding_plan  # noqa: F401

__all__ = ["IRGraph", "IRNode", "IRValue", "lower_to_backend_ops", "fuse_gemm_epilogue",
           "apply_kernel_selection", "compile_lowered", "lowered_to_text", "BindingPlan",
           "build_binding_plan", "allocate_static_env"]
