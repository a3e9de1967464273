"""The reference's recorded kid-trace graph (python_framework_test/
v2_kid_trace_by_id_test.py:221-328): f16, B=64, D=8, two Linear layers
with ReLU, MSE gradient, backward, and SGD (lr 0.01) on all four params.
Built here with this package's IR so that its IR / lowered / plan dumps and
its by-id runtime trace can be compared with the reference's artifacts."""
from __future__ import annotations

from .ir import IRGraph
from .lower import apply_kernel_selection, fuse_gemm_epilogue, lower_to_backend_ops
from .plan import build_binding_plan

F16 = "torch.float16"


def build_kid_trace_graph(B: int = 64, D: int = 8, lr: float = 1e-2, device: str = "cuda:0"):
    ir = IRGraph(name="v2_kid_trace_by_id_test")
    nv = lambda n, s: ir.new_value(name=n, shape=s, dtype=F16, device=device)  # noqa: E731
    lin = {"bias": True, "layout": "y = x @ W^T + b"}
    x = nv("x", (B, D))
    W0, b0 = nv("0.W", (D, D)), nv("0.b", (D,))
    lin0 = nv("lin0_out", (B, D))
    ir.emit(op="Linear", inputs=[x, W0, b0], outputs=[lin0], attrs=lin)
    r0 = nv("relu0_out", (B, D))
    ir.emit(op="ReLU", inputs=[lin0], outputs=[r0])
    r0s = nv("relu0_saved", (B, D))
    ir.emit(op="Save", inputs=[r0], outputs=[r0s])
    W1, b1 = nv("2.W", (D, D)), nv("2.b", (D,))
    lin1 = nv("lin1_out", (B, D))
    ir.emit(op="Linear", inputs=[r0, W1, b1], outputs=[lin1], attrs=lin)
    t = nv("t", (B, D))
    dY = nv("dY", (B, D))
    ir.emit(op="MseGrad", inputs=[lin1, t], outputs=[dY])
    d_r0, dW1, db1 = nv("d_relu0_out", (B, D)), nv("d_2.W", (D, D)), nv("d_2.b", (D,))
    ir.emit(op="LinearBwd", inputs=[r0, W1, dY], outputs=[d_r0, dW1, db1], attrs=lin)
    d_lin0 = nv("d_lin0_out", (B, D))
    ir.emit(op="ReluBwd", inputs=[d_r0, r0s], outputs=[d_lin0])
    dx, dW0, db0 = nv("d_x", (B, D)), nv("d_0.W", (D, D)), nv("d_0.b", (D,))
    ir.emit(op="LinearBwd", inputs=[x, W0, d_lin0], outputs=[dx, dW0, db0], attrs=lin)
    for p, g in ((W0, dW0), (b0, db0), (W1, dW1), (b1, db1)):
        ir.emit(op="SgdStep", inputs=[p, g], outputs=[p], attrs={"lr": lr})
    # reference order: StageA, StageB (kid pinning), StageC (fusion), fill the fused op's kid
    lowered = lower_to_backend_ops(ir)
    lowered = apply_kernel_selection(ir, lowered)
    lowered = fuse_gemm_epilogue(ir, [dict(it) for it in lowered])
    lowered = apply_kernel_selection(ir, lowered)
    plan = build_binding_plan(ir)
    return ir, lowered, plan
