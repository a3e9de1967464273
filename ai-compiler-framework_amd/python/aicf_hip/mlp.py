"""MLP train-step graphs on the plan runtime.

* build_mlp_xent: the reference-style 2-layer MLP (Linear -> ReLU ->
  Linear, softmax cross-entropy (mean), Adam); fp32.  At batch 64,
  784 -> 256 -> 10 this is the CPU-runnable configuration of the benchmark.
* build_mlp_mse: an L-layer bf16 MLP (GELU between layers, MSE loss) whose
  parameters, gradients and Adam moments each live in one flat fp32 buffer
  (bf16 shadow weights in a flat bf16 buffer), so the optimizer is one
  streaming AdamW launch over every parameter.  At batch 8192, 4 x 4096^2
  this is the hipGraph benchmark step.

Both return (ir, lowered, plan) ready for PlannedExecutor, plus helpers to
initialise inputs/parameters from a seed.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from .executor import ExecOptions, PlannedExecutor
from .ir import IRGraph
from .lower import compile_lowered
from .plan import BindingPlan, PlanOptions, build_binding_plan

F32, BF16, I32 = "torch.float32", "torch.bfloat16", "torch.int32"


# ============================================================ xent MLP (fp32)
def build_mlp_xent(B: int = 64, din: int = 784, dh: int = 256, dout: int = 10, *,
                   lr: float = 1e-3, beta1: float = 0.9, beta2: float = 0.999,
                   eps: float = 1e-8, device: str = "cuda:0", fuse_small=False):
    """fuse_small: StageF, the step in three launches (forward GEMM that
    also copies W0 for the input gradient, xent head that advances the step
    counter, gradient group with each AdamW update applied where its gradient
    is stored); "four": StageF with the updates in a multi-tensor AdamW
    launch of their own; off, the lowering is the reference pipeline's (17
    ops)."""
    ir = IRGraph(name=f"mlp_xent_{B}x{din}x{dh}x{dout}")
    nv = lambda n, s, dt=F32: ir.new_value(name=n, shape=s, dtype=dt, device=device)  # noqa: E731
    x = nv("x", (B, din))
    W0, b0 = nv("0.W", (dh, din)), nv("0.b", (dh,))
    lin0 = nv("lin0_out", (B, dh))
    h = nv("relu0_out", (B, dh))
    hs = nv("relu0_saved", (B, dh))
    W1, b1 = nv("2.W", (dout, dh)), nv("2.b", (dout,))
    logits = nv("logits", (B, dout))
    t = nv("t", (B,), I32)
    loss = nv("loss", ())
    dY = nv("dY", (B, dout))
    pred = nv("pred", (B,), I32)
    row_loss = nv("row_loss", (B,))
    dh_ = nv("d_relu0_out", (B, dh))
    dW1, db1 = nv("d_2.W", (dout, dh)), nv("d_2.b", (dout,))
    dlin0 = nv("d_lin0_out", (B, dh))
    dx = nv("d_x", (B, din))
    dW0, db0 = nv("d_0.W", (dh, din)), nv("d_0.b", (dh,))
    step = nv("opt.step", (), I32)
    lin = {"bias": True, "layout": "y = x @ W^T + b"}
    ir.emit(op="Linear", inputs=[x, W0, b0], outputs=[lin0], attrs=lin)
    ir.emit(op="ReLU", inputs=[lin0], outputs=[h])
    ir.emit(op="Save", inputs=[h], outputs=[hs])
    ir.emit(op="Linear", inputs=[h, W1, b1], outputs=[logits], attrs=lin)
    ir.emit(op="SoftmaxXent", inputs=[logits, t], outputs=[loss, dY, pred, row_loss])
    ir.emit(op="LinearBwd", inputs=[h, W1, dY], outputs=[dh_, dW1, db1], attrs=lin)
    ir.emit(op="ReluBwd", inputs=[dh_, hs], outputs=[dlin0])
    ir.emit(op="LinearBwd", inputs=[x, W0, dlin0], outputs=[dx, dW0, db0], attrs=lin)
    ir.emit(op="StepInc", inputs=[step], outputs=[step])
    hp = {"lr": lr, "beta1": beta1, "beta2": beta2, "eps": eps, "weight_decay": 0.0}
    for p, g in ((W0, dW0), (b0, db0), (W1, dW1), (b1, db1)):
        m = nv(f"opt.m.{p.name}", p.shape)
        v = nv(f"opt.v.{p.name}", p.shape)
        ir.emit(op="AdamWStep", inputs=[p, g, m, v, step], outputs=[p, m, v], attrs=hp)
    lowered = compile_lowered(ir, fuse_small=fuse_small)
    plan = build_binding_plan(ir)
    return ir, lowered, plan


def kaiming_uniform(rng: np.random.Generator, out_f: int, in_f: int) -> np.ndarray:
    b = math.sqrt(6.0 / in_f)
    return rng.uniform(-b, b, (out_f, in_f)).astype(np.float32)


def init_mlp_xent(B=64, din=784, dh=256, dout=10, seed=0):
    r = np.random.default_rng(seed)
    return {
        "x": r.standard_normal((B, din)).astype(np.float32),
        "t": r.integers(0, dout, B).astype(np.int32),
        "0.W": kaiming_uniform(r, dh, din), "0.b": np.zeros(dh, np.float32),
        "2.W": kaiming_uniform(r, dout, dh), "2.b": np.zeros(dout, np.float32),
    }


# ============================================================ bf16 MSE MLP
@dataclass
class FlatLayout:
    """Element offsets in the flat parameter buffer (and in the gradient,
    moment and bf16-shadow buffers laid out alike): the L weight matrices
    first, then the L biases, so that once the weight ranges are updated by
    fused GEMM epilogues the biases are one contiguous range for one AdamW
    launch."""
    D: int
    L: int

    @property
    def per_layer(self) -> int:
        return self.D * self.D + self.D

    @property
    def total(self) -> int:
        return self.per_layer * self.L

    def w_off(self, i: int) -> int:  # layer i in 1..L
        return (i - 1) * self.D * self.D

    def b_off(self, i: int) -> int:
        return self.L * self.D * self.D + (i - 1) * self.D


def build_mlp_mse(B: int = 8192, D: int = 4096, L: int = 4, *, lr: float = 1e-3,
                  beta1: float = 0.9, beta2: float = 0.999, eps: float = 1e-8,
                  weight_decay: float = 0.0, dead_dx: bool = True, nt_layout="cost",
                  nt_min_flops: float = 2.0 ** 30, fuse_optimizer: bool = False,
                  fuse_colsum: bool = False, fuse_tail: bool = False, device: str = "cuda:0"):
    """bf16 activations/weights, fp32 master parameters in one flat buffer.
    The GEMM kernel reads M/N-contiguous operands in place; StageD
    (nt_layout) may still insert explicit transposes: "cost" where a
    transpose is cheaper than the in-place read (none at the measured
    in-place cost of this kernel), True for every such operand, False for
    none.  fuse_optimizer: each weight-gradient GEMM applies AdamW to its
    layer's weights in its epilogue (StageE); the flat step then covers the
    biases only.  fuse_colsum: the bias gradients of the hidden layers are
    column-summed in the epilogue of the dGELU GEMM that produces their
    input (StageC').  fuse_tail: the loss, the bias gradients' column-sum
    finishes, step_inc and the bias AdamW in two launches (StageG)."""
    ir = IRGraph(name=f"mlp_mse_{B}x{D}x{L}")
    lay = FlatLayout(D, L)
    nv = lambda n, s, dt=F32, view=None: ir.new_value(name=n, shape=s, dtype=dt,  # noqa: E731
                                                      device=device, view_of=view)
    P = nv("flat.params", (lay.total,))
    Gf = nv("grad.flat", (lay.total,))
    Mf = nv("opt.m.flat", (lay.total,))
    Vf = nv("opt.v.flat", (lay.total,))
    Wb = nv("wb.flat", (lay.total,), BF16)
    step = nv("opt.step", (), I32)
    x = nv("x", (B, D), BF16)
    t = nv("t", (B, D))
    W, Wbv, bias, dW, db = {}, {}, {}, {}, {}
    for i in range(1, L + 1):
        W[i] = nv(f"{i}.W", (D, D), F32, (P.id, lay.w_off(i)))
        bias[i] = nv(f"{i}.b", (D,), F32, (P.id, lay.b_off(i)))
        Wbv[i] = nv(f"wb.{i}.W", (D, D), BF16, (Wb.id, lay.w_off(i)))
        dW[i] = nv(f"d_{i}.W", (D, D), F32, (Gf.id, lay.w_off(i)))
        db[i] = nv(f"d_{i}.b", (D,), F32, (Gf.id, lay.b_off(i)))
    lin = {"bias": True, "layout": "y = x @ W^T + b"}
    h: Dict[int, object] = {0: x}
    z: Dict[int, object] = {}
    for i in range(1, L):
        z[i] = nv(f"z{i}", (B, D), BF16)
        h[i] = nv(f"h{i}", (B, D), BF16)
        ir.emit(op="Linear", inputs=[h[i - 1], Wbv[i], bias[i]], outputs=[z[i]], attrs=lin)
        ir.emit(op="Gelu", inputs=[z[i]], outputs=[h[i]], attrs={"save_preact": True})
    y = nv("y", (B, D), BF16)
    ir.emit(op="Linear", inputs=[h[L - 1], Wbv[L], bias[L]], outputs=[y], attrs=lin)
    dY = nv("dY", (B, D), BF16)
    loss = nv("loss", ())
    # one partial per 2048 elements lets the loss kernel use its one-shot pass
    mse_ws = nv("mse.partials", (max(1024, -(-B * D // 2048)),))
    ir.emit(op="MseLoss", inputs=[y, t], outputs=[dY, loss, mse_ws])
    db_ws = nv("db.partials", (64, D))
    dcur = dY
    for i in range(L, 0, -1):
        dh = nv(f"d_h{i - 1}" if i > 1 else "d_x", (B, D), BF16)
        need_dx = i > 1 or dead_dx
        ir.emit(op="LinearBwd", inputs=[h[i - 1], Wbv[i], dcur], outputs=[dh, dW[i], db[i]],
                attrs=dict(lin, db_workspace=db_ws.id, need_dx=need_dx))
        if i > 1:
            dz = nv(f"d_z{i - 1}", (B, D), BF16)
            ir.emit(op="GeluBwd", inputs=[dh, z[i - 1]], outputs=[dz])
            dcur = dz
    ir.emit(op="StepInc", inputs=[step], outputs=[step])
    ir.emit(op="AdamWStep", inputs=[P, Gf, Mf, Vf, step], outputs=[P, Mf, Vf, Wb],
            attrs={"lr": lr, "beta1": beta1, "beta2": beta2, "eps": eps,
                   "weight_decay": weight_decay})
    lowered = compile_lowered(ir, fuse_bias=True, nt_layout=nt_layout, nt_min_flops=nt_min_flops,
                              fuse_optimizer=fuse_optimizer, fuse_colsum=fuse_colsum, fuse_tail=fuse_tail)
    plan = build_binding_plan(ir, opts=PlanOptions(param_names={"flat.params"}))
    return ir, lowered, plan


def init_mlp_mse(B: int, D: int, L: int, seed: int = 0, device: str = "cuda:0"):
    """Synthetic data and Kaiming-uniform weights generated on the device
    (seeded torch generator): x ~ N(0,1) in bf16, t ~ N(0,1) fp32, zero biases."""
    lay = FlatLayout(D, L)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    P = torch.zeros(lay.total, device=device, dtype=torch.float32)
    bound = math.sqrt(6.0 / D)
    for i in range(1, L + 1):
        w = P[lay.w_off(i):lay.w_off(i) + D * D]
        w.uniform_(-bound, bound, generator=gen)
    x = torch.randn((B, D), device=device, dtype=torch.float32, generator=gen).to(torch.bfloat16)
    t = torch.randn((B, D), device=device, dtype=torch.float32, generator=gen)
    return {"x": x, "t": t}, {"flat.params": P}


def make_executor(ir, lowered, plan, device="cuda:0", require_kernel_id=True,
                  own_graph=False) -> PlannedExecutor:
    return PlannedExecutor(ir=ir, lowered=lowered, plan=plan, device=torch.device(device),
                           opts=ExecOptions(require_kernel_id=require_kernel_id), own_graph=own_graph)


def refresh_shadow(ex: PlannedExecutor) -> None:
    """bf16 shadow of the fp32 master weights (before the first step)."""
    ex.value("wb.flat").copy_(ex.value("flat.params").to(torch.bfloat16))
