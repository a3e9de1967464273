"""Framework-level train-step handle over the plan runtime: host-managed
optimizer meta, warmup, eager steps, capture and replay.

Mirrors the reference's user-facing layer:
  * Adam (python/aicf_fw/optim/adam.py:6-50): per-parameter m/v state and
    the bias-correction meta bc1_inv = 1/(1-beta1^t), bc2_inv = 1/(1-beta2^t)
    as device scalars that update_meta() refills in place each step, so a
    captured graph reads the current values on every replay;
  * CompiledTrainStep (python/aicf_fw/fw/train_step.py:15-101): warmup runs
    before the first step or capture (fail-fast when warmup is required but
    disabled or has no inputs), train_step = update_meta + run, capture
    after warmup, replay(n, sync), reset;
  * build_fw_mvp: the graph of the reference's fw MVP user test
    (python/python_framework_test/python_framework_test.py:29-56):
    Linear(D, D) -> ReLU -> Linear(D, D), MSE gradient against t, Adam with
    the reference kernel contract adam_step(P, G, M, V, bc1_inv, bc2_inv)
    (adam_step/launcher.cu:257-293).  The reference's compile entry point
    (aicf_fw.fw.compile) is not in its tree; this builder produces the
    graph that test drives.
"""
from __future__ import annotations

from typing import Dict, Iterable, Optional, Tuple

import torch

from .executor import ExecOptions, PlannedExecutor
from .ir import IRGraph
from .lower import compile_lowered
from .plan import build_binding_plan

F32 = "torch.float32"
BC1_NAME = "opt.bc1_inv"
BC2_NAME = "opt.bc2_inv"


def opt_m_name(pname: str) -> str:
    return f"opt.m.{pname}"


def opt_v_name(pname: str) -> str:
    return f"opt.v.{pname}"


def _named(params) -> Iterable[Tuple[str, torch.Tensor]]:
    if hasattr(params, "named_parameters"):
        return list(params.named_parameters())
    return list(dict(params).items())


class Adam:
    """Host-managed Adam meta and state (optim/adam.py:6-50).  `params` is a
    model with named_parameters() or a name -> tensor mapping."""

    def __init__(self, params, lr: float = 1e-3, beta1: float = 0.9, beta2: float = 0.999,
                 eps: float = 1e-8, dtype: torch.dtype = torch.float32):
        self.lr, self.beta1, self.beta2, self.eps = float(lr), float(beta1), float(beta2), float(eps)
        named = _named(params)
        assert len(named) > 0
        dev = named[0][1].device
        self.step_host = 0
        self.bc1_inv = torch.ones((), device=dev, dtype=dtype)
        self.bc2_inv = torch.ones((), device=dev, dtype=dtype)
        self.m: Dict[str, torch.Tensor] = {n: torch.zeros_like(p) for n, p in named}
        self.v: Dict[str, torch.Tensor] = {n: torch.zeros_like(p) for n, p in named}

    def update_meta(self) -> None:
        """Advances the host step and refills the bias-correction scalars in
        place (fill_ on torch's current stream; a replay launched after it is
        ordered behind it)."""
        self.step_host += 1
        self.bc1_inv.fill_(float(1.0 / (1.0 - self.beta1 ** self.step_host)))
        self.bc2_inv.fill_(float(1.0 / (1.0 - self.beta2 ** self.step_host)))

    def named_state_tensors(self) -> Dict[str, torch.Tensor]:
        d: Dict[str, torch.Tensor] = {BC1_NAME: self.bc1_inv, BC2_NAME: self.bc2_inv}
        for n in self.m:
            d[opt_m_name(n)] = self.m[n]
            d[opt_v_name(n)] = self.v[n]
        return d

    def hyper(self) -> Dict[str, float]:
        return {"lr": self.lr, "beta1": self.beta1, "beta2": self.beta2, "eps": self.eps}


class CompiledTrainStep:
    """fw/train_step.py:15-101 over PlannedExecutor."""

    def __init__(self, *, ir, lowered, plan, ex: PlannedExecutor, params: Dict[str, torch.Tensor],
                 statics: Dict[str, torch.Tensor], optimizer, warmup_runs: int = 2,
                 warmup_required: bool = True):
        self.ir, self.lowered, self.plan, self.ex = ir, lowered, plan, ex
        self.params = params
        self.statics = statics
        self.optimizer = optimizer
        self.warmup_runs = int(warmup_runs)
        self.warmup_required = bool(warmup_required)
        self._warmed_up = False

    def _bind_all(self) -> Dict[str, torch.Tensor]:
        d: Dict[str, torch.Tensor] = {}
        d.update(self.params)
        d.update(self.statics)
        return d

    def _maybe_warmup(self, inputs: Optional[Dict[str, torch.Tensor]]) -> None:
        if self._warmed_up:
            return
        if self.warmup_runs <= 0:
            if self.warmup_required:
                raise RuntimeError(
                    "Warmup is disabled (warmup_runs=0 or AICF_WARMUP=0) but warmup_required=True.\n"
                    "This can lead to no-op updates due to unmaterialized static/state buffers.\n"
                    "Fix: set warmup_runs>=1, or pass warmup_inputs to compile_train_step(), "
                    "or disable warmup_required explicitly.")
            return
        if inputs is None:
            raise RuntimeError(
                "Warmup is required but no inputs were provided.\n"
                "Fix: call compiled.warmup(example_inputs) once, or pass warmup_inputs=... to "
                "compile_train_step().")
        self.warmup(inputs, n=self.warmup_runs)

    def warmup(self, inputs: Dict[str, torch.Tensor], n: int = 2, reuse_static: bool = True) -> None:
        for _ in range(int(n)):
            self.optimizer.update_meta()
            torch.cuda.synchronize()
            self.ex.run(inputs=inputs, params=self._bind_all(), reuse_static=reuse_static)
        self._warmed_up = True

    def run(self, inputs: Dict[str, torch.Tensor], reuse_static: bool = True):
        return self.ex.run(inputs=inputs, params=self._bind_all(), reuse_static=reuse_static)

    def train_step(self, inputs: Dict[str, torch.Tensor], reuse_static: bool = True):
        self._maybe_warmup(inputs)
        self.optimizer.update_meta()
        torch.cuda.synchronize()
        return self.run(inputs, reuse_static=reuse_static)

    def capture(self, inputs: Dict[str, torch.Tensor], reuse_static: bool = True) -> None:
        self._maybe_warmup(inputs)
        self.ex.reset_graph()
        self.ex.capture(inputs=inputs, params=self._bind_all(), reuse_static=reuse_static)

    def replay(self, n: int = 1, sync: bool = False) -> None:
        self.ex.replay(n=int(n))
        if sync:
            torch.cuda.synchronize()

    def reset(self) -> None:
        self.ex.reset_graph()


def build_fw_mvp(B: int = 64, D: int = 8, *, lr: float = 1e-3, beta1: float = 0.9,
                 beta2: float = 0.999, eps: float = 1e-8, device: str = "cuda:0"):
    """IR, lowered op list and binding plan of the fw MVP train step:
    y = Linear2(relu(Linear0(x))), dY = mse_grad(y, t) (scale 2/numel),
    backward through both layers, then adam_step on 0.W, 0.b, 2.W, 2.b with
    the host-managed bc1_inv / bc2_inv scalars."""
    ir = IRGraph(name=f"fw_mvp_train_step_{B}x{D}")
    nv = lambda n, s: ir.new_value(name=n, shape=s, dtype=F32, device=device)  # noqa: E731
    x, t = nv("x", (B, D)), nv("t", (B, D))
    W0, b0, W1, b1 = nv("0.W", (D, D)), nv("0.b", (D,)), nv("2.W", (D, D)), nv("2.b", (D,))
    lin0, h, hs, y = nv("lin0_out", (B, D)), nv("relu0_out", (B, D)), nv("relu0_saved", (B, D)), nv("y", (B, D))
    dY = nv("dY", (B, D))
    dh, dlin0, dx = nv("d_relu0_out", (B, D)), nv("d_lin0_out", (B, D)), nv("d_x", (B, D))
    dW1, db1, dW0, db0 = nv("d_2.W", (D, D)), nv("d_2.b", (D,)), nv("d_0.W", (D, D)), nv("d_0.b", (D,))
    bc1, bc2 = nv(BC1_NAME, ()), nv(BC2_NAME, ())
    lin = {"bias": True, "layout": "y = x @ W^T + b"}
    ir.emit(op="Linear", inputs=[x, W0, b0], outputs=[lin0], attrs=lin)
    ir.emit(op="ReLU", inputs=[lin0], outputs=[h])
    ir.emit(op="Save", inputs=[h], outputs=[hs])
    ir.emit(op="Linear", inputs=[h, W1, b1], outputs=[y], attrs=lin)
    ir.emit(op="MseGrad", inputs=[y, t], outputs=[dY])
    ir.emit(op="LinearBwd", inputs=[h, W1, dY], outputs=[dh, dW1, db1], attrs=lin)
    ir.emit(op="ReluBwd", inputs=[dh, hs], outputs=[dlin0])
    ir.emit(op="LinearBwd", inputs=[x, W0, dlin0], outputs=[dx, dW0, db0], attrs=lin)
    hp = {"lr": lr, "beta1": beta1, "beta2": beta2, "eps": eps}
    for p, g in ((W0, dW0), (b0, db0), (W1, dW1), (b1, db1)):
        m, v = nv(opt_m_name(p.name), p.shape), nv(opt_v_name(p.name), p.shape)
        ir.emit(op="AdamStep", inputs=[p, g, m, v, bc1, bc2], outputs=[p, m, v], attrs=hp)
    lowered = compile_lowered(ir)
    plan = build_binding_plan(ir)
    return ir, lowered, plan


def compile_fw_mvp(params: Dict[str, torch.Tensor], optimizer: Adam, *, B: int, D: int,
                   device: str = "cuda:0", warmup_runs: int = 2,
                   warmup_inputs: Optional[Dict[str, torch.Tensor]] = None,
                   warmup_required: bool = True, own_graph: bool = False) -> CompiledTrainStep:
    """Compiled train step of the fw MVP graph bound to `params` (names 0.W,
    0.b, 2.W, 2.b) and the optimizer's state; runs the warmup at once when
    warmup_inputs are given, as the reference's compile() does."""
    ir, lowered, plan = build_fw_mvp(B, D, lr=optimizer.lr, beta1=optimizer.beta1,
                                     beta2=optimizer.beta2, eps=optimizer.eps, device=device)
    ex = PlannedExecutor(ir=ir, lowered=lowered, plan=plan, device=torch.device(device),
                         opts=ExecOptions(require_kernel_id=True), own_graph=own_graph)
    ts = CompiledTrainStep(ir=ir, lowered=lowered, plan=plan, ex=ex, params=dict(params),
                           statics=optimizer.named_state_tensors(), optimizer=optimizer,
                           warmup_runs=warmup_runs, warmup_required=warmup_required)
    if warmup_inputs is not None:
        ts._maybe_warmup(warmup_inputs)
    return ts
