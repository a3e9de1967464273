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
initialise inputs/parameters from a seed and to check a step against the
CPU oracle (tests only: the oracle is imported lazily inside the checks).
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
                   eps: float = 1e-8, device: str = "cuda:0"):
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
    lowered = compile_lowered(ir)
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
                  fuse_colsum: bool = False, device: str = "cuda:0"):
    """bf16 activations/weights, fp32 master parameters in one flat buffer.
    The GEMM kernel reads M/N-contiguous operands in place; StageD
    (nt_layout) may still insert explicit transposes: "cost" where a
    transpose is cheaper than the in-place read (none at the measured
    in-place cost of this kernel), True for every such operand, False for
    none.  fuse_optimizer: each weight-gradient GEMM applies AdamW to its
    layer's weights in its epilogue (StageE); the flat step then covers the
    biases only.  fuse_colsum: the bias gradients of the hidden layers are
    column-summed in the epilogue of the dGELU GEMM that produces their
    input (StageC')."""
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
                              fuse_optimizer=fuse_optimizer, fuse_colsum=fuse_colsum)
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


# ============================================================ oracle checks
def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.float().numpy()
    return t.numpy()


def check_mlp_small(device: str = "cuda:0", verbose: bool = False, B=64, din=784, dh=256,
                    dout=10) -> Dict[str, object]:
    """Runs one eager step and one captured+replayed step of the xent MLP and
    checks loss, argmax, every gradient and every updated parameter against
    the CPU oracle (fp64 chain for loss/grads; the reference-exact AdamW
    restatement applied to the GPU's own gradients for the update)."""
    import oracle as orc  # test infrastructure

    ir, lowered, plan = build_mlp_xent(B, din, dh, dout, device=device)
    data = init_mlp_xent(B, din, dh, dout)
    params = {k: torch.from_numpy(v.copy()).to(device) for k, v in data.items() if "." in k}
    inputs = {"x": torch.from_numpy(data["x"]).to(device), "t": torch.from_numpy(data["t"]).to(device)}
    ex = make_executor(ir, lowered, plan, device)
    res: Dict[str, object] = {"ok": True}

    def expect(step_params, t):
        x = data["x"].astype(np.float64)
        W0, b0, W1, b1 = (step_params[k].astype(np.float64) for k in ("0.W", "0.b", "2.W", "2.b"))
        z1 = x @ W0.T + b0
        hh = np.maximum(z1, 0)
        logits = (hh @ W1.T + b1).astype(np.float32)
        loss, dz, am, _ = orc.softmax_xent_f64(logits, data["t"])
        grads = {"2.W": dz.T @ hh, "2.b": dz.sum(0)}
        dhh = (dz @ W1) * (hh > 0)
        grads["0.W"] = dhh.T @ x
        grads["0.b"] = dhh.sum(0)
        return loss, am, grads

    def check(tag, prev, t):
        loss, am, grads = expect(prev, t)
        gl = float(ex.value("loss").item())
        res[f"{tag}_loss_rel"] = abs(gl - loss) / abs(loss)
        ok = res[f"{tag}_loss_rel"] < 1e-5
        ok &= bool(np.array_equal(_np(ex.value("pred")), am))
        new = {}
        for k in ("0.W", "0.b", "2.W", "2.b"):
            g = _np(ex.value(f"d_{k}"))
            e = orc.rel_err(g, grads[k])
            res[f"{tag}_grad_{k}"] = e
            ok &= e < 1e-4
            m_prev = prev_m[k]
            v_prev = prev_v[k]
            pr, mr, vr = orc.adamw(prev[k], g, m_prev, v_prev, t)
            got = _np(params[k])
            ok &= bool(np.array_equal(got.ravel(), pr))
            res[f"{tag}_update_exact_{k}"] = bool(np.array_equal(got.ravel(), pr))
            new[k] = got.copy()
            prev_m[k], prev_v[k] = mr, vr
        return ok, new

    prev = {k: data[k].copy() for k in ("0.W", "0.b", "2.W", "2.b")}
    prev_m = {k: np.zeros(v.size, np.float32) for k, v in prev.items()}
    prev_v = {k: np.zeros(v.size, np.float32) for k, v in prev.items()}
    ex.run(inputs=inputs, params=params, reuse_static=False)
    torch.cuda.synchronize()
    ok, prev = check("eager", prev, 1)
    res["ok"] = bool(res["ok"] and ok)
    # capture the same step and replay it twice (steps 2 and 3)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    for t in (2, 3):
        ex.replay(1)
        torch.cuda.synchronize()
        ok, prev = check(f"replay{t}", prev, t)
        res["ok"] = bool(res["ok"] and ok)
    res["kernel_ids"] = sorted({it.get("kernel_id") for it in lowered})
    ex.reset_graph()
    if verbose:
        print("[mlp] check", res)
    return res


def check_mlp_mse_small(B: int = 256, D: int = 256, L: int = 4, device: str = "cuda:0",
                        steps: int = 3, nt_layout=False, fuse_colsum: bool = False) -> Dict[str, object]:
    """Runs the bf16 MSE MLP (same graph and kernels as the benchmark, smaller
    shape) eagerly for one step and as a captured graph for `steps`-1 more,
    and checks each step against the CPU oracle: an fp64 chain that rounds
    every stored bf16 tensor as the kernels do (loss, all dW / db, rel-err
    <= 1e-2), and the reference-exact AdamW restatement applied to the GPU's
    own gradients (updated parameters, moments and bf16 shadow bit-exact)."""
    import oracle as orc  # test infrastructure

    # nt_min_flops=0: with nt_layout, take the transpose + NT-kernel route at
    # every size
    ir, lowered, plan = build_mlp_mse(B, D, L, device=device, nt_layout=nt_layout, nt_min_flops=0,
                                      fuse_colsum=fuse_colsum)
    lay = FlatLayout(D, L)
    ex = make_executor(ir, lowered, plan, device)
    inputs, params = init_mlp_mse(B, D, L, seed=1, device=device)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    refresh_shadow(ex)
    torch.cuda.synchronize()
    X = _np(inputs["x"]).astype(np.float64)
    T = _np(inputs["t"]).astype(np.float64)
    q = lambda a: orc.bf16_round(np.asarray(a, np.float32)).astype(np.float64)  # noqa: E731
    res: Dict[str, object] = {"ok": True}
    Pm = _np(params["flat.params"]).copy()
    Mm = np.zeros_like(Pm)
    Vm = np.zeros_like(Pm)

    def expect(P):
        Wb = [q(P[lay.w_off(i):lay.w_off(i) + D * D].reshape(D, D)) for i in range(1, L + 1)]
        bs = [P[lay.b_off(i):lay.b_off(i) + D].astype(np.float64) for i in range(1, L + 1)]
        hs, zs = [X], []
        for i in range(L - 1):
            v = hs[-1] @ Wb[i].T + bs[i]
            zs.append(q(v))
            hs.append(q(orc.gelu_f64(v)))
        y = q(hs[-1] @ Wb[L - 1].T + bs[L - 1])
        n = B * D
        loss = float(np.mean((y - T) ** 2))
        dy = q((y - T) * np.float32(2.0 / n))
        grads = {}
        for i in range(L - 1, -1, -1):
            grads[f"{i + 1}.W"] = dy.T @ hs[i]
            grads[f"{i + 1}.b"] = dy.sum(0)
            if i > 0:
                dy = q((dy @ Wb[i]) * orc.gelu_grad_f64(zs[i - 1]))
        return loss, grads

    def check(tag, t):
        nonlocal Pm, Mm, Vm
        loss, grads = expect(Pm)
        gl = float(ex.value("loss").item())
        res[f"{tag}_loss_rel"] = abs(gl - loss) / loss
        ok = res[f"{tag}_loss_rel"] < 1e-2
        G = _np(ex.value("grad.flat"))
        for i in range(1, L + 1):
            for k, off, n in ((f"{i}.W", lay.w_off(i), D * D), (f"{i}.b", lay.b_off(i), D)):
                e = orc.rel_err(G[off:off + n], grads[k].ravel())
                res[f"{tag}_grad_{k}"] = e
                ok &= e < 1e-2
        Pr, Mr, Vr, Wr = orc.adamw(Pm, G, Mm, Vm, t, 1e-3, 0.9, 0.999, 1e-8, 0.0, shadow=True)
        exact = (np.array_equal(_np(ex.value("flat.params")), Pr)
                 and np.array_equal(_np(ex.value("opt.m.flat")), Mr)
                 and np.array_equal(_np(ex.value("opt.v.flat")), Vr)
                 and np.array_equal(ex.value("wb.flat").view(torch.int16).cpu().numpy().view(np.uint16), Wr))
        res[f"{tag}_adamw_exact"] = bool(exact)
        ok &= exact
        Pm, Mm, Vm = Pr, Mr, Vr
        res["ok"] = bool(res["ok"] and ok)

    ex.run(inputs=inputs, params=params, reuse_static=True)
    torch.cuda.synchronize()
    check("eager", 1)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    for t in range(2, steps + 1):
        ex.replay(1)
        torch.cuda.synchronize()
        check(f"replay{t}", t)
    ex.reset_graph()
    return res
