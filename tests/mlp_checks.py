"""CPU-oracle checks of the MLP train steps built by aicf_hip.mlp: one
eager step and captured+replayed steps, every loss, gradient and updated
parameter compared with the oracle.  Test infrastructure: imported by the
tests and by the driver's smoke entry point, never by the package."""
from __future__ import annotations

from typing import Dict

import numpy as np
import torch

from aicf_hip.mlp import (FlatLayout, build_mlp_mse, build_mlp_xent, init_mlp_mse, init_mlp_xent,
                          make_executor, refresh_shadow)


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.float().numpy()
    return t.numpy()


class XentOracle:
    """The oracle's view of the xent MLP (Linear -> ReLU -> Linear, softmax
    cross-entropy, AdamW with the in-kernel step) across steps.  check()
    takes the GPU state after one step on batch (x, labels): loss and
    argmax against an fp64 chain from the oracle's parameters, every
    gradient at rel-err <= 1e-4, then the reference-exact AdamW restatement
    applied to the GPU's own gradients must reproduce the GPU's parameters
    bit for bit; the oracle then carries those parameters and moments on.
    lr=0 and a held step model the AICF_WARMUP=1 branch (core_v2/exec.py:
    423-431): step_inc becomes a copy, Adam runs with lr 0."""

    NAMES = ("0.W", "0.b", "2.W", "2.b")

    def __init__(self, data: Dict[str, np.ndarray]):
        self.P = {k: data[k].astype(np.float32).copy() for k in self.NAMES}
        self.M = {k: np.zeros(v.size, np.float32) for k, v in self.P.items()}
        self.V = {k: np.zeros(v.size, np.float32) for k, v in self.P.items()}
        self.step = 0

    def expect(self, x, labels):
        import oracle as orc  # test infrastructure

        x = np.asarray(x, np.float64)
        W0, b0, W1, b1 = (self.P[k].astype(np.float64) for k in self.NAMES)
        hh = np.maximum(x @ W0.T + b0, 0)
        logits = (hh @ W1.T + b1).astype(np.float32)
        loss, dz, am, _ = orc.softmax_xent_f64(logits, labels)
        grads = {"2.W": dz.T @ hh, "2.b": dz.sum(0)}
        dhh = (dz @ W1) * (hh > 0)
        grads["0.W"] = dhh.T @ x
        grads["0.b"] = dhh.sum(0)
        return loss, am, grads

    def check(self, ex, params: Dict[str, torch.Tensor], x, labels, tag: str,
              res: Dict[str, object], warmup: bool = False) -> bool:
        import oracle as orc  # test infrastructure

        loss, am, grads = self.expect(x, labels)
        gl = float(ex.value("loss").item())
        res[f"{tag}_loss_rel"] = abs(gl - loss) / abs(loss)
        ok = res[f"{tag}_loss_rel"] < 1e-5
        ok &= bool(np.array_equal(_np(ex.value("pred")), am))
        step = self.step if warmup else self.step + 1
        lr = 0.0 if warmup else 1e-3
        ok &= int(ex.value("opt.step").item()) == step
        new = {}
        for k in self.NAMES:
            g = _np(ex.value(f"d_{k}"))
            e = orc.rel_err(g, grads[k])
            res[f"{tag}_grad_{k}"] = e
            ok &= e < 1e-4
            pr, mr, vr = orc.adamw(self.P[k], g, self.M[k], self.V[k], step, lr)
            got = _np(params[k])
            exact = (np.array_equal(got.ravel(), pr) and np.array_equal(_np(ex.value(f"opt.m.{k}")).ravel(), mr)
                     and np.array_equal(_np(ex.value(f"opt.v.{k}")).ravel(), vr))
            res[f"{tag}_update_exact_{k}"] = bool(exact)
            ok &= exact
            new[k] = (got.copy(), mr, vr)
        for k, (p, m, v) in new.items():
            self.P[k], self.M[k], self.V[k] = p, m, v
        self.step = step
        res["ok"] = bool(res.get("ok", True) and ok)
        return bool(ok)


def xent_setup(seed: int = 0, device: str = "cuda:0", own_graph: bool = False, B=64, din=784,
               dh=256, dout=10, fuse_small=False):
    """Executor, GPU inputs/params and oracle of the xent MLP from a seed
    (fuse_small: StageF, True for three launches, "four" for four)."""
    ir, lowered, plan = build_mlp_xent(B, din, dh, dout, device=device, fuse_small=fuse_small)
    data = init_mlp_xent(B, din, dh, dout, seed=seed)
    params = {k: torch.from_numpy(v.copy()).to(device) for k, v in data.items() if "." in k}
    inputs = {"x": torch.from_numpy(data["x"]).to(device), "t": torch.from_numpy(data["t"]).to(device)}
    ex = make_executor(ir, lowered, plan, device, own_graph=own_graph)
    return ex, inputs, params, XentOracle(data), data


def check_mlp_small(device: str = "cuda:0", verbose: bool = False, B=64, din=784, dh=256,
                    dout=10, fuse_small=False) -> Dict[str, object]:
    """Runs one eager step and two captured+replayed steps of the xent MLP and
    checks loss, argmax, every gradient and every updated parameter against
    the CPU oracle (fp64 chain for loss/grads; the reference-exact AdamW
    restatement applied to the GPU's own gradients for the update)."""
    ex, inputs, params, orc_state, data = xent_setup(0, device, False, B, din, dh, dout, fuse_small)
    res: Dict[str, object] = {"ok": True}
    ex.run(inputs=inputs, params=params, reuse_static=False)
    torch.cuda.synchronize()
    orc_state.check(ex, params, data["x"], data["t"], "eager", res)
    # capture the same step and replay it twice (steps 2 and 3)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    for t in (2, 3):
        ex.replay(1)
        torch.cuda.synchronize()
        orc_state.check(ex, params, data["x"], data["t"], f"replay{t}", res)
    res["kernel_ids"] = sorted({it[2] for it in ex.ops})
    ex.reset_graph()
    if verbose:
        print("[mlp] check", res)
    return res


class MvpOracle:
    """The oracle's view of the fw MVP step (Linear -> ReLU -> Linear, MSE
    gradient, adam_step with host-managed bc1_inv / bc2_inv).  check() after
    one GPU step on (x, t): every gradient against an fp64 chain from the
    oracle's parameters at rel-err <= 1e-4, then the reference-exact Adam
    restatement (adam_step/launcher.cu:276-291) with the bias-correction
    values the meta tensors held, applied to the GPU's own gradients, must
    reproduce the GPU's parameters and moments bit for bit."""

    NAMES = ("0.W", "0.b", "2.W", "2.b")

    def __init__(self, params: Dict[str, torch.Tensor]):
        self.P = {k: _np(params[k]).astype(np.float32).copy() for k in self.NAMES}
        self.M = {k: np.zeros(v.size, np.float32) for k, v in self.P.items()}
        self.V = {k: np.zeros(v.size, np.float32) for k, v in self.P.items()}

    def check(self, ts, x, t, tag: str, res: Dict[str, object], lr: float = 1e-3) -> bool:
        import oracle as orc  # test infrastructure

        x64, t64 = _np(x).astype(np.float64), _np(t).astype(np.float64)
        W0, b0, W1, b1 = (self.P[k].astype(np.float64) for k in self.NAMES)
        hh = np.maximum(x64 @ W0.T + b0, 0)
        y = hh @ W1.T + b1
        dy = (y - t64) * (2.0 / y.size)
        grads = {"2.W": dy.T @ hh, "2.b": dy.sum(0)}
        dhh = (dy @ W1) * (hh > 0)
        grads["0.W"], grads["0.b"] = dhh.T @ x64, dhh.sum(0)
        bc1 = np.float32(ts.optimizer.bc1_inv.item())
        bc2 = np.float32(ts.optimizer.bc2_inv.item())
        ex = ts.ex
        ok = True
        new = {}
        for k in self.NAMES:
            g = _np(ex.value(f"d_{k}"))
            e = orc.rel_err(g, grads[k])
            res[f"{tag}_grad_{k}"] = e
            ok &= e < 1e-4
            pr, mr, vr = orc.adam_ref(self.P[k], g, self.M[k], self.V[k], float(bc1), float(bc2), lr)
            got = _np(ts.params[k]).ravel()
            exact = (np.array_equal(got, pr) and np.array_equal(_np(ts.optimizer.m[k]).ravel(), mr)
                     and np.array_equal(_np(ts.optimizer.v[k]).ravel(), vr))
            res[f"{tag}_update_exact_{k}"] = bool(exact)
            ok &= exact
            new[k] = (got.reshape(self.P[k].shape).copy(), mr, vr)
        for k, (p, m, v) in new.items():
            self.P[k], self.M[k], self.V[k] = p, m, v
        res["ok"] = bool(res.get("ok", True) and ok)
        return bool(ok)


class MseOracle:
    """The oracle's view of the bf16 GELU/MSE/AdamW MLP (aicf_hip.mlp.
    build_mlp_mse, unfused optimizer) across steps.  check() after one GPU
    step: an fp64 chain from the oracle's parameters that rounds every stored
    bf16 tensor as the kernels do (loss and all dW / db at rel-err <= 1e-2),
    then the reference-exact AdamW restatement applied to the GPU's own
    gradients must reproduce the parameters, both moments and the bf16
    shadow bit for bit."""

    def __init__(self, inputs: Dict[str, torch.Tensor], params: Dict[str, torch.Tensor], B: int,
                 D: int, L: int):
        self.B, self.D, self.L = B, D, L
        self.lay = FlatLayout(D, L)
        self.X = _np(inputs["x"]).astype(np.float64)
        self.T = _np(inputs["t"]).astype(np.float64)
        self.P = _np(params["flat.params"]).copy()
        self.M = np.zeros_like(self.P)
        self.V = np.zeros_like(self.P)
        self.step = 0

    def expect(self):
        import oracle as orc  # test infrastructure

        B, D, L, lay = self.B, self.D, self.L, self.lay
        q = lambda a: orc.bf16_round(np.asarray(a, np.float32)).astype(np.float64)  # noqa: E731
        P = self.P
        Wb = [q(P[lay.w_off(i):lay.w_off(i) + D * D].reshape(D, D)) for i in range(1, L + 1)]
        bs = [P[lay.b_off(i):lay.b_off(i) + D].astype(np.float64) for i in range(1, L + 1)]
        hs, zs = [self.X], []
        for i in range(L - 1):
            v = hs[-1] @ Wb[i].T + bs[i]
            zs.append(q(v))
            hs.append(q(orc.gelu_f64(v)))
        y = q(hs[-1] @ Wb[L - 1].T + bs[L - 1])
        loss = float(np.mean((y - self.T) ** 2))
        dy = q((y - self.T) * np.float32(2.0 / (B * D)))
        grads = {}
        for i in range(L - 1, -1, -1):
            grads[f"{i + 1}.W"] = dy.T @ hs[i]
            grads[f"{i + 1}.b"] = dy.sum(0)
            if i > 0:
                dy = q((dy @ Wb[i]) * orc.gelu_grad_f64(zs[i - 1]))
        return loss, grads

    def check(self, ex, tag: str, res: Dict[str, object]) -> bool:
        import oracle as orc  # test infrastructure

        lay, D = self.lay, self.D
        loss, grads = self.expect()
        gl = float(ex.value("loss").item())
        res[f"{tag}_loss_rel"] = abs(gl - loss) / loss
        ok = res[f"{tag}_loss_rel"] < 1e-2
        G = _np(ex.value("grad.flat"))
        for i in range(1, self.L + 1):
            for k, off, n in ((f"{i}.W", lay.w_off(i), D * D), (f"{i}.b", lay.b_off(i), D)):
                e = orc.rel_err(G[off:off + n], grads[k].ravel())
                res[f"{tag}_grad_{k}"] = e
                ok &= e < 1e-2
        t = self.step + 1
        Pr, Mr, Vr, Wr = orc.adamw(self.P, G, self.M, self.V, t, 1e-3, 0.9, 0.999, 1e-8, 0.0, shadow=True)
        exact = (np.array_equal(_np(ex.value("flat.params")), Pr)
                 and np.array_equal(_np(ex.value("opt.m.flat")), Mr)
                 and np.array_equal(_np(ex.value("opt.v.flat")), Vr)
                 and np.array_equal(ex.value("wb.flat").view(torch.int16).cpu().numpy().view(np.uint16), Wr)
                 and int(ex.value("opt.step").item()) == t)
        res[f"{tag}_adamw_exact"] = bool(exact)
        ok &= exact
        self.P, self.M, self.V, self.step = Pr, Mr, Vr, t
        res["ok"] = bool(res.get("ok", True) and ok)
        return bool(ok)


def check_mlp_mse_small(B: int = 256, D: int = 256, L: int = 4, device: str = "cuda:0",
                        steps: int = 3, nt_layout=False, fuse_colsum: bool = False) -> Dict[str, object]:
    """Runs the bf16 MSE MLP (same graph and kernels as the benchmark, smaller
    shape) eagerly for one step and as a captured graph for `steps`-1 more,
    and checks each step against MseOracle."""
    # nt_min_flops=0: with nt_layout, take the transpose + NT-kernel route at
    # every size
    ir, lowered, plan = build_mlp_mse(B, D, L, device=device, nt_layout=nt_layout, nt_min_flops=0,
                                      fuse_colsum=fuse_colsum)
    ex = make_executor(ir, lowered, plan, device)
    inputs, params = init_mlp_mse(B, D, L, seed=1, device=device)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    refresh_shadow(ex)
    torch.cuda.synchronize()
    o = MseOracle(inputs, params, B, D, L)
    res: Dict[str, object] = {"ok": True}
    ex.run(inputs=inputs, params=params, reuse_static=True)
    torch.cuda.synchronize()
    o.check(ex, "eager", res)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    for t in range(2, steps + 1):
        ex.replay(1)
        torch.cuda.synchronize()
        o.check(ex, f"replay{t}", res)
    ex.reset_graph()
    return res
