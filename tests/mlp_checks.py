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
