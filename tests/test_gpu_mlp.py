"""End-to-end train steps on the plan runtime, eager and hipGraph-replayed,
checked step by step against the CPU oracle."""
from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


def test_mlp_xent_fp32_reference_config(C):
    """Batch 64, 784 -> 256 (ReLU) -> 10, softmax cross-entropy, Adam: loss,
    argmax, all gradients and all updated parameters (eager step, then two
    replays of the captured step)."""
    import mlp_checks

    res = mlp_checks.check_mlp_small()
    assert res["ok"], res


@pytest.mark.parametrize("B,D,L,nt,colsum", [(256, 256, 4, True, False), (512, 384, 3, True, False),
                                             (256, 256, 2, False, False), (256, 256, 4, False, True),
                                             (512, 512, 3, False, True)])
def test_mlp_mse_bf16_graph(C, B, D, L, nt, colsum):
    """The benchmark's bf16 GELU/MSE/AdamW graph at a reduced shape, with the
    transpose + NT-GEMM lowering (nt) and with the general GEMM kernel; with
    colsum the hidden layers' bias gradients come from the dGELU GEMMs'
    epilogue (GEPI kind 6)."""
    import mlp_checks
    from aicf_hip import mlp

    if colsum:
        ir, lowered, _ = mlp.build_mlp_mse(B, D, L, fuse_colsum=True)
        assert sum(bool(it["attrs"].get("epilogue_colsum")) for it in lowered) == L - 1
    res = mlp_checks.check_mlp_mse_small(B, D, L, nt_layout=nt, fuse_colsum=colsum)
    assert res["ok"], res


def _run_plan(B, D, L, steps, **kw):
    import torch

    from aicf_hip import mlp

    ir, lowered, plan = mlp.build_mlp_mse(B, D, L, **kw)
    ex = mlp.make_executor(ir, lowered, plan)
    inputs, params = mlp.init_mlp_mse(B, D, L, seed=3)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    mlp.refresh_shadow(ex)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    losses = []
    for _ in range(steps):
        ex.replay(1)
        torch.cuda.synchronize()
        losses.append(float(ex.value("loss").item()))
    out = {k: ex.value(k).cpu().clone() for k in ("flat.params", "opt.m.flat", "opt.v.flat", "wb.flat", "opt.step")}
    ex.reset_graph()
    return lowered, losses, out


@pytest.mark.parametrize("B,D,L", [(256, 3072, 3), (512, 4096, 2)])
def test_mlp_mse_fused_optimizer_plan_bit_identical(C, B, D, L):
    """The plan with AdamW fused into the weight-gradient GEMMs (StageE)
    against the unfused plan, three graph replays each from the same start:
    every loss, parameter, moment and shadow element bit for bit (the
    unfused plan is itself checked against the oracle above).  D >= 3072
    puts the unfused fp32-output dW GEMM on the same 256 x 256 tiles."""
    import torch

    low_f, loss_f, out_f = _run_plan(B, D, L, 3, fuse_optimizer=True)
    assert sum(it["op"] == "gemm_adamw" for it in low_f) == L
    assert sum(it["op"] == "adamw_step" for it in low_f) == 1
    low_u, loss_u, out_u = _run_plan(B, D, L, 3, fuse_optimizer=False)
    assert not any(it["op"] == "gemm_adamw" for it in low_u)
    assert loss_f == loss_u
    for k in out_f:
        assert torch.equal(out_f[k], out_u[k]), k
    assert int(out_f["opt.step"].item()) == 3


def test_mlp_mse_benchmark_shape_runs_finite(C):
    """Full benchmark shape (8192 x 4096, 4 layers): two replays, finite and
    decreasing loss, Adam moments populated (size-independent properties)."""
    import math

    import torch

    from aicf_hip import mlp

    ir, lowered, plan = mlp.build_mlp_mse(8192, 4096, 4)
    ex = mlp.make_executor(ir, lowered, plan)
    inputs, params = mlp.init_mlp_mse(8192, 4096, 4)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    mlp.refresh_shadow(ex)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    losses = []
    for _ in range(3):
        ex.replay(1)
        torch.cuda.synchronize()
        losses.append(float(ex.value("loss").item()))
    ex.reset_graph()
    assert all(math.isfinite(v) for v in losses), losses
    assert losses[-1] < losses[0], losses
    assert int(ex.value("opt.step").item()) == 3
    assert float(ex.value("opt.v.flat").abs().max().item()) > 0


def test_json_loaded_plan_runs_bit_identically(C):
    """The reference MLP written to the JSON IR document and read back
    (interchange.ir_to_json / ir_from_json, the format of core_v2/
    cuda_exec.py:306-371) lowers to the same op list; replayed as a graph,
    every step of the JSON-loaded plan matches the oracle (loss and argmax,
    all gradients <= 1e-4, AdamW bit-exact on the GPU's gradients) and is
    bit-identical to the natively built plan."""
    import mlp_checks
    import torch

    from aicf_hip import mlp
    from aicf_hip.interchange import ir_from_json, ir_to_json
    from aicf_hip.lower import compile_lowered, lowered_to_text
    from aicf_hip.plan import build_binding_plan

    ir, lowered, plan = mlp.build_mlp_xent()
    ir2 = ir_from_json(ir_to_json(ir))
    lowered2 = compile_lowered(ir2)
    assert lowered_to_text(lowered2, ir2.name) == lowered_to_text(lowered, ir.name)
    data = mlp.init_mlp_xent()
    results = []
    for tag, (g_ir, g_low, g_plan) in (("native", (ir, lowered, plan)),
                                       ("json", (ir2, lowered2, build_binding_plan(ir2)))):
        params = {k: torch.from_numpy(v.copy()).cuda() for k, v in data.items() if "." in k}
        inputs = {"x": torch.from_numpy(data["x"]).cuda(), "t": torch.from_numpy(data["t"]).cuda()}
        ex = mlp.make_executor(g_ir, g_low, g_plan)
        ex.build_env(inputs=inputs, params=params, reuse_static=False)
        ex.capture(inputs=inputs, params=params, reuse_static=True)
        orc_state = mlp_checks.XentOracle(data)
        res = {"ok": True}
        snaps = []
        for t in range(1, 4):
            ex.replay(1)
            torch.cuda.synchronize()
            assert orc_state.check(ex, params, data["x"], data["t"], f"{tag}_replay{t}", res), res
            snap = {k: ex.value(k).detach().cpu().clone() for k in ("loss", "pred", "d_0.W", "d_2.b")}
            snap.update({k: p.detach().cpu().clone() for k, p in params.items()})
            snaps.append(snap)
        ex.reset_graph()
        results.append(snaps)
    for a, b in zip(*results):
        for k in a:
            assert torch.equal(a[k], b[k]), k
