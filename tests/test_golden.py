"""The reference's only recorded fixtures: the kid-trace test artifacts
(artifacts/20260128_222814_v2_kid_trace_by_id_test/*.txt, copied to
tests/golden/kid_trace/).  The same graph built with aicf_hip must produce
the same IR dump, lowered op list (with pinned kernel ids), binding plan,
and - on the GPU - the same by-id runtime trace; its numbers are checked
against an fp64 chain that rounds every stored tensor to f16."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

GOLD = Path(__file__).resolve().parent / "golden" / "kid_trace"


def _ref(name: str) -> str:
    return (GOLD / name).read_text().rstrip("\n")


@pytest.fixture(scope="module")
def graph():
    from aicf_hip.kid_trace import build_kid_trace_graph

    return build_kid_trace_graph()


def test_ir_dump_matches_artifact(graph):
    ir, _, _ = graph
    assert ir.dump() == _ref("20_ir.txt")


def test_lowered_matches_artifact(graph):
    from aicf_hip import lowered_to_text

    ir, lowered, _ = graph
    assert lowered_to_text(lowered, ir.name) == _ref("30_lowered.txt")


def test_plan_matches_artifact(graph):
    _, _, plan = graph
    assert plan.dump() == _ref("40_plan.txt")


def test_executor_attr_packing():
    """Byte layouts of exec.py:211-277 (gemm <ii>, GEPI <iii>, ADAM <ffff>),
    plus the ops the reference left unpacked."""
    import struct

    from aicf_hip.executor import pack_attrs

    assert pack_attrs("gemm", {"transB": True}) == (0, struct.pack("<ii", 0, 1))
    assert pack_attrs("gemm_epilogue", {"transB": True, "epilogue_act": "relu", "epilogue_bias": True}) == \
        (int.from_bytes(b"GEPI", "little"), struct.pack("<iii", 0, 1, 0))
    assert pack_attrs("gemm_epilogue", {"epilogue": "bias_only"})[1] == struct.pack("<iii", 0, 0, 1)
    assert pack_attrs("adam_step", {}) == (int.from_bytes(b"ADAM", "little"),
                                           struct.pack("<ffff", 1e-3, 0.9, 0.999, 1e-8))
    assert pack_attrs("sgd_step", {"lr": 0.01}) == (int.from_bytes(b"SGDS", "little"), struct.pack("<f", 0.01))
    assert pack_attrs("relu", {}) == (0, b"")


@pytest.mark.gpu
def test_runtime_trace_and_numerics(C, graph):
    import torch

    import oracle as orc
    from aicf_hip.executor import ExecOptions, PlannedExecutor

    ir, lowered, plan = graph
    r = np.random.default_rng(0)
    B, D = 64, 8
    f16 = lambda a: a.astype(np.float16)  # noqa: E731
    x, t = f16(r.standard_normal((B, D))), f16(r.standard_normal((B, D)))
    W0, b0 = f16(r.standard_normal((D, D))), f16(r.standard_normal(D))
    W1, b1 = f16(r.standard_normal((D, D))), f16(r.standard_normal(D))
    dev = lambda a: torch.from_numpy(a.copy()).cuda()  # noqa: E731
    params = {"0.W": dev(W0), "0.b": dev(b0), "2.W": dev(W1), "2.b": dev(b1)}
    ex = PlannedExecutor(ir=ir, lowered=lowered, plan=plan, opts=ExecOptions(require_kernel_id=True))
    ex.trace_reset()
    ex.trace_enable(True)
    ex.run(inputs={"x": dev(x), "t": dev(t)}, params=params, reuse_static=False)
    ex.trace_enable(False)
    torch.cuda.synchronize()
    assert "\n".join(ex.trace_get()) == _ref("50_runtime_trace.txt")
    ex.trace_enable(True)

    # fp64 chain with f16 rounding of every stored tensor (fp32 accumulate)
    q = lambda a: np.asarray(a, np.float64).astype(np.float16).astype(np.float64)  # noqa: E731
    X, T = x.astype(np.float64), t.astype(np.float64)
    w0, c0, w1, c1 = (a.astype(np.float64) for a in (W0, b0, W1, b1))
    h = q(np.maximum(X @ w0.T + c0, 0))
    y = q(q(h @ w1.T) + c1)
    dY = q((y - T) * np.float32(2.0 / (B * D)))
    d_h = q(dY @ w1)
    dW1, db1 = q(dY.T @ h), q(dY.sum(0))
    d_l0 = np.where(h > 0, d_h, 0.0)
    dW0, db0 = q(d_l0.T @ X), q(d_l0.sum(0))
    for k, p, g in (("0.W", w0, dW0), ("0.b", c0, db0), ("2.W", w1, dW1), ("2.b", c1, db1)):
        want = q(p - 0.01 * g)  # SGDS lr is packed (the reference ran the default 1e-3)
        got = params[k].float().cpu().numpy().astype(np.float64)
        # within an f16 ulp or two of the emulated chain
        assert orc.rel_err(got, want) < 4e-3, k
        assert not np.array_equal(got, p), k  # the step did update


def test_stage_d_rewrites_backward_gemms_to_nt():
    """StageD turns every bf16 backward GEMM into transposes + the
    K-contiguous form and reuses a transposed copy until its source changes."""
    from aicf_hip import mlp

    ir, lowered, _ = mlp.build_mlp_mse(8192, 4096, 4, nt_layout=True)
    gemms = [it for it in lowered if it["op"] in ("gemm", "gemm_epilogue")]
    assert len(gemms) == 12
    for it in gemms:
        assert not it["attrs"].get("transA", False) and it["attrs"].get("transB", False)
    tr = [it for it in lowered if it["op"] == "transpose"]
    assert len(tr) == 12  # 4 weights, 4 output grads, 4 layer inputs
    srcs = [it["inputs"][0] for it in tr]
    assert len(set(srcs)) == len(srcs)
    # every transposed value is produced before it is consumed
    made = set()
    for it in lowered:
        for v in it["inputs"]:
            if ir.values[v].name.endswith("^T"):
                assert v in made
        made.update(it["outputs"])


def test_mlp_graph_without_stage_d_reads_operands_in_place():
    """Without StageD the backward GEMMs keep their stored layouts: forward
    X . W^T (K-contiguous both), dX = dZ . W (W M/N-contiguous), dW = dZ^T . H
    (both M/N-contiguous); no transposes are emitted."""
    from aicf_hip import mlp

    ir, lowered, _ = mlp.build_mlp_mse(8192, 4096, 4, nt_layout=False)
    assert not [it for it in lowered if it["op"] == "transpose"]
    layouts = {}
    for it in lowered:
        if it["op"] in ("gemm", "gemm_epilogue"):
            a = it["attrs"]
            key = (bool(a.get("transA", False)), bool(a.get("transB", False)))
            layouts[key] = layouts.get(key, 0) + 1
    # 4 forward, 4 dX (the first layer's dX too, as the reference computes it), 4 dW
    assert layouts == {(False, True): 4, (False, False): 4, (True, False): 4}


def test_stage_d_cost_policy_reads_every_operand_in_place():
    """StageD "cost" at the benchmark shape: the GEMM kernel reads
    M/N-contiguous operands at the K-contiguous rate, so no transpose pays
    for itself and the lowered step is the same as without StageD."""
    from aicf_hip import lower, mlp

    assert lower.MN_OPERAND_PENALTY == 0.0
    ir, lowered, _ = mlp.build_mlp_mse(8192, 4096, 4, nt_layout="cost")
    assert not [it for it in lowered if it["op"] == "transpose"]
    layouts = {}
    for it in lowered:
        if it["op"] in ("gemm", "gemm_epilogue"):
            a = it["attrs"]
            key = (bool(a.get("transA", False)), bool(a.get("transB", False)))
            layouts[key] = layouts.get(key, 0) + 1
    assert layouts == {(False, True): 4, (False, False): 4, (True, False): 4}


def test_stage_d_cost_policy_transposes_when_in_place_reads_cost_more(monkeypatch):
    """With a 10% in-place penalty (the model's input, not a measurement of
    this kernel), transposing a 4096^2 weight (32 MB) is cheaper than the
    penalty of its dX GEMM, transposing dZ or H (64 MB each) is not."""
    from aicf_hip import lower, mlp

    monkeypatch.setattr(lower, "MN_OPERAND_PENALTY", 0.10)
    ir, lowered, _ = mlp.build_mlp_mse(8192, 4096, 4, nt_layout="cost")
    tr = [it for it in lowered if it["op"] == "transpose"]
    assert sorted(ir.values[it["inputs"][0]].name for it in tr) == [f"wb.{i}.W" for i in range(1, 5)]
    layouts = {}
    for it in lowered:
        if it["op"] in ("gemm", "gemm_epilogue"):
            a = it["attrs"]
            key = (bool(a.get("transA", False)), bool(a.get("transB", False)))
            layouts[key] = layouts.get(key, 0) + 1
    assert layouts == {(False, True): 8, (True, False): 4}
