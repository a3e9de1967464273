"""Runtime protocols checked step by step against the CPU oracle: the
AICF_WARMUP branch of the executor (core_v2/exec.py:396,423-431), the fw
MVP user flow (python_framework_test/python_framework_test.py:29-116:
warmup, train_step, capture, replay, meta mutation between replays, an
unsynchronised replay), and the ordering of a replay against work queued on
torch's default stream before and after it."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_aicf_warmup_branch_then_real_steps(C, monkeypatch):
    """AICF_WARMUP=1: step_inc is a copy and AdamW runs with lr 0, so the
    parameters and the step counter stay bit-identical while the moments
    take the oracle's values; a graph captured under it replays the warmup
    step.  Unset, a fresh capture replays real steps from that state."""
    import mlp_checks

    ex, inputs, params, orc_state, data = mlp_checks.xent_setup(seed=4)
    P0 = {k: p.detach().cpu().clone() for k, p in params.items()}
    res = {"ok": True}
    monkeypatch.setenv("AICF_WARMUP", "1")
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    for i in range(2):
        ex.run(inputs={}, params={}, reuse_static=True)
        torch.cuda.synchronize()
        assert orc_state.check(ex, params, data["x"], data["t"], f"warm{i}", res, warmup=True), res
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    ex.replay(1)
    torch.cuda.synchronize()
    assert orc_state.check(ex, params, data["x"], data["t"], "warm_replay", res, warmup=True), res
    for k, p in params.items():
        assert torch.equal(p.cpu(), P0[k]), k
    assert int(ex.value("opt.step").item()) == 0
    assert float(ex.value("opt.v.0.W").abs().max().item()) > 0
    monkeypatch.delenv("AICF_WARMUP")
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    for t in (1, 2):
        ex.replay(1)
        torch.cuda.synchronize()
        assert orc_state.check(ex, params, data["x"], data["t"], f"replay{t}", res), res
    assert int(ex.value("opt.step").item()) == 2
    ex.reset_graph()


def _mvp_setup(seed=0, B=64, D=8, device="cuda:0", **kw):
    from aicf_hip import fw

    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    x = torch.randn(B, D, generator=g).to(device)
    t = torch.randn(B, D, generator=g).to(device)
    bound = 1.0 / np.sqrt(D)
    params = {"0.W": ((torch.rand(D, D, generator=g) * 2 - 1) * bound).to(device),
              "0.b": ((torch.rand(D, generator=g) * 2 - 1) * bound).to(device),
              "2.W": ((torch.rand(D, D, generator=g) * 2 - 1) * bound).to(device),
              "2.b": ((torch.rand(D, generator=g) * 2 - 1) * bound).to(device)}
    opt = fw.Adam(params, lr=1e-3)
    ts = fw.compile_fw_mvp(params, opt, B=B, D=D, device=device, **kw)
    return ts, opt, params, {"x": x, "t": t}


def test_fw_mvp_user_flow_against_oracle(C):
    """The fw MVP user test's sequence with every step checked against the
    oracle (gradients <= 1e-4, Adam update bit-exact with the meta values the
    GPU read): two warmup steps, train_step, capture, three replays, a replay
    with bc1_inv = bc2_inv = 1, a replay with them restored (the two updates
    differ, python_framework_test.py:80-100), and a replay whose result is
    read on torch's stream without synchronising."""
    import mlp_checks

    ts, opt, params, batch = _mvp_setup()
    orc_state = mlp_checks.MvpOracle(params)
    res = {"ok": True}
    W0 = params["0.W"]
    for i in range(2):
        ts.warmup(batch, n=1)
        assert orc_state.check(ts, batch["x"], batch["t"], f"warmup{i}", res), res
    assert opt.step_host == 2
    W0_before = W0.clone()
    ts.train_step(batch)
    torch.cuda.synchronize()
    assert orc_state.check(ts, batch["x"], batch["t"], "train_step", res), res
    assert float((W0 - W0_before).abs().max().item()) > 0
    ts.capture(batch)
    for i in range(3):
        ts.replay(n=1, sync=True)
        assert orc_state.check(ts, batch["x"], batch["t"], f"replay{i}", res), res
    bc1_before, bc2_before = float(opt.bc1_inv.item()), float(opt.bc2_inv.item())
    W0_m0 = W0.clone()
    opt.bc1_inv.fill_(1.0)
    opt.bc2_inv.fill_(1.0)
    ts.replay(n=1, sync=True)
    assert orc_state.check(ts, batch["x"], batch["t"], "mutated", res), res
    d_mut = float((W0 - W0_m0).abs().max().item())
    W0_m1 = W0.clone()
    opt.bc1_inv.fill_(bc1_before)
    opt.bc2_inv.fill_(bc2_before)
    ts.replay(n=1, sync=True)
    assert orc_state.check(ts, batch["x"], batch["t"], "restored", res), res
    d_rest = float((W0 - W0_m1).abs().max().item())
    assert abs(d_mut - d_rest) >= 1e-12, (d_mut, d_rest)
    # unsynchronised replay: the clone below is queued on torch's stream and
    # must still see the replay's update
    W0_a0 = W0.clone()
    ts.replay(n=1, sync=False)
    W0_after = W0.clone()
    torch.cuda.synchronize()
    assert orc_state.check(ts, batch["x"], batch["t"], "async", res), res
    assert torch.equal(W0_after, W0) and not torch.equal(W0_after, W0_a0)
    ts.reset()


def test_fw_mvp_compile_warmup_and_fail_fast(C):
    """A required warmup that is disabled or has no inputs fails before any
    launch, with the reference's messages (fw/train_step.py:47-66); compile
    with warmup_inputs runs the warmup_runs steps at once (the meta is at
    step 2 and the weights moved)."""
    from aicf_hip import fw

    ts, opt, params, batch = _mvp_setup(seed=1)
    W = params["0.W"].clone()
    with pytest.raises(RuntimeError, match="Warmup is required but no inputs"):
        ts._maybe_warmup(None)
    ts.warmup_runs = 0
    with pytest.raises(RuntimeError, match="Warmup is disabled"):
        ts.train_step(batch)
    torch.cuda.synchronize()
    assert opt.step_host == 0 and torch.equal(params["0.W"], W)
    opt2 = fw.Adam(params, lr=1e-3)
    ts2 = fw.compile_fw_mvp(params, opt2, B=64, D=8, warmup_inputs=batch)
    torch.cuda.synchronize()
    assert opt2.step_host == 2 and ts2._warmed_up and not torch.equal(params["0.W"], W)


def test_replay_ordered_against_default_stream(C):
    """A new batch copied into the bound input on torch's default stream
    behind a long-running kernel, then a replay with no synchronisation, then
    a read queued on the same stream: the replay runs after the copy and the
    read after the replay, so the step matches the oracle on the new batch
    (the graph stream is non-blocking and waits on the default stream only
    through the launch's event edges)."""
    import mlp_checks

    assert torch.cuda.current_stream().cuda_stream == 0  # the null stream
    ex, inputs, params, orc_state, data = mlp_checks.xent_setup(seed=6)
    res = {"ok": True}
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    ex.replay(1)
    torch.cuda.synchronize()
    assert orc_state.check(ex, params, data["x"], data["t"], "first", res), res
    r = np.random.default_rng(12)
    x2 = r.standard_normal(data["x"].shape).astype(np.float32)
    t2 = r.integers(0, 10, data["t"].shape).astype(np.int32)
    x2_d, t2_d = torch.from_numpy(x2).cuda(), torch.from_numpy(t2).cuda()
    a = torch.randn(4096, 4096, device="cuda")
    torch.cuda.synchronize()
    for _ in range(8):  # a few ms of work ahead of the copies
        a = a @ a
        a = a / a.norm()
    ex.value("x").copy_(x2_d)
    ex.value("t").copy_(t2_d)
    ex.replay(1)
    snap = {k: ex.value(k).clone() for k in ("loss", "pred", "d_0.W", "d_2.b")}
    torch.cuda.synchronize()
    assert orc_state.check(ex, params, x2, t2, "after_copy", res), res
    for k, v in snap.items():
        assert torch.equal(v, ex.value(k)), k
    ex.reset_graph()
