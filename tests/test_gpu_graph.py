"""Graph lifecycle beyond the process-wide graph: several executors each
holding an instantiated graph of their own, replayed interleaved, and
re-capture with other input buffers updating the executable in place.

Each graph replay is checked against the CPU oracle (loss and argmax, all
gradients <= 1e-4, the AdamW update bit-exact on the GPU's gradients; the
oracle follows each executor's own sequence of batches) and compared bit
for bit with eager execution of the same plan on separately allocated
copies of the same data.  The process-wide graph (handle 0, the reference's
singleton, src/python_bindings/bindings.cpp:137-187,475-547) keeps working
alongside.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

KEYS = ("loss", "pred", "d_0.W", "d_2.b")


def _xent_setup(seed, own_graph):
    import mlp_checks

    ex, inputs, params, _, _ = mlp_checks.xent_setup(seed, own_graph=own_graph)
    return ex, inputs, params


def _oracle(seed):
    import mlp_checks
    from aicf_hip import mlp

    data = mlp.init_mlp_xent(seed=seed)
    return mlp_checks.XentOracle(data), data


def _snap(ex, params):
    out = {k: ex.value(k).detach().cpu().clone() for k in KEYS}
    out.update({k: p.detach().cpu().clone() for k, p in params.items()})
    return out


def _eager_steps(seed, n, feed=None):
    """n eager steps; feed(i) optionally returns new inputs for step i."""
    ex, inputs, params = _xent_setup(seed, own_graph=False)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    snaps = []
    for i in range(n):
        if feed is not None and feed(i) is not None:
            ex.build_env(inputs=feed(i), params=params, reuse_static=True)
        ex.run(inputs={}, params={}, reuse_static=True)
        torch.cuda.synchronize()
        snaps.append(_snap(ex, params))
    return snaps


def _assert_same(a, b, tag):
    for k in a:
        assert torch.equal(a[k], b[k]), f"{tag}: {k} differs"


def test_executors_with_own_graphs_replay_interleaved(C):
    """Two plans (different data) instantiated at once on their own handles,
    plus a third on the process-wide graph; replays alternate between them
    and each matches its own eager run bit for bit."""
    want = {seed: _eager_steps(seed, 3) for seed in (1, 2, 3)}
    oracles = {seed: _oracle(seed) for seed in (1, 2, 3)}
    res = {"ok": True}
    exs = {}
    for seed in (1, 2, 3):
        ex, inputs, params = _xent_setup(seed, own_graph=(seed != 3))
        ex.build_env(inputs=inputs, params=params, reuse_static=False)
        ex.capture(inputs=inputs, params=params, reuse_static=True)
        exs[seed] = (ex, params)
    h1, h2 = exs[1][0].graph_handle, exs[2][0].graph_handle
    assert h1 and h2 and h1 != h2 and exs[3][0].graph_handle is None
    assert C.graph_state_h(h1) == 2 and C.graph_state_h(h2) == 2 and C.graph_state_h(0) == 2
    assert C.graph_stream_h(h1) != C.graph_stream_h(h2)
    for step in range(3):
        for seed in (2, 3, 1):
            ex, params = exs[seed]
            ex.replay(1)
            torch.cuda.synchronize()
            o, data = oracles[seed]
            assert o.check(ex, params, data["x"], data["t"], f"s{seed}_{step}", res), res
            _assert_same(_snap(ex, params), want[seed][step], f"seed {seed} step {step}")
    for seed, (ex, _) in exs.items():
        if seed == 3:
            ex.reset_graph()
        else:
            ex.close()
    assert C.graph_state_h(h1) == -1 and C.graph_state_h(0) == 0
    with pytest.raises(RuntimeError, match="unknown graph handle"):
        C.graph_launch_h(h1)


def test_recapture_with_new_inputs_updates_in_place(C):
    """Capture, replay, bind another batch (new tensors at new addresses) and
    capture again on the same handle: the executable is updated, not
    rebuilt, and the replays match eager steps fed the same batches."""
    r = np.random.default_rng(11)
    x2 = torch.from_numpy(r.standard_normal((64, 784)).astype(np.float32)).cuda()
    t2 = torch.from_numpy(r.integers(0, 10, 64).astype(np.int32)).cuda()
    batch2 = {"x": x2.clone(), "t": t2.clone()}
    want = _eager_steps(5, 4, feed=lambda i: batch2 if i == 2 else None)

    o, data = _oracle(5)
    res = {"ok": True}
    ex, inputs, params = _xent_setup(5, own_graph=True)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    assert ex.graph_updates == 0
    for step in range(2):
        ex.replay(1)
        torch.cuda.synchronize()
        assert o.check(ex, params, data["x"], data["t"], f"step{step}", res), res
        _assert_same(_snap(ex, params), want[step], f"step {step}")
    old_x = ex.value("x").data_ptr()
    ex.recapture(inputs={"x": x2, "t": t2})
    assert ex.value("x").data_ptr() == x2.data_ptr() != old_x
    assert ex.graph_updates == 1
    xb, tb = x2.cpu().numpy(), t2.cpu().numpy()
    for step in range(2, 4):
        ex.replay(1)
        torch.cuda.synchronize()
        assert o.check(ex, params, xb, tb, f"step{step}", res), res
        _assert_same(_snap(ex, params), want[step], f"step {step}")
    ex.close()


def _env_snapshot(ex):
    return {vid: t.detach().cpu().clone() for vid, t in ex.env.items()}


def test_recapture_of_a_different_plan_reinstantiates(C):
    """A capture whose op sequence differs from the executable's (another
    plan captured on the same handle) cannot be an update: the handle builds
    a new executable; each replay matches the oracle (the xent and the bf16
    MSE steps, gradients and the AdamW update) and equals eager execution
    (every value of the plan compared)."""
    import mlp_checks
    from aicf_hip import mlp

    def xent():
        ir, lowered, plan = mlp.build_mlp_xent()
        data = mlp.init_mlp_xent(seed=7)
        params = {k: torch.from_numpy(v.copy()).cuda() for k, v in data.items() if "." in k}
        inputs = {"x": torch.from_numpy(data["x"]).cuda(), "t": torch.from_numpy(data["t"]).cuda()}
        o = mlp_checks.XentOracle(data)
        check = lambda ex, res: o.check(ex, params, data["x"], data["t"], "xent", res)  # noqa: E731
        return ir, lowered, plan, inputs, params, None, check

    def mse():
        ir, lowered, plan = mlp.build_mlp_mse(256, 256, 2)
        inputs, params = mlp.init_mlp_mse(256, 256, 2, seed=8)
        o = mlp_checks.MseOracle(inputs, params, 256, 256, 2)
        return ir, lowered, plan, inputs, params, mlp.refresh_shadow, lambda ex, res: o.check(ex, "mse", res)

    h = C.graph_create()
    try:
        for make in (xent, mse):
            snaps = []
            for graph in (False, True):
                ir, lowered, plan, inputs, params, prep, check = make()
                ex = mlp.make_executor(ir, lowered, plan)
                ex.build_env(inputs=inputs, params=params, reuse_static=False)
                for vid in plan.statics:  # defined contents for never-written scratch
                    if ir.values[vid].view_of is None:
                        ex.env[vid].zero_()
                if prep is not None:
                    prep(ex)
                torch.cuda.synchronize()
                if graph:
                    s = C.graph_begin_h(h)
                    ex._execute_lowered(stream=s)
                    C.graph_end_h(h)
                    C.graph_launch_h(h)
                else:
                    ex.run(inputs={}, params={}, reuse_static=True)
                torch.cuda.synchronize()
                res = {"ok": True}
                assert check(ex, res), res
                snaps.append(_env_snapshot(ex))
            assert snaps[0].keys() == snaps[1].keys()
            for vid in snaps[0]:
                assert torch.equal(snaps[0][vid], snaps[1][vid]), f"{make.__name__}: vid {vid}"
        assert C.graph_updates_h(h) == 0
    finally:
        C.graph_destroy(h)


def test_graph_handle_misuse(C):
    h = C.graph_create()
    with pytest.raises(RuntimeError, match="no captured graph"):
        C.graph_launch_h(h)
    with pytest.raises(RuntimeError, match="not capturing"):
        C.graph_end_h(h)
    with pytest.raises(RuntimeError, match="process-wide graph"):
        C.graph_destroy(0)
    C.graph_destroy(h)
    with pytest.raises(RuntimeError, match="unknown graph handle"):
        C.graph_begin_h(h)
