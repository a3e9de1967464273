"""GPU parity at the benchmark configurations' full sizes.

The full outputs are too large for the fp64 oracle to recompute in
seconds, so each test checks what does not depend on size:
  * C2 row kernels (16384 rows x C): row max bit-exact on every row (max is
    order-free), every softmax row sums to 1, the all -1e4 row is exactly
    1/C, and sampled rows against the fp64 oracle;
  * C3 AdamW over 2^28 parameters, t = 1..10: the update is elementwise, so
    a sample of 2^20 parameters run through the oracle's fp32 restatement
    must match the GPU bit for bit after every step;
  * C4 GEMM + epilogue at every configured shape: rows are independent, so
    sampled rows against an fp64 product of the same stored (bf16-rounded)
    operands.
Inputs follow BASELINE.json's configs (N(0,4) rows, N(0,0.02) / N(0,1e-3)
Adam buffers, U(-1,1)/sqrt(K) GEMM operands), generated on the GPU from a
seeded torch generator.
"""
from __future__ import annotations

import math
import struct

import numpy as np
import pytest
import torch

import oracle as orc

pytestmark = pytest.mark.gpu

RRED = int.from_bytes(b"RRED", "little")
ADAM = int.from_bytes(b"ADAM", "little")
GEPI = int.from_bytes(b"GEPI", "little")


def _host(t):
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return orc.bf16_bits_to_f32(t.view(torch.int16).numpy().view(np.uint16)).reshape(t.shape)
    return t.numpy()


@pytest.mark.parametrize("cols", [128, 1024, 8192, 32768])
def test_c2_row_softmax_max_sum_full_size(C, cols):
    rows = 16384
    gen = torch.Generator(device="cuda")
    gen.manual_seed(cols)
    x = torch.randn((rows, cols), device="cuda", generator=gen) * 2.0  # N(0, 4)
    x[-1].fill_(-1e4)
    y = torch.empty_like(x)
    mx = torch.empty(rows, device="cuda")
    sx = torch.empty(rows, device="cuda")
    C.op_call(int(C.OpKind.RowSoftmax), [x], [y, mx, sx], 0, b"", 0)
    rmax = torch.empty(rows, device="cuda")
    rsum = torch.empty(rows, device="cuda")
    C.op_call(int(C.OpKind.RowReduce), [x], [rmax], RRED, struct.pack("<i", 1), 0)
    C.op_call(int(C.OpKind.RowReduce), [x], [rsum], RRED, struct.pack("<i", 0), 0)
    xh = x.cpu().numpy()
    yh = y.cpu().numpy()
    ref_max = xh.max(axis=1)
    assert np.array_equal(mx.cpu().numpy(), ref_max)
    assert np.array_equal(rmax.cpu().numpy(), ref_max)
    row_tot = yh.sum(axis=1, dtype=np.float64)
    assert np.abs(row_tot - 1.0).max() < 1e-5
    assert np.all(yh[-1] == np.float32(1.0 / cols))
    sample = np.random.default_rng(cols).choice(rows - 1, 64, replace=False)
    sample = np.append(sample, rows - 1)
    ry, rmx, rsx = orc.softmax_rows_f64(xh[sample])
    assert orc.rel_err(yh[sample], ry) < 1e-5
    assert orc.rel_err(sx.cpu().numpy()[sample], rsx) < 1e-5
    assert orc.rel_err(rsum.cpu().numpy()[sample], rsx) < 1e-5


def test_c3_adamw_2p28_ten_steps_bit_exact_on_a_sample(C):
    n = 1 << 28
    gen = torch.Generator(device="cuda")
    gen.manual_seed(28)
    P = torch.randn(n, device="cuda", generator=gen) * 0.02
    G = torch.randn(n, device="cuda", generator=gen) * 1e-3
    M = torch.zeros(n, device="cuda")
    V = torch.zeros(n, device="cuda")
    step = torch.zeros((), dtype=torch.int32, device="cuda")
    lr, b1, b2, eps, wd = 1e-3, 0.9, 0.999, 1e-8, 0.01
    pay = struct.pack("<fffff", lr, b1, b2, eps, wd)
    idx = torch.from_numpy(np.sort(np.random.default_rng(28).choice(n, 1 << 20, replace=False))).cuda()
    p, gr = P[idx].cpu().numpy(), G[idx].cpu().numpy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for t in range(1, 11):
        C.launch_by_id("step_inc_v0", C.OpKind.StepInc, [step], [step])
        C.launch_by_id("adamw_step_f32_v1", C.OpKind.AdamStep, [P, G, M, V, step], [P, M, V], ADAM, pay)
        p, m, v = orc.adamw(p, gr, m, v, t, lr=lr, beta1=b1, beta2=b2, eps=eps, wd=wd)
        assert np.array_equal(P[idx].cpu().numpy(), p), f"step {t}"
        assert np.array_equal(M[idx].cpu().numpy(), m), f"step {t}"
        assert np.array_equal(V[idx].cpu().numpy(), v), f"step {t}"
    assert int(step.item()) == 10


# Every (dtype, shape) the benchmark times for C4, each with the three
# epilogues it times (GEPI kinds 1 bias only, 0 bias+ReLU, 3 bias+GELU): the
# dispatcher picks the tile configuration from the shape and the epilogue
# (64 x 64 8-stage, 128 x 128 for K <= 256, 4-wave and 8-wave 256 x 256,
# persistent), so each point pins the path it reaches.  Plus K = 512, the
# 8-wave persistent tiles with two tiles per workgroup.
C4_SHAPES = [(1024, 1024, 1024), (4096, 4096, 4096), (8192, 8192, 8192), (8192, 4096, 256), (8192, 4096, 11008)]
C4_CASES = [(dt, *shp) for dt in ("bf16", "fp32") for shp in C4_SHAPES] + [("bf16", 8192, 4096, 512)]
ACT_KIND = {"none": 1, "relu": 0, "gelu": 3}


@pytest.mark.parametrize("dt,M,N,K", C4_CASES)
def test_c4_gemm_epilogue_full_size_sampled_rows(C, dt, M, N, K):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(M + N + K)
    s = 1.0 / math.sqrt(K)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    X = ((torch.rand((M, K), device="cuda", generator=gen) * 2 - 1) * s).to(tdt)
    W = ((torch.rand((N, K), device="cuda", generator=gen) * 2 - 1) * s).to(tdt)
    b = (torch.rand(N, device="cuda", generator=gen) * 2 - 1) * s
    rows = torch.from_numpy(np.sort(np.random.default_rng(K).choice(M, 16, replace=False))).cuda()
    xs = _host(X[rows]).astype(np.float64)
    wh = _host(W).astype(np.float64)
    z = xs @ wh.T + b.cpu().numpy().astype(np.float64)[None, :]
    del wh
    kid = "gemm_epilogue_bf16_mfma_v0" if dt == "bf16" else "gemm_epilogue_f32_mfma_v0"
    tol = 1e-2 if dt == "bf16" else 1e-4
    for act in ("none", "relu", "gelu"):
        print(f"[c4] {dt} {M}x{N}x{K} {act}", flush=True)
        Y = torch.full((M, N), float("nan"), device="cuda", dtype=tdt)
        C.launch_by_id(kid, C.OpKind.GemmEpilogue, [X, W, b], [Y], GEPI,
                       struct.pack("<iii", 0, 1, ACT_KIND[act]))
        ref = {"none": z, "relu": np.maximum(z, 0.0), "gelu": orc.gelu_f64(z)}[act]
        assert orc.rel_err(_host(Y[rows]), ref) < tol, act
        # every element written: no NaN left from the fill
        assert not torch.isnan(Y).any(), act
        del Y


@pytest.mark.parametrize("colsum", [False, True])
def test_c5_mlp_step_full_shape_forward_rows_and_adamw_bit_exact(C, colsum):
    """C5 at its full shape (batch 8192, 4 x 4096^2, GELU, MSE, AdamW) replayed
    once from its captured graph.  Forward rows are independent: 16 sampled
    rows of every stored activation (z_i, h_i, y) against an fp64 chain from
    the same bf16 inputs and weights that rounds each stored tensor to bf16.
    The optimizer is elementwise: the oracle's AdamW applied to the GPU's own
    gradients over all 67,125,248 parameters must reproduce the updated fp32
    parameters, both moments and the bf16 shadow bit for bit.  Every bias
    gradient matches the fp64 column sum of the stored output gradient it
    comes from (with colsum: taken in the dGELU GEMMs' epilogue), 4096
    sampled weight-gradient entries per layer match fp64 dots over the 8192
    stored rows, and 16 sampled rows of every input gradient match the fp64
    chain through the dGELU epilogue."""
    from aicf_hip import mlp

    B, D, L = 8192, 4096, 4
    ir, lowered, plan = mlp.build_mlp_mse(B, D, L, fuse_colsum=colsum)
    ex = mlp.make_executor(ir, lowered, plan)
    inputs, params = mlp.init_mlp_mse(B, D, L)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    mlp.refresh_shadow(ex)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    P0 = ex.value("flat.params").cpu().numpy().copy()
    Wb0 = ex.value("wb.flat").cpu().clone()
    ex.replay(1)
    torch.cuda.synchronize()

    rows = torch.from_numpy(np.sort(np.random.default_rng(5).choice(B, 16, replace=False))).cuda()
    lay = mlp.FlatLayout(D, L)
    bf = lambda a: orc.bf16_round(a.astype(np.float32)).astype(np.float64)  # noqa: E731
    h = _host(ex.value("x")[rows]).astype(np.float64)
    wb0 = orc.bf16_bits_to_f32(Wb0.view(torch.int16).numpy().view(np.uint16))
    for i in range(1, L + 1):
        W = wb0[lay.w_off(i):lay.w_off(i) + D * D].reshape(D, D).astype(np.float64)
        b = P0[lay.b_off(i):lay.b_off(i) + D].astype(np.float64)
        z = bf(h @ W.T + b[None, :])
        name = f"z{i}" if i < L else "y"
        assert orc.rel_err(_host(ex.value(name)[rows]), z) < 1e-2, name
        if i < L:
            h = bf(orc.gelu_f64(z))
            assert orc.rel_err(_host(ex.value(f"h{i}")[rows]), h) < 1e-2, f"h{i}"

    G = ex.value("grad.flat").cpu().numpy()
    Z = np.zeros_like(P0)
    Pr, Mr, Vr, Wr = orc.adamw(P0, G, Z, Z, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, shadow=True)
    assert np.array_equal(ex.value("flat.params").cpu().numpy(), Pr)
    assert np.array_equal(ex.value("opt.m.flat").cpu().numpy(), Mr)
    assert np.array_equal(ex.value("opt.v.flat").cpu().numpy(), Vr)
    assert np.array_equal(ex.value("wb.flat").cpu().view(torch.int16).numpy().view(np.uint16), Wr)
    assert np.isfinite(G).all() and np.abs(G).max() > 0
    # bias gradients: column sums of the stored (bf16) output gradient of each layer
    for i in range(1, L + 1):
        dz = _host(ex.value("dY" if i == L else f"d_z{i}")).astype(np.float64).sum(axis=0)
        assert orc.rel_err(G[lay.b_off(i):lay.b_off(i) + D], dz) < 1e-5, i
    # weight gradients dW_i = dz_i^T . h_{i-1} (core_v2/lower.py:100-104): a
    # 64 x 64 block of sampled (output, input) pairs per layer, 4096 entries,
    # each an fp64 dot over all 8192 stored bf16 rows of both operands
    r = np.random.default_rng(9)
    for i in range(1, L + 1):
        o_idx = np.sort(r.choice(D, 64, replace=False))
        j_idx = np.sort(r.choice(D, 64, replace=False))
        dz = ex.value("dY" if i == L else f"d_z{i}")[:, torch.from_numpy(o_idx).cuda()]
        hp = ex.value("x" if i == 1 else f"h{i - 1}")[:, torch.from_numpy(j_idx).cuda()]
        ref = _host(dz).astype(np.float64).T @ _host(hp).astype(np.float64)
        got = G[lay.w_off(i):lay.w_off(i) + D * D].reshape(D, D)[np.ix_(o_idx, j_idx)]
        assert orc.rel_err(got, ref) < 1e-4, f"dW{i}"
    # input gradients of 16 sampled rows: d_z{i-1} = bf16((dz_i . Wb_i) *
    # gelu'(z_{i-1})) through the dGELU epilogue, d_x = bf16(dz_1 . Wb_1)
    for i in range(L, 0, -1):
        W = wb0[lay.w_off(i):lay.w_off(i) + D * D].reshape(D, D).astype(np.float64)
        dzr = _host(ex.value("dY" if i == L else f"d_z{i}")[rows]).astype(np.float64)
        v = dzr @ W
        if i > 1:
            v = bf(v * orc.gelu_grad_f64(_host(ex.value(f"z{i - 1}")[rows]).astype(np.float64)))
            assert orc.rel_err(_host(ex.value(f"d_z{i - 1}")[rows]), v) < 1e-2, f"d_z{i - 1}"
        else:
            assert orc.rel_err(_host(ex.value("d_x")[rows]), bf(v)) < 1e-2, "d_x"
    ex.reset_graph()


def test_c5_fused_optimizer_plan_bit_identical_at_full_shape(C):
    """C5 at its full shape with AdamW fused into the four weight-gradient
    GEMMs against the unfused plan (pinned to the oracle above), one replay
    each from the same start: loss, all 67,125,248 parameters, both moments
    and the bf16 shadow bit for bit."""
    from aicf_hip import mlp

    B, D, L = 8192, 4096, 4
    outs = []
    for fuse in (True, False):
        ir, lowered, plan = mlp.build_mlp_mse(B, D, L, fuse_optimizer=fuse)
        assert sum(it["op"] == "gemm_adamw" for it in lowered) == (L if fuse else 0)
        ex = mlp.make_executor(ir, lowered, plan)
        inputs, params = mlp.init_mlp_mse(B, D, L)
        ex.build_env(inputs=inputs, params=params, reuse_static=False)
        mlp.refresh_shadow(ex)
        ex.capture(inputs=inputs, params=params, reuse_static=True)
        ex.replay(1)
        torch.cuda.synchronize()
        outs.append({k: ex.value(k).cpu().clone() for k in ("loss", "flat.params", "opt.m.flat", "opt.v.flat",
                                                             "wb.flat")})
        ex.reset_graph()
        del ex
        torch.cuda.empty_cache()
    for k in outs[0]:
        assert torch.equal(outs[0][k], outs[1][k]), k


def test_c5_tail_plan_bit_identical_at_full_shape(C):
    """C5 at its full shape with the loss and bias tail in two launches
    (StageG) against the same plan without it, one replay each from the same
    start: all 67,125,248 parameters, both moments, the bf16 shadow, the bias
    gradients and the step counter bit for bit, the loss (summed in another
    order) to 1e-6."""
    from aicf_hip import mlp

    B, D, L = 8192, 4096, 4
    outs = []
    for tail in (True, False):
        ir, lowered, plan = mlp.build_mlp_mse(B, D, L, fuse_optimizer=True, fuse_colsum=True, fuse_tail=tail)
        assert ("mse_colsum" in [it["op"] for it in lowered]) == tail
        ex = mlp.make_executor(ir, lowered, plan)
        inputs, params = mlp.init_mlp_mse(B, D, L)
        ex.build_env(inputs=inputs, params=params, reuse_static=False)
        mlp.refresh_shadow(ex)
        ex.capture(inputs=inputs, params=params, reuse_static=True)
        ex.replay(1)
        torch.cuda.synchronize()
        b0 = mlp.FlatLayout(D, L).b_off(1)
        o = {k: ex.value(k).cpu().clone() for k in ("flat.params", "opt.m.flat", "opt.v.flat", "wb.flat", "opt.step")}
        o["bias_grads"] = ex.value("grad.flat")[b0:b0 + L * D].cpu().clone()
        o["loss"] = float(ex.value("loss").item())
        outs.append(o)
        ex.reset_graph()
        del ex
        torch.cuda.empty_cache()
    assert abs(outs[0].pop("loss") - outs[1]["loss"]) <= 1e-6 * abs(outs[1].pop("loss"))
    for k in outs[0]:
        assert torch.equal(outs[0][k], outs[1][k]), k
    assert int(outs[0]["opt.step"].item()) == 1


def test_c5_headline_plan_against_oracle_at_full_shape(C):
    """The exact plan the benchmark times (AdamW in the dW GEMMs' epilogue,
    the hidden bias gradients in the dGELU GEMMs' epilogue, the loss and bias
    tail in two launches) at the full C5 shape, replayed once from its graph,
    against the oracle directly.  The weight gradients exist only inside the
    GEMM epilogue; at t = 1 from zero moments m = fl((1 - b1) g) and
    v = fl((1 - b2) fl(g g)), so 4096 sampled m and v entries per layer pin
    them against fp64 dots over the 8192 stored rows (core_v2/lower.py:100-104),
    and the updated weights of those entries follow the oracle's AdamW from
    that gradient (adam_step/launcher.cu:276-291 with in-kernel bias
    correction).  Also: forward rows, the loss against fp64 mean((y - t)^2) on
    the stored y, dY bit for bit against the oracle's mse_grad
    (mse_grad/launcher.cu:61-71), bias gradients against fp64 column sums,
    the bias updates bit for bit, the bf16 shadow as the rounding of every
    updated weight, and the step counter."""
    from aicf_hip import mlp

    B, D, L = 8192, 4096, 4
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-8
    ir, lowered, plan = mlp.build_mlp_mse(B, D, L, fuse_optimizer=True, fuse_colsum=True, fuse_tail=True)
    ops = [it["op"] for it in lowered]
    assert ops.count("gemm_adamw") == L and "mse_colsum" in ops and "colsum_adamw" in ops
    ex = mlp.make_executor(ir, lowered, plan)
    inputs, params = mlp.init_mlp_mse(B, D, L)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    mlp.refresh_shadow(ex)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    P0 = ex.value("flat.params").cpu().numpy().copy()
    Wb0 = ex.value("wb.flat").cpu().clone()
    ex.replay(1)
    torch.cuda.synchronize()
    assert int(ex.value("opt.step").item()) == 1

    lay = mlp.FlatLayout(D, L)
    rows = torch.from_numpy(np.sort(np.random.default_rng(15).choice(B, 16, replace=False))).cuda()
    bf = lambda a: orc.bf16_round(a.astype(np.float32)).astype(np.float64)  # noqa: E731
    wb0 = orc.bf16_bits_to_f32(Wb0.view(torch.int16).numpy().view(np.uint16))
    # forward rows of every stored activation
    h = _host(ex.value("x")[rows]).astype(np.float64)
    for i in range(1, L + 1):
        W = wb0[lay.w_off(i):lay.w_off(i) + D * D].reshape(D, D).astype(np.float64)
        b = P0[lay.b_off(i):lay.b_off(i) + D].astype(np.float64)
        z = bf(h @ W.T + b[None, :])
        name = f"z{i}" if i < L else "y"
        assert orc.rel_err(_host(ex.value(name)[rows]), z) < 1e-2, name
        if i < L:
            h = bf(orc.gelu_f64(z))
            assert orc.rel_err(_host(ex.value(f"h{i}")[rows]), h) < 1e-2, f"h{i}"
    # loss and the output gradient (mse_colsum)
    y = _host(ex.value("y"))
    t = ex.value("t").cpu().numpy()
    ref_loss = orc.mse_loss_f64(y, t)
    assert abs(float(ex.value("loss").item()) - ref_loss) <= 1e-5 * ref_loss
    rs = rows.cpu().numpy()
    d = orc.mse_grad_f32(y[rs], t[rs], scale=np.float32(2.0) / np.float32(B * D))
    dY_bits = ex.value("dY")[rows].cpu().contiguous().view(torch.int16).numpy().view(np.uint16).ravel()
    assert np.array_equal(dY_bits, orc.bf16_bits_from_f32(d))
    del y, t

    G = ex.value("grad.flat").cpu().numpy()
    P1 = ex.value("flat.params").cpu().numpy()
    M1 = ex.value("opt.m.flat").cpu().numpy()
    V1 = ex.value("opt.v.flat").cpu().numpy()
    W1 = ex.value("wb.flat").cpu().view(torch.int16).numpy().view(np.uint16)
    # the shadow is the bf16 rounding of every updated parameter; no weight
    # moved by more than lr (at t = 1 the step is lr g / (|g| + eps))
    assert np.array_equal(W1, orc.bf16_bits_from_f32(P1))
    assert np.isfinite(P1).all() and np.isfinite(M1).all() and (V1 >= 0).all()
    assert np.abs(P1 - P0).max() <= lr * (1 + 1e-5)
    # bias gradients (column sums of the stored output gradients) and their
    # update, bit for bit from those gradients
    b0_, nb = lay.b_off(1), L * D
    for i in range(1, L + 1):
        dz = _host(ex.value("dY" if i == L else f"d_z{i}")).astype(np.float64).sum(axis=0)
        assert orc.rel_err(G[lay.b_off(i):lay.b_off(i) + D], dz) < 1e-5, f"db{i}"
    Zb = np.zeros(nb, np.float32)
    Pr, Mr, Vr, Wr = orc.adamw(P0[b0_:b0_ + nb], G[b0_:b0_ + nb], Zb, Zb, 1, lr, b1, b2, eps, 0.0, shadow=True)
    assert np.array_equal(P1[b0_:b0_ + nb], Pr) and np.array_equal(M1[b0_:b0_ + nb], Mr)
    assert np.array_equal(V1[b0_:b0_ + nb], Vr) and np.array_equal(W1[b0_:b0_ + nb], Wr)
    # weight gradients through the moments, and the weights' update from them
    omb1 = np.float64(np.float32(1.0) - np.float32(b1))
    omb2 = np.float64(np.float32(1.0) - np.float32(b2))
    r = np.random.default_rng(16)
    for i in range(1, L + 1):
        o_idx = np.sort(r.choice(D, 64, replace=False))
        j_idx = np.sort(r.choice(D, 64, replace=False))
        dz = ex.value("dY" if i == L else f"d_z{i}")[:, torch.from_numpy(o_idx).cuda()]
        hp = ex.value("x" if i == 1 else f"h{i - 1}")[:, torch.from_numpy(j_idx).cuda()]
        g = _host(dz).astype(np.float64).T @ _host(hp).astype(np.float64)
        sel = lambda a: a[lay.w_off(i):lay.w_off(i) + D * D].reshape(D, D)[np.ix_(o_idx, j_idx)]  # noqa: E731
        m, v = sel(M1), sel(V1)
        assert orc.rel_err(m, omb1 * g) < 1e-4, f"m{i}"
        assert orc.rel_err(v, omb2 * g * g) < 2e-4, f"v{i}"
        # the oracle's AdamW from the gradient these moments hold
        g32 = (m.astype(np.float64) / omb1).astype(np.float32)
        Z = np.zeros(g32.size, np.float32)
        pr, mr, vr = orc.adamw(sel(P0), g32, Z, Z, 1, lr, b1, b2, eps, 0.0)
        step_gpu = (sel(P1).astype(np.float64) - sel(P0)).ravel()
        step_ref = (pr.astype(np.float64) - sel(P0).ravel())
        assert orc.rel_err(step_gpu, step_ref) < 1e-5, f"P{i}"
        assert orc.rel_err(v.ravel(), vr) < 1e-6, f"v{i} vs m{i}"
    ex.reset_graph()
