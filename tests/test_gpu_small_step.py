"""The small-step kernels against the CPU oracle: the small fp32 GEMM path
(every operand layout, ragged sizes, the bias+ReLU epilogue, the copy of B),
the fused classifier head (with and without the step counter), the gradient
group with and without AdamW at the store, the multi-tensor AdamW, and the
reference MLP's step in its three- and four-launch lowerings, eager and
replayed, under AICF_WARMUP too, and bit-identical to each other."""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

GGRP = int.from_bytes(b"GGRP", "little")
GGRA = int.from_bytes(b"GGRA", "little")
XHST = int.from_bytes(b"XHST", "little")
GEPI = int.from_bytes(b"GEPI", "little")
ADAM = int.from_bytes(b"ADAM", "little")
STEP_OPS = {True: ["gemm_epilogue_bcopy", "xent_head", "grad_group_adamw"],
            "four": ["gemm_epilogue", "xent_head", "grad_group", "adamw_multi"]}


def _orc():
    import oracle as orc  # test infrastructure

    return orc


def g(a, dt=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dt is None else t.to(dt)


SMALL = [(64, 256, 784), (256, 784, 64), (64, 784, 256), (10, 256, 64), (1, 1, 1), (17, 33, 5),
         (100, 3, 1000), (31, 47, 130), (48, 16, 4096), (7, 19, 803), (33, 9, 517)]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_small_gemm_every_layout(C, ta, tb):
    """Problems with fewer than 128 tiles of 64 x 64 take the small-GEMM path
    (one 16 x 16 tile per wave, K split over the workgroup): fp32 rel-err
    <= 1e-4 against fp64 for every transposition and ragged M, N, K."""
    orc = _orc()
    r = np.random.default_rng(11 + 2 * ta + tb)
    for M, N, K in SMALL:
        A = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
        B = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
        o = torch.empty((M, N), device="cuda")
        C.op_call(int(C.OpKind.Gemm), [g(A), g(B)], [o], 0, struct.pack("<ii", ta, tb), 0)
        torch.cuda.synchronize()
        e = orc.rel_err(o.cpu().numpy(), orc.gemm_f64(A, B, bool(ta), bool(tb)))
        assert e < 1e-4, (M, N, K, ta, tb, e)


def test_small_gemm_bias_relu_epilogue_and_views(C):
    """gemm_bias_relu_f32_naive_v0 on the reference MLP's first layer shape
    (64 x 784 . 256 x 784^T + b, ReLU) and on strided operand views."""
    orc = _orc()
    r = np.random.default_rng(5)
    x = r.standard_normal((64, 784)).astype(np.float32)
    W = r.standard_normal((256, 784)).astype(np.float32) * 0.05
    b = r.standard_normal(256).astype(np.float32)
    o = torch.empty((64, 256), device="cuda")
    gpel = int.from_bytes(b"GPEL", "big")
    C.launch_by_id("gemm_bias_relu_f32_naive_v0", C.OpKind.GemmEpilogue, [g(x), g(W), g(b)], [o], gpel,
                   struct.pack("<iii", 0, 1, 1), 0)
    torch.cuda.synchronize()
    ref = np.maximum(orc.gemm_f64(x, W, False, True) + b, 0)
    assert orc.rel_err(o.cpu().numpy(), ref) < 1e-4
    # views with row strides larger than the row: the small path reads them in place
    big = g(r.standard_normal((70, 900)).astype(np.float32))
    wb = g(r.standard_normal((40, 900)).astype(np.float32))
    av, bv = big[3:67, 5:805], wb[:, 100:900]
    o2 = torch.empty((64, 40), device="cuda")
    C.op_call(int(C.OpKind.Gemm), [av, bv], [o2], 0, struct.pack("<ii", 0, 1), 0)
    torch.cuda.synchronize()
    ref2 = orc.gemm_f64(av.cpu().numpy(), bv.cpu().numpy(), False, True)
    assert orc.rel_err(o2.cpu().numpy(), ref2) < 1e-4


@pytest.mark.parametrize("B,K,Cn", [(64, 256, 10), (37, 72, 7), (5, 2048, 32), (130, 516, 16)])
def test_xent_head_against_oracle(C, B, K, Cn):
    """logits, dlogits (rel <= 1e-5), argmax (exact), row loss (rel <= 1e-5),
    dH = dlogits . W and the ReLU backward (rel <= 1e-5; dX exact zeros where
    the saved output is not positive); an out-of-range label gives a NaN row
    loss and no one-hot term."""
    orc = _orc()
    r = np.random.default_rng(B + K + Cn)
    H = np.maximum(r.standard_normal((B, K)), 0).astype(np.float32)
    W = (r.standard_normal((Cn, K)) / np.sqrt(K)).astype(np.float32)
    b = r.standard_normal(Cn).astype(np.float32)
    t = r.integers(0, Cn, B).astype(np.int32)
    t[B // 2] = Cn  # out of range
    H[1, :] = 0.0
    outs = [torch.empty((B, Cn), device="cuda"), torch.empty((B, Cn), device="cuda"),
            torch.empty(B, dtype=torch.int32, device="cuda"), torch.empty(B, device="cuda"),
            torch.empty((B, K), device="cuda"), torch.empty((B, K), device="cuda")]
    Hd = g(H)
    C.launch_by_id("xent_head_f32_v0", C.OpKind.XentHead, [Hd, g(W), g(b), g(t), Hd], outs, 0, b"", 0)
    torch.cuda.synchronize()
    z = H.astype(np.float64) @ W.T.astype(np.float64) + b
    zg = outs[0].cpu().numpy()
    assert orc.rel_err(zg, z) < 1e-5
    _, dz, am, rl = orc.softmax_xent_f64(zg, t)
    assert np.array_equal(outs[2].cpu().numpy(), am)
    rlg = outs[3].cpu().numpy()
    valid = np.arange(B) != B // 2
    assert np.isnan(rlg[B // 2]) and orc.rel_err(rlg[valid], rl[valid]) < 1e-5
    assert orc.rel_err(outs[1].cpu().numpy(), dz) < 1e-5
    dH = outs[1].cpu().numpy().astype(np.float64) @ W.astype(np.float64)
    assert orc.rel_err(outs[4].cpu().numpy(), dH) < 1e-5
    dX = outs[5].cpu().numpy()
    assert np.array_equal(dX == 0, (H <= 0) | (outs[4].cpu().numpy() == 0))
    assert np.array_equal(dX[H > 0], outs[4].cpu().numpy()[H > 0])


def _group(C, ins, outs, jobs):
    pay = struct.pack("<i", len(jobs)) + b"".join(struct.pack("<iiiiii", *j) for j in jobs)
    C.launch_by_id("grad_group_f32_v0", C.OpKind.GradGroup, ins, outs, GGRP, pay, 0)


def test_grad_group_jobs_against_oracle(C):
    """Every job type in one launch: three GEMMs (plain, A transposed, B
    transposed) at rel <= 1e-4, two column sums at rel <= 1e-5, the loss
    mean bit-identical to softmax_xent's, the step counter +1."""
    orc = _orc()
    r = np.random.default_rng(3)
    dY = r.standard_normal((64, 10)).astype(np.float32)
    h = r.standard_normal((64, 256)).astype(np.float32)
    dl = r.standard_normal((64, 256)).astype(np.float32)
    W0 = r.standard_normal((256, 784)).astype(np.float32)
    x = r.standard_normal((64, 784)).astype(np.float32)
    logits = r.standard_normal((64, 10)).astype(np.float32)
    lab = r.integers(0, 10, 64).astype(np.int32)
    # softmax_xent on the GPU for its row losses and its mean
    xl, xd = torch.empty((), device="cuda"), torch.empty((64, 10), device="cuda")
    xa, xr = torch.empty(64, dtype=torch.int32, device="cuda"), torch.empty(64, device="cuda")
    C.op_call(int(C.OpKind.SoftmaxXent), [g(logits), g(lab)], [xl, xd, xa, xr], 0, b"", 0)
    step = torch.tensor(41, dtype=torch.int32, device="cuda")
    ins = [g(dY), g(h), g(dl), g(W0), g(x), xr, step]
    dW1 = torch.empty((10, 256), device="cuda")
    db1 = torch.empty(10, device="cuda")
    dx = torch.empty((64, 784), device="cuda")
    dW0 = torch.empty((256, 784), device="cuda")
    db0 = torch.empty(256, device="cuda")
    loss = torch.empty((), device="cuda")
    xT = torch.empty((64, 64), device="cuda")
    outs = [dW1, db1, dx, dW0, db0, loss, step, xT]
    jobs = [(0, 0, 1, 0, 1, 0), (1, 0, 0, 1, 0, 0), (0, 2, 3, 2, 0, 0), (0, 2, 4, 3, 1, 0),
            (1, 2, 0, 4, 0, 0), (2, 5, 0, 5, 0, 0), (3, 6, 0, 6, 1, 0), (0, 4, 4, 7, 0, 1)]
    _group(C, ins, outs, jobs)
    torch.cuda.synchronize()
    assert orc.rel_err(dW1.cpu().numpy(), orc.gemm_f64(dY, h, True, False)) < 1e-4
    assert orc.rel_err(dx.cpu().numpy(), orc.gemm_f64(dl, W0, False, False)) < 1e-4
    assert orc.rel_err(dW0.cpu().numpy(), orc.gemm_f64(dl, x, True, False)) < 1e-4
    assert orc.rel_err(xT.cpu().numpy(), orc.gemm_f64(x, x, False, True)) < 1e-4
    assert orc.rel_err(db1.cpu().numpy(), orc.colsum_f64(dY)) < 1e-5
    assert orc.rel_err(db0.cpu().numpy(), orc.colsum_f64(dl)) < 1e-5
    assert torch.equal(loss, xl)
    assert int(step.item()) == 42
    # the warmup form of the step job copies
    _group(C, [step], [step], [(3, 0, 0, 0, 0, 0)])
    torch.cuda.synchronize()
    assert int(step.item()) == 42


def test_adamw_multi_bit_identical_to_adamw_step(C):
    """Four tensors (sizes with every tail length) updated in one launch for
    three steps match four adamw_step launches bit for bit, and the oracle."""
    orc = _orc()
    r = np.random.default_rng(9)
    sizes = (1000, 7, 4099, 1)
    P = [r.standard_normal(n).astype(np.float32) for n in sizes]
    G = [[r.standard_normal(n).astype(np.float32) * 1e-2 for n in sizes] for _ in range(3)]
    pay = struct.pack("<fffff", 1e-3, 0.9, 0.999, 1e-8, 0.01)
    a = [[g(p), torch.zeros(p.size, device="cuda"), torch.zeros(p.size, device="cuda")] for p in P]
    b = [[g(p), torch.zeros(p.size, device="cuda"), torch.zeros(p.size, device="cuda")] for p in P]
    sa = torch.zeros((), dtype=torch.int32, device="cuda")
    Mo = [np.zeros(n, np.float32) for n in sizes]
    Vo = [np.zeros(n, np.float32) for n in sizes]
    Po = [p.copy() for p in P]
    for t in range(3):
        sa.fill_(t + 1)
        ins, outs = [], []
        for k in range(4):
            gk = g(G[t][k])
            ins += [a[k][0], gk, a[k][1], a[k][2]]
            outs += [a[k][0], a[k][1], a[k][2]]
            C.launch_by_id("adamw_step_f32_v1", C.OpKind.AdamStep, [b[k][0], gk, b[k][1], b[k][2], sa],
                           [b[k][0], b[k][1], b[k][2]], ADAM, pay, 0)
        C.launch_by_id("adamw_multi_f32_v0", C.OpKind.AdamWMulti, ins + [sa], outs, ADAM, pay, 0)
        torch.cuda.synchronize()
        for k in range(4):
            for u, v in zip(a[k], b[k]):
                assert torch.equal(u, v), (t, k)
            Po[k], Mo[k], Vo[k] = orc.adamw(Po[k], G[t][k], Mo[k], Vo[k], t + 1, 1e-3, wd=0.01)
            assert np.array_equal(a[k][0].cpu().numpy(), Po[k]), (t, k)


@pytest.mark.parametrize("fuse_small", [True, "four"])
@pytest.mark.parametrize("seed,shape", [(0, (64, 784, 256, 10)), (1, (37, 100, 72, 7)),
                                        (2, (200, 64, 512, 32))])
def test_fused_step_against_oracle(C, seed, shape, fuse_small):
    """The reference MLP's step in three launches (StageF) and in four: an
    eager step and three replays of the captured step, each against the
    oracle (loss rel <= 1e-5, argmax exact, gradients <= 1e-4, AdamW
    bit-exact on the GPU's gradients), at the reference shape and at ragged
    ones."""
    import mlp_checks

    B, din, dh, dout = shape
    ex, inputs, params, orc_state, data = mlp_checks.xent_setup(seed, B=B, din=din, dh=dh, dout=dout,
                                                                fuse_small=fuse_small)
    assert [op for op, *_ in ex.ops] == STEP_OPS[fuse_small]
    res = {"ok": True}
    ex.run(inputs=inputs, params=params, reuse_static=False)
    torch.cuda.synchronize()
    assert orc_state.check(ex, params, data["x"], data["t"], "eager", res), res
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    for t in range(3):
        ex.replay(1)
        torch.cuda.synchronize()
        assert orc_state.check(ex, params, data["x"], data["t"], f"replay{t}", res), res
    ex.reset_graph()


@pytest.mark.parametrize("fuse_small", [True, "four"])
def test_fused_step_warmup_branch(C, monkeypatch, fuse_small):
    """AICF_WARMUP=1 on the three- and four-launch steps: the step increment
    (in the head, or the group's step job) adds 0 and every AdamW update runs
    with lr 0 (parameters and step unchanged, moments as the oracle's);
    unset, replays take real steps."""
    import mlp_checks

    ex, inputs, params, orc_state, data = mlp_checks.xent_setup(7, fuse_small=fuse_small)
    assert [op for op, *_ in ex.ops] == STEP_OPS[fuse_small]
    P0 = {k: p.detach().cpu().clone() for k, p in params.items()}
    res = {"ok": True}
    monkeypatch.setenv("AICF_WARMUP", "1")
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    ex.run(inputs={}, params={}, reuse_static=True)
    torch.cuda.synchronize()
    assert orc_state.check(ex, params, data["x"], data["t"], "warm", res, warmup=True), res
    for k, p in params.items():
        assert torch.equal(p.cpu(), P0[k]), k
    assert int(ex.value("opt.step").item()) == 0
    monkeypatch.delenv("AICF_WARMUP")
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    for t in (1, 2):
        ex.replay(1)
        torch.cuda.synchronize()
        assert orc_state.check(ex, params, data["x"], data["t"], f"replay{t}", res), res
    assert int(ex.value("opt.step").item()) == 2
    ex.reset_graph()


@pytest.mark.parametrize("shape", [(64, 784, 256, 10), (37, 100, 72, 7)])
def test_three_launch_step_bit_identical_to_four(C, shape):
    """The three-launch step (forward GEMM writing W0's copy, head advancing
    the step, AdamW at the group's stores) and the four-launch step give the
    same bits for every value the step writes, eager and over three replays:
    the GEMM tiles, column sums and AdamW element updates are the same code
    in the same order, and the copy of W0 is W0."""
    import mlp_checks

    B, din, dh, dout = shape
    runs = {}
    for fs in (True, "four"):
        ex, inputs, params, orc_state, data = mlp_checks.xent_setup(3, B=B, din=din, dh=dh, dout=dout,
                                                                    fuse_small=fs)
        snaps = []
        ex.run(inputs=inputs, params=params, reuse_static=False)
        torch.cuda.synchronize()
        names = ["loss", "logits", "dY", "pred", "row_loss", "d_x", "d_0.W", "d_0.b", "d_2.W", "d_2.b",
                 "opt.step", "opt.m.0.W", "opt.v.0.W", "opt.m.2.b", "opt.v.2.b"]
        snap = lambda: {**{k: ex.value(k).detach().cpu().clone() for k in names},  # noqa: E731
                        **{k: p.detach().cpu().clone() for k, p in params.items()}}
        snaps.append(snap())
        ex.capture(inputs=inputs, params=params, reuse_static=True)
        for _ in range(3):
            ex.replay(1)
            torch.cuda.synchronize()
            snaps.append(snap())
        ex.reset_graph()
        runs[fs] = snaps
    for t, (a, b) in enumerate(zip(runs[True], runs["four"])):
        for k in a:
            assert torch.equal(a[k], b[k]), (t, k)
    assert int(runs[True][-1]["opt.step"].item()) == 4


def _bias_corrections(C, step, lr=1e-3, b1=0.9, b2=0.999):
    """{lr / bc1, 1 / bc2} of the counter's step, written by the head's
    counter workgroup (a one-row head, the counter advanced by 0)."""
    H = torch.ones((1, 4), device="cuda")
    W = torch.ones((1, 4), device="cuda")
    outs = [torch.empty((1, 1), device="cuda"), torch.empty((1, 1), device="cuda"),
            torch.empty(1, dtype=torch.int32, device="cuda"), torch.empty(1, device="cuda"),
            torch.empty((1, 4), device="cuda"), torch.empty((1, 4), device="cuda")]
    scal = torch.full((2,), float("nan"), device="cuda")
    C.launch_by_id("xent_head_step_f32_v0", C.OpKind.XentHead,
                   [H, W, torch.zeros(1, device="cuda"), torch.zeros(1, dtype=torch.int32, device="cuda"), H, step],
                   outs + [step, scal], XHST, struct.pack("<ifff", 0, lr, b1, b2), 0)
    return scal


def _ggra(C, ins, outs, jobs, si, lr=1e-3, wd=0.01):
    head = struct.pack("<ifffffi", len(jobs), lr, 0.9, 0.999, 1e-8, wd, si)
    pay = head + b"".join(struct.pack("<" + "i" * 12, *j) for j in jobs)
    C.launch_by_id("grad_group_adamw_f32_v0", C.OpKind.GradGroup, ins, outs, GGRA, pay, 0)


@pytest.mark.parametrize("M,N,K", [(10, 256, 64), (256, 784, 64), (33, 47, 5), (16, 100, 300)])
def test_grad_group_adamw_bit_identical_to_adamw_step(C, M, N, K):
    """GEMM and column-sum jobs with AdamW at the store (bias corrections
    from the head's counter workgroup), over two steps, against the same
    group without AdamW followed by adamw_step on its outputs (bias
    corrections from the counter): gradients and P, M, V bit-identical
    (ragged tiles, K split over the waves, columns past 64), and a job
    without AdamW beside them."""
    r = np.random.default_rng(M + N + K)
    A = g(r.standard_normal((K, M)).astype(np.float32))    # read transposed: dW = A^T . X
    X = g(r.standard_normal((K, N)).astype(np.float32))
    Y = g(r.standard_normal((K, M)).astype(np.float32))    # column sums of Y
    pay = struct.pack("<fffff", 1e-3, 0.9, 0.999, 1e-8, 0.01)

    def state():
        return [g(r2.standard_normal(n).astype(np.float32)) for n in (M * N, M * N, M * N, M, M, M)]

    r2 = np.random.default_rng(1)
    fused = state()
    r2 = np.random.default_rng(1)
    ref = state()
    for P in (fused, ref):
        P[2].abs_()
        P[5].abs_()  # second moments are not negative
    sf = torch.zeros((), dtype=torch.int32, device="cuda")
    sr = torch.zeros((), dtype=torch.int32, device="cuda")
    for t in range(2):
        sf.fill_(t + 1)
        sr.fill_(t + 1)
        dW, db, xx = (torch.empty((M, N), device="cuda"), torch.empty(M, device="cuda"),
                      torch.empty((N, N), device="cuda"))
        W, Wm, Wv, b, bm, bv = fused
        ins = [A, X, Y, W.view(M, N), Wm, Wv, b, bm, bv, _bias_corrections(C, sf)]
        outs = [dW, W.view(M, N), Wm, Wv, db, b, bm, bv, xx]
        jobs = [[0, 0, 1, 0, 1, 0, 3, 4, 5, 1, 2, 3],
                [1, 2, 0, 4, 0, 0, 6, 7, 8, 5, 6, 7],
                [0, 1, 1, 8, 1, 0, -1, -1, -1, -1, -1, -1]]
        _ggra(C, ins, outs, jobs, 9)
        rW, rb, rx = (torch.empty((M, N), device="cuda"), torch.empty(M, device="cuda"),
                      torch.empty((N, N), device="cuda"))
        _group(C, [A, X, Y], [rW, rb, rx], [(0, 0, 1, 0, 1, 0), (1, 2, 0, 1, 0, 0), (0, 1, 1, 2, 1, 0)])
        for P, Gd, Mm, Vv in ((ref[0], rW.view(-1), ref[1], ref[2]), (ref[3], rb, ref[4], ref[5])):
            C.launch_by_id("adamw_step_f32_v1", C.OpKind.AdamStep, [P, Gd, Mm, Vv, sr], [P, Mm, Vv], ADAM, pay, 0)
        torch.cuda.synchronize()
        assert torch.equal(dW, rW) and torch.equal(db, rb) and torch.equal(xx, rx), t
        for k in range(6):
            assert torch.equal(fused[k], ref[k]), (t, k)


@pytest.mark.parametrize("M,N,K", [(64, 256, 784), (5, 33, 12), (100, 40, 516)])
def test_gemm_bcopy_writes_b_and_the_same_c(C, M, N, K):
    """gemm_small_bcopy_f32_v0: C bit-identical to the plain small-GEMM
    epilogue on the same call, and the second output is B exactly (K split
    over 1, 8 and 16 waves, N and K tails)."""
    r = np.random.default_rng(M * N + K)
    A = g(r.standard_normal((M, K)).astype(np.float32))
    W = g(r.standard_normal((N, K)).astype(np.float32))
    b = g(r.standard_normal(N).astype(np.float32))
    for kind in (0, 1, 2):
        c1, c2 = torch.empty((M, N), device="cuda"), torch.empty((M, N), device="cuda")
        wc = torch.full((N, K), float("nan"), device="cuda")
        attr = struct.pack("<iii", 0, 1, kind)
        C.launch_by_id("gemm_small_bcopy_f32_v0", C.OpKind.GemmEpilogue, [A, W, b], [c1, wc], GEPI, attr, 0)
        C.launch_by_id("gemm_bias_relu_f32_naive_v0", C.OpKind.GemmEpilogue, [A, W, b], [c2], GEPI, attr, 0)
        torch.cuda.synchronize()
        assert torch.equal(c1, c2), kind
        assert torch.equal(wc, W), kind


def test_xent_head_step_variant_matches_the_plain_head(C):
    """xent_head_step_f32_v0 writes the plain head's bits and advances the
    counter by 1, or by 0 (the warmup form)."""
    r = np.random.default_rng(4)
    B, K, Cn = 64, 256, 10
    H = g(np.maximum(r.standard_normal((B, K)), 0).astype(np.float32))
    W = g((r.standard_normal((Cn, K)) / 16).astype(np.float32))
    b = g(r.standard_normal(Cn).astype(np.float32))
    t = g(r.integers(0, Cn, B).astype(np.int32))

    def outs():
        return [torch.empty((B, Cn), device="cuda"), torch.empty((B, Cn), device="cuda"),
                torch.empty(B, dtype=torch.int32, device="cuda"), torch.empty(B, device="cuda"),
                torch.empty((B, K), device="cuda"), torch.empty((B, K), device="cuda")]

    ref = outs()
    C.launch_by_id("xent_head_f32_v0", C.OpKind.XentHead, [H, W, b, t, H], ref, 0, b"", 0)
    step = torch.tensor(5, dtype=torch.int32, device="cuda")
    for inc, want in ((1, 6), (0, 6), (1, 7)):
        o = outs()
        C.launch_by_id("xent_head_step_f32_v0", C.OpKind.XentHead, [H, W, b, t, H, step], o + [step], XHST,
                       struct.pack("<i", inc), 0)
        torch.cuda.synchronize()
        assert int(step.item()) == want
        for u, v in zip(o, ref):
            assert torch.equal(u, v), inc
    # with the hyperparameters: the bias corrections of the advanced step
    # (fp64 powers rounded to fp32 once; bit-exactness against adamw_step is
    # checked through the group's updates)
    scal = torch.empty(2, device="cuda")
    o = outs()
    C.launch_by_id("xent_head_step_f32_v0", C.OpKind.XentHead, [H, W, b, t, H, step], o + [step, scal], XHST,
                   struct.pack("<ifff", 1, 2e-3, 0.8, 0.99), 0)
    torch.cuda.synchronize()
    assert int(step.item()) == 8
    for u, v in zip(o, ref):
        assert torch.equal(u, v)
    want = (np.float32(2e-3) / np.float32(1 - 0.8 ** 8), 1 / np.float32(1 - 0.99 ** 8))
    assert np.allclose(scal.cpu().numpy(), want, rtol=1e-6), (scal, want)


def test_graph_of_several_steps_matches_single_step_replays(C):
    """capture(steps=3): one replay of the three-launch step's graph advances
    three steps, bit-identical to three replays of the one-step graph
    (replayed with the C++ n-launch loop); steps < 1 is refused."""
    import mlp_checks

    runs = {}
    for per, replays in ((1, 6), (3, 2)):
        ex, inputs, params, orc_state, data = mlp_checks.xent_setup(5, fuse_small=True)
        ex.build_env(inputs=inputs, params=params, reuse_static=False)
        ex.capture(inputs=inputs, params=params, reuse_static=True, steps=per)
        assert ex.steps_per_replay == per
        ex.replay(replays)
        torch.cuda.synchronize()
        runs[per] = {k: p.detach().cpu().clone() for k, p in params.items()}
        runs[per]["loss"] = ex.value("loss").detach().cpu().clone()
        runs[per]["step"] = int(ex.value("opt.step").item())
        with pytest.raises(ValueError):
            ex.capture(inputs=inputs, params=params, reuse_static=True, steps=0)
        ex.reset_graph()
    assert runs[1]["step"] == runs[3]["step"] == 6
    for k in runs[1]:
        if k != "step":
            assert torch.equal(runs[1][k], runs[3][k]), k
