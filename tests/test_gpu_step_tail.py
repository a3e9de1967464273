"""The tail ops of the large MSE step against the CPU oracle and against the
ops they replace: mse_colsum (gradient bits from the oracle, column partials
bit-identical to the two-pass column sum's workspace, loss from the fp64
oracle, step counter), colsum_adamw (the finish order restated in fp32 and
the oracle's AdamW, bit for bit), the dGELU partials epilogue (kind 7)
against kind 6, and the StageG plan against the plans without it, replayed
as graphs and under AICF_WARMUP."""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MSCS = int.from_bytes(b"MSCS", "little")
CADW = int.from_bytes(b"CADW", "little")
GEPI = int.from_bytes(b"GEPI", "little")
RSUM = int.from_bytes(b"RSUM", "big")


def _orc():
    import oracle as orc  # test infrastructure

    return orc


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    return t.view(torch.int16).numpy() if t.dtype in (torch.bfloat16, torch.float16) else t.view(torch.int32).numpy()


@pytest.mark.parametrize("bf", [True, False])
@pytest.mark.parametrize("M,N,P", [(512, 1024, 8), (8192, 4096, 64), (384, 520, 3)])
def test_mse_colsum_against_oracle_and_column_sum(C, bf, M, N, P):
    orc = _orc()
    if not bf and N % 4 or bf and N % 8:
        pytest.skip("width off the vector path")
    g = torch.Generator(device="cuda")
    g.manual_seed(M + N)
    pred = torch.randn((M, N), device="cuda", generator=g)
    pred = pred.to(torch.bfloat16) if bf else pred
    tgt = torch.randn((M, N), device="cuda", generator=g)
    step = torch.full((), 5, dtype=torch.int32, device="cuda")
    dY = torch.empty_like(pred)
    loss = torch.empty((), device="cuda")
    lp = torch.empty(8192, device="cuda")
    cp = torch.full((P, N), float("nan"), device="cuda")
    C.op_call(int(C.OpKind.MseColsum), [pred, tgt, step], [dY, loss, lp, cp, step], MSCS,
              struct.pack("<fi", 0.0, 1), 0)
    torch.cuda.synchronize()
    p32 = pred.float().cpu().numpy()
    t32 = tgt.cpu().numpy()
    d = orc.mse_grad_f32(p32, t32)
    if bf:
        assert np.array_equal(_bits(dY).view(np.uint16).ravel(), orc.bf16_bits_from_f32(d))
    else:
        assert np.array_equal(dY.cpu().numpy().ravel(), d)
    ref_loss = orc.mse_loss_f64(p32, t32)
    assert abs(float(loss.item()) - ref_loss) <= 1e-6 * ref_loss
    assert int(step.item()) == 6
    # every partial row is the fp64 column sum of its M / P rows of the stored gradient to
    # fp32 rounding; for bf16 it is the two-pass column sum's workspace, bit for bit
    dYh = dY.float().cpu().numpy()
    rows = M // P
    for q in range(P):
        e = orc.rel_err(cp[q].cpu().numpy(), orc.colsum_f64(dYh[q * rows:(q + 1) * rows]))
        assert e < 1e-5, (q, e)
    if bf:
        db = torch.empty(N, device="cuda")
        ws = torch.empty((P, N), device="cuda")
        C.op_call(int(C.OpKind.ReduceSum), [dY], [db, ws], RSUM, struct.pack("<q", 0), 0)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(cp), _bits(ws))
    # step += 0 under the warmup attribute
    C.op_call(int(C.OpKind.MseColsum), [pred, tgt, step], [dY, loss, lp, cp, step], MSCS,
              struct.pack("<fi", 0.0, 0), 0)
    torch.cuda.synchronize()
    assert int(step.item()) == 6


def _finish_f32(c: np.ndarray) -> np.ndarray:
    """The column-sum finish order in fp32: four row strides of 4 (rows
    16 at a time as (a0 + a1) + (a2 + a3), then one at a time), combined
    (s0 + s1) + (s2 + s3)."""
    R = c.shape[0]
    f = np.float32
    s4 = []
    for w in range(4):
        s = np.zeros(c.shape[1], f)
        r = w
        while r + 12 < R:
            s = (s + ((c[r] + c[r + 4]).astype(f) + (c[r + 8] + c[r + 12]).astype(f))).astype(f)
            r += 16
        while r < R:
            s = (s + c[r]).astype(f)
            r += 4
        s4.append(s)
    return ((s4[0] + s4[1]).astype(f) + (s4[2] + s4[3]).astype(f)).astype(f)


@pytest.mark.parametrize("shapes,wd", [([(32, 256), (64, 128), (5, 64)], 0.0), ([(2, 4096)], 0.01),
                                       ([(17, 96)] * 8, 0.0)])
def test_colsum_adamw_against_oracle(C, shapes, wd):
    orc = _orc()
    r = np.random.default_rng(len(shapes) * 100 + shapes[0][0])
    parts = [r.standard_normal(s).astype(np.float32) * 1e-2 for s in shapes]
    n = sum(s[1] for s in shapes)
    P = r.standard_normal(n).astype(np.float32) * 0.02
    M = r.standard_normal(n).astype(np.float32) * 1e-3
    V = np.abs(r.standard_normal(n).astype(np.float32)) * 1e-5
    step = 3
    dev = [torch.from_numpy(p).cuda() for p in parts]
    Pd, Md, Vd = (torch.from_numpy(a.copy()).cuda() for a in (P, M, V))
    S = torch.full((), step, dtype=torch.int32, device="cuda")
    G = torch.empty(n, device="cuda")
    W = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    pay = struct.pack("<ifffff", len(shapes), 1e-3, 0.9, 0.999, 1e-8, wd)
    C.op_call(int(C.OpKind.ColsumAdamW), dev + [Pd, Md, Vd, S], [G, Pd, Md, Vd, W], CADW, pay, 0)
    torch.cuda.synchronize()
    g = np.concatenate([_finish_f32(p) for p in parts])
    assert np.array_equal(G.cpu().numpy(), g)
    Pr, Mr, Vr, Wr = orc.adamw(P, g, M, V, step, 1e-3, 0.9, 0.999, 1e-8, wd, shadow=True)
    assert np.array_equal(Pd.cpu().numpy(), Pr)
    assert np.array_equal(Md.cpu().numpy(), Mr)
    assert np.array_equal(Vd.cpu().numpy(), Vr)
    assert np.array_equal(_bits(W).view(np.uint16), Wr)


@pytest.mark.parametrize("M,N,K", [(512, 768, 320), (8192, 4096, 4096)])
def test_dgelu_partials_epilogue_matches_kind6(C, M, N, K):
    """GEPI kind 7 writes the same dZ and the same per-tile column sums as
    kind 6 (whose finished column sums the plan tests pin to the oracle)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(M + K)
    s = 1.0 / np.sqrt(K)
    A = (torch.randn((M, K), device="cuda", generator=g) * s).to(torch.bfloat16)
    B = (torch.randn((K, N), device="cuda", generator=g) * s).to(torch.bfloat16)
    Z = torch.randn((M, N), device="cuda", generator=g).to(torch.bfloat16)
    C6, C7 = torch.empty((M, N), dtype=torch.bfloat16, device="cuda"), torch.empty((M, N), dtype=torch.bfloat16,
                                                                                  device="cuda")
    db = torch.empty(N, device="cuda")
    ws = torch.empty((M // 256, N), device="cuda")
    part = torch.full((M // 256, N), float("nan"), device="cuda")
    C.op_call(int(C.OpKind.GemmEpilogue), [A, B, Z], [C6, db, ws], GEPI, struct.pack("<iii", 0, 0, 6), 0)
    C.op_call(int(C.OpKind.GemmEpilogue), [A, B, Z], [C7, part], GEPI, struct.pack("<iii", 0, 0, 7), 0)
    torch.cuda.synchronize()
    assert torch.equal(C6, C7)
    assert np.array_equal(_bits(part), _bits(ws))
    assert np.array_equal(_finish_f32(part.cpu().numpy()), db.cpu().numpy())


def _run_plan(B, D, L, steps, **kw):
    from aicf_hip import mlp

    ir, lowered, plan = mlp.build_mlp_mse(B, D, L, **kw)
    ex = mlp.make_executor(ir, lowered, plan)
    inputs, params = mlp.init_mlp_mse(B, D, L, seed=4)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    mlp.refresh_shadow(ex)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    losses = []
    for _ in range(steps):
        ex.replay(1)
        torch.cuda.synchronize()
        losses.append(float(ex.value("loss").item()))
    lay = mlp.FlatLayout(D, L)
    b0 = lay.b_off(1)
    out = {k: ex.value(k).cpu().clone() for k in ("flat.params", "opt.m.flat", "opt.v.flat", "wb.flat", "opt.step")}
    out["bias_grads"] = ex.value("grad.flat")[b0:b0 + L * D].cpu().clone()
    ex.reset_graph()
    return lowered, losses, out


@pytest.mark.parametrize("B,D,L,unfused", [(512, 1024, 3, False), (256, 3072, 2, True)])
def test_tail_plan_bit_identical_to_the_plans_without_it(C, B, D, L, unfused):
    """StageG against StageE + StageC' (and, at D >= 3072 where the unfused
    dW GEMM runs on the same tiles, against StageC' alone, which the oracle
    pins step by step): three replays, every parameter, moment, shadow
    element, bias gradient and the step counter bit for bit; the loss, summed
    in another order, to 1e-6."""
    low_t, loss_t, out_t = _run_plan(B, D, L, 3, fuse_optimizer=True, fuse_colsum=True, fuse_tail=True)
    assert [it["op"] for it in low_t].count("mse_colsum") == 1
    refs = [dict(fuse_optimizer=True, fuse_colsum=True)] + ([dict(fuse_colsum=True)] if unfused else [])
    for kw in refs:
        low_r, loss_r, out_r = _run_plan(B, D, L, 3, **kw)
        assert "mse_colsum" not in [it["op"] for it in low_r]
        for a, b in zip(loss_t, loss_r):
            assert abs(a - b) <= 1e-6 * abs(b), (loss_t, loss_r)
        for k in out_t:
            assert torch.equal(out_t[k], out_r[k]), (kw, k)
    assert int(out_t["opt.step"].item()) == 3


def test_tail_plan_warmup_branch(C, monkeypatch):
    """AICF_WARMUP=1: mse_colsum leaves the step counter alone and the bias
    AdamW runs with lr 0 (as the weight updates do), so the parameters stay;
    unset, replays take real steps."""
    from aicf_hip import mlp

    B, D, L = 512, 512, 2
    ir, lowered, plan = mlp.build_mlp_mse(B, D, L, fuse_optimizer=True, fuse_colsum=True, fuse_tail=True)
    assert "mse_colsum" in [it["op"] for it in lowered]
    ex = mlp.make_executor(ir, lowered, plan)
    inputs, params = mlp.init_mlp_mse(B, D, L, seed=6)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    mlp.refresh_shadow(ex)
    P0 = ex.value("flat.params").cpu().clone()
    monkeypatch.setenv("AICF_WARMUP", "1")
    ex.run(inputs={}, params={}, reuse_static=True)
    torch.cuda.synchronize()
    assert torch.equal(ex.value("flat.params").cpu(), P0)
    assert int(ex.value("opt.step").item()) == 0
    monkeypatch.delenv("AICF_WARMUP")
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    ex.replay(2)
    torch.cuda.synchronize()
    assert int(ex.value("opt.step").item()) == 2
    assert not torch.equal(ex.value("flat.params").cpu(), P0)
    ex.reset_graph()
