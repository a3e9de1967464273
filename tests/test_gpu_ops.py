"""GPU parity of every op family against the CPU oracle.

Calls go through aicf_cuda._C (op_call / launch_by_id), which calls the
C-ABI of libaicf_hip.  Inputs are seeded numpy arrays; expected values come
from oracle/ (reference-exact fp32 restatements, or fp64 with the
tolerances of the north star: bit-exact for integer/index work and
order-free ops, rel-err <= 1e-5 for fp32 softmax/reduce/Adam, <= 1e-4 for
fp32 GEMM, <= 1e-2 for bf16 GEMM).  Shapes follow the reference probes
(python/cuda_binding_test/*.py) plus edge cases.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

import oracle as orc

pytestmark = pytest.mark.gpu

ADAM = int.from_bytes(b"ADAM", "little")
BCOR = int.from_bytes(b"BCOR", "little")
SGDS = int.from_bytes(b"SGDS", "little")
MSEG = int.from_bytes(b"MSEG", "little")
RSUM = int.from_bytes(b"RSUM", "big")
BADD = int.from_bytes(b"BADD", "little")
GEMM = int.from_bytes(b"GEMM", "big")
GPEL = int.from_bytes(b"GPEL", "big")
GEPI = int.from_bytes(b"GEPI", "little")
RRED = int.from_bytes(b"RRED", "little")
GADW = int.from_bytes(b"GADW", "little")


def g(a, dtype=None):
    """numpy -> cuda tensor (uint16 arrays are reinterpreted as `dtype`)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16)).view(dtype or torch.float16)
    else:
        t = torch.from_numpy(a)
    return t.cuda()


def h(t):
    """cuda tensor -> numpy (16-bit floats come back as raw uint16 bits)."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def rng(seed):
    return np.random.default_rng(seed)


def scalar(v, dtype=torch.float32):
    """0-d device tensor (np.ascontiguousarray would promote 0-d to 1-d)."""
    return torch.tensor(v, dtype=dtype, device="cuda")


def assert_bits_equal(got, ref, *inputs):
    """Bit-exact check that reports the first mismatching elements."""
    got = np.asarray(got).ravel()
    ref = np.asarray(ref).ravel()
    bad = np.nonzero(got != ref)[0]
    if bad.size:
        rows = [f"i={i} got={got[i]} ref={ref[i]} in={[np.asarray(a).ravel()[i] for a in inputs]}"
                for i in bad[:8]]
        raise AssertionError(f"{bad.size} mismatches\n" + "\n".join(rows))


# ============================================================== optimizer
@pytest.mark.parametrize("shape,inplace", [((1024,), False), ((64, 256), False),
                                           ((8, 32, 128), False), ((64, 256), True),
                                           ((1001,), False), ((3,), True)])
def test_adam_reference_contract_bit_exact(C, shape, inplace):
    # v2_adam_step_probe.py:41-92 shapes; bc = 1 - beta^3 (:53-54)
    r = rng(1)
    P, G, M = (r.standard_normal(shape).astype(np.float32) for _ in range(3))
    V = np.abs(r.standard_normal(shape)).astype(np.float32)
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-8
    bc1, bc2 = np.float32(1 - b1 ** 3), np.float32(1 - b2 ** 3)
    tP, tG, tM, tV = g(P), g(G), g(M), g(V)
    outs = [tP, tM, tV] if inplace else [torch.empty_like(tP) for _ in range(3)]
    C.op_call(int(C.OpKind.AdamStep),
              [tP, tG, tM, tV, scalar(float(bc1)), scalar(float(bc2))], outs, ADAM,
              struct.pack("<ffff", lr, b1, b2, eps), 0)
    Pr, Mr, Vr = orc.adam_ref(P, G, M, V, bc1, bc2, lr, b1, b2, eps)
    assert np.array_equal(h(outs[0]).ravel(), Pr)
    assert np.array_equal(h(outs[1]).ravel(), Mr)
    assert np.array_equal(h(outs[2]).ravel(), Vr)
    if not inplace:
        assert np.array_equal(h(tP), P)  # inputs untouched


@pytest.mark.parametrize("n,shadow", [(4096, False), (4099, True), (1 << 20, True)])
def test_adamw_in_kernel_bias_correction(C, n, shadow):
    r = rng(2)
    P = (0.02 * r.standard_normal(n)).astype(np.float32)
    G = (1e-3 * r.standard_normal(n)).astype(np.float32)
    M = np.zeros(n, np.float32)
    V = np.zeros(n, np.float32)
    tP, tG, tM, tV = g(P), g(G), g(M), g(V)
    step = torch.zeros((), dtype=torch.int32, device="cuda")
    outs = [tP, tM, tV] + ([torch.empty(n, dtype=torch.bfloat16, device="cuda")] if shadow else [])
    pay = struct.pack("<fffff", 1e-3, 0.9, 0.999, 1e-8, 0.01)
    Pc, Mc, Vc = P.copy(), M.copy(), V.copy()
    for t in range(1, 4):
        C.launch_by_id("step_inc_v0", C.OpKind.StepInc, [step], [step])
        C.launch_by_id("adamw_step_f32_v1", C.OpKind.AdamStep, [tP, tG, tM, tV, step], outs,
                       ADAM, pay)
        res = orc.adamw(Pc, G, Mc, Vc, t, 1e-3, 0.9, 0.999, 1e-8, 0.01, shadow=shadow)
        Pc, Mc, Vc = res[0], res[1], res[2]
    assert int(step.item()) == 3
    assert np.array_equal(h(tP), Pc)
    assert np.array_equal(h(tM), Mc)
    assert np.array_equal(h(tV), Vc)
    if shadow:
        assert np.array_equal(h(outs[3]), res[3])


@pytest.mark.parametrize("step", [1, 10, 0])
@pytest.mark.parametrize("rank1", [False, True])
def test_bias_corr(C, step, rank1):
    s = torch.tensor([step] if rank1 else step, dtype=torch.int32, device="cuda")
    shp = (1,) if rank1 else ()
    o1, o2 = torch.empty(shp, device="cuda"), torch.empty(shp, device="cuda")
    C.op_call(int(C.OpKind.BiasCorr), [s], [o1, o2], BCOR, struct.pack("<ff", 0.9, 0.999), 0)
    r1, r2 = orc.bias_corr(step, 0.9, 0.999)
    # device powf vs host powf: within 2 ulp
    assert abs(float(o1.item()) - r1) <= 2 * np.spacing(np.float32(r1))
    assert abs(float(o2.item()) - r2) <= 2 * np.spacing(np.float32(r2))


@pytest.mark.parametrize("shape", [(1,), (1024,), (64, 256), ()])
def test_step_inc(C, shape):
    s = torch.arange(int(np.prod(shape)) if shape else 1, dtype=torch.int32, device="cuda").reshape(shape)
    ref = s.clone()
    C.op_call(int(C.OpKind.StepInc), [s], [s], 0, b"", 0)
    assert torch.equal(s, ref + 1)
    # out-of-place increments the output buffer (step_inc/launcher.cu:140-141)
    o = torch.full_like(s, 7)
    C.op_call(int(C.OpKind.StepInc), [s], [o], 0, b"", 0)
    assert torch.equal(o, torch.full_like(s, 8))


def test_sgd(C):
    r = rng(3)
    for n in (1024, 1023):
        P = r.standard_normal(n).astype(np.float32)
        G = r.standard_normal(n).astype(np.float32)
        tP, tG = g(P), g(G)
        C.op_call(int(C.OpKind.SgdStep), [tP, tG], [tP], SGDS, struct.pack("<f", 0.01), 0)
        assert np.array_equal(h(tP), orc.sgd_f32(P, G, 0.01))
        Ph = P.astype(np.float16).view(np.uint16)
        Gh = G.astype(np.float16).view(np.uint16)
        tPh, tGh = g(Ph), g(Gh)
        C.op_call(int(C.OpKind.SgdStep), [tPh, tGh], [tPh], 0, b"", 0)  # default lr 1e-3
        assert_bits_equal(h(tPh), orc.sgd_f16(Ph, Gh, 1e-3), Ph, Gh)
    with pytest.raises(RuntimeError):
        C.op_call(int(C.OpKind.SgdStep), [tP, tG], [tG], 0, b"", 0)  # O aliases G


# ============================================================== elementwise
SHAPES = [(1024,), (64, 256), (8, 32, 128), (7, 33, 127)]


@pytest.mark.parametrize("shape", SHAPES)
def test_add_relu_relu_bwd_copy_zero(C, shape):
    r = rng(4)
    a = r.standard_normal(shape).astype(np.float32)
    b = r.standard_normal(shape).astype(np.float32)
    ta, tb = g(a), g(b)
    o = torch.empty_like(ta)
    C.op_call(int(C.OpKind.EltwiseAdd), [ta, tb], [o], 0, b"", 0)
    assert np.array_equal(h(o).ravel(), orc.add_f32(a, b))
    C.op_call(int(C.OpKind.EltwiseRelu), [ta], [o], 0, b"", 0)
    assert np.array_equal(h(o).ravel(), orc.relu_f32(a))
    C.op_call(int(C.OpKind.ReluBwd), [tb, ta], [o], 0, b"", 0)
    assert np.array_equal(h(o).ravel(), orc.relu_bwd_f32(b, a))
    C.op_call(int(C.OpKind.Copy), [ta], [o], 0, b"", 0)
    assert np.array_equal(h(o), a)
    C.op_call(int(C.OpKind.GradZero), [o], [o], 0, b"", 0)
    assert not h(o).any()
    ah = a.astype(np.float16).view(np.uint16)
    bh = b.astype(np.float16).view(np.uint16)
    tah, tbh = g(ah), g(bh)
    oh = torch.empty_like(tah)
    C.op_call(int(C.OpKind.EltwiseAdd), [tah, tbh], [oh], 0, b"", 0)
    assert np.array_equal(h(oh).ravel(), orc.add_f16(ah, bh))
    C.op_call(int(C.OpKind.EltwiseRelu), [tah], [oh], 0, b"", 0)
    assert np.array_equal(h(oh).ravel(), orc.relu_f16(ah))
    C.op_call(int(C.OpKind.ReluBwd), [tbh, tah], [oh], 0, b"", 0)
    assert np.array_equal(h(oh).ravel(), orc.relu_bwd_f16(bh, ah))
    C.op_call(int(C.OpKind.Copy), [tah], [oh], 0, b"", 0)
    assert np.array_equal(h(oh), ah)


def test_relu_special_values(C):
    x = np.array([1.5, -2.0, 0.0, -0.0, np.nan, np.inf, -np.inf, 1e-40], np.float32)
    tx = g(x)
    o = torch.empty_like(tx)
    C.op_call(int(C.OpKind.EltwiseRelu), [tx], [o], 0, b"", 0)
    assert np.array_equal(h(o).view(np.uint32), orc.relu_f32(x).view(np.uint32))


@pytest.mark.parametrize("shape", [(64, 256), (8, 32, 128), (7, 33, 127), (3, 5)])
def test_bias_add(C, shape):
    r = rng(5)
    y = r.standard_normal(shape).astype(np.float32)
    b = r.standard_normal(shape[-1]).astype(np.float32)
    ty = g(y)
    C.op_call(int(C.OpKind.BiasAdd), [ty, g(b)], [ty], BADD, struct.pack("<q", -1), 0)
    assert np.array_equal(h(ty).ravel(), orc.bias_add_f32(y, b))
    yh = y.astype(np.float16).view(np.uint16)
    bh = b.astype(np.float16).view(np.uint16)
    tyh = g(yh)
    C.op_call(int(C.OpKind.BiasAdd), [tyh, g(bh)], [tyh], 0, b"", 0)
    assert np.array_equal(h(tyh).ravel(), orc.bias_add_f16(yh, bh))


@pytest.mark.parametrize("shape", [(64, 256), (8, 32, 128), (7, 33, 127)])
def test_mse_grad(C, shape):
    r = rng(6)
    p = r.standard_normal(shape).astype(np.float32)
    t = r.standard_normal(shape).astype(np.float32)
    o = torch.empty(shape, device="cuda")
    C.op_call(int(C.OpKind.MseGrad), [g(p), g(t)], [o], 0, b"", 0)
    assert np.array_equal(h(o).ravel(), orc.mse_grad_f32(p, t))
    C.op_call(int(C.OpKind.MseGrad), [g(p), g(t)], [o], MSEG, struct.pack("<f", 0.125), 0)
    assert np.array_equal(h(o).ravel(), orc.mse_grad_f32(p, t, 0.125))
    ph = p.astype(np.float16).view(np.uint16)
    th = t.astype(np.float16).view(np.uint16)
    oh = torch.empty(shape, dtype=torch.float16, device="cuda")
    C.op_call(int(C.OpKind.MseGrad), [g(ph), g(th)], [oh], MSEG, struct.pack("<f", 0.125), 0)
    half = int(np.prod(shape)) % 2 == 0  # the f16 variant's half2 path (mse_grad/launcher.cu:272)
    assert np.array_equal(h(oh).ravel(), orc.mse_grad_f16(ph, th, 0.125, half_math=half))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape,nparts", [((64, 256), 1024), ((513, 1000), 1024), ((2048, 4096), 1024),
                                          ((2048, 4096), 4096), ((37, 123), 1024)])
def test_mse_loss_grad_fused(C, dtype, shape, nparts):
    """Pass 1 one-shot (a partial per 2048 elements fits the buffer, n a
    multiple of 8) or grid-stride (2048 x 4096 with 1024 partials; n = 4551)."""
    r = rng(7)
    p = r.standard_normal(shape).astype(np.float32)
    t = r.standard_normal(shape).astype(np.float32)
    if dtype == "bf16":
        pb = orc.bf16_bits_from_f32(p)
        tp = g(pb, torch.bfloat16)
        p = orc.bf16_bits_to_f32(pb).reshape(shape)
    else:
        tp = g(p)
    d = torch.empty_like(tp)
    loss = torch.empty((), device="cuda")
    part = torch.empty(nparts, device="cuda")
    C.launch_by_id("mse_loss_grad_v0", C.OpKind.MseGrad, [tp, g(t)], [d, loss, part])
    ref = orc.mse_grad_f32(p, t)
    if dtype == "bf16":
        assert np.array_equal(h(d).ravel(), orc.bf16_bits_from_f32(ref))
    else:
        assert np.array_equal(h(d).ravel(), ref)
    assert abs(loss.item() - orc.mse_loss_f64(p, t)) / orc.mse_loss_f64(p, t) < 1e-5


def test_gelu_and_gelu_bwd(C):
    r = rng(8)
    x = (3 * r.standard_normal(100003)).astype(np.float32)
    d = r.standard_normal(100003).astype(np.float32)
    o = torch.empty(100003, device="cuda")
    C.op_call(int(C.OpKind.EltwiseGelu), [g(x)], [o], 0, b"", 0)
    assert orc.rel_err(h(o), orc.gelu_f64(x.astype(np.float64))) < 1e-5
    C.op_call(int(C.OpKind.GeluBwd), [g(d), g(x)], [o], 0, b"", 0)
    assert orc.rel_err(h(o), d * orc.gelu_grad_f64(x.astype(np.float64))) < 1e-5
    xb = orc.bf16_bits_from_f32(x)
    ob = torch.empty(100003, dtype=torch.bfloat16, device="cuda")
    C.op_call(int(C.OpKind.EltwiseGelu), [g(xb, torch.bfloat16)], [ob], 0, b"", 0)
    ref = orc.gelu_f64(orc.bf16_bits_to_f32(xb).astype(np.float64))
    assert orc.rel_err(orc.bf16_bits_to_f32(h(ob)), ref) < 8e-3


# ============================================================== reductions
def test_reduce_sum_columns(C):
    # v2_reduce_sum_probe.py:24-75: f32 128x64 (seed 0), f16->f32 257x64 (seed 1)
    x = rng(0).standard_normal((128, 64)).astype(np.float32)
    o = torch.empty(64, device="cuda")
    C.op_call(int(C.OpKind.ReduceSum), [g(x)], [o], RSUM, struct.pack("<q", 0), 0)
    assert orc.rel_err(h(o), orc.colsum_f64(x)) < 1e-5
    xh = rng(1).standard_normal((257, 64)).astype(np.float16)
    o = torch.empty(64, device="cuda")
    C.op_call(int(C.OpKind.ReduceSum), [g(xh.view(np.uint16))], [o], 0, b"", 0)
    assert orc.rel_err(h(o), orc.colsum_f64(xh.astype(np.float32))) < 1e-5
    oh = torch.empty(64, dtype=torch.float16, device="cuda")
    C.op_call(int(C.OpKind.ReduceSum), [g(xh.view(np.uint16))], [oh], 0, b"", 0)
    assert orc.rel_err(orc.f16_bits_to_f64(h(oh)), orc.colsum_f64(xh.astype(np.float32))) < 1e-3
    # bf16 -> f32 with a partials buffer (two-pass, 8192 x 4096 like the MLP bias grads)
    xb = orc.bf16_bits_from_f32(rng(2).standard_normal((8192, 4096)).astype(np.float32))
    o = torch.empty(4096, device="cuda")
    part = torch.empty((64, 4096), device="cuda")
    C.launch_by_id("reduce_sum_keep_lastdim_bf16_to_f32_v0", C.OpKind.ReduceSum,
                   [g(xb, torch.bfloat16)], [o, part])
    ref = orc.colsum_f64(orc.bf16_bits_to_f32(xb).reshape(8192, 4096))
    assert orc.rel_err(h(o), ref) < 1e-5
    o1 = torch.empty(4096, device="cuda")
    C.launch_by_id("reduce_sum_keep_lastdim_bf16_to_f32_v0", C.OpKind.ReduceSum,
                   [g(xb, torch.bfloat16)], [o1])
    assert orc.rel_err(h(o1), ref) < 1e-5


@pytest.mark.parametrize("rows,cols", [(1, 8), (3, 96), (129, 4104), (1000, 256), (4097, 520), (8192, 96)])
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_reduce_sum_one_output_narrow_blocks(C, rows, cols, dt):
    """The reference's one-output column sum (no partials buffer) on narrow
    column blocks over all rows: single rows, column counts that are not a
    multiple of a block or of 8 blocks (no XCD remap), and long columns, vs
    the fp64 column sum of the same stored values."""
    x = rng(rows * 7 + cols).standard_normal((rows, cols)).astype(np.float32)
    if dt == "f32":
        t, ref = g(x), orc.colsum_f64(x)
        kid = "reduce_sum_keep_lastdim_f32_v0"
    elif dt == "bf16":
        xb = orc.bf16_bits_from_f32(x)
        t, ref = g(xb, torch.bfloat16), orc.colsum_f64(orc.bf16_bits_to_f32(xb).reshape(rows, cols))
        kid = "reduce_sum_keep_lastdim_bf16_to_f32_v0"
    else:
        xh = x.astype(np.float16)
        t, ref = g(xh.view(np.uint16)), orc.colsum_f64(xh.astype(np.float32))
        kid = "reduce_sum_keep_lastdim_f16_to_f32_v0"
    o = torch.full((cols,), float("nan"), device="cuda")
    C.launch_by_id(kid, C.OpKind.ReduceSum, [t], [o])
    assert orc.rel_err(h(o), ref) < 1e-5


@pytest.mark.parametrize("cols,rows", [(128, 64), (1024, 64), (8192, 64), (32768, 16), (1000, 64), (64, 64),
                                       (2048, 64), (4096, 64), (256, 37), (128, 37), (1024, 37), (512, 5),
                                       (16384, 3)])
def test_row_softmax_and_stats(C, cols, rows):
    """Register-resident shapes (one row per lane group, wave or workgroup,
    including partial workgroups: 37 rows at 16 rows per workgroup) and the
    looping kernel (C = 1000)."""
    x = (2.0 * rng(cols).standard_normal((rows, cols))).astype(np.float32)  # N(0, 4)
    x[-1, :] = -1e4
    y = torch.empty((rows, cols), device="cuda")
    mx = torch.empty(rows, device="cuda")
    sx = torch.empty(rows, device="cuda")
    C.op_call(int(C.OpKind.RowSoftmax), [g(x)], [y, mx, sx], 0, b"", 0)
    ry, rmx, rsx = orc.softmax_rows_f64(x)
    yy = h(y)
    assert orc.rel_err(yy, ry) < 1e-5
    assert np.array_equal(h(mx), rmx.astype(np.float32))  # max is order-free: bit-exact
    assert orc.rel_err(h(sx)[:-1], rsx[:-1]) < 1e-5
    assert orc.rel_err(h(sx), rsx) < 1e-5
    assert np.all(yy[-1] == np.float32(1.0 / cols))  # stable row: exactly 1/C
    # RowReduce sum / max
    o = torch.empty(rows, device="cuda")
    C.op_call(int(C.OpKind.RowReduce), [g(x)], [o], RRED, struct.pack("<i", 1), 0)
    assert np.array_equal(h(o), rmx.astype(np.float32))
    C.op_call(int(C.OpKind.RowReduce), [g(x)], [o], RRED, struct.pack("<i", 0), 0)
    assert orc.rel_err(h(o), rsx) < 1e-5
    # softmax only
    C.op_call(int(C.OpKind.RowSoftmax), [g(x)], [y], 0, b"", 0)
    assert orc.rel_err(h(y), ry) < 1e-5


@pytest.mark.parametrize("B,Ccls", [(64, 10), (64, 1024), (37, 1000), (256, 128), (37, 128), (9, 8192),
                                    (5, 32768)])
def test_softmax_xent(C, B, Ccls):
    r = rng(B * Ccls)
    z = (3 * r.standard_normal((B, Ccls))).astype(np.float32)
    z[1, 3] = z[1, 5] = z[1].max() + 2.0  # tie -> first index
    if Ccls >= 512:  # tie between columns held by different waves of the row
        z[2, 300] = z[2, 7] = z[2].max() + 3.0
    lab = r.integers(0, Ccls, B).astype(np.int32)
    loss = torch.empty((), device="cuda")
    dz = torch.empty((B, Ccls), device="cuda")
    am = torch.empty(B, dtype=torch.int32, device="cuda")
    rl = torch.empty(B, device="cuda")
    C.op_call(int(C.OpKind.SoftmaxXent), [g(z), g(lab)], [loss, dz, am, rl], 0, b"", 0)
    rloss, rdz, ram, rrl = orc.softmax_xent_f64(z, lab)
    assert np.array_equal(h(am), ram)
    assert h(am)[1] == 3
    if Ccls >= 512:
        assert h(am)[2] == 7
    assert abs(loss.item() - rloss) / abs(rloss) < 1e-5
    assert orc.rel_err(h(dz), rdz) < 1e-5
    assert orc.rel_err(h(rl), rrl) < 1e-5


@pytest.mark.parametrize("Ccls", [128, 1024, 1000])  # register-resident rows, and the looping kernel
def test_softmax_xent_row_loss_of_extreme_rows(C, Ccls):
    """Rows of equal values far from zero (+-1e4) have row loss log(C) for any
    label, and rows offset by 1e4 have the loss of the unshifted row: each
    row's loss against the fp64 oracle row by row (not normwise), so a
    cancellation after rounding log(S) shows up."""
    B = 8
    r = rng(Ccls + 7)
    z = r.standard_normal((B, Ccls)).astype(np.float32)
    z[0], z[1] = -1e4, 1e4
    z[2:5] += np.float32(1e4)
    z[5:] -= np.float32(1e4)
    lab = r.integers(0, Ccls, B).astype(np.int32)
    loss = torch.empty((), device="cuda")
    dz = torch.empty((B, Ccls), device="cuda")
    am = torch.empty(B, dtype=torch.int32, device="cuda")
    rl = torch.empty(B, device="cuda")
    C.op_call(int(C.OpKind.SoftmaxXent), [g(z), g(lab)], [loss, dz, am, rl], 0, b"", 0)
    _, _, _, rrl = orc.softmax_xent_f64(z, lab)
    got = h(rl).astype(np.float64)
    assert np.abs(got[:2] - np.log(Ccls)).max() <= 2e-6 * np.log(Ccls)
    assert (np.abs(got - rrl) / np.abs(rrl)).max() < 1e-5


# ============================================================== GEMM
def _gemm_ref(A, B, ta, tb):
    return orc.gemm_f64(A, B, ta, tb)


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_f32_probe_shapes(C, ta, tb):
    # v2_gemm_probe.py:92-119: M,K,N = 64,48,80, all trans combos
    r = rng(10)
    M, K, N = 64, 48, 80
    A = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    o = torch.empty((M, N), device="cuda")
    C.op_call(int(C.OpKind.Gemm), [g(A), g(B)], [o], 0, struct.pack("<ii", ta, tb), 0)
    assert orc.rel_err(h(o), _gemm_ref(A, B, ta, tb)) < 1e-4
    C.launch_by_id("gemm_f32_naive_v0", C.OpKind.Gemm, [g(A), g(B)], [o], GEMM,
                   struct.pack("<ii", ta, tb))
    assert orc.rel_err(h(o), _gemm_ref(A, B, ta, tb)) < 1e-4


def test_gemm_f32_strided_views(C):
    r = rng(11)
    A = r.standard_normal((96, 70)).astype(np.float32)
    B = r.standard_normal((90, 50)).astype(np.float32)
    tA, tB = g(A), g(B)
    a_view = tA[:64:1, 3:51]     # [64, 48], row stride 70
    b_view = tB[5:53, 10:40:1]   # [48, 30], row stride 50
    o_full = torch.zeros((64, 61), device="cuda")
    o = o_full[:, 1:31]          # non-contiguous output
    C.op_call(int(C.OpKind.Gemm), [a_view, b_view], [o], 0, b"", 0)
    ref = A[:64, 3:51].astype(np.float64) @ B[5:53, 10:40].astype(np.float64)
    assert orc.rel_err(h(o), ref) < 1e-4
    assert not h(o_full)[:, 0].any() and not h(o_full)[:, 31:].any()
    # column-strided (gather) operand: every other column
    a2 = tA[:, ::2][:64, :32]
    o2 = torch.empty((64, 30), device="cuda")
    C.op_call(int(C.OpKind.Gemm), [a2, tB[:32, :30]], [o2], 0, b"", 0)
    ref2 = A[:64, ::2][:, :32].astype(np.float64) @ B[:32, :30].astype(np.float64)
    assert orc.rel_err(h(o2), ref2) < 1e-4


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_f16_probe_shapes(C, ta, tb):
    r = rng(12)
    M = K = N = 64
    A = r.standard_normal((M, K)).astype(np.float16)
    B = r.standard_normal((K, N)).astype(np.float16)
    o = torch.empty((M, N), dtype=torch.float16, device="cuda")
    C.op_call(int(C.OpKind.Gemm), [g(A.view(np.uint16)), g(B.view(np.uint16))], [o], 0,
              struct.pack("<ii", ta, tb), 0)
    ref = _gemm_ref(A.astype(np.float32), B.astype(np.float32), ta, tb)
    assert orc.rel_err(orc.f16_bits_to_f64(h(o)), ref) < 2e-3


@pytest.mark.parametrize("M,N,K,ta,tb", [
    (4096, 4096, 128, False, True),   # 256x256 tiles
    (2048, 1024, 128, False, True),   # 128x128 tiles
    (1024, 1024, 1024, False, True),  # 64x64 tiles, 8 LDS stages (16 K-steps: no tail loop)
    (1024, 512, 1088, False, True),   # 64x64, 8 stages, 17 K-steps: the tail loop's waits
    (1024, 1024, 4096, False, True),  # 64x64, 8 stages, 64 K-steps
    (2048, 2048, 2048, False, True),  # 128x128 tiles, 4 stages
    (2048, 2048, 1088, False, True),  # 128x128, 4 stages, 17 K-steps
    (100, 72, 784, False, True),
    (64, 256, 784, False, True),
    (256, 4096, 256, False, True),
    (512, 384, 640, False, False),
    (384, 512, 1024, True, False),
    (200, 136, 96, True, True),
])
def test_gemm_bf16(C, M, N, K, ta, tb):
    r = rng(M + N + K)
    s = 1.0 / np.sqrt(K)
    A = r.uniform(-s, s, (K, M) if ta else (M, K)).astype(np.float32)
    B = r.uniform(-s, s, (N, K) if tb else (K, N)).astype(np.float32)
    Ab, Bb = orc.bf16_bits_from_f32(A), orc.bf16_bits_from_f32(B)
    ref = _gemm_ref(orc.bf16_bits_to_f32(Ab).reshape(A.shape), orc.bf16_bits_to_f32(Bb).reshape(B.shape), ta, tb)
    o = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    C.op_call(int(C.OpKind.Gemm), [g(Ab, torch.bfloat16), g(Bb, torch.bfloat16)], [o], 0,
              struct.pack("<ii", ta, tb), 0)
    assert orc.rel_err(orc.bf16_bits_to_f32(h(o)), ref) < 1e-2
    of = torch.empty((M, N), device="cuda")
    C.launch_by_id("gemm_bf16_mfma_f32out_v0", C.OpKind.Gemm,
                   [g(Ab, torch.bfloat16), g(Bb, torch.bfloat16)], [of], 0, struct.pack("<ii", ta, tb))
    assert orc.rel_err(h(of), ref) < 1e-5  # fp32 out: only accumulation-order error


@pytest.mark.parametrize("K", [64, 192, 576, 640])
@pytest.mark.parametrize("ta,tb", [(False, True), (False, False), (True, True), (True, False)])
def test_gemm_bf16_256_tiles_all_operand_layouts(C, ta, tb, K):
    """256x256-tile path with each operand K-contiguous or MN-contiguous
    (the latter read through the transposing LDS loads).  Both operands
    K-contiguous with K <= 512 and a one-output epilogue take the 128x128
    tiles instead; K = 576 and 640 (odd and even K-step counts) keep that
    layout on the 256x256 tiles."""
    M = N = 4096
    r = rng(K + 2 * ta + tb)
    s = 1.0 / np.sqrt(K)
    A = r.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = r.uniform(-s, s, (N, K) if tb else (K, N)).astype(np.float32)
    Ab, Bb = orc.bf16_bits_from_f32(A), orc.bf16_bits_from_f32(B)
    ref = _gemm_ref(orc.bf16_bits_to_f32(Ab).reshape(A.shape), orc.bf16_bits_to_f32(Bb).reshape(B.shape), ta, tb)
    of = torch.empty((M, N), device="cuda")
    C.launch_by_id("gemm_bf16_mfma_f32out_v0", C.OpKind.Gemm,
                   [g(Ab, torch.bfloat16), g(Bb, torch.bfloat16)], [of], 0, struct.pack("<ii", ta, tb))
    assert orc.rel_err(h(of), ref) < 1e-5
    o = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    C.op_call(int(C.OpKind.Gemm), [g(Ab, torch.bfloat16), g(Bb, torch.bfloat16)], [o], 0,
              struct.pack("<ii", ta, tb), 0)
    assert orc.rel_err(orc.bf16_bits_to_f32(h(o)), ref) < 1e-2


def test_gemm_bf16_dgelu_with_mn_contiguous_weight_256_tiles(C):
    """dX = (dY . W) * gelu'(Z) with W stored [out, in] (MN-contiguous B), on
    the 256x256-tile path: the backward GEMM of a Linear layer without a
    transposed copy of W."""
    M, N, K = 8192, 1024, 128  # dY [M, K], W [K, N] row-major, Z [M, N]
    r = rng(77)
    dY = orc.bf16_bits_from_f32(r.standard_normal((M, K)).astype(np.float32))
    W = orc.bf16_bits_from_f32(r.uniform(-0.1, 0.1, (K, N)).astype(np.float32))
    Z = orc.bf16_bits_from_f32(r.standard_normal((M, N)).astype(np.float32))
    dz = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    C.launch_by_id("gemm_epilogue_bf16_mfma_v0", C.OpKind.GemmEpilogue,
                   [g(dY, torch.bfloat16), g(W, torch.bfloat16), g(Z, torch.bfloat16)], [dz], GEPI,
                   struct.pack("<iii", 0, 0, 5))
    ref = _gemm_ref(orc.bf16_bits_to_f32(dY).reshape(M, K), orc.bf16_bits_to_f32(W).reshape(K, N),
                    False, False) * orc.gelu_grad_f64(orc.bf16_bits_to_f32(Z).reshape(M, N).astype(np.float64))
    assert orc.rel_err(orc.bf16_bits_to_f32(h(dz)).reshape(M, N), ref) < 1e-2


@pytest.mark.parametrize("ta,tb,K", [(0, 1, 128), (1, 0, 128), (0, 0, 128), (1, 1, 128), (0, 1, 192),
                                     (0, 0, 192), (0, 1, 576), (0, 1, 640)])
def test_gemm_bf16_persistent_tiles(C, ta, tb, K):
    """More 256x256 tiles (17 x 16 = 272) than CUs: one persistent workgroup
    per CU loops over its tiles, 16 of them take a second tile.  All operand
    layouts (fp32 output at 1e-5), bias+GELU with the pre-activation, and
    dGELU epilogues.  K = 128 and 192 (2 and 3 K-steps) put the pre-activation
    rows loaded during the last K-step in either stage buffer; with both
    operands K-contiguous the fp32-output GEMM takes the 128x128 tiles up to
    K = 512, so that layout also runs at K = 576 and 640 (9 and 10 K-steps)."""
    M, N = 17 * 256, 16 * 256
    r = rng(300 + 2 * ta + tb)
    s = 1.0 / np.sqrt(K)
    A = r.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = r.uniform(-s, s, (N, K) if tb else (K, N)).astype(np.float32)
    Ab, Bb = orc.bf16_bits_from_f32(A), orc.bf16_bits_from_f32(B)
    Af, Bf = orc.bf16_bits_to_f32(Ab).reshape(A.shape), orc.bf16_bits_to_f32(Bb).reshape(B.shape)
    ref = _gemm_ref(Af, Bf, ta, tb)
    ga, gb = g(Ab, torch.bfloat16), g(Bb, torch.bfloat16)
    of = torch.empty((M, N), device="cuda")
    C.launch_by_id("gemm_bf16_mfma_f32out_v0", C.OpKind.Gemm, [ga, gb], [of], 0, struct.pack("<ii", ta, tb))
    assert orc.rel_err(h(of), ref) < 1e-5
    bias = r.uniform(-s, s, N).astype(np.float32)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    z = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    C.launch_by_id("gemm_epilogue_bf16_mfma_v0", C.OpKind.GemmEpilogue, [ga, gb, g(bias)], [y, z], GEPI,
                   struct.pack("<iii", ta, tb, 3))
    z_ref = ref + bias[None, :]
    assert orc.rel_err(orc.bf16_bits_to_f32(h(z)).reshape(M, N), z_ref) < 1e-2
    assert orc.rel_err(orc.bf16_bits_to_f32(h(y)).reshape(M, N), orc.gelu_f64(z_ref)) < 1e-2
    Zb = orc.bf16_bits_from_f32(r.standard_normal((M, N)).astype(np.float32))
    dz = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    C.launch_by_id("gemm_epilogue_bf16_mfma_v0", C.OpKind.GemmEpilogue, [ga, gb, g(Zb, torch.bfloat16)], [dz],
                   GEPI, struct.pack("<iii", ta, tb, 5))
    d_ref = ref * orc.gelu_grad_f64(orc.bf16_bits_to_f32(Zb).reshape(M, N).astype(np.float64))
    assert orc.rel_err(orc.bf16_bits_to_f32(h(dz)).reshape(M, N), d_ref) < 1e-2


@pytest.mark.parametrize("M,N,K", [(256, 256, 96), (512, 384, 160), (2048, 1024, 96), (4096, 4096, 64)])
def test_gemm_f32_tiled_paths(C, M, N, K):
    """fp32 X[M,K] . W[N,K]^T on the tiled MFMA paths (64x64, 128x128 and
    256x256 tiles, 32x32x2 fp32 MFMA), plain and with the bias+GELU /
    bias+ReLU epilogues, vs the fp64 oracle."""
    r = rng(M + N + K)
    X = r.uniform(-1, 1, (M, K)).astype(np.float32)
    W = (r.uniform(-1, 1, (N, K)) / np.sqrt(K)).astype(np.float32)
    b = r.uniform(-1, 1, N).astype(np.float32)
    ref = _gemm_ref(X, W, False, True)
    o = torch.empty((M, N), device="cuda")
    C.op_call(int(C.OpKind.Gemm), [g(X), g(W)], [o], 0, struct.pack("<ii", 0, 1), 0)
    assert orc.rel_err(h(o), ref) < 1e-4
    C.op_call(int(C.OpKind.GemmEpilogue), [g(X), g(W), g(b)], [o], GEPI, struct.pack("<iii", 0, 1, 3), 0)
    assert orc.rel_err(h(o), orc.gelu_f64(ref + b[None, :])) < 1e-4
    C.op_call(int(C.OpKind.GemmEpilogue), [g(X), g(W), g(b)], [o], GPEL, struct.pack("<iii", 0, 1, 1), 0)
    want = np.maximum(ref + b[None, :], 0)
    assert orc.rel_err(h(o), want) < 1e-4
    assert np.all(h(o)[want == 0] == 0)


@pytest.mark.parametrize("K", [32, 96, 288])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (True, True), (False, True)])
def test_gemm_f32_256_tiles_all_operand_layouts(C, ta, tb, K):
    """fp32 on the 256x256 tiles with each operand K-contiguous or
    M/N-contiguous (one 4-byte LDS read per K-row), including the reference's
    default layout (no transposes: A [M, K], B [K, N]); plain and with the
    bias+GELU epilogue, vs the fp64 oracle.  K = 32 is one K-step; 96 and
    288 odd counts."""
    M, N = 2048, 4096  # 128 tiles of 256 x 256
    r = rng(K + 2 * ta + tb + 1000)
    A = r.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = (r.uniform(-1, 1, (N, K) if tb else (K, N)) / np.sqrt(K)).astype(np.float32)
    bias = r.uniform(-1, 1, N).astype(np.float32)
    ref = _gemm_ref(A, B, ta, tb)
    o = torch.empty((M, N), device="cuda")
    C.op_call(int(C.OpKind.Gemm), [g(A), g(B)], [o], 0, struct.pack("<ii", ta, tb), 0)
    assert orc.rel_err(h(o), ref) < 1e-4
    C.op_call(int(C.OpKind.GemmEpilogue), [g(A), g(B), g(bias)], [o], GEPI, struct.pack("<iii", ta, tb, 3), 0)
    assert orc.rel_err(h(o), orc.gelu_f64(ref + bias[None, :])) < 1e-4


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("M,N,K", [(1024, 1024, 1024), (2048, 2048, 256), (1024, 512, 2048), (512, 256, 64)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (True, True)])
def test_gemm_small_tiles_mn_contiguous_operands(C, ta, tb, M, N, K, dt):
    """Problems with fewer than 128 tiles of 256 x 256 in the layouts with an
    M/N-contiguous operand: 128 x 128 tiles (4 LDS stages for 16-bit with
    >= 16 K-steps), and 64 x 64 tiles for fp32 (1024^3, 512 x 256), plain
    and with bias+ReLU, vs the fp64 oracle."""
    r = rng(M + N + K + 4 * ta + 2 * tb + (dt == "bf16"))
    A = r.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = (r.uniform(-1, 1, (N, K) if tb else (K, N)) / np.sqrt(K)).astype(np.float32)
    bias = r.uniform(-1, 1, N).astype(np.float32)
    if dt == "bf16":
        Ab, Bb = orc.bf16_bits_from_f32(A), orc.bf16_bits_from_f32(B)
        A = orc.bf16_bits_to_f32(Ab).reshape(A.shape)
        B = orc.bf16_bits_to_f32(Bb).reshape(B.shape)
        ta_, tb_ = g(Ab, torch.bfloat16), g(Bb, torch.bfloat16)
        o = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        back, tol = (lambda t: orc.bf16_bits_to_f32(h(t)).reshape(M, N)), 1e-2
    else:
        ta_, tb_ = g(A), g(B)
        o = torch.empty((M, N), device="cuda")
        back, tol = h, 1e-4
    ref = _gemm_ref(A, B, ta, tb)
    C.op_call(int(C.OpKind.Gemm), [ta_, tb_], [o], 0, struct.pack("<ii", ta, tb), 0)
    assert orc.rel_err(back(o), ref) < tol
    C.op_call(int(C.OpKind.GemmEpilogue), [ta_, tb_, g(bias)], [o], GEPI, struct.pack("<iii", ta, tb, 0), 0)
    assert orc.rel_err(back(o), np.maximum(ref + bias[None, :], 0)) < tol


@pytest.mark.parametrize("relu", [1, 0])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, True)])
def test_gemm_epilogue_f32_gpel(C, relu, ta, tb):
    # v2_gemm_epilogue_probe.py:108-158: f32 64,48,80 x trans x relu
    r = rng(13)
    M, K, N = 64, 48, 80
    A = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    bias = r.standard_normal(N).astype(np.float32)
    o = torch.empty((M, N), device="cuda")
    C.op_call(int(C.OpKind.GemmEpilogue), [g(A), g(B), g(bias)], [o], GPEL,
              struct.pack("<iii", ta, tb, relu), 0)
    ref = _gemm_ref(A, B, ta, tb) + bias[None, :]
    if relu:
        ref = np.maximum(ref, 0)
    assert orc.rel_err(h(o), ref) < 1e-4
    if relu:
        assert np.all(h(o)[ref < -1e-3] == 0)


def test_gemm_epilogue_default_is_bias_relu_and_gepi_kinds(C):
    r = rng(14)
    M, K, N = 64, 64, 64
    A = r.standard_normal((M, K)).astype(np.float32)
    B = r.standard_normal((K, N)).astype(np.float32)
    bias = r.standard_normal(N).astype(np.float32)
    base = _gemm_ref(A, B, False, False)
    o = torch.empty((M, N), device="cuda")
    C.op_call(int(C.OpKind.GemmEpilogue), [g(A), g(B), g(bias)], [o], 0, b"", 0)
    assert orc.rel_err(h(o), np.maximum(base + bias, 0)) < 1e-4
    for kind, fn in [(0, lambda x: np.maximum(x + bias, 0)), (1, lambda x: x + bias),
                     (2, lambda x: np.maximum(x, 0)),
                     (3, lambda x: orc.gelu_f64(x + bias)), (4, lambda x: orc.gelu_f64(x))]:
        C.op_call(int(C.OpKind.GemmEpilogue), [g(A), g(B), g(bias)], [o], GEPI,
                  struct.pack("<iii", 0, 0, kind), 0)
        assert orc.rel_err(h(o), fn(base)) < 1e-4, kind


@pytest.mark.parametrize("M,N,K", [(256, 512, 384), (1024, 1024, 1024), (100, 200, 64),
                                   (4096, 4096, 64), (2048, 2048, 1024)])
def test_gemm_epilogue_bf16_gelu_aux_and_dgelu(C, M, N, K):
    """bias+GELU with the pre-activation (1024^3: 64x64 tiles, 8 LDS stages;
    2048 x 2048 x 1024: 128x128 tiles, 4 stages) and the dGELU epilogue."""
    r = rng(15)
    s = 1.0 / np.sqrt(K)
    X = orc.bf16_bits_from_f32(r.uniform(-1, 1, (M, K)).astype(np.float32))
    W = orc.bf16_bits_from_f32(r.uniform(-s, s, (N, K)).astype(np.float32))
    bias = r.uniform(-s, s, N).astype(np.float32)
    Xf = orc.bf16_bits_to_f32(X).reshape(M, K)
    Wf = orc.bf16_bits_to_f32(W).reshape(N, K)
    z_ref = _gemm_ref(Xf, Wf, False, True) + bias[None, :]
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    z = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    C.launch_by_id("gemm_epilogue_bf16_mfma_v0", C.OpKind.GemmEpilogue,
                   [g(X, torch.bfloat16), g(W, torch.bfloat16), g(bias)], [y, z], GEPI,
                   struct.pack("<iii", 0, 1, 3))
    zz = orc.bf16_bits_to_f32(h(z)).reshape(M, N)
    assert orc.rel_err(zz, z_ref) < 1e-2
    assert orc.rel_err(orc.bf16_bits_to_f32(h(y)).reshape(M, N), orc.gelu_f64(z_ref)) < 1e-2
    # dgelu epilogue: dZ = (dY . W) * gelu'(Z), dY [M,N] . W [N,K] -> [M,K]
    dY = orc.bf16_bits_from_f32(r.standard_normal((M, N)).astype(np.float32))
    Zk = orc.bf16_bits_from_f32(r.standard_normal((M, K)).astype(np.float32))
    dz = torch.empty((M, K), dtype=torch.bfloat16, device="cuda")
    C.launch_by_id("gemm_epilogue_bf16_mfma_v0", C.OpKind.GemmEpilogue,
                   [g(dY, torch.bfloat16), g(W, torch.bfloat16), g(Zk, torch.bfloat16)], [dz], GEPI,
                   struct.pack("<iii", 0, 0, 5))
    ref = _gemm_ref(orc.bf16_bits_to_f32(dY).reshape(M, N), Wf, False, False) * \
        orc.gelu_grad_f64(orc.bf16_bits_to_f32(Zk).reshape(M, K).astype(np.float64))
    assert orc.rel_err(orc.bf16_bits_to_f32(h(dz)).reshape(M, K), ref) < 1e-2


@pytest.mark.parametrize("M,N,K,ta,tb", [(512, 768, 128, 0, 0), (4096, 4096, 64, 0, 1),
                                         (17 * 256, 16 * 256, 128, 0, 0), (1024, 512, 320, 1, 0)])
def test_gemm_dgelu_with_column_sums(C, M, N, K, ta, tb):
    """GEPI kind 6: the dGELU GEMM that also column-sums its stored output
    (one partial per 256-row tile, then a fixed-order finish).  The output is
    the same bits as kind 5; db against the fp64 column sum of that stored
    bf16 output; the workspace may have more rows than M/256."""
    r = rng(M + N + K)
    A = orc.bf16_bits_from_f32(r.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
    B = orc.bf16_bits_from_f32(r.uniform(-0.1, 0.1, (N, K) if tb else (K, N)).astype(np.float32))
    Z = orc.bf16_bits_from_f32(r.standard_normal((M, N)).astype(np.float32))
    ga, gb, gz = g(A, torch.bfloat16), g(B, torch.bfloat16), g(Z, torch.bfloat16)
    d5 = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    C.launch_by_id("gemm_epilogue_bf16_mfma_v0", C.OpKind.GemmEpilogue, [ga, gb, gz], [d5], GEPI,
                   struct.pack("<iii", ta, tb, 5))
    d6 = torch.empty_like(d5)
    db = torch.empty(N, device="cuda")
    ws = torch.full((M // 256 + 3, N), float("nan"), device="cuda")
    C.launch_by_id("gemm_epilogue_bf16_mfma_v0", C.OpKind.GemmEpilogue, [ga, gb, gz], [d6, db, ws], GEPI,
                   struct.pack("<iii", ta, tb, 6))
    assert torch.equal(d5, d6)
    ref = orc.bf16_bits_to_f32(h(d6)).reshape(M, N).astype(np.float64).sum(axis=0)
    assert orc.rel_err(h(db), ref) < 1e-5
    assert np.isnan(h(ws)[M // 256:]).all()  # rows past M/256 untouched


def test_gemm_dgelu_column_sums_rejects(C):
    """Kind 6 needs the bf16 256 x 256 path and a [>= M/256, N] fp32 workspace."""
    def call(M, N, K, P):
        A = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda")
        B = torch.zeros((K, N), dtype=torch.bfloat16, device="cuda")
        Z = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
        C.launch_by_id("gemm_epilogue_bf16_mfma_v0", C.OpKind.GemmEpilogue, [A, B, Z],
                       [torch.empty((M, N), dtype=torch.bfloat16, device="cuda"), torch.empty(N, device="cuda"),
                        torch.empty((P, N), device="cuda")], GEPI, struct.pack("<iii", 0, 0, 6))
    with pytest.raises(RuntimeError):
        call(512, 256, 64, 1)      # workspace rows < M/256
    with pytest.raises(RuntimeError):
        call(384, 256, 64, 2)      # M not a multiple of 256
    with pytest.raises(RuntimeError):
        call(512, 256, 96, 2)      # K not a multiple of 64
    call(512, 256, 64, 2)
    torch.cuda.synchronize()


def test_gemm_neg_cases_raise(C):
    A = torch.zeros((64, 48), device="cuda")
    B = torch.zeros((48, 80), device="cuda")
    with pytest.raises(RuntimeError, match="status=NotImplemented"):
        C.op_call(int(C.OpKind.Gemm), [A, B], [torch.empty((64, 81), device="cuda")], 0, b"", 0)
    with pytest.raises(RuntimeError, match="kernel_id=gemm_f32_naive_v0"):
        C.launch_by_id("gemm_f32_naive_v0", C.OpKind.Gemm, [A, B],
                       [torch.empty((64, 81), device="cuda")])
    with pytest.raises(RuntimeError):
        C.op_call(int(C.OpKind.Gemm), [A.cpu(), B], [torch.empty((64, 80), device="cuda")])


# (M, N, K, transA, transB): both operand layouts per side; 4096 x 2048 is the
# smallest shape on which the plain fp32-output GEMM also takes 256 x 256
# tiles; 17 x 16 tiles exceed the CU count (persistent workgroups).
GADW_CASES = [(4096, 4096, 64, 1, 0), (4096, 4096, 192, 0, 1), (4096, 2048, 128, 0, 0),
              (4096, 2048, 128, 1, 1), (17 * 256, 16 * 256, 128, 1, 0)]


@pytest.mark.parametrize("M,N,K,ta,tb", GADW_CASES)
def test_gemm_adamw_matches_gemm_then_adamw_bit_exact(C, M, N, K, ta, tb):
    """gemm_adamw (weight-gradient GEMM with AdamW in its epilogue) against
    the fp32-output GEMM followed by the streaming AdamW with bf16 shadow,
    over two steps with different gradients and weight decay: parameters,
    both moments and the shadow bit for bit.  The unfused gradient run
    through the oracle's AdamW gives the same bits."""
    r = rng(M + N + K + 2 * ta + tb)
    s = 1.0 / np.sqrt(K)
    As = [orc.bf16_bits_from_f32(r.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)) for _ in range(2)]
    Bs = [orc.bf16_bits_from_f32(r.uniform(-s, s, (N, K) if tb else (K, N)).astype(np.float32)) for _ in range(2)]
    P0 = (0.02 * r.standard_normal((M, N))).astype(np.float32)
    Pf, Mf, Vf = g(P0), torch.zeros((M, N), device="cuda"), torch.zeros((M, N), device="cuda")
    Pu, Mu, Vu = g(P0), torch.zeros((M, N), device="cuda"), torch.zeros((M, N), device="cuda")
    Wf = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    Wu = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    G = torch.empty((M, N), device="cuda")
    sf = torch.zeros((), dtype=torch.int32, device="cuda")
    su = torch.zeros((), dtype=torch.int32, device="cuda")
    hp = (1e-3, 0.9, 0.999, 1e-8, 0.01)
    Pc, Mc, Vc = P0.ravel().copy(), np.zeros(M * N, np.float32), np.zeros(M * N, np.float32)
    for t in range(1, 3):
        ga, gb = g(As[t - 1], torch.bfloat16), g(Bs[t - 1], torch.bfloat16)
        C.launch_by_id("step_inc_v0", C.OpKind.StepInc, [sf], [sf])
        C.launch_by_id("gemm_adamw_bf16_v0", C.OpKind.GemmAdamW, [ga, gb, Pf, Mf, Vf, sf], [Pf, Mf, Vf, Wf],
                       GADW, struct.pack("<iifffff", ta, tb, *hp))
        C.launch_by_id("step_inc_v0", C.OpKind.StepInc, [su], [su])
        C.launch_by_id("gemm_bf16_mfma_f32out_v0", C.OpKind.Gemm, [ga, gb], [G], 0, struct.pack("<ii", ta, tb))
        C.launch_by_id("adamw_step_f32_v1", C.OpKind.AdamStep, [Pu, G, Mu, Vu, su], [Pu, Mu, Vu, Wu], ADAM,
                       struct.pack("<fffff", *hp))
        Pc, Mc, Vc, Wc = orc.adamw(Pc, h(G).ravel(), Mc, Vc, t, *hp, shadow=True)
        assert_bits_equal(h(Pf), h(Pu))
        assert_bits_equal(h(Mf), h(Mu))
        assert_bits_equal(h(Vf), h(Vu))
        assert_bits_equal(h(Wf), h(Wu))
        assert_bits_equal(h(Pf), Pc)
        assert_bits_equal(h(Wf), Wc)
    assert int(sf.item()) == 2


def test_gemm_adamw_rejects_what_it_does_not_cover(C):
    """Shapes off the 256 x 256 tiles, P/M/V outputs not aliasing the inputs,
    and a NaN hyper-parameter are rejected on the host."""
    def args(M, N, K):
        A = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda")
        B = torch.zeros((K, N), dtype=torch.bfloat16, device="cuda")
        P, Mm, V = (torch.zeros((M, N), device="cuda") for _ in range(3))
        W = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        st = torch.ones((), dtype=torch.int32, device="cuda")
        return [A, B, P, Mm, V, st], [P, Mm, V, W]
    pay = struct.pack("<iifffff", 0, 0, 1e-3, 0.9, 0.999, 1e-8, 0.0)
    ins, outs = args(384, 256, 64)
    with pytest.raises(RuntimeError):
        C.launch_by_id("gemm_adamw_bf16_v0", C.OpKind.GemmAdamW, ins, outs, GADW, pay)
    ins, outs = args(256, 256, 96)
    with pytest.raises(RuntimeError):
        C.launch_by_id("gemm_adamw_bf16_v0", C.OpKind.GemmAdamW, ins, outs, GADW, pay)
    ins, outs = args(256, 256, 64)
    with pytest.raises(RuntimeError):
        C.launch_by_id("gemm_adamw_bf16_v0", C.OpKind.GemmAdamW, ins, [outs[0].clone()] + outs[1:], GADW, pay)
    with pytest.raises(RuntimeError):
        C.launch_by_id("gemm_adamw_bf16_v0", C.OpKind.GemmAdamW, ins, outs, GADW,
                       struct.pack("<iifffff", 0, 0, float("nan"), 0.9, 0.999, 1e-8, 0.0))
    C.launch_by_id("gemm_adamw_bf16_v0", C.OpKind.GemmAdamW, ins, outs, GADW, pay)
    torch.cuda.synchronize()
    assert float(outs[0].abs().max().item()) == 0.0  # zero gradient, zero decay: P stays 0


@pytest.mark.parametrize("R,Ccols,dtype", [(64, 64, "bf16"), (4096, 8192, "bf16"), (100, 37, "f32"),
                                           (300, 129, "bf16"), (8192, 256, "f32")])
def test_transpose(C, R, Ccols, dtype):
    r = rng(R * Ccols)
    x = r.standard_normal((R, Ccols)).astype(np.float32)
    if dtype == "bf16":
        xb = orc.bf16_bits_from_f32(x)
        tx, want = g(xb, torch.bfloat16), np.ascontiguousarray(xb.reshape(R, Ccols).T)
    else:
        tx, want = g(x), np.ascontiguousarray(x.T)
    y = torch.empty((Ccols, R), dtype=tx.dtype, device="cuda")
    C.op_call(int(C.OpKind.Transpose), [tx], [y], 0, b"", 0)
    assert np.array_equal(h(y), want)  # pure data movement: bit-exact


# ============================================================== graph
def test_graph_capture_replay_matches_eager(C):
    """Captured elementwise + Adam sequence, replayed 3x with eager work and
    host-side scalar updates between replays; each replay checked."""
    r = rng(16)
    n = 1 << 16
    P = r.standard_normal(n).astype(np.float32)
    G = r.standard_normal(n).astype(np.float32)
    tP, tG = g(P), g(G)
    tM, tV = torch.zeros_like(tP), torch.zeros_like(tP)
    bc1 = torch.tensor(1.0, device="cuda")
    bc2 = torch.tensor(1.0, device="cuda")
    pay = struct.pack("<ffff", 1e-3, 0.9, 0.999, 1e-8)
    C.graph_reset()
    s = C.graph_begin()
    assert s != 0 and C.graph_stream() == s
    C.launch_by_id("adam_step_f32_v0", C.OpKind.AdamStep, [tP, tG, tM, tV, bc1, bc2],
                   [tP, tM, tV], ADAM, pay, s)
    C.graph_end()
    trace = C.trace_get()
    assert trace == ["kid:adam_step_f32_v0 kind:adam_step"]
    Pc, Mc, Vc = P.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for t in range(1, 4):
        b1, b2 = np.float32(1 - 0.9 ** t), np.float32(1 - 0.999 ** t)
        bc1.fill_(float(b1))
        bc2.fill_(float(b2))
        _ = (tG * 2).sum()  # unrelated eager work on torch's stream
        C.graph_launch()
        torch.cuda.synchronize()
        Pc, Mc, Vc = orc.adam_ref(Pc, G, Mc, Vc, b1, b2)
        assert np.array_equal(h(tP), Pc), f"replay {t}"
        assert np.array_equal(h(tV), Vc), f"replay {t}"
    C.graph_reset()
    with pytest.raises(RuntimeError, match="no captured graph"):
        C.graph_launch()
    with pytest.raises(RuntimeError, match="not capturing"):
        C.graph_end()


def test_trace_api(C):
    C.trace_reset()
    C.trace_enable(True)
    x = torch.ones(16, device="cuda")
    C.op_call(int(C.OpKind.EltwiseRelu), [x], [x])
    C.launch_by_id("relu_f32_v0", C.OpKind.EltwiseRelu, [x], [x])
    assert C.trace_get() == ["relu", "kid:relu_f32_v0 kind:relu"]
    C.trace_enable(False)
    C.op_call(int(C.OpKind.EltwiseRelu), [x], [x])
    assert len(C.trace_get()) == 2
    C.trace_enable(True)
    C.trace_reset()
    assert C.trace_get() == []


def test_diag_mfma_loop_runs_and_rate_is_plausible(C):
    """The measurement aid behind bench.py's MFMA ceiling: returns Ok, rejects
    bad arguments, and its rate lies between a fraction of and the dense bf16
    peak (2.5 PFLOP/s)."""
    import ctypes

    from aicf_cuda import abi

    lib = abi.load()
    out = torch.zeros(1, device="cuda")
    s = torch.cuda.current_stream()
    assert lib.aicf_diag_mfma_loop(None, 256, 10, 1, None) == abi.STATUS_INVALID_ARGUMENT
    assert lib.aicf_diag_mfma_loop(ctypes.c_void_p(out.data_ptr()), 0, 10, 1, None) == abi.STATUS_INVALID_ARGUMENT
    blocks, iters = 1024, 2000
    for k in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        assert lib.aicf_diag_mfma_loop(ctypes.c_void_p(out.data_ptr()), blocks, iters, k + 1,
                                       ctypes.c_void_p(s.cuda_stream)) == abi.STATUS_OK
        e1.record(s)
        torch.cuda.synchronize()
    tflops = blocks * 4.0 * iters * 8 * 32768 / (e0.elapsed_time(e1) * 1e-3) / 1e12
    assert 300.0 < tflops < 2600.0, tflops
    # the 16 x 16 x 32 form: same flop per round, rejected forms
    assert lib.aicf_diag_mfma_loop_form(ctypes.c_void_p(out.data_ptr()), 4, 10, 1, 8, None) == \
        abi.STATUS_INVALID_ARGUMENT
    for k in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        assert lib.aicf_diag_mfma_loop_form(ctypes.c_void_p(out.data_ptr()), blocks, iters, k + 1, 16,
                                            ctypes.c_void_p(s.cuda_stream)) == abi.STATUS_OK
        e1.record(s)
        torch.cuda.synchronize()
    tflops16 = blocks * 4.0 * iters * 16 * 16384 / (e0.elapsed_time(e1) * 1e-3) / 1e12
    assert 300.0 < tflops16 < 2600.0, tflops16
