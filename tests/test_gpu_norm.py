"""GPU parity of LayerNorm (f32, f16) and BatchNorm (f16 NCHW) against the
CPU oracle (fp64 restatements of layernorm/launcher.cu and
batchnorm/launcher.cu, pinned against torch in test_oracle.py).  Cases follow
python/cuda_binding_test/v2_layernorm_probe.py and v2_batchnorm_probe.py
(shapes, affine / non-affine, training / inference, NEG cases) plus rows
longer than the register-resident LayerNorm path (N > 2048).

Tolerances (normwise rel-err vs fp64 on the stored inputs): fp32 outputs and
the fp32 statistics <= 1e-5; f16 outputs <= 2e-3 (one f16 rounding).
"""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

import oracle as orc

pytestmark = pytest.mark.gpu

LNEP = int.from_bytes(b"LNEP", "little")
BNEP = int.from_bytes(b"BNEP", "little")


def rng(seed):
    return np.random.default_rng(seed)


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).cuda()


def host(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def stored(a, dtype):
    """The values a tensor of `dtype` holds (f16 rounding applied)."""
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).double().numpy()


LN_SHAPES = [(8, 128), (64, 256), (7, 33), (5, 2048), (6, 3000), (3, 1)]


@pytest.mark.parametrize("M,N", LN_SHAPES)
@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_layernorm_fwd_bwd(C, M, N, affine, dtype):
    r = rng(M * 7 + N)
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    x = dev(r.standard_normal((M, N)) * 2 + 0.5, dtype)
    g = dev(r.standard_normal(N), dtype) if affine else None
    b = dev(r.standard_normal(N), dtype) if affine else None
    y = torch.empty_like(x)
    mean = torch.empty(M, device="cuda")
    rstd = torch.empty(M, device="cuda")
    ins = [x, g, b] if affine else [x]
    C.op_call(C.OpKind.LayerNormFwd, ins, [y, mean, rstd], LNEP, struct.pack("<f", 1e-5))
    xs = host(x)
    gs, bs = (host(g), host(b)) if affine else (None, None)
    y_ref, mu_ref, rs_ref = orc.layernorm_fwd_f64(xs, gs, bs, eps=1e-5)
    assert orc.rel_err(host(mean), mu_ref) < 1e-5
    assert orc.rel_err(host(rstd), rs_ref) < 1e-5
    if N > 1:
        assert orc.rel_err(host(y), y_ref) < tol

    # backward with the statistics the forward produced
    dy = dev(r.standard_normal((M, N)), dtype)
    dx = torch.empty_like(x)
    if affine:
        dg = torch.empty(N, device="cuda")
        db = torch.empty(N, device="cuda")
        C.op_call(C.OpKind.LayerNormBwd, [x, dy, g, mean, rstd], [dx, dg, db])
    else:
        C.op_call(C.OpKind.LayerNormBwd, [x, dy, mean, rstd], [dx])
    dx_ref, dg_ref, db_ref = orc.layernorm_bwd_f64(xs, host(dy), host(mean), host(rstd), gs)
    if N > 1:
        assert orc.rel_err(host(dx), dx_ref) < tol
    if affine:
        assert orc.rel_err(host(dg), dg_ref) < 1e-5
        assert orc.rel_err(host(db), db_ref) < 1e-5


def test_layernorm_eps_attr_and_by_id(C):
    """LNEP eps is honoured; by-id dispatch of the f32 id; a constant row
    normalises to exactly 0 with rstd = 1/sqrt(eps)."""
    x = torch.full((4, 64), 2.5, device="cuda")
    x[1] = torch.arange(64, device="cuda", dtype=torch.float32)
    y = torch.empty_like(x)
    mean = torch.empty(4, device="cuda")
    rstd = torch.empty(4, device="cuda")
    C.launch_by_id("layernorm_fwd_f32_v0", C.OpKind.LayerNormFwd, [x], [y, mean, rstd], LNEP,
                   struct.pack("<f", 0.25))
    assert torch.all(y[0] == 0) and float(mean[0]) == 2.5
    assert abs(float(rstd[0]) - 2.0) < 1e-6  # 1/sqrt(0 + 0.25)
    ref, _, rs = orc.layernorm_fwd_f64(host(x), eps=0.25)
    assert orc.rel_err(host(y), ref) < 1e-5 and orc.rel_err(host(rstd), rs) < 1e-6


def test_layernorm_neg_cases(C):
    x3 = torch.randn(2, 3, 4, device="cuda")
    with pytest.raises(RuntimeError, match="NotImplemented"):  # v2_layernorm_probe NEG rank
        C.op_call(C.OpKind.LayerNormFwd, [x3], [torch.empty_like(x3), torch.empty(2, device="cuda"),
                                                torch.empty(2, device="cuda")], LNEP, struct.pack("<f", 1e-5))
    x = torch.randn(4, 8, device="cuda")
    outs = [torch.empty_like(x), torch.empty(4, device="cuda"), torch.empty(4, device="cuda")]
    with pytest.raises(RuntimeError, match="NotImplemented"):  # schema gate (LNEP required)
        C.op_call(C.OpKind.LayerNormFwd, [x], outs, 0, b"")
    with pytest.raises(RuntimeError, match="InvalidArgument"):
        C.launch_by_id("layernorm_fwd_f32_v0", C.OpKind.LayerNormFwd, [x], outs, 0, b"")


BN_SHAPES = [(8, 16, 8, 8), (16, 32, 16, 16), (7, 33, 5, 7)]


@pytest.mark.parametrize("shape", BN_SHAPES)
@pytest.mark.parametrize("affine", [True, False])
def test_batchnorm_training_fwd_bwd(C, shape, affine):
    r = rng(sum(shape) + affine)
    Nb, Cc, H, W = shape
    x = dev(r.standard_normal(shape) * 1.5 + 0.25, torch.float16)
    g = dev(r.standard_normal(Cc), torch.float16) if affine else None
    b = dev(r.standard_normal(Cc), torch.float16) if affine else None
    y = torch.empty_like(x)
    sm = torch.zeros(Cc, device="cuda")
    sr = torch.zeros(Cc, device="cuda")
    C.op_call(C.OpKind.BatchNormFwd, [x, g, b] if affine else [x], [y, sm, sr], BNEP,
              struct.pack("<fI", 1e-5, 0))
    xs = host(x)
    gs, bs = (host(g), host(b)) if affine else (None, None)
    y_ref, mu_ref, rs_ref = orc.batchnorm_fwd_train_f64(xs, gs, bs, eps=1e-5)
    assert orc.rel_err(host(sm), mu_ref) < 1e-5
    assert orc.rel_err(host(sr), rs_ref) < 1e-5
    assert orc.rel_err(host(y), y_ref) < 2e-3
    if not affine:
        # non-affine backward: accepted by supported(), NotImplemented at launch
        dy = torch.randn_like(x)
        with pytest.raises(RuntimeError, match="NotImplemented"):
            C.op_call(C.OpKind.BatchNormBwd, [x, dy, sm, sr], [torch.empty_like(x)])
        return
    dy = dev(r.standard_normal(shape), torch.float16)
    dx = torch.empty_like(x)
    dg = torch.zeros(Cc, device="cuda")
    db = torch.zeros(Cc, device="cuda")
    C.op_call(C.OpKind.BatchNormBwd, [x, dy, g, sm, sr], [dx, dg, db])
    dx_ref, dg_ref, db_ref = orc.batchnorm_bwd_f64(xs, host(dy), gs, host(sm), host(sr))
    assert orc.rel_err(host(dx), dx_ref) < 2e-3
    assert orc.rel_err(host(dg), dg_ref) < 1e-5
    assert orc.rel_err(host(db), db_ref) < 1e-5


@pytest.mark.parametrize("shape", BN_SHAPES)
@pytest.mark.parametrize("affine", [True, False])
def test_batchnorm_inference(C, shape, affine):
    r = rng(sum(shape) * 3 + affine)
    Cc = shape[1]
    x = dev(r.standard_normal(shape), torch.float16)
    rm = dev(r.standard_normal(Cc), torch.float32)
    rv = dev(r.uniform(0.5, 1.5, Cc), torch.float32)
    g = dev(r.standard_normal(Cc), torch.float16) if affine else None
    b = dev(r.standard_normal(Cc), torch.float16) if affine else None
    y = torch.empty_like(x)
    ins = [x, g, b, rm, rv] if affine else [x, rm, rv]
    C.op_call(C.OpKind.BatchNormFwd, ins, [y], BNEP, struct.pack("<fI", 1e-5, 1))
    ref = orc.batchnorm_fwd_infer_f64(host(x), host(rm), host(rv),
                                      host(g) if affine else None, host(b) if affine else None, eps=1e-5)
    assert orc.rel_err(host(y), ref) < 2e-3


def test_batchnorm_neg_cases(C):
    x2 = torch.randn(8, 16, device="cuda", dtype=torch.float16)
    with pytest.raises(RuntimeError, match="NotImplemented"):  # wrong rank
        C.op_call(C.OpKind.BatchNormFwd, [x2], [torch.empty_like(x2)], BNEP, struct.pack("<fI", 1e-5, 1))
    x = torch.randn(8, 16, 8, 8, device="cuda", dtype=torch.float16)
    rm = torch.zeros(16, device="cuda")
    rv = torch.ones(16, device="cuda")
    with pytest.raises(RuntimeError, match="NotImplemented"):  # wrong schema
        C.op_call(C.OpKind.BatchNormFwd, [x, rm, rv], [torch.empty_like(x)], 0x12345678, b"\x00" * 8)
    # training outputs with use_running_stats set -> InvalidArgument
    with pytest.raises(RuntimeError, match="InvalidArgument"):
        C.op_call(C.OpKind.BatchNormFwd, [x], [torch.empty_like(x), torch.empty(16, device="cuda"),
                                               torch.empty(16, device="cuda")], BNEP, struct.pack("<fI", 1e-5, 1))
