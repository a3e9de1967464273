"""Pins the CPU oracle before it is trusted as the parity reference.

Each oracle function is checked against something independent of its own
formula: the reference probes' closed forms, an independent library
(numpy, torch on the CPU in float64), brute force, or special cases whose
answer is fixed by the mathematics.  The checks are chosen so that a
plausible slip (swapped betas, a dropped bias-correction term, a wrong
index, an off-by-one rounding) fails at least one of them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as orc


def rng(seed=0):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- formats
def test_f16_conversion_matches_numpy_correct_rounding():
    r = rng(1)
    x = np.concatenate([  # includes overflow to inf on purpose
        r.standard_normal(20000) * 10.0 ** r.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]),
    ])
    got = orc.f16_bits_from_f64(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)  # numpy rounds double->half once, RNE
    assert np.array_equal(got, ref)
    back = orc.f16_bits_to_f64(got)
    assert np.array_equal(back, ref.view(np.float16).astype(np.float64))


def test_bf16_conversion_matches_torch():
    r = rng(2)
    x = (r.standard_normal(50000) * 10.0 ** r.integers(-30, 30, 50000)).astype(np.float32)
    x[:4] = [0.0, -0.0, np.inf, -np.inf]
    got = orc.bf16_bits_from_f32(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    assert np.array_equal(orc.bf16_bits_to_f32(got),
                          torch.from_numpy(x).to(torch.bfloat16).float().numpy())


# ---------------------------------------------------------------- adam
def _adam_probe_formula(P, G, M, V, bc1, bc2, lr, b1, b2, eps):
    # v2_adam_step_probe.py:32-38 (torch expression), here in float64 on the
    # fp32 values the kernel receives (attrs are packed as <ffff>)
    lr, b1, b2, eps = (float(np.float32(v)) for v in (lr, b1, b2, eps))
    P, G, M, V = (torch.from_numpy(a.astype(np.float64)) for a in (P, G, M, V))
    m_new = b1 * M + (1.0 - b1) * G
    v_new = b2 * V + (1.0 - b2) * (G * G)
    P_new = P - lr * ((m_new / bc1) / (torch.sqrt(v_new / bc2) + eps))
    return P_new.numpy(), m_new.numpy(), v_new.numpy()


@pytest.mark.parametrize("t", [1, 3, 10])
def test_adam_ref_matches_probe_formula(t):
    r = rng(3)
    n = 4096
    P = r.standard_normal(n).astype(np.float32)
    G = r.standard_normal(n).astype(np.float32)
    M = (0.1 * r.standard_normal(n)).astype(np.float32)
    V = np.abs(r.standard_normal(n)).astype(np.float32)
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-8
    bc1, bc2 = np.float32(1 - b1 ** t), np.float32(1 - b2 ** t)
    Po, Mo, Vo = orc.adam_ref(P, G, M, V, bc1, bc2, lr, b1, b2, eps)
    Pr, Mr, Vr = _adam_probe_formula(P, G, M, V, float(bc1), float(bc2), lr, b1, b2, eps)
    assert orc.rel_err(Mo, Mr) < 1e-6
    assert orc.rel_err(Vo, Vr) < 1e-6
    # P' within the rounding of P' plus a few ulp of the step (the m update
    # can cancel, which amplifies its fp32 rounding)
    tol = 1.5 * np.spacing(np.abs(Pr).astype(np.float32)) + 2.0 ** -19 * np.abs(Pr - P)
    assert np.all(np.abs(Po - Pr) <= tol)
    assert orc.rel_err(Po, Pr) < 1e-6
    f = lambda v: float(np.float32(v))  # noqa: E731  attrs arrive as fp32
    Pd, Md, Vd = orc.adam_f64(P, G, M, V, float(bc1), float(bc2), f(lr), f(b1), f(b2), f(eps))
    assert orc.rel_err(Pd - P, Pr - P) < 1e-12
    assert orc.rel_err(Md, Mr) < 1e-12


def test_adam_first_step_closed_form():
    # t=1, m=v=0, bc=1-beta: m_hat = g, v_hat = g^2 -> p' = p - lr*g/(|g|+eps)
    r = rng(4)
    g = r.uniform(0.5, 2.0, 1000).astype(np.float32) * np.sign(r.standard_normal(1000)).astype(np.float32)
    p = r.standard_normal(1000).astype(np.float32)
    z = np.zeros_like(p)
    Po, Mo, Vo = orc.adam_ref(p, g, z, z, np.float32(0.1), np.float32(1 - 0.999))
    expect = p.astype(np.float64) - 1e-3 * g / (np.abs(g) + 1e-8)
    assert np.max(np.abs(Po - expect)) < 2e-6
    assert np.allclose(Mo, 0.1 * g, rtol=1e-6)
    omb2 = float(np.float32(1) - np.float32(0.999))  # 1 - beta2 formed in fp32
    assert np.allclose(Vo, omb2 * g.astype(np.float64) ** 2, rtol=1e-6)


def test_adamw_reduces_to_adam_and_applies_decoupled_wd():
    r = rng(5)
    n = 2048
    P = r.standard_normal(n).astype(np.float32)
    G = r.standard_normal(n).astype(np.float32)
    M = (0.1 * r.standard_normal(n)).astype(np.float32)
    V = np.abs(r.standard_normal(n)).astype(np.float32)
    for t in (1, 7):
        # bias correction from the fp32 betas, rounded to fp32 once
        bc1 = float(np.float32(1 - float(np.float32(0.9)) ** t))
        bc2 = float(np.float32(1 - float(np.float32(0.999)) ** t))
        Po, Mo, Vo = orc.adamw(P, G, M, V, t, wd=0.0)
        Pr, Mr, Vr = _adam_probe_formula(P, G, M, V, bc1, bc2, 1e-3, 0.9, 0.999, 1e-8)
        ulp = np.spacing(np.abs(Pr).astype(np.float32)) + 2.0 ** -19 * np.abs(Pr - P)
        assert np.all(np.abs(Po - Pr) <= 1.5 * ulp)
        assert orc.rel_err(Mo, Mr) < 1e-6
        wd = 0.01
        Pw, _, _ = orc.adamw(P, G, M, V, t, wd=wd)
        Pwr = P.astype(np.float64) * float(np.float32(1) - np.float32(1e-3) * np.float32(wd)) + (Pr - P)
        assert np.all(np.abs(Pw - Pwr) <= 2.5 * ulp)
        # weight decay moved every parameter towards zero by lr*wd*|p|
        assert np.all(np.abs(Pw - Po) <= 1e-5 * np.abs(P) + 2 * ulp)
    # step 0 is clamped to 1
    a = orc.adamw(P, G, M, V, 0)
    b = orc.adamw(P, G, M, V, 1)
    assert np.array_equal(a[0], b[0])
    _, _, _, Wb = orc.adamw(P, G, M, V, 2, shadow=True)
    assert np.array_equal(Wb, orc.bf16_bits_from_f32(orc.adamw(P, G, M, V, 2)[0]))


@pytest.mark.parametrize("step", [0, 1, 2, 10, 1000])
def test_bias_corr_matches_probe(step):
    # v2_biascorr_probe.py:32-40: t = max(step, 1), out = 1/(1 - beta^t)
    t = max(step, 1)
    o1, o2 = orc.bias_corr(step, 0.9, 0.999)
    assert abs(o1 - 1 / (1 - 0.9 ** t)) / (1 / (1 - 0.9 ** t)) < 2e-6
    assert abs(o2 - 1 / (1 - 0.999 ** t)) / (1 / (1 - 0.999 ** t)) < 2e-5
    # beta = 1 makes 1 - beta^t = 0, clamped to 1e-20
    o1, _ = orc.bias_corr(step, 1.0, 0.5)
    assert o1 == np.float32(1e20)


def test_sgd_matches_formula():
    r = rng(6)
    P = r.standard_normal(1000).astype(np.float32)
    G = r.standard_normal(1000).astype(np.float32)
    O = orc.sgd_f32(P, G, 0.01)
    assert np.max(np.abs(O - (P.astype(np.float64) - 0.01 * G))) <= np.max(np.abs(P)) * 2 ** -23
    Ph = P.astype(np.float16).view(np.uint16)
    Gh = G.astype(np.float16).view(np.uint16)
    Oh = orc.sgd_f16(Ph, Gh, 0.01)
    ref = (Ph.view(np.float16).astype(np.float64) - 0.01 * Gh.view(np.float16).astype(np.float64))
    assert np.max(np.abs(Oh.view(np.float16).astype(np.float64) - ref)) < 2e-3


# ---------------------------------------------------------------- elementwise
def test_add_f16_is_correctly_rounded():
    r = rng(7)
    a = (r.standard_normal(5000) * 10.0 ** r.integers(-4, 4, 5000)).astype(np.float16)
    b = (r.standard_normal(5000) * 10.0 ** r.integers(-4, 4, 5000)).astype(np.float16)
    got = orc.add_f16(a.view(np.uint16), b.view(np.uint16))
    exact = a.astype(np.float64) + b.astype(np.float64)
    assert np.array_equal(got, exact.astype(np.float16).view(np.uint16))


def test_add_f32_is_numpy_float32_add():
    """orc_add_f32 (add/launcher.cu:44-50: out = a + b in fp32) against
    numpy's IEEE float32 addition: bit-identical on random magnitudes
    spanning cancellation, denormals and the special values."""
    r = rng(17)
    a = (r.standard_normal(20000) * 10.0 ** r.integers(-40, 38, 20000)).astype(np.float32)
    b = (r.standard_normal(20000) * 10.0 ** r.integers(-40, 38, 20000)).astype(np.float32)
    b[:500] = -a[:500]                       # exact cancellation gives +0
    b[500:1000] = np.nextafter(-a[500:1000], np.float32(0))  # one-ulp differences
    sp = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 1e-45, -1e-45, 3.4e38], np.float32)
    a = np.concatenate([a, np.repeat(sp, sp.size)])
    b = np.concatenate([b, np.tile(sp, sp.size)])
    got = orc.add_f32(a, b)
    want = (a + b).astype(np.float32)
    assert np.array_equal(got.view(np.uint32)[~np.isnan(want)], want.view(np.uint32)[~np.isnan(want)])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    # inf + -inf is NaN, -0 + -0 keeps its sign
    i = a.size - sp.size * sp.size
    assert np.isnan(got[i + 1]) and got.view(np.uint32)[i + 4 * 8 + 4] == np.float32(-0.0).view(np.uint32)


def test_relu_bwd_f16_matches_numpy_mask():
    """orc_relu_bwd_f16 (relu_bwd/launcher.cu:47-56: dY = Y > 0 ? dOut : +0,
    as half bits) against a numpy float16 mask over every one of the 65536
    half bit patterns of Y (NaN and -0 give +0, positive denormals pass dOut)."""
    y = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    r = rng(18)
    dout = r.standard_normal(65536).astype(np.float16).view(np.uint16)
    got = orc.relu_bwd_f16(dout, y)
    want = np.where(y.view(np.float16) > np.float16(0), dout, np.uint16(0)).astype(np.uint16)
    assert np.array_equal(got, want)
    assert got[0x0001] == dout[0x0001] and got[0x8000] == 0 and got[0x7E00] == 0


def test_relu_special_values():
    x = np.array([1.5, -2.0, 0.0, -0.0, np.nan, np.inf, -np.inf, 1e-40], np.float32)
    y = orc.relu_f32(x)
    assert np.array_equal(y.view(np.uint32), np.array([1.5, 0, 0, 0, 0, np.inf, 0, 1e-40],
                                                      np.float32).view(np.uint32))
    yh = orc.relu_f16(x.astype(np.float16).view(np.uint16))
    assert np.array_equal(yh, np.array([1.5, 0, 0, 0, 0, np.inf, 0, 0], np.float16).view(np.uint16))
    d = orc.relu_bwd_f32(np.full(8, 3.0, np.float32), x)
    assert np.array_equal(d, np.array([3, 0, 0, 0, 0, 3, 0, 3], np.float32))


def test_bias_add_broadcasts_last_dim():
    r = rng(8)
    y = r.standard_normal((7, 5)).astype(np.float32)
    b = r.standard_normal(5).astype(np.float32)
    assert np.array_equal(orc.bias_add_f32(y, b).reshape(7, 5), y + b[None, :])
    yh, bh = y.astype(np.float16), b.astype(np.float16)
    got = orc.bias_add_f16(yh.view(np.uint16), bh.view(np.uint16)).view(np.float16).reshape(7, 5)
    exact = (yh.astype(np.float64) + bh.astype(np.float64)[None, :]).astype(np.float16)
    assert np.array_equal(got, exact)


def test_mse_grad_default_scale_and_half_math():
    r = rng(9)
    p = r.standard_normal((64, 256)).astype(np.float32)
    t = r.standard_normal((64, 256)).astype(np.float32)
    d = orc.mse_grad_f32(p, t)
    # mse_grad/launcher.cu:213-215: scale = 2/numel
    assert np.allclose(d, (p - t).ravel() * (2.0 / p.size), rtol=1e-6, atol=0)
    ph, th = p.astype(np.float16), t.astype(np.float16)
    dh = orc.mse_grad_f16(ph.view(np.uint16), th.view(np.uint16), 0.125, half_math=True)
    # numpy float16 ops round each result to half (exact here: |values| < 8)
    ref = ((ph - th) * np.float16(0.125)).ravel()
    assert np.array_equal(dh.view(np.float16), ref)
    ds = orc.mse_grad_f16(ph.view(np.uint16), th.view(np.uint16), 0.1)
    ref2 = ((ph.astype(np.float32) - th.astype(np.float32)) * np.float32(0.1)).astype(np.float16).ravel()
    assert np.array_equal(ds.view(np.float16), ref2)
    assert abs(orc.mse_loss_f64(p, t) - np.mean((p.astype(np.float64) - t) ** 2)) < 1e-12


def test_gelu_matches_torch():
    x = np.linspace(-8, 8, 4001)
    xt = torch.from_numpy(x).requires_grad_(True)
    y = torch.nn.functional.gelu(xt, approximate="tanh")
    y.sum().backward()
    assert np.max(np.abs(orc.gelu_f64(x) - y.detach().numpy())) < 1e-14
    assert np.max(np.abs(orc.gelu_grad_f64(x) - xt.grad.numpy())) < 1e-13


# ---------------------------------------------------------------- reductions
def test_colsum_matches_numpy():
    x = rng(10).standard_normal((257, 64)).astype(np.float32)
    assert np.allclose(orc.colsum_f64(x), x.astype(np.float64).sum(0), rtol=0, atol=1e-12)


@pytest.mark.parametrize("C", [10, 128, 1000])
def test_softmax_matches_torch_and_stable_row(C):
    x = (2.0 * rng(11).standard_normal((33, C))).astype(np.float32)
    x[-1, :] = -1e4
    y, mx, sx = orc.softmax_rows_f64(x)
    ref = torch.softmax(torch.from_numpy(x).double(), dim=1).numpy()
    assert np.max(np.abs(y - ref)) < 1e-15
    assert np.array_equal(mx, x.max(1).astype(np.float64))
    assert np.allclose(sx, x.astype(np.float64).sum(1), rtol=1e-12)
    assert np.all(y[-1] == 1.0 / C)


def test_softmax_xent_matches_torch():
    r = rng(12)
    z = (3 * r.standard_normal((64, 10))).astype(np.float32)
    z[5, 2] = z[5, 7] = z[5].max() + 1.0  # tie: first index wins
    lab = r.integers(0, 10, 64).astype(np.int32)
    loss, dz, am, rl = orc.softmax_xent_f64(z, lab)
    zt = torch.from_numpy(z).double().requires_grad_(True)
    lt = torch.nn.functional.cross_entropy(zt, torch.from_numpy(lab).long())
    lt.backward()
    assert abs(loss - lt.item()) < 1e-13
    assert np.max(np.abs(dz - zt.grad.numpy())) < 1e-15
    assert np.array_equal(am, np.argmax(z, axis=1))
    assert am[5] == 2


# ---------------------------------------------------------------- gemm
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_f64_matches_numpy(ta, tb):
    r = rng(13)
    M, K, N = 64, 48, 80  # v2_gemm_probe.py:92-119 shapes
    A = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    ref = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
    got = orc.gemm_f64(A, B, ta, tb)
    assert np.max(np.abs(got - ref)) < 1e-12
    g32 = orc.gemm_ref_f32(A, B, ta, tb)
    assert orc.rel_err(g32, ref) < 1e-6
    part = orc.gemm_ref_f32(A, B, ta, tb, rows=(8, 16))
    assert np.array_equal(part[8:16], g32[8:16]) and not part[:8].any()


# ---------------------------------------------------------------- LayerNorm / BatchNorm
@pytest.mark.parametrize("affine", [False, True])
def test_layernorm_matches_torch(affine):
    r = rng(21)
    M, N = 7, 33  # v2_layernorm_probe.py shapes include (7, 33)
    x = r.standard_normal((M, N)) * 3 + 1.5
    dy = r.standard_normal((M, N))
    g = r.standard_normal(N) if affine else None
    b = r.standard_normal(N) if affine else None
    y, mu, rs = orc.layernorm_fwd_f64(x, g, b, eps=1e-5)
    xt = torch.from_numpy(x).requires_grad_(True)
    gt = torch.from_numpy(g).requires_grad_(True) if affine else None
    bt = torch.from_numpy(b).requires_grad_(True) if affine else None
    yt = torch.nn.functional.layer_norm(xt, (N,), gt, bt, eps=1e-5)
    assert np.max(np.abs(y - yt.detach().numpy())) < 1e-12
    assert np.max(np.abs(mu - x.mean(1))) < 1e-13
    assert np.max(np.abs(rs - 1 / np.sqrt(x.var(1) + 1e-5))) < 1e-12
    yt.backward(torch.from_numpy(dy))
    dx, dg, db = orc.layernorm_bwd_f64(x, dy, mu, rs, g)
    assert np.max(np.abs(dx - xt.grad.numpy())) < 1e-11
    if affine:
        assert np.max(np.abs(dg - gt.grad.numpy())) < 1e-11
        assert np.max(np.abs(db - bt.grad.numpy())) < 1e-11
    else:
        assert dg is None and db is None


def test_layernorm_constant_row_closed_form():
    x = np.full((2, 16), 3.25)
    y, mu, rs = orc.layernorm_fwd_f64(x, eps=1e-5)
    assert np.all(y == 0) and np.all(mu == 3.25)
    assert np.allclose(rs, 1 / np.sqrt(1e-5), rtol=1e-15)


@pytest.mark.parametrize("affine", [False, True])
def test_batchnorm_matches_torch(affine):
    r = rng(22)
    Nb, C, H, W = 7, 5, 5, 3
    x = r.standard_normal((Nb, C, H, W)) * 2 - 0.5
    dy = r.standard_normal((Nb, C, H, W))
    g = r.standard_normal(C) if affine else None
    b = r.standard_normal(C) if affine else None
    y, mu, rs = orc.batchnorm_fwd_train_f64(x, g, b, eps=1e-5)
    xt = torch.from_numpy(x).requires_grad_(True)
    gt = torch.from_numpy(g).requires_grad_(True) if affine else None
    bt = torch.from_numpy(b).requires_grad_(True) if affine else None
    yt = torch.nn.functional.batch_norm(xt, None, None, gt, bt, training=True, momentum=0.0, eps=1e-5)
    assert np.max(np.abs(y - yt.detach().numpy())) < 1e-12
    if affine:
        yt.backward(torch.from_numpy(dy))
        dx, dg, db = orc.batchnorm_bwd_f64(x, dy, g, mu, rs)
        assert np.max(np.abs(dx - xt.grad.numpy())) < 1e-11
        assert np.max(np.abs(dg - gt.grad.numpy())) < 1e-11
        assert np.max(np.abs(db - bt.grad.numpy())) < 1e-11
    rm, rv = r.standard_normal(C), r.uniform(0.5, 1.5, C)
    yi = orc.batchnorm_fwd_infer_f64(x, rm, rv, g, b, eps=1e-5)
    yti = torch.nn.functional.batch_norm(torch.from_numpy(x), torch.from_numpy(rm), torch.from_numpy(rv),
                                         None if g is None else torch.from_numpy(g),
                                         None if b is None else torch.from_numpy(b), training=False, eps=1e-5)
    assert np.max(np.abs(yi - yti.numpy())) < 1e-12
