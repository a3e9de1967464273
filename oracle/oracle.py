"""Python face of the CPU oracle (oracle/aicf_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product path.  Each function
names the reference code it restates (paths relative to
ai-compiler-framework/ in the reference tree).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"

_lib = None

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
I64, F32, F64, I32 = ctypes.c_int64, ctypes.c_float, ctypes.c_double, ctypes.c_int32


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB.exists():
        build()
    L = ctypes.CDLL(str(LIB))
    sig = {
        "orc_threads": (I32, []),
        "orc_set_threads": (None, [I32]),
        "orc_f16_from_f64": (ctypes.c_uint16, [F64]),
        "orc_f16_to_f64": (F64, [ctypes.c_uint16]),
        "orc_bf16_from_f32": (ctypes.c_uint16, [F32]),
        "orc_f32_to_bf16_array": (None, [f32p, u16p, I64]),
        "orc_bf16_to_f32_array": (None, [u16p, f32p, I64]),
        "orc_f64_to_f16_array": (None, [f64p, u16p, I64]),
        "orc_adam_ref_f32": (None, [f32p, f32p, f32p, f32p, f32p, f32p, f32p, I64, F32, F32, F32,
                                    F32, F32, F32]),
        "orc_adam_f64": (None, [f32p, f32p, f32p, f32p, f64p, f64p, f64p, I64, F64, F64, F64, F64,
                                F64, F64]),
        "orc_adamw_f32": (None, [f32p, f32p, f32p, f32p, f32p, f32p, f32p, ctypes.c_void_p, I64,
                                 F32, F32, F32, F32, F32, I32]),
        "orc_bias_corr": (None, [I32, F32, F32, ctypes.POINTER(F32), ctypes.POINTER(F32)]),
        "orc_sgd_f32": (None, [f32p, f32p, f32p, I64, F32]),
        "orc_sgd_f16": (None, [u16p, u16p, u16p, I64, F32]),
        "orc_add_f16": (None, [u16p, u16p, u16p, I64]),
        "orc_add_f32": (None, [f32p, f32p, f32p, I64]),
        "orc_relu_f32": (None, [f32p, f32p, I64]),
        "orc_relu_f16": (None, [u16p, u16p, I64]),
        "orc_relu_bwd_f32": (None, [f32p, f32p, f32p, I64]),
        "orc_relu_bwd_f16": (None, [u16p, u16p, u16p, I64]),
        "orc_bias_add_f32": (None, [f32p, f32p, f32p, I64, I64]),
        "orc_bias_add_f16": (None, [u16p, u16p, u16p, I64, I64]),
        "orc_mse_grad_f32": (None, [f32p, f32p, f32p, I64, F32]),
        "orc_mse_grad_f16_scalar": (None, [u16p, u16p, u16p, I64, F32]),
        "orc_mse_grad_f16_half": (None, [u16p, u16p, u16p, I64, F32]),
        "orc_mse_loss_f64": (F64, [f32p, f32p, I64]),
        "orc_gelu_f64": (None, [f64p, f64p, I64]),
        "orc_gelu_grad_f64": (None, [f64p, f64p, I64]),
        "orc_colsum_f64": (None, [f32p, f64p, I64, I64]),
        "orc_softmax_rows_f64": (None, [f32p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                        I64, I64]),
        "orc_softmax_xent_f64": (F64, [f32p, i32p, f64p, i32p, f64p, I64, I64]),
        "orc_gemm_f64": (None, [f32p, I64, I64, f32p, I64, I64, f64p, I64, I64, I64]),
        "orc_gemm_ref_f32": (None, [f32p, I64, I64, f32p, I64, I64, f32p, I64, I64, I64, I64,
                                    I64]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


# ---------------------------------------------------------------- formats
def f16_bits_from_f64(x) -> np.ndarray:
    x = _c(x, np.float64)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f64_to_f16_array(x.ravel(), out.ravel(), x.size)
    return out


def f16_bits_to_f64(h) -> np.ndarray:
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float64)


def bf16_bits_from_f32(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_array(x.ravel(), out.ravel(), x.size)
    return out


def bf16_bits_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def bf16_round(x) -> np.ndarray:
    """fp32 values rounded to bf16 and widened back to fp32."""
    return bf16_bits_to_f32(bf16_bits_from_f32(x))


# ---------------------------------------------------------------- optimizer
def adam_ref(P, G, M, V, bc1, bc2, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8):
    """adam_step/launcher.cu:276-291, fp32, bit-level restatement."""
    P, G, M, V = (_c(a, np.float32).ravel() for a in (P, G, M, V))
    Po, Mo, Vo = (np.empty_like(P) for _ in range(3))
    lib().orc_adam_ref_f32(P, G, M, V, Po, Mo, Vo, P.size, lr, beta1, beta2, eps, bc1, bc2)
    return Po, Mo, Vo


def adam_f64(P, G, M, V, bc1, bc2, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8):
    P, G, M, V = (_c(a, np.float32).ravel() for a in (P, G, M, V))
    Po, Mo, Vo = (np.empty(P.size, np.float64) for _ in range(3))
    lib().orc_adam_f64(P, G, M, V, Po, Mo, Vo, P.size, lr, beta1, beta2, eps, bc1, bc2)
    return Po, Mo, Vo


def adamw(P, G, M, V, step, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, wd=0.0, shadow=False):
    """Appended AdamW variant (in-kernel bias correction from an int32 step)."""
    P, G, M, V = (_c(a, np.float32).ravel() for a in (P, G, M, V))
    Po, Mo, Vo = (np.empty_like(P) for _ in range(3))
    Wb = np.empty(P.size, np.uint16) if shadow else None
    lib().orc_adamw_f32(P, G, M, V, Po, Mo, Vo, _ptr(Wb), P.size, lr, beta1, beta2, eps, wd,
                        int(step))
    return (Po, Mo, Vo, Wb) if shadow else (Po, Mo, Vo)


def bias_corr(step, beta1, beta2):
    """biascorr/launcher.cu:86-99."""
    o1, o2 = F32(), F32()
    lib().orc_bias_corr(int(step), beta1, beta2, ctypes.byref(o1), ctypes.byref(o2))
    return np.float32(o1.value), np.float32(o2.value)


def sgd_f32(P, G, lr):
    P, G = _c(P, np.float32).ravel(), _c(G, np.float32).ravel()
    O = np.empty_like(P)
    lib().orc_sgd_f32(P, G, O, P.size, lr)
    return O


def sgd_f16(P, G, lr):
    P, G = _c(P, np.uint16).ravel(), _c(G, np.uint16).ravel()
    O = np.empty_like(P)
    lib().orc_sgd_f16(P, G, O, P.size, lr)
    return O


# ---------------------------------------------------------------- elementwise
def add_f16(a, b):
    a, b = _c(a, np.uint16).ravel(), _c(b, np.uint16).ravel()
    o = np.empty_like(a)
    lib().orc_add_f16(a, b, o, a.size)
    return o


def add_f32(a, b):
    a, b = _c(a, np.float32).ravel(), _c(b, np.float32).ravel()
    o = np.empty_like(a)
    lib().orc_add_f32(a, b, o, a.size)
    return o


def relu_f32(x):
    x = _c(x, np.float32).ravel()
    y = np.empty_like(x)
    lib().orc_relu_f32(x, y, x.size)
    return y


def relu_f16(x):
    x = _c(x, np.uint16).ravel()
    y = np.empty_like(x)
    lib().orc_relu_f16(x, y, x.size)
    return y


def relu_bwd_f32(dout, y):
    dout, y = _c(dout, np.float32).ravel(), _c(y, np.float32).ravel()
    o = np.empty_like(y)
    lib().orc_relu_bwd_f32(dout, y, o, y.size)
    return o


def relu_bwd_f16(dout, y):
    dout, y = _c(dout, np.uint16).ravel(), _c(y, np.uint16).ravel()
    o = np.empty_like(y)
    lib().orc_relu_bwd_f16(dout, y, o, y.size)
    return o


def bias_add_f32(y, b):
    y = _c(y, np.float32)
    M, N = int(np.prod(y.shape[:-1])), y.shape[-1]
    o = np.empty(y.size, np.float32)
    lib().orc_bias_add_f32(y.ravel(), _c(b, np.float32).ravel(), o, M, N)
    return o


def bias_add_f16(y, b):
    y = _c(y, np.uint16)
    M, N = int(np.prod(y.shape[:-1])), y.shape[-1]
    o = np.empty(y.size, np.uint16)
    lib().orc_bias_add_f16(y.ravel(), _c(b, np.uint16).ravel(), o, M, N)
    return o


def mse_grad_f32(p, t, scale=None):
    p, t = _c(p, np.float32).ravel(), _c(t, np.float32).ravel()
    s = np.float32(2.0) / np.float32(p.size) if scale is None else scale
    d = np.empty_like(p)
    lib().orc_mse_grad_f32(p, t, d, p.size, float(s))
    return d


def mse_grad_f16(p, t, scale=None, half_math=False):
    p, t = _c(p, np.uint16).ravel(), _c(t, np.uint16).ravel()
    s = np.float32(2.0) / np.float32(p.size) if scale is None else scale
    d = np.empty_like(p)
    fn = lib().orc_mse_grad_f16_half if half_math else lib().orc_mse_grad_f16_scalar
    fn(p, t, d, p.size, float(s))
    return d


def mse_loss_f64(p, t):
    p, t = _c(p, np.float32).ravel(), _c(t, np.float32).ravel()
    return lib().orc_mse_loss_f64(p, t, p.size)


def gelu_f64(x):
    x = _c(x, np.float64)
    y = np.empty_like(x)
    lib().orc_gelu_f64(x.ravel(), y.ravel(), x.size)
    return y


def gelu_grad_f64(x):
    x = _c(x, np.float64)
    y = np.empty_like(x)
    lib().orc_gelu_grad_f64(x.ravel(), y.ravel(), x.size)
    return y


# ---------------------------------------------------------------- reductions
def colsum_f64(x):
    """reduce_sum/launcher.cu:140-155 (keep-lastdim column sum), fp64."""
    x = _c(x, np.float32)
    M, N = int(np.prod(x.shape[:-1])), x.shape[-1]
    out = np.empty(N, np.float64)
    lib().orc_colsum_f64(x.ravel(), out, M, N)
    return out


def softmax_rows_f64(x, want_y=True):
    x = _c(x, np.float32)
    R, C = int(np.prod(x.shape[:-1])), x.shape[-1]
    y = np.empty((R, C), np.float64) if want_y else None
    mx, sx = np.empty(R, np.float64), np.empty(R, np.float64)
    lib().orc_softmax_rows_f64(x.ravel(), _ptr(y), _ptr(mx), _ptr(sx), R, C)
    return y, mx, sx


def softmax_xent_f64(z, labels):
    z = _c(z, np.float32)
    B, C = z.shape
    labels = _c(labels, np.int32)
    dz = np.empty((B, C), np.float64)
    am = np.empty(B, np.int32)
    rl = np.empty(B, np.float64)
    loss = lib().orc_softmax_xent_f64(z, labels, dz, am, rl, B, C)
    return loss, dz, am, rl


# ---------------------------------------------------------------- gemm
def gemm_f64(A, B, transA=False, transB=False):
    """C = op(A) op(B) in fp64 on fp32-stored inputs (gemm/launcher.cu:98-148 views)."""
    A, B = _c(A, np.float32), _c(B, np.float32)
    ars, acs = (A.shape[1], 1) if not transA else (1, A.shape[1])
    M, K = (A.shape[0], A.shape[1]) if not transA else (A.shape[1], A.shape[0])
    brs, bcs = (B.shape[1], 1) if not transB else (1, B.shape[1])
    N = B.shape[1] if not transB else B.shape[0]
    C = np.empty((M, N), np.float64)
    lib().orc_gemm_f64(A.ravel(), ars, acs, B.ravel(), brs, bcs, C, M, N, K)
    return C


def gemm_ref_f32(A, B, transA=False, transB=False, rows=None):
    """gemm/launcher.cu:155-172: per-output sequential-k fp32 (reference algorithm)."""
    A, B = _c(A, np.float32), _c(B, np.float32)
    ars, acs = (A.shape[1], 1) if not transA else (1, A.shape[1])
    M, K = (A.shape[0], A.shape[1]) if not transA else (A.shape[1], A.shape[0])
    brs, bcs = (B.shape[1], 1) if not transB else (1, B.shape[1])
    N = B.shape[1] if not transB else B.shape[0]
    r0, r1 = (0, M) if rows is None else rows
    C = np.zeros((M, N), np.float32)
    lib().orc_gemm_ref_f32(A.ravel(), ars, acs, B.ravel(), brs, bcs, C.ravel(), N, r0, r1, N, K)
    return C


# ---------------------------------------------------------------- metrics
# ---------------------------------------------------------------- LayerNorm
def layernorm_fwd_f64(x, gamma=None, beta=None, eps=1e-5):
    """layernorm/launcher.cu:128-216 (layernorm_fwd_*_kernel): per row mean,
    biased variance, rstd = 1/sqrt(var + eps), y = (x - mean) rstd [* gamma +
    beta].  fp64, on the stored inputs."""
    x = np.asarray(x, np.float64)
    mu = x.mean(axis=1)
    var = ((x - mu[:, None]) ** 2).mean(axis=1)
    rs = 1.0 / np.sqrt(var + eps)
    y = (x - mu[:, None]) * rs[:, None]
    if gamma is not None:
        y = y * np.asarray(gamma, np.float64)[None, :] + np.asarray(beta, np.float64)[None, :]
    return y, mu, rs


def layernorm_bwd_f64(x, dy, mean, rstd, gamma=None):
    """layernorm/launcher.cu:221-371 (bwd_dx and bwd_dg_db kernels):
    dyh = dy * gamma, xhat = (x - mean) rstd,
    dx = (N dyh - sum(dyh) - xhat sum(dyh xhat)) rstd / N,
    dgamma = sum_m dy xhat, dbeta = sum_m dy (None without gamma)."""
    x, dy = np.asarray(x, np.float64), np.asarray(dy, np.float64)
    mean, rstd = np.asarray(mean, np.float64), np.asarray(rstd, np.float64)
    N = x.shape[1]
    xh = (x - mean[:, None]) * rstd[:, None]
    dyh = dy if gamma is None else dy * np.asarray(gamma, np.float64)[None, :]
    s1 = dyh.sum(axis=1, keepdims=True)
    s2 = (dyh * xh).sum(axis=1, keepdims=True)
    dx = (N * dyh - s1 - xh * s2) * (rstd[:, None] / N)
    if gamma is None:
        return dx, None, None
    return dx, (dy * xh).sum(axis=0), dy.sum(axis=0)


# ---------------------------------------------------------------- BatchNorm (NCHW)
def batchnorm_fwd_train_f64(x, gamma=None, beta=None, eps=1e-5):
    """batchnorm/launcher.cu:113-188,402-440 (training): per channel batch
    mean and biased variance over N, H, W; rstd = 1/sqrt(var + eps);
    y = (x - mean) rstd [* gamma + beta].  Returns (y, mean, rstd)."""
    x = np.asarray(x, np.float64)
    mu = x.mean(axis=(0, 2, 3))
    var = ((x - mu[None, :, None, None]) ** 2).mean(axis=(0, 2, 3))
    rs = 1.0 / np.sqrt(var + eps)
    y = (x - mu[None, :, None, None]) * rs[None, :, None, None]
    if gamma is not None:
        y = y * np.asarray(gamma, np.float64)[None, :, None, None] + \
            np.asarray(beta, np.float64)[None, :, None, None]
    return y, mu, rs


def batchnorm_fwd_infer_f64(x, rmean, rvar, gamma=None, beta=None, eps=1e-5):
    """batchnorm/launcher.cu:190-222 (bn_infer_apply_f16): running statistics."""
    x = np.asarray(x, np.float64)
    rs = 1.0 / np.sqrt(np.asarray(rvar, np.float64) + eps)
    y = (x - np.asarray(rmean, np.float64)[None, :, None, None]) * rs[None, :, None, None]
    if gamma is not None:
        y = y * np.asarray(gamma, np.float64)[None, :, None, None] + \
            np.asarray(beta, np.float64)[None, :, None, None]
    return y


def batchnorm_bwd_f64(x, dy, gamma, mean, rstd):
    """batchnorm/launcher.cu:224-290,528-590 (affine training backward):
    dbeta = sum dy, dgamma = sum dy xhat,
    dx = (NHW dy - dbeta - xhat dgamma) gamma rstd / NHW."""
    x, dy = np.asarray(x, np.float64), np.asarray(dy, np.float64)
    mean, rstd = np.asarray(mean, np.float64), np.asarray(rstd, np.float64)
    g = np.asarray(gamma, np.float64)
    cnt = x.shape[0] * x.shape[2] * x.shape[3]
    xh = (x - mean[None, :, None, None]) * rstd[None, :, None, None]
    s1 = dy.sum(axis=(0, 2, 3))
    s2 = (dy * xh).sum(axis=(0, 2, 3))
    dx = (cnt * dy - s1[None, :, None, None] - xh * s2[None, :, None, None]) * \
        (g * rstd / cnt)[None, :, None, None]
    return dx, s2, s1


def rel_err(y, r) -> float:
    """Normwise relative error max|y - r| / max(max|r|, 1e-30)."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.max(np.abs(y - r)) / max(float(np.max(np.abs(r))), 1e-30))


def threads() -> int:
    return int(lib().orc_threads())


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))
