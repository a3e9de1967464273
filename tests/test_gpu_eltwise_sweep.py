"""Randomised parity sweep of the streaming element-wise and optimizer ops:
48 seeded draws of op, dtype, length (1, odd lengths, lengths around the 2-,
4- and 8-element vector widths) and base offset (0, or 1 element: a
misaligned view that must take the scalar path), bit-exact against the
oracle's restatements of the reference kernels."""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

import oracle as orc

pytestmark = pytest.mark.gpu

ADAM = int.from_bytes(b"ADAM", "little")
MSEG = int.from_bytes(b"MSEG", "little")
SGDS = int.from_bytes(b"SGDS", "little")
LENS = [1, 2, 3, 5, 7, 8, 9, 15, 16, 17, 31, 33, 127, 1000, 4097, 65537]
OPS = ["add", "relu", "relu_bwd", "copy", "grad_zero", "bias_add", "mse_grad", "sgd", "adamw"]


def _draws(n=48, seed=11):
    r = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        op = OPS[int(r.integers(len(OPS)))]
        dt = "f32" if op == "adamw" else ["f32", "f16"][int(r.integers(2))]
        out.append((op, dt, int(r.choice(LENS)), int(r.integers(2))))
    return out


def _view(a: np.ndarray, off: int) -> torch.Tensor:
    """Device copy of `a` starting `off` elements into a larger buffer."""
    flat = a.reshape(-1)
    base = torch.zeros(flat.size + 8, dtype=torch.int16 if a.dtype == np.uint16 else torch.float32,
                       device="cuda")
    src = torch.from_numpy(flat.view(np.int16) if a.dtype == np.uint16 else flat).cuda()
    base[off:off + flat.size].copy_(src)
    t = base[off:off + flat.size].view(a.shape)
    return t.view(torch.float16) if a.dtype == np.uint16 else t


def _host(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.float16 else t.numpy()


@pytest.mark.parametrize("op,dt,n,off", _draws())
def test_eltwise_random_lengths_and_offsets(C, op, dt, n, off):
    r = np.random.default_rng(n * 31 + off + OPS.index(op))
    f = lambda *s: r.standard_normal(s).astype(np.float32)  # noqa: E731
    enc = (lambda x: x) if dt == "f32" else (lambda x: x.astype(np.float16).view(np.uint16))  # noqa: E731
    if op in ("add", "relu_bwd"):
        a, b = enc(f(n)), enc(f(n))
        o = _view(np.zeros_like(a), off)
        kind = int(C.OpKind.EltwiseAdd if op == "add" else C.OpKind.ReluBwd)
        C.op_call(kind, [_view(a, off), _view(b, off)], [o], 0, b"", 0)
        if op == "add":
            ref = orc.add_f32(a, b) if dt == "f32" else orc.add_f16(a, b)
        else:
            ref = orc.relu_bwd_f32(a, b) if dt == "f32" else orc.relu_bwd_f16(a, b)
        assert np.array_equal(_host(o).ravel(), ref)
    elif op in ("relu", "copy"):
        a = enc(f(n))
        o = _view(np.zeros_like(a), off)
        C.op_call(int(C.OpKind.EltwiseRelu if op == "relu" else C.OpKind.Copy), [_view(a, off)], [o], 0, b"", 0)
        ref = (orc.relu_f32(a) if dt == "f32" else orc.relu_f16(a)) if op == "relu" else a.ravel()
        assert np.array_equal(_host(o).ravel(), ref)
    elif op == "grad_zero":
        o = _view(enc(f(n)), off)
        C.op_call(int(C.OpKind.GradZero), [o], [o], 0, b"", 0)
        assert not _host(o).any()
    elif op == "bias_add":
        rows = 3 if n % 3 == 0 and n > 3 else 1
        y, b = enc(f(rows, n // rows)), enc(f(n // rows))
        ty = _view(y, off)
        C.op_call(int(C.OpKind.BiasAdd), [ty, _view(b, off)], [ty], 0, b"", 0)
        ref = orc.bias_add_f32(y, b) if dt == "f32" else orc.bias_add_f16(y, b)
        assert np.array_equal(_host(ty).ravel(), ref)
    elif op == "mse_grad":
        p, t = enc(f(n)), enc(f(n))
        o = _view(np.zeros_like(p), off)
        C.op_call(int(C.OpKind.MseGrad), [_view(p, off), _view(t, off)], [o], MSEG, struct.pack("<f", 0.125), 0)
        if dt == "f32":
            ref = orc.mse_grad_f32(p, t, 0.125)
        else:  # half2 math when the length is even and every pointer 4-byte aligned
            ref = orc.mse_grad_f16(p, t, 0.125, half_math=(n % 2 == 0 and off % 2 == 0))
        assert np.array_equal(_host(o).ravel(), ref)
    elif op == "sgd":
        p, gr = enc(f(n)), enc(f(n))
        tp = _view(p, off)
        C.op_call(int(C.OpKind.SgdStep), [tp, _view(gr, off)], [tp], SGDS, struct.pack("<f", 0.01), 0)
        ref = orc.sgd_f32(p, gr, 0.01) if dt == "f32" else orc.sgd_f16(p, gr, 0.01)
        assert np.array_equal(_host(tp).ravel(), ref)
    else:  # adamw, in place, bf16 shadow, two steps
        P, G = 0.02 * f(n), 1e-3 * f(n)
        tP, tG = _view(P, off), _view(G, off)
        tM, tV = _view(np.zeros(n, np.float32), off), _view(np.zeros(n, np.float32), off)
        Wb = torch.empty(n, dtype=torch.bfloat16, device="cuda")
        step = torch.zeros((), dtype=torch.int32, device="cuda")
        Pc, Mc, Vc = P.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
        for t in (1, 2):
            C.launch_by_id("step_inc_v0", C.OpKind.StepInc, [step], [step])
            C.launch_by_id("adamw_step_f32_v1", C.OpKind.AdamStep, [tP, tG, tM, tV, step], [tP, tM, tV, Wb],
                           ADAM, struct.pack("<fffff", 1e-3, 0.9, 0.999, 1e-8, 0.01))
            Pc, Mc, Vc, Wc = orc.adamw(Pc, G, Mc, Vc, t, 1e-3, 0.9, 0.999, 1e-8, 0.01, shadow=True)
        assert np.array_equal(_host(tP).ravel(), Pc)
        assert np.array_equal(_host(tM).ravel(), Mc)
        assert np.array_equal(_host(tV).ravel(), Vc)
        assert np.array_equal(Wb.cpu().view(torch.int16).numpy().view(np.uint16), Wc)
