"""Randomised GEMM parity sweep: 48 seeded draws of shape (including 1, odd
sizes and sizes just past a tile boundary), operand layouts (transA,
transB), dtype (fp32, f16, bf16) and epilogue (plain, bias, bias+ReLU,
bias+GELU), each dispatched by the registry (op_call, as the reference's
executor does without kernel ids) and compared with the fp64 oracle product
of the same stored operands: max error over the largest pre-activation
magnitude <= 1e-4 (fp32), 2e-3 (f16 out), 1e-2 (bf16 out)."""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

import oracle as orc

pytestmark = pytest.mark.gpu

GEPI = int.from_bytes(b"GEPI", "little")
SIZES_MN = [1, 7, 64, 129, 256, 384, 520, 1000]
SIZES_K = [1, 3, 16, 64, 100, 256, 520, 1100]
TOL = {"f32": 1e-4, "f16": 2e-3, "bf16": 1e-2}


def _draws(n=48, seed=2024):
    r = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        dt = ["f32", "f16", "bf16"][int(r.integers(3))]
        epis = ["plain", "bias", "relu"] + (["gelu"] if dt != "f16" else [])
        out.append((int(r.choice(SIZES_MN)), int(r.choice(SIZES_MN)), int(r.choice(SIZES_K)),
                    bool(r.integers(2)), bool(r.integers(2)), dt, epis[int(r.integers(len(epis)))]))
    return out


def _dev(a, dt):
    """float32 numpy -> device tensor of dtype dt, and the values it holds."""
    if dt == "f32":
        return torch.from_numpy(a).cuda(), a.astype(np.float64)
    if dt == "f16":
        h = a.astype(np.float16)
        return torch.from_numpy(h.view(np.int16)).view(torch.float16).cuda(), h.astype(np.float64)
    bits = orc.bf16_bits_from_f32(a)
    return (torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda(),
            orc.bf16_bits_to_f32(bits).reshape(a.shape).astype(np.float64))


def _host(t):
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return orc.bf16_bits_to_f32(t.view(torch.int16).numpy().view(np.uint16)).reshape(t.shape).astype(np.float64)
    return t.float().numpy().astype(np.float64)


@pytest.mark.parametrize("M,N,K,ta,tb,dt,epi", _draws())
def test_gemm_random_shapes_layouts_dtypes_epilogues(C, M, N, K, ta, tb, dt, epi):
    r = np.random.default_rng(M * 1000003 + N * 1009 + K)
    s = 1.0 / np.sqrt(K)
    A32 = r.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B32 = r.uniform(-s, s, (N, K) if tb else (K, N)).astype(np.float32)
    A, Ah = _dev(A32, dt)
    B, Bh = _dev(B32, dt)
    ref = z = orc.gemm_f64(Ah, Bh, ta, tb)
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dt]
    out = torch.empty((M, N), dtype=tdt, device="cuda")
    if epi == "plain":
        C.op_call(int(C.OpKind.Gemm), [A, B], [out], 0, struct.pack("<ii", ta, tb), 0)
    else:
        bias = r.uniform(-s, s, N).astype(np.float32)
        kind = {"bias": 1, "relu": 0, "gelu": 3}[epi]
        C.op_call(int(C.OpKind.GemmEpilogue), [A, B, torch.from_numpy(bias).cuda()], [out], GEPI,
                  struct.pack("<iii", ta, tb, kind), 0)
        ref = z = ref + bias.astype(np.float64)[None, :]
        if epi == "relu":
            ref = np.maximum(ref, 0.0)
        elif epi == "gelu":
            ref = orc.gelu_f64(ref)
    torch.cuda.synchronize()
    got = _host(out)
    assert np.isfinite(got).all()
    # normwise against the pre-activation's scale (a ReLU output may be all zero)
    err = np.abs(got - ref).max() / max(np.abs(z).max(), 1e-30)
    assert err < TOL[dt], (M, N, K, ta, tb, dt, epi, err)
