"""The direct column-sum entry point aicf_reduce_sum_lastdim_f32 (the C-ABI
counterpart of the reference's reduce_sum/api.hpp:6, implemented at
reduce_sum/launcher.cu:494-503: dB[n] = sum_m dY[m, n] over a row-major
[M, N] fp32 matrix) called through the C-ABI with ctypes, against the fp64
column sum of the oracle: at the shapes of the reference probe
(v2_reduce_sum_probe.py:24-75: 128 x 64 from seed 0, 257 x 64), ragged
shapes, one row, one column, and the step's 8192 x 4096.  The host-side
rejections (M or N not positive, null pointers) need no GPU."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from aicf_cuda import abi


@pytest.fixture(scope="module")
def lib():
    return abi.load()


def _call(lib, dY, dB, M, N, stream):
    return lib.aicf_reduce_sum_lastdim_f32(ctypes.c_void_p(dY), ctypes.c_void_p(dB), M, N, ctypes.c_void_p(stream))


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,seed", [(128, 64, 0), (257, 64, 1), (1, 1, 2), (1, 4097, 3), (3000, 1, 4),
                                      (1000, 333, 5), (4097, 520, 6), (8192, 4096, 7)])
def test_reduce_sum_lastdim_f32_against_oracle(lib, M, N, seed):
    import torch

    import oracle as orc  # test infrastructure

    print(f"[reduce_api] M={M} N={N} seed={seed}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    dY = torch.randn((M, N), device="cuda", generator=g)
    dB = torch.full((N,), float("nan"), device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    st = _call(lib, dY.data_ptr(), dB.data_ptr(), M, N, s)
    assert st == abi.STATUS_OK, lib.aicf_last_error()
    torch.cuda.synchronize()
    ref = orc.colsum_f64(dY.cpu().numpy())
    got = dB.cpu().numpy()
    assert np.isfinite(got).all()
    assert orc.rel_err(got, ref) < 1e-5
    # the result is reproducible (fixed summation order)
    dB2 = torch.full((N,), float("nan"), device="cuda")
    assert _call(lib, dY.data_ptr(), dB2.data_ptr(), M, N, s) == abi.STATUS_OK
    torch.cuda.synchronize()
    assert torch.equal(dB, dB2)


@pytest.mark.gpu
def test_reduce_sum_lastdim_f32_runs_on_the_given_stream(lib):
    """The launch goes on the stream passed in: a sum queued on a side
    stream behind a fill of the input sees the filled values."""
    import torch

    side = torch.cuda.Stream()
    dY = torch.zeros((512, 256), device="cuda")
    dB = torch.empty(256, device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        dY.fill_(0.5)
        assert _call(lib, dY.data_ptr(), dB.data_ptr(), 512, 256, side.cuda_stream) == abi.STATUS_OK
    side.synchronize()
    assert torch.equal(dB.cpu(), torch.full((256,), 256.0))


def test_reduce_sum_lastdim_f32_rejects_on_the_host(lib):
    fake = 0x100000
    inv = abi.STATUS_INVALID_ARGUMENT
    assert _call(lib, fake, fake + (1 << 20), 0, 64, 0) == inv
    assert _call(lib, fake, fake + (1 << 20), 64, 0, 0) == inv
    assert _call(lib, fake, fake + (1 << 20), -1, 64, 0) == inv
    assert lib.aicf_reduce_sum_lastdim_f32(None, ctypes.c_void_p(fake), 4, 4, None) == inv
    assert lib.aicf_reduce_sum_lastdim_f32(ctypes.c_void_p(fake), None, 4, 4, None) == inv
