"""The no-allocation MSE loss + gradient entry point
(aicf_mse_loss_grad_noalloc, include/aicf_hip.h) called through the C-ABI,
against the existing entry point it is a variant of (kernel
mse_loss_grad_v0 through aicf_dispatch_by_id_v0, with a partials buffer
the caller allocates): dPred and the loss bit for bit, on two calls in a
row, the second with a smaller input, for bf16 and fp32 predictions and for
the one-shot (n % 8 == 0) and strided pass-1 paths.  The host-side
rejections need no GPU."""
from __future__ import annotations

import ctypes
import struct

import numpy as np
import pytest

from aicf_cuda import abi

MSEG = int.from_bytes(b"MSEG", "little")


@pytest.fixture(scope="module")
def lib():
    return abi.load()


def _noalloc(lib, p, t, d, loss, scale, stream):
    import torch

    dtype = abi.DTYPE_BF16 if p.dtype == torch.bfloat16 else abi.DTYPE_F32
    return lib.aicf_mse_loss_grad_noalloc(ctypes.c_void_p(p.data_ptr()), ctypes.c_void_p(t.data_ptr()),
                                          ctypes.c_void_p(d.data_ptr()), ctypes.c_void_p(loss.data_ptr()),
                                          p.numel(), dtype, scale, ctypes.c_void_p(stream))


def _desc(x):
    import torch

    code = {torch.float32: abi.DTYPE_F32, torch.bfloat16: abi.DTYPE_BF16}[x.dtype]
    return abi.make_desc(x.data_ptr(), code, tuple(x.shape), tuple(x.stride()), x.is_contiguous())


def _existing(lib, p, t, d, loss, ws, scale, stream):
    ins = abi.desc_array([_desc(p), _desc(t)])
    outs = abi.desc_array([_desc(d), _desc(loss), _desc(ws)])
    blob, keep = abi.make_blob(MSEG, struct.pack("<f", scale))
    return lib.aicf_dispatch_by_id_v0(5, b"mse_loss_grad_v0", ins, 2, outs, 3, ctypes.byref(blob),
                                      ctypes.c_void_p(stream))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("sizes", [((8192, 4096), (1000, 64)), ((4099, 37), (256, 3))])
def test_noalloc_matches_the_allocating_entry_point(lib, dtype, sizes):
    import torch

    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    s = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device="cuda")
    g.manual_seed(sum(sizes[0]))
    for shape in sizes:  # second call smaller than the first
        n = shape[0] * shape[1]
        print(f"[noalloc] dtype={dtype} shape={shape}", flush=True)
        p = torch.randn(shape, device="cuda", generator=g).to(tdt)
        t = torch.randn(shape, device="cuda", generator=g)
        scale = 2.0 / n
        d0, l0 = torch.full_like(p, float("nan")), torch.full((), float("nan"), device="cuda")
        ws = torch.empty(max(1024, -(-n // 2048)), device="cuda")
        assert _existing(lib, p, t, d0, l0, ws, scale, s) == abi.STATUS_OK
        d1, l1 = torch.full_like(p, float("nan")), torch.full((), float("nan"), device="cuda")
        st = _noalloc(lib, p, t, d1, l1, scale, s)
        assert st == abi.STATUS_OK, lib.aicf_last_error()
        torch.cuda.synchronize()
        assert torch.equal(d0.view(torch.int16) if dtype == "bf16" else d0.view(torch.int32),
                           d1.view(torch.int16) if dtype == "bf16" else d1.view(torch.int32))
        assert torch.equal(l0, l1) and torch.isfinite(l1)
        ref = float(((p.double() - t.double()) ** 2).mean())
        assert abs(float(l1) - ref) <= 1e-5 * ref


def test_noalloc_rejects_on_the_host(lib):
    """Beyond the 2^27-element maximum, a foreign dtype, a null pointer or a
    misaligned pointer: INVALID_ARGUMENT with a message, before any device
    call (fake addresses are never touched)."""
    fake = ctypes.c_void_p(0x100000)
    f = lib.aicf_mse_loss_grad_noalloc
    assert f(fake, fake, fake, fake, (1 << 27) + 1, abi.DTYPE_F32, 1.0, None) == abi.STATUS_INVALID_ARGUMENT
    assert b"134217728" in lib.aicf_last_error()
    assert f(fake, fake, fake, fake, 64, abi.DTYPE_F16, 1.0, None) == abi.STATUS_INVALID_ARGUMENT
    assert f(None, fake, fake, fake, 64, abi.DTYPE_F32, 1.0, None) == abi.STATUS_INVALID_ARGUMENT
    assert f(fake, fake, fake, fake, 0, abi.DTYPE_F32, 1.0, None) == abi.STATUS_INVALID_ARGUMENT
    odd = ctypes.c_void_p(0x100004)
    assert f(odd, fake, fake, fake, 64, abi.DTYPE_F32, 1.0, None) == abi.STATUS_INVALID_ARGUMENT
    assert b"misaligned" in lib.aicf_last_error()
