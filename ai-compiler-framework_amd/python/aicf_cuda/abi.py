"""ctypes view of the C-ABI declared in include/aicf_hip.h.

Used by the tests and by callers that want the boundary without pybind.
Struct layouts match include/aicf_hip.h exactly.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libaicf_hip.so"

MAX_RANK = 4
DTYPE_UNKNOWN, DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_I32 = 0, 1, 2, 3, 4
STATUS_OK, STATUS_INVALID_ARGUMENT, STATUS_NOT_IMPLEMENTED, STATUS_INTERNAL = 0, 1, 2, 3


class TensorDesc(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_uint8),
        ("rank", ctypes.c_int32),
        ("shape", ctypes.c_int64 * MAX_RANK),
        ("stride", ctypes.c_int64 * MAX_RANK),
        ("contiguous", ctypes.c_bool),
        ("alignment", ctypes.c_int32),
        ("device", ctypes.c_int32),
    ]


class AttrBlob(ctypes.Structure):
    _fields_ = [("schema_id", ctypes.c_uint32), ("bytes", ctypes.c_uint32), ("data", ctypes.c_void_p)]


# Exported symbols and their signatures (restype, argtypes).
SIGNATURES = {
    "aicf_dispatch_v0": (ctypes.c_int32, [ctypes.c_int32, ctypes.POINTER(TensorDesc), ctypes.c_int32,
                                          ctypes.POINTER(TensorDesc), ctypes.c_int32,
                                          ctypes.POINTER(AttrBlob), ctypes.c_void_p]),
    "aicf_dispatch_by_id_v0": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_char_p,
                                                ctypes.POINTER(TensorDesc), ctypes.c_int32,
                                                ctypes.POINTER(TensorDesc), ctypes.c_int32,
                                                ctypes.POINTER(AttrBlob), ctypes.c_void_p]),
    "aicf_cuda_register_all_kernels": (None, []),
    "aicf_reduce_sum_lastdim_f32": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
                                                     ctypes.c_int32, ctypes.c_void_p]),
    "aicf_diag_mfma_loop": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_uint32,
                                             ctypes.c_void_p]),
    "aicf_diag_mfma_loop_form": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                                  ctypes.c_uint32, ctypes.c_int32, ctypes.c_void_p]),
    "aicf_mse_loss_grad_noalloc": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                    ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                                    ctypes.c_float, ctypes.c_void_p]),
    "aicf_registry_count": (ctypes.c_int32, [ctypes.c_int32]),
    "aicf_registry_kernel_id": (ctypes.c_char_p, [ctypes.c_int32, ctypes.c_int32]),
    "aicf_registry_priority": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_int32]),
    "aicf_registry_schema": (ctypes.c_uint32, [ctypes.c_int32, ctypes.c_int32]),
    "aicf_registry_has": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_char_p]),
    "aicf_status_name": (ctypes.c_char_p, [ctypes.c_int32]),
    "aicf_opkind_name": (ctypes.c_char_p, [ctypes.c_int32]),
    "aicf_graph_begin": (ctypes.c_int32, [ctypes.POINTER(ctypes.c_uint64)]),
    "aicf_graph_end": (ctypes.c_int32, []),
    "aicf_graph_launch": (ctypes.c_int32, [ctypes.c_void_p]),
    "aicf_graph_reset": (ctypes.c_int32, []),
    "aicf_graph_stream": (ctypes.c_uint64, []),
    "aicf_graph_state": (ctypes.c_int32, []),
    "aicf_graph_create": (ctypes.c_int32, [ctypes.POINTER(ctypes.c_uint64)]),
    "aicf_graph_destroy": (ctypes.c_int32, [ctypes.c_uint64]),
    "aicf_graph_begin_h": (ctypes.c_int32, [ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)]),
    "aicf_graph_end_h": (ctypes.c_int32, [ctypes.c_uint64]),
    "aicf_graph_launch_h": (ctypes.c_int32, [ctypes.c_uint64, ctypes.c_void_p]),
    "aicf_graph_reset_h": (ctypes.c_int32, [ctypes.c_uint64]),
    "aicf_graph_stream_h": (ctypes.c_uint64, [ctypes.c_uint64]),
    "aicf_graph_state_h": (ctypes.c_int32, [ctypes.c_uint64]),
    "aicf_graph_updates_h": (ctypes.c_uint64, [ctypes.c_uint64]),
    "aicf_last_error": (ctypes.c_char_p, []),
}

_lib = None


def load() -> ctypes.CDLL:
    """Loads libaicf_hip.so (import torch first in processes that use the GPU)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run ai-compiler-framework_amd/build.py")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def make_desc(data: int, dtype: int, shape, stride=None, contiguous=None) -> TensorDesc:
    """Builds a TensorDesc from a raw pointer (device or fake) and a shape."""
    d = TensorDesc()
    d.data = data
    d.dtype = dtype
    d.rank = len(shape)
    if stride is None:
        stride, acc = [], 1
        for s in reversed(shape):
            stride.insert(0, acc)
            acc *= s
    for i, (s, st) in enumerate(zip(shape, stride)):
        d.shape[i] = s
        d.stride[i] = st
    if contiguous is None:
        exp, acc, contiguous = [], 1, True
        for i in reversed(range(len(shape))):
            if shape[i] != 1 and stride[i] != acc:
                contiguous = False
            acc *= shape[i]
    d.contiguous = bool(contiguous)
    return d


def desc_array(descs):
    arr = (TensorDesc * max(1, len(descs)))()
    for i, d in enumerate(descs):
        arr[i] = d
    return arr


def make_blob(schema_id: int, payload: bytes):
    """Returns (AttrBlob, keepalive buffer)."""
    buf = ctypes.create_string_buffer(payload, len(payload)) if payload else None
    b = AttrBlob()
    b.schema_id = schema_id
    b.bytes = len(payload)
    b.data = ctypes.cast(buf, ctypes.c_void_p) if buf is not None else None
    return b, buf
