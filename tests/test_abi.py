"""C-ABI boundary tests that need no GPU.

The library must load, export every function include/aicf_hip.h declares,
keep the reference's struct layouts and numeric ABI constants, register the
reference's kernel ids with the reference priorities, and map contract
violations to the reference's status codes (registry.cpp:16-64,144-195).
Fake device pointers are used only where the call is rejected before any
HIP call is made.
"""
from __future__ import annotations

import ctypes
import re
import struct
from pathlib import Path

import pytest

from aicf_cuda import abi

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "aicf_hip.h"

OK, INV, NOTIMPL = abi.STATUS_OK, abi.STATUS_INVALID_ARGUMENT, abi.STATUS_NOT_IMPLEMENTED
F32, F16, BF16, I32 = abi.DTYPE_F32, abi.DTYPE_F16, abi.DTYPE_BF16, abi.DTYPE_I32

# register_all.cpp:105-257 of the reference: (OpKind, kernel_id, priority)
REFERENCE_IDS = [
    (4, "reduce_sum_keep_lastdim_f16_v0", 115),
    (4, "reduce_sum_keep_lastdim_f16_to_f32_v0", 110),
    (4, "reduce_sum_keep_lastdim_f32_v0", 100),
    (2, "gemm_f16_tc_wmma_out_f16_v0", 20),
    (2, "gemm_f32_naive_v0", 0),
    (17, "gemm_bias_relu_f16_tc_wmma_out_f16_v0", 20),
    (17, "gemm_bias_relu_f32_naive_v0", 0),
    (3, "bias_add_f16_vec2_v0", 30),
    (3, "bias_add_f16_v0", 20),
    (3, "bias_add_f32_v0", 0),
    (0, "add_f16_vec2_v0", 30),
    (0, "add_f16_v0", 20),
    (0, "add_f32_v0", 0),
    (1, "relu_f16_vec2_v0", 30),
    (1, "relu_f16_v0", 20),
    (1, "relu_f32_v0", 0),
    (5, "mse_grad_f16_v0", 20),
    (5, "mse_grad_f32_v0", 0),
    (6, "relu_bwd_f16_vec2_v0", 30),
    (6, "relu_bwd_f16_v0", 20),
    (6, "relu_bwd_f32_v0", 0),
    (7, "sgd_step_f16_half2_v0", 30),
    (7, "sgd_step_f16_v0", 20),
    (7, "sgd_step_f32_v0", 0),
    (8, "copy_f16_v0", 20),
    (8, "copy_f32_v0", 0),
    (9, "grad_zero_v0", 0),
    (10, "adam_step_f32_v0", 0),
    (11, "step_inc_v0", 0),
    (12, "bias_corr_v0", 0),
    (13, "layernorm_fwd_f16_v0", 10),
    (13, "layernorm_fwd_f32_v0", 0),
    (14, "layernorm_bwd_f16_v0", 10),
    (14, "layernorm_bwd_f32_v0", 0),
    (15, "batchnorm_fwd_f16_v0", 10),
    (16, "batchnorm_bwd_f16_v0", 10),
]
# register_all.cpp:259-290: schema gates (0 = none)
REFERENCE_GATES = {"layernorm_fwd_f16_v0": int.from_bytes(b"LNEP", "little"),
                   "layernorm_fwd_f32_v0": int.from_bytes(b"LNEP", "little"),
                   "layernorm_bwd_f16_v0": 0, "layernorm_bwd_f32_v0": 0,
                   "batchnorm_fwd_f16_v0": int.from_bytes(b"BNEP", "little"),
                   "batchnorm_bwd_f16_v0": 0}

FAKE = 0x100000  # never dereferenced: every call below is rejected on the host


@pytest.fixture(scope="module")
def lib():
    return abi.load()


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aicf_\w+)\s*\(", text)))


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 18
    for n in names:
        assert hasattr(lib, n), f"{n} declared in aicf_hip.h but not exported"
    assert set(names) == set(abi.SIGNATURES), "abi.py signature table out of date"


def test_struct_layout_matches_reference():
    # tensor_desc.hpp:88-106: void*, uint8 dtype, int32 rank union,
    # int64 shape[4], int64 stride[4], bool contiguous, int32 alignment, int32 device
    assert ctypes.sizeof(abi.TensorDesc) == 96
    assert abi.TensorDesc.rank.offset == 12
    assert abi.TensorDesc.shape.offset == 16
    assert abi.TensorDesc.stride.offset == 48
    assert abi.TensorDesc.contiguous.offset == 80
    assert abi.TensorDesc.device.offset == 88
    assert ctypes.sizeof(abi.AttrBlob) == 16


def test_header_constants():
    text = HEADER.read_text()
    consts = dict(re.findall(r"#define (AICF_\w+) (0x[0-9A-Fa-f]+|\d+)", text))
    v = {k: int(x.rstrip("u"), 0) for k, x in consts.items()}
    # fourcc schema ids (numeric ABI, exec.py:203-217 and the launchers)
    assert v["AICF_SCHEMA_ADAM"] == int.from_bytes(b"ADAM", "little")
    assert v["AICF_SCHEMA_GEPI"] == int.from_bytes(b"GEPI", "little")
    assert v["AICF_SCHEMA_GEMM"] == int.from_bytes(b"GEMM", "big")
    assert v["AICF_SCHEMA_GPEL"] == int.from_bytes(b"GPEL", "big")
    assert v["AICF_SCHEMA_RSUM"] == int.from_bytes(b"RSUM", "big")
    assert v["AICF_SCHEMA_BCOR"] == int.from_bytes(b"BCOR", "little")
    assert v["AICF_SCHEMA_MSEG"] == int.from_bytes(b"MSEG", "little")
    assert v["AICF_SCHEMA_SGDS"] == int.from_bytes(b"SGDS", "little")
    assert v["AICF_SCHEMA_BADD"] == int.from_bytes(b"BADD", "little")
    assert v["AICF_OP_GEMM_EPILOGUE"] == 17 and v["AICF_OP_ADAM_STEP"] == 10
    assert v["AICF_DTYPE_BF16"] == 3 and v["AICF_DTYPE_I32"] == 4


def test_reference_kernel_ids_and_priorities(lib):
    for kind, kid, prio in REFERENCE_IDS:
        assert lib.aicf_registry_has(kind, kid.encode()) == 1, kid
        n = lib.aicf_registry_count(kind)
        ids = [lib.aicf_registry_kernel_id(kind, i).decode() for i in range(n)]
        prios = [lib.aicf_registry_priority(kind, i) for i in range(n)]
        assert prios[ids.index(kid)] == prio, kid
        assert prios == sorted(prios, reverse=True), f"kind {kind} not in priority order"
    for kind, kid, _ in REFERENCE_IDS:
        if kid in REFERENCE_GATES:
            n = lib.aicf_registry_count(kind)
            ids = [lib.aicf_registry_kernel_id(kind, i).decode() for i in range(n)]
            assert lib.aicf_registry_schema(kind, ids.index(kid)) == REFERENCE_GATES[kid], kid
    # reference schema gates: Adam requires ADAM, BiasCorr requires BCOR
    assert lib.aicf_registry_schema(10, [lib.aicf_registry_kernel_id(10, i).decode()
                                         for i in range(2)].index("adam_step_f32_v0")) == \
        int.from_bytes(b"ADAM", "little")
    assert lib.aicf_registry_schema(12, 0) == int.from_bytes(b"BCOR", "little")


def test_names(lib):
    assert lib.aicf_status_name(0) == b"Ok"
    assert lib.aicf_status_name(2) == b"NotImplemented"
    assert lib.aicf_opkind_name(17) == b"gemm_epilogue"
    assert lib.aicf_opkind_name(99) == b"unknown"


def _call(lib, kind, ins, outs, schema=0, payload=b"", kid=None):
    ia, oa = abi.desc_array(ins), abi.desc_array(outs)
    blob, keep = abi.make_blob(schema, payload)
    bp = ctypes.byref(blob) if (schema or payload) else None
    if kid is None:
        return lib.aicf_dispatch_v0(kind, ia, len(ins), oa, len(outs), bp, None)
    return lib.aicf_dispatch_by_id_v0(kind, kid.encode() if kid else b"", ia, len(ins), oa,
                                      len(outs), bp, None)


def d(shape, dtype=F32, ptr=FAKE, stride=None, contiguous=None):
    return abi.make_desc(ptr, dtype, shape, stride, contiguous)


def test_dispatch_neg_cases(lib):
    # op_call path: no supported variant -> NotImplemented (registry.cpp:181)
    # v2_relu_probe NEG: dtype mismatch, shape mismatch
    assert _call(lib, 1, [d((8, 7))], [d((8, 7), F16)]) == NOTIMPL
    assert _call(lib, 1, [d((8, 7))], [d((8, 8))]) == NOTIMPL
    # v2_add_probe NEG
    assert _call(lib, 0, [d((8, 7)), d((8, 8))], [d((8, 7))]) == NOTIMPL
    assert _call(lib, 0, [d((8, 7)), d((8, 7), F16)], [d((8, 7))]) == NOTIMPL
    # v2_copy_probe / v2_grad_zero_probe NEG
    assert _call(lib, 8, [d((128,))], [d((128,), F16)]) == NOTIMPL
    assert _call(lib, 8, [d((128,))], [d((256,))]) == NOTIMPL
    assert _call(lib, 9, [d((128,))], [d((128,), F16)]) == NOTIMPL
    assert _call(lib, 9, [d((128,))], [d((129,))]) == NOTIMPL
    # v2_adam_step_probe NEG: f16 dtype; G aliasing Pout
    sc = d((), F32)
    adam = int.from_bytes(b"ADAM", "little")
    pay = struct.pack("<ffff", 1e-3, 0.9, 0.999, 1e-8)
    h = [d((128,), F16, FAKE + i * 4096) for i in range(4)]
    assert _call(lib, 10, h + [sc, sc], [d((128,), F16, FAKE + 8192 * 4)] * 3, adam, pay) == NOTIMPL
    P, G, M, V = (d((128,), F32, FAKE + i * 4096) for i in range(4))
    assert _call(lib, 10, [P, G, M, V, sc, sc], [G, M, V], adam, pay) == NOTIMPL
    # Adam without the ADAM schema never passes the gate
    assert _call(lib, 10, [P, G, M, V, sc, sc], [P, M, V]) == NOTIMPL
    assert _call(lib, 10, [P, G, M, V, sc, sc], [P, M, V], kid="adam_step_f32_v0") == INV
    # v2_gemm_probe NEG: wrong C shape
    assert _call(lib, 2, [d((64, 48)), d((48, 80))], [d((64, 81))]) == NOTIMPL
    # v2_gemm_epilogue_probe NEG: bias length; dtype mix
    assert _call(lib, 17, [d((64, 48)), d((48, 80)), d((79,))], [d((64, 80))]) == NOTIMPL
    assert _call(lib, 17, [d((64, 48)), d((48, 80), F16), d((80,))], [d((64, 80))]) == NOTIMPL
    # v2_reduce_sum_probe NEG: axis = 1 under RSUM
    rsum = int.from_bytes(b"RSUM", "big")
    assert _call(lib, 4, [d((128, 64))], [d((64,))], rsum, struct.pack("<q", 1)) == NOTIMPL
    # v2_bias_add_probe NEG: axis = 0; bias length
    badd = int.from_bytes(b"BADD", "little")
    assert _call(lib, 3, [d((64, 256)), d((256,))], [d((64, 256))], badd, struct.pack("<q", 0)) == NOTIMPL
    assert _call(lib, 3, [d((64, 256)), d((255,))], [d((64, 256))]) == NOTIMPL
    # v2_mse_grad_probe NEG: shape; dtype
    assert _call(lib, 5, [d((64, 256)), d((64, 255))], [d((64, 256))]) == NOTIMPL
    assert _call(lib, 5, [d((64, 256)), d((64, 256), F16)], [d((64, 256))]) == NOTIMPL
    # v2_step_inc_probe NEG: dtype; shape
    assert _call(lib, 11, [d((4,), F32)], [d((4,), F32)]) == NOTIMPL
    assert _call(lib, 11, [d((4,), I32)], [d((5,), I32)]) == NOTIMPL
    # v2_biascorr_probe NEG: wrong schema; float step
    bcor = int.from_bytes(b"BCOR", "little")
    st = d((), I32)
    assert _call(lib, 12, [st], [sc, sc], adam, struct.pack("<ff", 0.9, 0.999)) == NOTIMPL
    assert _call(lib, 12, [d((), F32)], [sc, sc], bcor, struct.pack("<ff", 0.9, 0.999)) == NOTIMPL
    # v2_sgd_step_probe NEG: dtype; shape; O aliasing G (rejected in launch, before HIP)
    assert _call(lib, 7, [d((128,)), d((128,), F16)], [d((128,))]) == NOTIMPL
    assert _call(lib, 7, [d((128,)), d((127,))], [d((128,))]) == NOTIMPL
    Pp, Gp = d((128,), F32, FAKE), d((128,), F32, FAKE + 4096)
    assert _call(lib, 7, [Pp, Gp], [Gp]) == INV


def test_dgelu_colsum_supported_only_where_it_runs(lib):
    """GEPI kind 6 (dGELU + column sums) is supported exactly where its
    bf16 256 x 256-tile path runs: M and N multiples of 256, K of 64, a
    workspace of at least M/256 rows.  Everything else is refused by
    supported() (no variant for op_call; INVALID_ARGUMENT by id), on the
    host, before any launch."""
    gepi = int.from_bytes(b"GEPI", "little")
    pay = struct.pack("<iii", 0, 0, 6)
    kid = "gemm_epilogue_bf16_mfma_v0"

    def call(M, N, K, P, by_id):
        ins = [d((M, K), BF16, FAKE), d((K, N), BF16, FAKE + (1 << 24)), d((M, N), BF16, FAKE + (2 << 24))]
        outs = [d((M, N), BF16, FAKE + (3 << 24)), d((N,), F32, FAKE + (4 << 24)),
                d((P, N), F32, FAKE + (5 << 24))]
        return _call(lib, 17, ins, outs, gepi, pay, kid=kid if by_id else None)

    for M, N, K, P in ((384, 256, 64, 2), (512, 320, 64, 2), (512, 256, 96, 2), (512, 256, 64, 1),
                       (128, 256, 64, 1), (128, 256, 64, 0)):
        assert call(M, N, K, P, True) == INV, (M, N, K, P)
        assert call(M, N, K, P, False) == NOTIMPL, (M, N, K, P)
    # an f16 call with kind 6 has no supporting variant either
    ins = [d((512, 64), F16), d((64, 256), F16), d((512, 256), F16)]
    outs = [d((512, 256), F16), d((256,), F32), d((2, 256), F32)]
    assert _call(lib, 17, ins, outs, gepi, pay) == NOTIMPL


def test_zero_size_inputs_follow_the_reference(lib):
    """Zero-element tensors get the reference's statuses, decided on the host:
    copy, grad_zero and Adam accept n = 0 and return Ok without a launch
    (copy/launcher.cu:81,110; grad_zero/launcher.cu:79,107;
    adam_step/launcher.cu:174-175,211-212); the other ops require a positive
    size, so no variant supports the call (relu/launcher.cu:131-132,
    add/launcher.cu:108, bias_add/launcher.cu:142-150,
    reduce_sum/launcher.cu:44-53, mse_grad/launcher.cu:131,
    relu_bwd/launcher.cu:110, sgd_step/launcher.cu:66-70,
    step_inc/launcher.cu:105, gemm/launcher.cu:141)."""
    adam = int.from_bytes(b"ADAM", "little")
    pay = struct.pack("<ffff", 1e-3, 0.9, 0.999, 1e-8)
    sc = d((), F32)
    z = lambda k=0, dt=F32: d((0,), dt, FAKE + k * 4096)  # noqa: E731
    assert _call(lib, 8, [z(0)], [z(1)]) == OK                                   # copy
    assert _call(lib, 9, [z(0)], [z(0)]) == OK                                   # grad_zero
    assert _call(lib, 10, [z(0), z(1), z(2), z(3), sc, sc], [z(0), z(2), z(3)], adam, pay) == OK
    assert _call(lib, 1, [z()], [z()]) == NOTIMPL                                # relu
    assert _call(lib, 0, [z(), z(1)], [z(2)]) == NOTIMPL                         # add
    assert _call(lib, 3, [d((0, 8)), d((8,))], [d((0, 8))]) == NOTIMPL          # bias_add
    assert _call(lib, 4, [d((0, 8))], [d((8,))]) == NOTIMPL                     # reduce_sum
    assert _call(lib, 5, [z(), z(1)], [z(2)]) == NOTIMPL                         # mse_grad
    assert _call(lib, 6, [z(), z(1)], [z(2)]) == NOTIMPL                         # relu_bwd
    assert _call(lib, 7, [z(), z(1)], [z()]) == NOTIMPL                          # sgd
    assert _call(lib, 11, [z(0, I32)], [z(0, I32)]) == NOTIMPL                  # step_inc
    assert _call(lib, 2, [d((0, 8)), d((8, 8))], [d((0, 8))]) == NOTIMPL        # gemm


def test_by_id_status_rules(lib):
    P = d((128,))
    # empty id -> InvalidArgument; unknown id -> NotImplemented
    assert _call(lib, 1, [P], [P], kid="") == INV
    assert _call(lib, 1, [P], [P], kid="no_such_kernel_v0") == NOTIMPL
    # LayerNorm fwd is schema-gated (LNEP): schema 0 by id -> InvalidArgument,
    # by op_call -> no eligible variant -> NotImplemented (registry.cpp:35-38,181-190)
    assert _call(lib, 13, [P], [P], kid="layernorm_fwd_f32_v0") == INV
    assert _call(lib, 13, [P], [P]) == NOTIMPL
    lnep = int.from_bytes(b"LNEP", "little")
    # right schema, wrong rank (v2_layernorm_probe NEG rank) -> unsupported
    x3 = d((2, 3, 4))
    assert _call(lib, 13, [x3], [x3, d((2,)), d((2,))], lnep, struct.pack("<f", 1e-5)) == NOTIMPL
    assert _call(lib, 13, [x3], [x3, d((2,)), d((2,))], lnep, struct.pack("<f", 1e-5),
                 kid="layernorm_fwd_f32_v0") == INV
    # BatchNorm: wrong rank -> NotImplemented; wrong schema -> NotImplemented (v2_batchnorm_probe)
    bnep = int.from_bytes(b"BNEP", "little")
    x2 = d((8, 16), F16)
    assert _call(lib, 15, [x2], [x2], bnep, struct.pack("<fI", 1e-5, 1)) == NOTIMPL
    x4 = d((8, 16, 8, 8), F16)
    assert _call(lib, 15, [x4, d((16,)), d((16,))], [x4], 0x12345678, b"\x00" * 8) == NOTIMPL
    # unsupported call to an existing id -> InvalidArgument
    assert _call(lib, 1, [d((8, 7))], [d((8, 8))], kid="relu_f32_v0") == INV
    # kid registered under another kind -> NotImplemented
    assert _call(lib, 0, [P], [P], kid="relu_f32_v0") == NOTIMPL
    # bad kind value
    assert _call(lib, 99, [P], [P]) == INV
    assert lib.aicf_dispatch_v0(1, None, 1, None, 0, None, None) == INV


def test_graph_misuse_is_rejected_without_a_gpu(lib):
    # bindings.cpp:507-509,529-531 of the reference: end without begin and
    # launch before capture are errors
    assert lib.aicf_graph_state() == 0
    assert lib.aicf_graph_end() == INV
    assert b"not capturing" in lib.aicf_last_error()
    assert lib.aicf_graph_launch(None) == INV
    assert b"no captured graph" in lib.aicf_last_error()
    assert lib.aicf_graph_stream() == 0


def test_graph_handles_without_a_gpu(lib):
    """Handle bookkeeping needs no device: create / query / misuse / destroy."""
    import ctypes

    h = ctypes.c_uint64(0)
    assert lib.aicf_graph_create(ctypes.byref(h)) == 0 and h.value != 0
    h2 = ctypes.c_uint64(0)
    assert lib.aicf_graph_create(ctypes.byref(h2)) == 0 and h2.value not in (0, h.value)
    hv = ctypes.c_uint64(h.value)
    assert lib.aicf_graph_state_h(hv) == 0
    assert lib.aicf_graph_stream_h(hv) == 0
    assert lib.aicf_graph_updates_h(hv) == 0
    assert lib.aicf_graph_end_h(hv) == INV
    assert b"not capturing" in lib.aicf_last_error()
    assert lib.aicf_graph_launch_h(hv, None) == INV
    assert b"no captured graph" in lib.aicf_last_error()
    assert lib.aicf_graph_reset_h(hv) == 0
    assert lib.aicf_graph_destroy(ctypes.c_uint64(0)) == INV
    assert lib.aicf_graph_destroy(hv) == 0
    assert lib.aicf_graph_state_h(hv) == -1
    assert lib.aicf_graph_destroy(hv) == INV
    assert b"unknown graph handle" in lib.aicf_last_error()
    assert lib.aicf_graph_launch_h(hv, None) == INV
    assert lib.aicf_graph_destroy(ctypes.c_uint64(h2.value)) == 0
    # handle 0 is the process-wide graph and always exists
    assert lib.aicf_graph_state_h(ctypes.c_uint64(0)) == lib.aicf_graph_state()
