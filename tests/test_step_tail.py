"""StageG (the loss and bias tail of the large MSE step) and the host-side
contracts of its two ops, without a GPU: the benchmark step lowers to 12
GEMMs plus mse_colsum and colsum_adamw, every value the unfused tail writes
is still written, the lowering falls back where the partition does not
match, the warmup rewrite reaches both ops, and supported() refuses what the
kernels cannot run before any launch."""
from __future__ import annotations

import struct

import pytest

from aicf_cuda import abi

OK, INV, NOTIMPL = abi.STATUS_OK, abi.STATUS_INVALID_ARGUMENT, abi.STATUS_NOT_IMPLEMENTED
F32, BF16, I32 = abi.DTYPE_F32, abi.DTYPE_BF16, abi.DTYPE_I32
MSCS = int.from_bytes(b"MSCS", "little")
CADW = int.from_bytes(b"CADW", "little")
GEPI = int.from_bytes(b"GEPI", "little")
MSE_COLSUM, COLSUM_ADAMW, GEMM_EPILOGUE = 28, 29, 17
MB = 1 << 24  # spacing of fake device addresses: every call below is rejected on the host


@pytest.fixture(scope="module")
def lib():
    return abi.load()


def d(shape, dtype=F32, ptr=0x100000, stride=None):
    return abi.make_desc(ptr, dtype, shape, stride, None)


def call(lib, kind, ins, outs, schema=0, payload=b"", kid=None):
    import ctypes

    ia, oa = abi.desc_array(ins), abi.desc_array(outs)
    blob, keep = abi.make_blob(schema, payload)
    bp = ctypes.byref(blob) if (schema or payload) else None
    if kid is None:
        return lib.aicf_dispatch_v0(kind, ia, len(ins), oa, len(outs), bp, None)
    return lib.aicf_dispatch_by_id_v0(kind, kid.encode(), ia, len(ins), oa, len(outs), bp, None)


def _tail(B=8192, D=4096, L=4, **kw):
    from aicf_hip import mlp

    return mlp.build_mlp_mse(B, D, L, fuse_optimizer=True, fuse_colsum=True, fuse_tail=True, device="cpu", **kw)


def test_benchmark_step_lowers_to_twelve_gemms_and_two_tail_ops():
    ir, lowered, _ = _tail()
    ops = [it["op"] for it in lowered]
    assert len(lowered) == 14
    assert ops.count("mse_colsum") == 1 and ops.count("colsum_adamw") == 1
    assert sum(o in ("gemm", "gemm_epilogue", "gemm_adamw") for o in ops) == 12
    for gone in ("mse_loss", "reduce_sum", "step_inc", "adamw_step"):
        assert gone not in ops, gone
    name = {v.id: v.name for v in ir.values.values()}
    shape = {v.id: v.shape for v in ir.values.values()}
    mc = lowered[ops.index("mse_colsum")]
    assert [name[v] for v in mc["inputs"]] == ["y", "t", "opt.step"]
    assert [name[v] for v in mc["outputs"]] == ["dY", "loss", "mse.partials", "d_4.b.partials", "opt.step"]
    assert shape[mc["outputs"][3]] == (64, 4096)  # the reduce_sum's workspace rows: its bits
    # the loss op increments the step before every reader of the counter
    first_reader = min(i for i, it in enumerate(lowered) if mc["inputs"][2] in it["inputs"] and it is not mc)
    assert ops.index("mse_colsum") < first_reader
    dg = [it for it in lowered if it["attrs"].get("epilogue_colsum") == "partials"]
    assert len(dg) == 3
    for it in dg:
        assert len(it["outputs"]) == 2 and shape[it["outputs"][1]] == (8192 // 256, 4096)
    ca = lowered[-1]
    assert ca["op"] == "colsum_adamw" and ca["attrs"]["tensors"] == 4
    assert [name[v] for v in ca["inputs"][:4]] == [f"d_{i}.b.partials" for i in (1, 2, 3, 4)]
    assert [name[v] for v in ca["outputs"]][0] == "grad.flat[67108864:67125248]"
    assert ca["kernel_id"] == "colsum_adamw_f32_v0" and mc["kernel_id"] == "mse_colsum_v0"


def test_tail_needs_the_pattern():
    """Without StageE the bias step is the whole flat range, and at a batch
    below twice the workspace rows the column-sum partition is another one:
    both keep the unfused tail."""
    from aicf_hip import mlp

    _, low, _ = mlp.build_mlp_mse(512, 512, 4, fuse_colsum=True, fuse_tail=True, device="cpu")
    assert "mse_colsum" not in [it["op"] for it in low]
    _, low, _ = _tail(B=64, D=512)
    assert "mse_colsum" not in [it["op"] for it in low]


def test_tail_lowering_round_trips_through_the_text_dump():
    from aicf_hip.interchange import lowered_from_text
    from aicf_hip.lower import lowered_to_text

    ir, lowered, _ = _tail(B=512, D=512)
    assert lowered_from_text(lowered_to_text(lowered, ir.name)) == lowered


def test_warmup_and_packing_of_the_tail_ops():
    from aicf_hip.executor import epilogue_kind, pack_attrs, warmup_attrs

    _, lowered, _ = _tail(B=512, D=512)
    mc = next(it for it in lowered if it["op"] == "mse_colsum")
    ca = next(it for it in lowered if it["op"] == "colsum_adamw")
    assert pack_attrs("mse_colsum", mc["attrs"]) == (MSCS, struct.pack("<fi", 0.0, 1))
    assert pack_attrs("mse_colsum", warmup_attrs("mse_colsum", mc["attrs"])) == (MSCS, struct.pack("<fi", 0.0, 0))
    schema, pay = pack_attrs("colsum_adamw", ca["attrs"])
    assert schema == CADW and struct.unpack("<ifffff", pay)[:2] == (4, pytest.approx(1e-3))
    assert struct.unpack("<ifffff", pack_attrs("colsum_adamw", warmup_attrs("colsum_adamw", ca["attrs"]))[1])[1] == 0
    assert epilogue_kind({"epilogue_act": "dgelu", "epilogue_colsum": "partials"}) == 7
    assert epilogue_kind({"epilogue_act": "dgelu", "epilogue_colsum": True}) == 6


def _mse_args(M=256, N=512, P=4, pdt=BF16, base=MB):
    ins = [d((M, N), pdt, base), d((M, N), F32, base + MB), d((), I32, base + 2 * MB)]
    outs = [d((M, N), pdt, base + 3 * MB), d((), F32, base + 4 * MB), d((4096,), F32, base + 5 * MB),
            d((P, N), F32, base + 6 * MB), ins[2]]
    return ins, outs


def test_mse_colsum_refuses_what_the_kernel_cannot_run(lib):
    kid = "mse_colsum_v0"
    pay = struct.pack("<fi", 0.0, 1)

    def rejected(ins, outs, schema=MSCS, p=pay):
        return call(lib, MSE_COLSUM, ins, outs, schema, p, kid) == INV

    ins, outs = _mse_args(M=250, P=4)  # rows not a multiple of the partial rows
    assert rejected(ins, outs)
    ins, outs = _mse_args(N=500)  # bf16 columns not a multiple of 8
    assert rejected(ins, outs)
    ins, outs = _mse_args()
    outs[4] = d((), I32, 40 * MB)  # the step counter is updated in place
    assert rejected(ins, outs)
    ins, outs = _mse_args()
    outs[3] = d((4, 511), F32, 10 * MB)  # partials of another width
    assert rejected(ins, outs)
    ins, outs = _mse_args()
    outs[2] = d((3,), F32, 10 * MB)  # fewer loss partials than workgroups
    assert rejected(ins, outs)
    ins, outs = _mse_args()
    assert rejected(ins, outs, MSCS, struct.pack("<fi", 0.0, 2))  # step += 0 or 1 only
    assert rejected(ins, outs, GEPI, pay)  # another schema
    ins, outs = _mse_args()
    assert rejected(ins[:2], outs)
    assert call(lib, MSE_COLSUM, *_mse_args(N=500)) == NOTIMPL  # no variant takes it


def _cadw_args(T=2, n_t=(256, 128), rows=(4, 8), base=MB):
    parts = [d((rows[t], n_t[t]), F32, base + t * MB) for t in range(T)]
    n = sum(n_t)
    P, M, V = (d((n,), F32, base + (10 + k) * MB) for k in range(3))
    S = d((), I32, base + 20 * MB)
    G, W = d((n,), F32, base + 21 * MB), d((n,), BF16, base + 22 * MB)
    return parts + [P, M, V, S], [G, P, M, V, W]


def _cadw_pay(T=2):
    return struct.pack("<ifffff", T, 1e-3, 0.9, 0.999, 1e-8, 0.0)


def test_colsum_adamw_refuses_what_the_kernel_cannot_run(lib):
    kid = "colsum_adamw_f32_v0"

    def rejected(ins, outs, pay=None):
        return call(lib, COLSUM_ADAMW, ins, outs, CADW, pay or _cadw_pay(), kid) == INV

    ins, outs = _cadw_args()
    assert rejected(ins, outs, _cadw_pay(3))  # T does not match the inputs
    assert rejected(ins, outs, _cadw_pay(9))  # at most 8 tensors
    ins, outs = _cadw_args()
    outs[1] = d((384,), F32, 40 * MB)  # out of place
    assert rejected(ins, outs)
    ins, outs = _cadw_args()
    outs[0] = d((384,), F32, ins[2].data)  # G written over P
    assert rejected(ins, outs)
    ins, outs = _cadw_args()
    outs[0] = d((384,), F32, ins[0].data)  # G written over a partial tensor
    assert rejected(ins, outs)
    ins, outs = _cadw_args()
    outs[4] = d((383,), BF16, 50 * MB)  # shadow of another length
    assert rejected(ins, outs)
    ins, outs = _cadw_args(n_t=(256, 127))
    ins[2] = d((384,), F32, 30 * MB)  # P longer than the partial widths
    assert rejected(ins, outs)
    ins, outs = _cadw_args()
    ins[5] = d((), F32, 60 * MB)  # the step counter is int32
    assert rejected(ins, outs)


def test_dgelu_partials_epilogue_refusals(lib):
    """GEPI kind 7 takes (C, partials [M/256, N]) on the 256 x 256 bf16 path
    only: a partial tensor with extra rows (its reader sums every row) or a
    shape off that path is refused."""
    kid = "gemm_epilogue_bf16_mfma_v0"
    pay = struct.pack("<iii", 0, 0, 7)
    A, B, Z = d((512, 256), BF16, MB), d((256, 512), BF16, 2 * MB), d((512, 512), BF16, 3 * MB)
    C = d((512, 512), BF16, 4 * MB)
    assert call(lib, GEMM_EPILOGUE, [A, B, Z], [C, d((3, 512), F32, 5 * MB)], GEPI, pay, kid) == INV
    assert call(lib, GEMM_EPILOGUE, [A, B, Z], [C, d((2, 512), F32, 5 * MB), d((512,), F32, 6 * MB)],
                GEPI, pay, kid) == INV
    A2, Z2, C2 = d((500, 256), BF16, MB), d((500, 512), BF16, 3 * MB), d((500, 512), BF16, 4 * MB)
    assert call(lib, GEMM_EPILOGUE, [A2, B, Z2], [C2, d((1, 512), F32, 5 * MB)], GEPI, pay, kid) == INV


def test_tail_sizes_the_loss_partials_for_wide_rows():
    """mse_colsum writes ceil(N / 512) x P loss partials (bf16, 64 lanes of 8
    columns per workgroup); where the loss op's own buffer is smaller (here
    1024 elements against 32 x 64 = 2048 for N = 16384, P = 64) the tail
    gets a buffer of its own instead of an op that fails at launch."""
    from aicf_hip import mlp

    ir, low, _ = mlp.build_mlp_mse(128, 16384, 1, fuse_optimizer=True, fuse_colsum=True, fuse_tail=True,
                                   device="cpu")
    assert ir.by_name("mse.partials").shape == (1024,)
    mc = next(it for it in low if it["op"] == "mse_colsum")
    ws = ir.values[mc["outputs"][2]]
    assert ws.name != "mse.partials" and ws.shape == (2048,) and "float32" in ws.dtype
    # at the benchmark shape the loss op's buffer is large enough and is reused
    ir, low, _ = _tail(B=512, D=512)
    mc = next(it for it in low if it["op"] == "mse_colsum")
    assert ir.values[mc["outputs"][2]].name == "mse.partials"


def test_lowering_constants_match_the_kernels():
    """The lowering's copies of kernel limits are the kernels' own values."""
    import re
    from pathlib import Path

    from aicf_hip import lower

    csrc = Path(__file__).resolve().parents[1] / "ai-compiler-framework_amd" / "csrc"
    elt = (csrc / "kernels" / "eltwise.hip").read_text()
    hdr = (csrc / "common" / "smallstep.hpp").read_text()
    assert int(re.search(r"kMseColsumVecBf16\s*=\s*(\d+)", elt).group(1)) == lower.MSE_COLSUM_VEC_BF16
    assert int(re.search(r"kSmallGemmMaxTiles64\s*=\s*(\d+)", hdr).group(1)) == lower.SMALL_GEMM_MAX_TILES64


def test_mse_colsum_refuses_overlapping_outputs(lib):
    """Written buffers that overlap an input or each other are refused, also
    when only part of the byte ranges meet."""
    kid = "mse_colsum_v0"
    pay = struct.pack("<fi", 0.0, 1)
    # gradient over the second half of the prediction
    ins, outs = _mse_args()
    outs[0] = d((256, 512), BF16, ins[0].data + 256 * 512)
    assert call(lib, MSE_COLSUM, ins, outs, MSCS, pay, kid) == INV
    # loss scalar inside the target
    ins, outs = _mse_args()
    outs[1] = d((), F32, ins[1].data + 64)
    assert call(lib, MSE_COLSUM, ins, outs, MSCS, pay, kid) == INV
    # column partials overlapping the loss partials
    ins, outs = _mse_args()
    outs[3] = d((4, 512), F32, outs[2].data + 4000 * 4)
    assert call(lib, MSE_COLSUM, ins, outs, MSCS, pay, kid) == INV
    # loss partials over the step counter
    ins, outs = _mse_args()
    outs[2] = d((4096,), F32, ins[2].data - 8)
    assert call(lib, MSE_COLSUM, ins, outs, MSCS, pay, kid) == INV
