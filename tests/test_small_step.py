"""StageF (the small-step lowering) and the host-side contracts of its three
ops, without a GPU: the reference MLP's step lowers to four launches whose
jobs are independent, the unfused values the oracle reads are all produced,
the AICF_WARMUP rewrite reaches the fused ops, and supported() refuses what
the kernels cannot run (overlapping group jobs, aliasing Adam buffers,
heads wider than the kernel) before any launch."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from aicf_cuda import abi

OK, INV, NOTIMPL = abi.STATUS_OK, abi.STATUS_INVALID_ARGUMENT, abi.STATUS_NOT_IMPLEMENTED
F32, I32 = abi.DTYPE_F32, abi.DTYPE_I32
GGRP = int.from_bytes(b"GGRP", "little")
ADAM = int.from_bytes(b"ADAM", "little")
XENT_HEAD, GRAD_GROUP, ADAMW_MULTI = 25, 26, 27
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


def _fused():
    from aicf_hip import mlp

    return mlp.build_mlp_xent(fuse_small=True)


def test_reference_step_lowers_to_four_launches():
    ir, lowered, _ = _fused()
    assert [(it["op"], it["kernel_id"]) for it in lowered] == [
        ("gemm_epilogue", "gemm_bias_relu_f32_naive_v0"), ("xent_head", "xent_head_f32_v0"),
        ("grad_group", "grad_group_f32_v0"), ("adamw_multi", "adamw_multi_f32_v0")]
    name = {v.id: v.name for v in ir.values.values()}
    g = lowered[2]
    kinds = sorted(j[0] for j in g["attrs"]["jobs"])
    assert kinds == [0, 0, 0, 1, 1, 2, 3]  # dW1, dx, dW0 | db1, db0 | loss mean | step
    written = {name[v] for it in lowered for v in it["outputs"]}
    for k in ("loss", "pred", "row_loss", "logits", "dY", "d_relu0_out", "d_lin0_out", "d_x", "opt.step",
              "d_0.W", "d_0.b", "d_2.W", "d_2.b", "0.W", "0.b", "2.W", "2.b"):
        assert k in written, k
    # the saved ReLU output is read from the ReLU output itself (nothing rewrites it)
    assert lowered[1]["inputs"][0] == lowered[1]["inputs"][4] == lowered[0]["outputs"][0]


def test_group_jobs_are_independent():
    ir, lowered, _ = _fused()
    from aicf_hip.lower import _base

    g = lowered[2]
    ins, outs = g["inputs"], g["outputs"]
    jobs = g["attrs"]["jobs"]
    for a, ja in enumerate(jobs):
        wa = _base(ir, outs[ja[3]])
        for b, jb in enumerate(jobs):
            if a == b:
                continue
            reads = {_base(ir, ins[jb[1]])} | ({_base(ir, ins[jb[2]])} if jb[0] == 0 else set())
            assert wa not in reads and wa != _base(ir, outs[jb[3]]), (ja, jb)


def test_unfused_lowering_is_the_reference_one():
    from aicf_hip import mlp

    _, lowered, _ = mlp.build_mlp_xent()
    assert len(lowered) == 17 and lowered[1]["op"] == "copy_saved"


def test_warmup_rewrites_reach_the_fused_ops():
    from aicf_hip.executor import pack_attrs, warmup_attrs

    _, lowered, _ = _fused()
    g, a = lowered[2], lowered[3]
    wg = warmup_attrs("grad_group", g["attrs"])
    assert [j[4] for j in wg["jobs"] if j[0] == 3] == [0]
    assert [j[4] for j in g["attrs"]["jobs"] if j[0] == 3] == [1]  # the original is unchanged
    assert [j[:4] for j in wg["jobs"]] == [j[:4] for j in g["attrs"]["jobs"]]
    assert warmup_attrs("adamw_multi", a["attrs"])["lr"] == 0.0
    schema, pay = pack_attrs("grad_group", g["attrs"])
    assert schema == GGRP and len(pay) == 4 + 24 * len(g["attrs"]["jobs"])
    assert struct.unpack_from("<i", pay)[0] == 7
    schema, pay = pack_attrs("adamw_multi", a["attrs"])
    assert schema == ADAM and struct.unpack("<fffff", pay)[0] == pytest.approx(1e-3)


def test_fused_lowering_round_trips_through_the_text_dump():
    from aicf_hip.interchange import lowered_from_text
    from aicf_hip.lower import lowered_to_text

    ir, lowered, _ = _fused()
    text = lowered_to_text(lowered, ir.name)
    assert lowered_from_text(text) == lowered


def test_head_fusion_needs_the_pattern():
    """A head wider than 32 classes keeps the softmax_xent path; the other
    passes still group what they can."""
    from aicf_hip import mlp

    _, lowered, _ = mlp.build_mlp_xent(B=64, din=784, dh=256, dout=40, fuse_small=True)
    ops = [it["op"] for it in lowered]
    assert "xent_head" not in ops and "softmax_xent" in ops and "adamw_multi" in ops


def _group_payload(jobs):
    return struct.pack("<i", len(jobs)) + b"".join(struct.pack("<iiiiii", *j) for j in jobs)


def test_grad_group_refuses_conflicting_jobs(lib):
    kid = "grad_group_f32_v0"
    A, B, C2 = d((64, 32), ptr=1 * MB), d((32, 16), ptr=2 * MB), d((64, 16), ptr=3 * MB)
    col = d((16,), ptr=4 * MB)
    # a GEMM and a column sum of its own output in one group: refused
    jobs = [(0, 0, 1, 0, 0, 0), (1, 2, 0, 1, 0, 0)]
    assert call(lib, GRAD_GROUP, [A, B, C2], [C2, col], GGRP, _group_payload(jobs), kid) == INV
    # two jobs writing overlapping memory: refused
    jobs = [(1, 0, 0, 0, 0, 0), (1, 1, 0, 1, 0, 0)]
    o1, o2 = d((32,), ptr=5 * MB), d((32,), ptr=5 * MB + 64)
    assert call(lib, GRAD_GROUP, [A, d((64, 32), ptr=6 * MB)], [o1, o2], GGRP, _group_payload(jobs), kid) == INV
    # more than 8 jobs, an unknown type, an index out of range, the wrong schema
    many = [(3, 0, 0, 0, 1, 0)] * 9
    step = d((), I32, ptr=7 * MB)
    assert call(lib, GRAD_GROUP, [step], [step], GGRP, _group_payload(many), kid) == INV
    assert call(lib, GRAD_GROUP, [step], [step], GGRP, _group_payload([(4, 0, 0, 0, 0, 0)]), kid) == INV
    assert call(lib, GRAD_GROUP, [step], [step], GGRP, _group_payload([(3, 1, 0, 0, 1, 0)]), kid) == INV
    assert call(lib, GRAD_GROUP, [step], [step], ADAM, _group_payload([(3, 0, 0, 0, 1, 0)]), kid) == INV
    # a step job adds 0 or 1 only
    assert call(lib, GRAD_GROUP, [step], [step], GGRP, _group_payload([(3, 0, 0, 0, 2, 0)]), kid) == INV
    # GEMM shapes must chain
    jobs = [(0, 0, 1, 0, 0, 0)]
    assert call(lib, GRAD_GROUP, [A, d((31, 16), ptr=2 * MB)], [C2], GGRP, _group_payload(jobs), kid) == INV


def test_adamw_multi_refuses_aliasing_and_bad_layouts(lib):
    kid = "adamw_multi_f32_v0"
    pay = struct.pack("<fffff", 1e-3, 0.9, 0.999, 1e-8, 0.0)

    def tensors(base, n=64):
        return [d((n,), ptr=base + k * MB) for k in range(4)]

    step = d((), I32, ptr=60 * MB)
    t0, t1 = tensors(10 * MB), tensors(20 * MB)
    ok_in = t0 + t1 + [step]
    outs = [t0[0], t0[2], t0[3], t1[0], t1[2], t1[3]]
    # out of place is refused (the fused update is in place)
    bad = list(outs)
    bad[0] = d((64,), ptr=40 * MB)
    assert call(lib, ADAMW_MULTI, ok_in, bad, ADAM, pay, kid) == INV
    # G aliasing M
    t2 = tensors(30 * MB)
    t2[1] = t2[2]
    assert call(lib, ADAMW_MULTI, t2 + [step], [t2[0], t2[2], t2[3]], ADAM, pay, kid) == INV
    # two tensors sharing a buffer
    t3 = tensors(10 * MB)
    assert call(lib, ADAMW_MULTI, t0 + t3 + [step], outs[:3] + [t3[0], t3[2], t3[3]], ADAM, pay, kid) == INV
    # wrong counts, unaligned, mismatched sizes
    assert call(lib, ADAMW_MULTI, ok_in[:-1], outs, ADAM, pay, kid) == INV
    t4 = [d((64,), ptr=50 * MB + k * MB + 4) for k in range(4)]
    assert call(lib, ADAMW_MULTI, t4 + [step], [t4[0], t4[2], t4[3]], ADAM, pay, kid) == INV
    t5 = tensors(10 * MB)
    t5[1] = d((63,), ptr=11 * MB)
    assert call(lib, ADAMW_MULTI, t5 + [step], [t5[0], t5[2], t5[3]], ADAM, pay, kid) == INV


def test_xent_head_refuses_what_the_kernel_cannot_run(lib):
    kid = "xent_head_f32_v0"

    def args(B=64, K=256, C=10, ptr=MB):
        ins = [d((B, K), ptr=ptr), d((C, K), ptr=ptr + MB), d((C,), ptr=ptr + 2 * MB), d((B,), I32, ptr=ptr + 3 * MB),
               d((B, K), ptr=ptr)]
        outs = [d((B, C), ptr=ptr + 5 * MB), d((B, C), ptr=ptr + 6 * MB), d((B,), I32, ptr=ptr + 7 * MB),
                d((B,), ptr=ptr + 8 * MB), d((B, K), ptr=ptr + 9 * MB), d((B, K), ptr=ptr + 10 * MB)]
        return ins, outs

    for B, K, C in ((64, 256, 33), (64, 254, 10), (64, 4096, 10), (64, 256, 0)):
        ins, outs = args(B, K, C)
        assert call(lib, XENT_HEAD, ins, outs, kid=kid) == INV, (B, K, C)
        assert call(lib, XENT_HEAD, ins, outs) == NOTIMPL, (B, K, C)
    ins, outs = args()
    outs[4] = ins[1]  # dH written over W
    assert call(lib, XENT_HEAD, ins, outs, kid=kid) == INV
    ins, outs = args()
    ins[3] = d((64,), F32, ptr=4 * MB)  # labels must be int32
    assert call(lib, XENT_HEAD, ins, outs, kid=kid) == INV


def _view_params(ir, names, elem_offset):
    """Re-declare parameters `names` of a built IR as views of one flat fp32
    buffer, the first one at `elem_offset` elements (the rest follow it)."""
    import dataclasses

    total = elem_offset + sum(int(np.prod(ir.by_name(n).shape)) for n in names)
    flat = ir.new_value(name="flat.extra", shape=(total,), dtype="torch.float32", device="cpu")
    off = elem_offset
    for n in names:
        v = ir.by_name(n)
        ir.values[v.id] = dataclasses.replace(v, view_of=(flat.id, off))
        off += int(np.prod(v.shape))


def _relower(ir):
    from aicf_hip.lower import compile_lowered

    return compile_lowered(ir, fuse_small=True)


def test_small_step_keeps_unaligned_views_off_the_vector_kernels():
    """adamw_multi and xent_head move 16-byte vectors: a head weight that is
    a view at an offset of one float keeps adamw_step (which has an unaligned
    path) and the unfused head; at a 16-byte offset the fusions apply."""
    from aicf_hip import mlp

    ir, low, _ = mlp.build_mlp_xent(fuse_small=True)
    _view_params(ir, ["2.W"], 4)  # 16 bytes: still aligned
    ops = [it["op"] for it in _relower(ir)]
    assert "xent_head" in ops and ops.count("adamw_multi") == 1 and "adamw_step" not in ops
    ir, low, _ = mlp.build_mlp_xent(fuse_small=True)
    _view_params(ir, ["2.W"], 1)
    ops = [it["op"] for it in _relower(ir)]
    assert "xent_head" not in ops and "softmax_xent" in ops
    name = {v.id: v.name for v in ir.values.values()}
    low = _relower(ir)
    multi = [it for it in low if it["op"] == "adamw_multi"]
    fused_params = {name[v] for it in multi for v in it["inputs"][0::4][:-1]}
    assert "2.W" not in fused_params
    assert any(it["op"] == "adamw_step" and name[it["inputs"][0]] == "2.W" for it in low)


def _save_graph(extra_reader_before=False, dst_name="relu0_saved"):
    """relu(x) -> h; copy_saved(h) -> s; relu_bwd(d, s) -> dx as a lowered list."""
    from aicf_hip.ir import IRGraph

    ir = IRGraph(name="saves")
    nv = lambda n: ir.new_value(name=n, shape=(4, 8), dtype="torch.float32", device="cpu").id  # noqa: E731
    x, h, s, d_, dx, y = nv("a_in"), nv("h"), nv(dst_name), nv("d_h"), nv("d_a"), nv("y")
    low = [{"op": "relu", "inputs": [x], "outputs": [h], "attrs": {}}]
    if extra_reader_before:
        low.append({"op": "relu", "inputs": [s], "outputs": [y], "attrs": {}})
    low += [{"op": "copy_saved", "inputs": [h], "outputs": [s], "attrs": {}},
            {"op": "relu_bwd", "inputs": [d_, s], "outputs": [dx], "attrs": {}}]
    return ir, low, s, h


def test_drop_dead_saves_keeps_copies_something_else_reads():
    from aicf_hip.lower import drop_dead_saves

    ir, low, s, h = _save_graph()
    out = drop_dead_saves(ir, low)
    assert [it["op"] for it in out] == ["relu", "relu_bwd"] and out[1]["inputs"] == [low[2]["inputs"][0], h]
    # an op before the copy reads the previous step's save: the copy stays
    ir, low, s, h = _save_graph(extra_reader_before=True)
    assert [it["op"] for it in drop_dead_saves(ir, low)] == ["relu", "relu", "copy_saved", "relu_bwd"]
    # the caller reads the save after the step
    ir, low, s, h = _save_graph()
    assert "copy_saved" in [it["op"] for it in drop_dead_saves(ir, low, keep=[s])]
    # a save bound by the caller (an input or parameter name) is not the copy's to drop
    for nm in ("x", "0.W"):
        ir, low, s, h = _save_graph(dst_name=nm)
        assert "copy_saved" in [it["op"] for it in drop_dead_saves(ir, low)], nm


def test_xent_head_refuses_partially_overlapping_outputs(lib):
    kid = "xent_head_f32_v0"
    B, K, C = 64, 256, 10
    ins = [d((B, K), ptr=MB), d((C, K), ptr=2 * MB), d((C,), ptr=3 * MB), d((B,), I32, ptr=4 * MB),
           d((B, K), ptr=5 * MB)]

    def outs():
        return [d((B, C), ptr=6 * MB), d((B, C), ptr=7 * MB), d((B,), I32, ptr=8 * MB), d((B,), ptr=9 * MB),
                d((B, K), ptr=10 * MB), d((B, K), ptr=11 * MB)]

    o = outs()
    o[5] = d((B, K), ptr=5 * MB + 1024)  # dX over the second row onwards of S
    assert call(lib, XENT_HEAD, ins, o, kid=kid) == INV
    o = outs()
    o[1] = d((B, C), ptr=6 * MB + 16)  # dlogits overlapping logits
    assert call(lib, XENT_HEAD, ins, o, kid=kid) == INV
    o = outs()
    o[3] = d((B,), ptr=MB + 4096)  # row loss inside H
    assert call(lib, XENT_HEAD, ins, o, kid=kid) == INV
