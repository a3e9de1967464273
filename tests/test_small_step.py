"""StageF (the small-step lowering) and the host-side contracts of its ops,
without a GPU: the reference MLP's step lowers to three launches (four with
the AdamW updates in a launch of their own) whose jobs are independent, the
unfused values the oracle reads are all produced, the AICF_WARMUP rewrite
reaches the fused ops, and supported() refuses what the kernels cannot run
(overlapping group jobs, aliasing Adam buffers, heads wider than the
kernel, updates of a tensor another job reads) before any launch."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from aicf_cuda import abi

OK, INV, NOTIMPL = abi.STATUS_OK, abi.STATUS_INVALID_ARGUMENT, abi.STATUS_NOT_IMPLEMENTED
F32, I32 = abi.DTYPE_F32, abi.DTYPE_I32
GGRP = int.from_bytes(b"GGRP", "little")
GGRA = int.from_bytes(b"GGRA", "little")
XHST = int.from_bytes(b"XHST", "little")
GEPI = int.from_bytes(b"GEPI", "little")
ADAM = int.from_bytes(b"ADAM", "little")
GEMM_EPILOGUE, XENT_HEAD, GRAD_GROUP, ADAMW_MULTI = 17, 25, 26, 27
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


def _fused(fuse_small=True):
    from aicf_hip import mlp

    return mlp.build_mlp_xent(fuse_small=fuse_small)


def test_reference_step_lowers_to_three_launches():
    ir, lowered, _ = _fused()
    assert [(it["op"], it["kernel_id"]) for it in lowered] == [
        ("gemm_epilogue_bcopy", "gemm_small_bcopy_f32_v0"), ("xent_head", "xent_head_step_f32_v0"),
        ("grad_group_adamw", "grad_group_adamw_f32_v0")]
    name = {v.id: v.name for v in ir.values.values()}
    fwd, head, g = lowered
    # the forward GEMM writes the copy of 0.W that the input gradient reads
    assert [name[v] for v in fwd["outputs"]] == ["relu0_out", "0.W.copy"]
    # the head advances the step counter in place and writes the step's
    # AdamW bias corrections, which the group reads
    assert name[head["inputs"][5]] == name[head["outputs"][6]] == "opt.step" and head["attrs"]["step_inc"] == 1
    assert name[head["outputs"][7]] == "opt.step.adamw_scalars"
    assert (head["attrs"]["lr"], head["attrs"]["beta1"], head["attrs"]["beta2"]) == (1e-3, 0.9, 0.999)
    ins, outs = g["inputs"], g["outputs"]
    jobs = g["attrs"]["jobs"]
    assert sorted(j[0] for j in jobs) == [0, 0, 0, 1, 1, 2]  # dW1, dx, dW0 | db1, db0 | loss mean; no step job
    upd = {name[outs[j[3]]]: [name[ins[j[6 + k]]] for k in range(3)] for j in jobs if j[6] >= 0}
    assert upd == {"d_2.W": ["2.W", "opt.m.2.W", "opt.v.2.W"], "d_2.b": ["2.b", "opt.m.2.b", "opt.v.2.b"],
                   "d_0.W": ["0.W", "opt.m.0.W", "opt.v.0.W"], "d_0.b": ["0.b", "opt.m.0.b", "opt.v.0.b"]}
    for j in jobs:  # in place
        if j[6] >= 0:
            assert [ins[j[6 + k]] for k in range(3)] == [outs[j[9 + k]] for k in range(3)]
    dx = [j for j in jobs if name[outs[j[3]]] == "d_x"][0]
    assert name[ins[dx[2]]] == "0.W.copy"
    assert name[ins[g["attrs"]["scalars_input"]]] == "opt.step.adamw_scalars"
    assert "opt.step" not in {name[v] for v in list(ins) + list(outs)}
    written = {name[v] for it in lowered for v in it["outputs"]}
    for k in ("loss", "pred", "row_loss", "logits", "dY", "d_relu0_out", "d_lin0_out", "d_x", "opt.step",
              "d_0.W", "d_0.b", "d_2.W", "d_2.b", "0.W", "0.b", "2.W", "2.b"):
        assert k in written, k
    # nothing in the group reads a tensor it updates
    upd_ids = {ins[j[6 + k]] for j in jobs if j[6] >= 0 for k in range(3)}
    assert not upd_ids & {ins[j[1]] for j in jobs} and not upd_ids & {ins[j[2]] for j in jobs if j[0] == 0}


def test_reference_step_lowers_to_four_launches():
    ir, lowered, _ = _fused("four")
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


@pytest.mark.parametrize("fuse_small", [True, "four"])
def test_group_jobs_are_independent(fuse_small):
    ir, lowered, _ = _fused(fuse_small)
    from aicf_hip.lower import _base

    g = lowered[2]
    ins, outs = g["inputs"], g["outputs"]
    jobs = g["attrs"]["jobs"]
    for a, ja in enumerate(jobs):
        wa = {_base(ir, outs[ja[3]])}
        if len(ja) == 12 and ja[6] >= 0:
            wa |= {_base(ir, ins[ja[6 + k]]) for k in range(3)}
        for b, jb in enumerate(jobs):
            if a == b:
                continue
            reads = {_base(ir, ins[jb[1]])} | ({_base(ir, ins[jb[2]])} if jb[0] == 0 else set())
            writes = {_base(ir, outs[jb[3]])}
            if len(jb) == 12 and jb[6] >= 0:
                writes |= {_base(ir, ins[jb[6 + k]]) for k in range(3)}
            assert not wa & reads and not wa & writes, (ja, jb)


def test_unfused_lowering_is_the_reference_one():
    from aicf_hip import mlp

    _, lowered, _ = mlp.build_mlp_xent()
    assert len(lowered) == 17 and lowered[1]["op"] == "copy_saved"


def test_warmup_rewrites_reach_the_three_launch_ops():
    from aicf_hip.executor import pack_attrs, warmup_attrs

    _, lowered, _ = _fused()
    head, g = lowered[1], lowered[2]
    wh = warmup_attrs("xent_head", head["attrs"])
    assert (wh["step_inc"], wh["lr"]) == (0, 0.0) and (head["attrs"]["step_inc"], head["attrs"]["lr"]) == (1, 1e-3)
    assert warmup_attrs("xent_head", {}) == {}  # the plain head has no step part
    assert warmup_attrs("grad_group_adamw", g["attrs"])["lr"] == 0.0 and g["attrs"]["lr"] == pytest.approx(1e-3)
    schema, pay = pack_attrs("xent_head", head["attrs"])
    assert schema == XHST and struct.unpack("<ifff", pay) == (1, pytest.approx(1e-3), pytest.approx(0.9),
                                                              pytest.approx(0.999))
    assert struct.unpack("<i", pack_attrs("xent_head", {"step_inc": 0})[1]) == (0,)
    assert pack_attrs("xent_head", {})[0] == 0
    schema, pay = pack_attrs("grad_group_adamw", g["attrs"])
    n = len(g["attrs"]["jobs"])
    assert schema == GGRA and len(pay) == 28 + 48 * n
    cnt, lr, b1, b2, eps, wd, si = struct.unpack_from("<ifffffi", pay)
    assert (cnt, si) == (n, g["attrs"]["scalars_input"]) and (b1, wd) == (pytest.approx(0.9), 0.0)
    assert [list(struct.unpack_from("<" + "i" * 12, pay, 28 + 48 * k)) for k in range(n)] == g["attrs"]["jobs"]
    schema, pay = pack_attrs("gemm_epilogue_bcopy", lowered[0]["attrs"])
    assert schema == GEPI and struct.unpack("<iii", pay) == (0, 1, 0)


def test_warmup_rewrites_reach_the_fused_ops():
    from aicf_hip.executor import pack_attrs, warmup_attrs

    _, lowered, _ = _fused("four")
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


@pytest.mark.parametrize("fuse_small", [True, "four"])
def test_fused_lowering_round_trips_through_the_text_dump(fuse_small):
    from aicf_hip.interchange import lowered_from_text
    from aicf_hip.lower import lowered_to_text

    ir, lowered, _ = _fused(fuse_small)
    text = lowered_to_text(lowered, ir.name)
    assert lowered_from_text(text) == lowered


def test_head_fusion_needs_the_pattern():
    """A head wider than 32 classes keeps the softmax_xent path; the other
    passes still group what they can."""
    from aicf_hip import mlp

    _, lowered, _ = mlp.build_mlp_xent(B=64, din=784, dh=256, dout=40, fuse_small=True)
    ops = [it["op"] for it in lowered]
    assert "xent_head" not in ops and "softmax_xent" in ops and "adamw_multi" in ops
    # with no head to take the step counter the updates stay in adamw_multi
    # (a step_inc launch of their own would cost what the fusion saves)
    assert "grad_group_adamw" not in ops and "gemm_epilogue_bcopy" not in ops


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
    # an operand spanning 2^31 bytes or more (the small GEMM's buffer offsets are 32-bit)
    wide_a, wide_b = d((16, 1 << 27), ptr=1 << 40), d((1 << 27, 16), ptr=1 << 42)
    assert call(lib, GRAD_GROUP, [wide_a, wide_b], [d((16, 16), ptr=3 * MB)], GGRP, _group_payload(jobs), kid) == INV


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


def _relower(ir, fuse_small=True):
    from aicf_hip.lower import compile_lowered

    return compile_lowered(ir, fuse_small=fuse_small)


def test_small_step_keeps_unaligned_views_off_the_vector_kernels():
    """adamw_multi and xent_head move 16-byte vectors: a head weight that is
    a view at an offset of one float keeps adamw_step (which has an unaligned
    path) and the unfused head; at a 16-byte offset the fusions apply."""
    from aicf_hip import mlp

    ir, low, _ = mlp.build_mlp_xent(fuse_small=True)
    _view_params(ir, ["2.W"], 4)  # 16 bytes: still aligned
    ops = [it["op"] for it in _relower(ir, "four")]
    assert "xent_head" in ops and ops.count("adamw_multi") == 1 and "adamw_step" not in ops
    # the group's updates take any offset
    ops = [it["op"] for it in _relower(ir)]
    assert ops == ["gemm_epilogue_bcopy", "xent_head", "grad_group_adamw"]
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


def _ggra_payload(jobs, scalars_input, lr=1e-3, b1=0.9, b2=0.999, eps=1e-8, wd=0.0):
    head = struct.pack("<ifffffi", len(jobs), lr, b1, b2, eps, wd, scalars_input)
    return head + b"".join(struct.pack("<" + "i" * 12, *j) for j in jobs)


def _ggra_case():
    """A GEMM dW = dY^T . X (16 x 32) with AdamW on W, a column sum db of dY
    with AdamW on b, and a dX = dY . Wc job reading a copy Wc of W."""
    dY, X = d((64, 16), ptr=1 * MB), d((64, 32), ptr=2 * MB)
    W, Wm, Wv = d((16, 32), ptr=3 * MB), d((16, 32), ptr=4 * MB), d((16, 32), ptr=5 * MB)
    b, bm, bv = d((16,), ptr=6 * MB), d((16,), ptr=7 * MB), d((16,), ptr=8 * MB)
    Wc, scal = d((16, 32), ptr=9 * MB), d((2,), ptr=10 * MB)
    dW, db, dX = d((16, 32), ptr=11 * MB), d((16,), ptr=12 * MB), d((64, 32), ptr=13 * MB)
    ins = [dY, X, W, Wm, Wv, b, bm, bv, Wc, scal]
    outs = [dW, W, Wm, Wv, db, b, bm, bv, dX]
    jobs = [[0, 0, 1, 0, 1, 0, 2, 3, 4, 1, 2, 3],
            [1, 0, 0, 4, 0, 0, 5, 6, 7, 5, 6, 7],
            [0, 0, 8, 8, 0, 0, -1, -1, -1, -1, -1, -1]]
    return ins, outs, jobs, 9


def test_grad_group_adamw_refuses_what_would_race(lib, monkeypatch):
    kid = "grad_group_adamw_f32_v0"
    ins, outs, jobs, si = _ggra_case()

    def ok(ins=ins, outs=outs, jobs=jobs, si=si, schema=GGRA, **hp):
        return call(lib, GRAD_GROUP, ins, outs, schema, _ggra_payload(jobs, si, **hp), kid)

    # the well-formed case passes every host check: it only fails at the
    # launch, which this container cannot do (no GPU)
    assert ok() != INV
    # the copy job reads W itself while W is updated: refused
    j = [list(x) for x in jobs]
    j[2][2] = 2
    assert ok(jobs=j) == INV
    # AdamW on the loss-mean type, or on a step job in the group
    j = [list(x) for x in jobs]
    j[1][0] = 2
    assert ok(jobs=j) == INV
    j = [list(x) for x in jobs] + [[3, 9, 0, 9, 1, 0] + [-1] * 6]
    assert ok(ins=ins, outs=outs + [ins[9]], jobs=j) == INV
    # not in place: the P output is another buffer
    o = list(outs)
    o[1] = d((16, 32), ptr=20 * MB)
    assert ok(outs=o) == INV
    # M of the wrong size, an update overlapping another job's output
    i2 = list(ins)
    i2[3] = d((16, 31), ptr=4 * MB)
    o2 = list(outs)
    o2[2] = i2[3]
    assert ok(ins=i2, outs=o2) == INV
    i3, o3 = list(ins), list(outs)
    i3[6] = o3[6] = d((16,), ptr=13 * MB + 64)  # b's M inside dX
    assert ok(ins=i3, outs=o3) == INV
    # the bias corrections overlapping an updated tensor, of the wrong type or
    # size; a NaN hyperparameter, the GGRP schema, an index out of range
    i4 = list(ins)
    i4[9] = d((2,), ptr=6 * MB + 4)
    assert ok(ins=i4) == INV
    for bad in (d((2,), I32, ptr=10 * MB), d((3,), ptr=10 * MB)):
        i4[9] = bad
        assert ok(ins=i4) == INV
    assert ok(lr=float("nan")) == INV
    assert ok(schema=GGRP) == INV
    j = [list(x) for x in jobs]
    j[0][8] = 10
    assert ok(jobs=j) == INV
    # a GEMM output that is not row-major contiguous
    o5 = list(outs)
    o5[0] = d((16, 32), ptr=11 * MB, stride=(64, 1))
    assert ok(outs=o5) == INV


def test_xent_head_step_refuses_bad_counters(lib):
    kid = "xent_head_step_f32_v0"
    B, K, C = 64, 256, 10
    step = d((), I32, ptr=20 * MB)
    ins = [d((B, K), ptr=MB), d((C, K), ptr=2 * MB), d((C,), ptr=3 * MB), d((B,), I32, ptr=4 * MB),
           d((B, K), ptr=5 * MB), step]
    outs = [d((B, C), ptr=6 * MB), d((B, C), ptr=7 * MB), d((B,), I32, ptr=8 * MB), d((B,), ptr=9 * MB),
            d((B, K), ptr=10 * MB), d((B, K), ptr=11 * MB), step]
    inc1 = struct.pack("<i", 1)
    assert call(lib, XENT_HEAD, ins, outs, XHST, inc1, kid) != INV
    assert call(lib, XENT_HEAD, ins, outs, XHST, struct.pack("<i", 2), kid) == INV
    assert call(lib, XENT_HEAD, ins, outs, GGRP, inc1, kid) == INV
    assert call(lib, XENT_HEAD, ins[:5], outs[:6], XHST, inc1, kid) == INV
    o = list(outs)
    o[6] = d((), I32, ptr=21 * MB)  # not in place
    assert call(lib, XENT_HEAD, ins, o, XHST, inc1, kid) == INV
    # with the hyperparameters an 8th output takes the bias corrections
    hp = inc1 + struct.pack("<fff", 1e-3, 0.9, 0.999)
    scal = d((2,), ptr=22 * MB)
    assert call(lib, XENT_HEAD, ins, outs + [scal], XHST, hp, kid) != INV
    assert call(lib, XENT_HEAD, ins, outs, XHST, hp, kid) == INV
    assert call(lib, XENT_HEAD, ins, outs + [scal], XHST, inc1, kid) == INV
    assert call(lib, XENT_HEAD, ins, outs + [d((3,), ptr=22 * MB)], XHST, hp, kid) == INV
    assert call(lib, XENT_HEAD, ins, outs + [d((2,), ptr=9 * MB)], XHST, hp, kid) == INV  # over the row loss
    nan = inc1 + struct.pack("<fff", float("nan"), 0.9, 0.999)
    assert call(lib, XENT_HEAD, ins, outs + [scal], XHST, nan, kid) == INV
    i2, o2 = list(ins), list(outs)
    i2[5] = o2[6] = d((), I32, ptr=9 * MB + 8)  # inside the row loss
    assert call(lib, XENT_HEAD, i2, o2, XHST, inc1, kid) == INV
    i3, o3 = list(ins), list(outs)
    i3[5] = o3[6] = d((2,), I32, ptr=20 * MB)  # not a scalar
    assert call(lib, XENT_HEAD, i3, o3, XHST, inc1, kid) == INV


def test_gemm_bcopy_refuses_what_it_cannot_copy(lib):
    kid = "gemm_small_bcopy_f32_v0"
    M, N, K = 64, 256, 784
    A, W, b = d((M, K), ptr=MB), d((N, K), ptr=4 * MB), d((N,), ptr=8 * MB)
    C, Wc = d((M, N), ptr=9 * MB), d((N, K), ptr=12 * MB)

    def run(ins, outs, ta=0, tb=1, kind=0, schema=GEPI):
        return call(lib, GEMM_EPILOGUE, ins, outs, schema, struct.pack("<iii", ta, tb, kind), kid)

    assert run([A, W, b], [C, Wc]) != INV
    assert run([A, W, b], [C, Wc], kind=2) != INV  # ReLU without bias
    assert run([A, d((K, N), ptr=4 * MB), b], [C, d((K, N), ptr=12 * MB)], tb=0) == INV  # B not K-contiguous
    assert run([A, W, b], [C, Wc], kind=3) == INV  # GELU is not the small path's
    assert run([A, W, b], [C, d((N, K - 4), ptr=12 * MB)]) == INV  # copy of another shape
    assert run([A, W, b], [C, d((N, K), ptr=MB + 64)]) == INV  # copy over A
    assert run([A, W, b], [C, d((N, K), ptr=12 * MB + 4)]) == INV  # unaligned copy
    assert run([d((M, 786), ptr=MB), d((N, 786), ptr=4 * MB), b], [C, d((N, 786), ptr=12 * MB)]) == INV  # K % 4
    assert run([A, W, b], [C]) == INV  # no copy output
    big = d((8192, K), ptr=16 * MB)
    assert run([big, W, b], [d((8192, N), ptr=40 * MB), Wc]) == INV  # not a small problem
    # the general epilogue variants refuse the two-output call
    assert call(lib, GEMM_EPILOGUE, [A, W, b], [C, Wc], GEPI, struct.pack("<iii", 0, 1, 0),
                "gemm_bias_relu_f32_naive_v0") == INV


def test_group_jobs_refuse_operands_past_32_bit_offsets():
    """The small GEMM reads through 32-bit buffer offsets: a GEMM whose
    operand spans 2^31 bytes or more stays out of the group (the host check
    of the kernel refuses it too)."""
    from aicf_hip.ir import IRGraph
    from aicf_hip.lower import _job_of

    ir = IRGraph(name="wide")
    nv = lambda n, s: ir.new_value(name=n, shape=s, dtype="torch.float32", device="cpu").id  # noqa: E731
    a, b, c = nv("a", (16, 1 << 27)), nv("b", (1 << 27, 16)), nv("c", (16, 16))
    it = {"op": "gemm", "inputs": [a, b], "outputs": [c], "attrs": {}}
    assert _job_of(ir, it) is None  # 16 x 2^27 floats = 8 GiB
    a2, b2 = nv("a2", (16, 1 << 20)), nv("b2", (1 << 20, 16))
    assert _job_of(ir, {"op": "gemm", "inputs": [a2, b2], "outputs": [c], "attrs": {}}) is not None
