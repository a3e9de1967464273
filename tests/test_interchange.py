"""Plan interchange (JSON IR of core_v2/cuda_exec.py:306-371, lowered list of
core_v2/lower.py:9-21): round trips reproduce the reference's recorded
artifacts byte for byte, and externally produced plans lower and bind like
graphs built in Python."""
from __future__ import annotations

import json
from pathlib import Path

import pytest

GOLD = Path(__file__).resolve().parent / "golden" / "kid_trace"


def _ref(name: str) -> str:
    return (GOLD / name).read_text().rstrip("\n")


def _kid_trace_lowering(ir):
    """The reference's stage order for the kid-trace graph: A, B, C, B."""
    from aicf_hip.lower import apply_kernel_selection, fuse_gemm_epilogue, lower_to_backend_ops

    low = apply_kernel_selection(ir, lower_to_backend_ops(ir))
    low = fuse_gemm_epilogue(ir, [dict(it) for it in low])
    return apply_kernel_selection(ir, low)


def test_json_ir_round_trip_reproduces_artifacts():
    from aicf_hip.interchange import ir_from_json, ir_to_json
    from aicf_hip.kid_trace import build_kid_trace_graph
    from aicf_hip.lower import lowered_to_text
    from aicf_hip.plan import build_binding_plan

    ir, _, _ = build_kid_trace_graph()
    doc = ir_to_json(ir)
    root = json.loads(doc)
    assert set(root) == {"graph", "values", "nodes"}
    assert root["values"]["0"] == {"id": 0, "name": "x", "shape": [64, 8], "dtype": "torch.float16",
                                   "device": "cuda:0"}
    ir2 = ir_from_json(doc)
    assert ir2.dump() == _ref("20_ir.txt")
    low2 = _kid_trace_lowering(ir2)
    assert lowered_to_text(low2, ir2.name) == _ref("30_lowered.txt")
    assert build_binding_plan(ir2).dump() == _ref("40_plan.txt")
    # new values continue after the document's highest id
    assert ir2.new_value(name="extra", shape=(1,), dtype="torch.float32").id == max(ir.values) + 1


def test_lowered_text_round_trip():
    from aicf_hip.interchange import lowered_from_json, lowered_from_text, lowered_to_json
    from aicf_hip.lower import lowered_to_text

    text = _ref("30_lowered.txt")
    low = lowered_from_text(text)
    assert len(low) == 16
    assert low[0] == {"op": "gemm_epilogue", "inputs": [0, 1, 2], "outputs": [4],
                      "attrs": {"epilogue_act": "relu", "epilogue_bias": True, "transB": True},
                      "kernel_id": "gemm_bias_relu_f16_tc_wmma_out_f16_v0"}
    assert low[12]["attrs"] == {"lr": 0.01}
    assert lowered_to_text(low, "v2_kid_trace_by_id_test") == text
    assert lowered_from_json(lowered_to_json(low)) == low


def test_json_with_lowered_nodes_passes_through():
    """A document whose nodes are already lowered ops (as the reference's
    JSON executable accepts, cuda_exec.py:155-162) lowers to the same list."""
    from aicf_hip.interchange import ir_from_dict, ir_to_dict, lowered_from_text
    from aicf_hip.kid_trace import build_kid_trace_graph
    from aicf_hip.lower import apply_kernel_selection, lower_to_backend_ops, lowered_to_text

    ir, lowered, _ = build_kid_trace_graph()
    root = ir_to_dict(ir)
    root["nodes"] = [{"op": it["op"], "inputs": it["inputs"], "outputs": it["outputs"],
                      "attrs": it.get("attrs", {})} for it in lowered_from_text(_ref("30_lowered.txt"))]
    ir2 = ir_from_dict(root)
    low2 = apply_kernel_selection(ir2, lower_to_backend_ops(ir2))
    assert lowered_to_text(low2, ir2.name) == _ref("30_lowered.txt")


def test_flat_buffer_views_survive_the_round_trip():
    from aicf_hip import mlp
    from aicf_hip.interchange import ir_from_json, ir_to_json
    from aicf_hip.plan import PlanOptions, build_binding_plan

    ir, lowered, plan = mlp.build_mlp_mse(256, 128, 2)
    ir2 = ir_from_json(ir_to_json(ir))
    assert ir2.values == ir.values
    assert any(v.view_of is not None for v in ir2.values.values())
    assert build_binding_plan(ir2, opts=PlanOptions(param_names={"flat.params"})).dump() == plan.dump()


def test_reader_errors():
    from aicf_hip.interchange import ir_from_dict, lowered_from_text

    with pytest.raises(ValueError, match="missing 'values'"):
        ir_from_dict({"nodes": []})
    with pytest.raises(ValueError, match="missing 'nodes'"):
        ir_from_dict({"values": {}})
    v = {"0": {"id": 0, "name": "x", "shape": [2], "dtype": "torch.float32", "device": "cuda:0"}}
    with pytest.raises(ValueError, match="invalid input vid=3"):
        ir_from_dict({"values": v, "nodes": [{"op": "relu", "inputs": [3], "outputs": [0]}]})
    with pytest.raises(ValueError, match="invalid output vid=5"):
        ir_from_dict({"values": v, "nodes": [{"op": "relu", "inputs": [0], "outputs": [5]}]})
    with pytest.raises(ValueError, match="unparsable"):
        lowered_from_text("  #000 gemm (0, 1 -> (2)")
