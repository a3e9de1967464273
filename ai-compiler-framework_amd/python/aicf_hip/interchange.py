"""Plan interchange: the JSON IR and lowered-list formats of the reference.

* JSON IR — the document the reference's JSON executable reads
  (core_v2/cuda_exec.py:306-371): ``{"graph": name, "values": {key: {"id",
  "name", "shape", "dtype", "device"}}, "nodes": [{"op", "inputs",
  "outputs", "attrs"}]}``, inputs/outputs as value ids.  Nodes may be IR ops
  (Linear, ReLU, LinearBwd, ...) or ops that are already lowered (gemm,
  bias_add, ...); both go through the same lowering (StageA passes lowered
  ops through).  An optional ``"view_of": [base_id, element_offset]`` on a
  value carries this build's flat-buffer views; readers that do not know it
  ignore it.
* Lowered list — the dicts ``{"op", "inputs", "outputs", "attrs",
  "kernel_id"}`` of core_v2/lower.py:9-21 and their text dump
  (``30_lowered.txt`` layout, written by ``lower.lowered_to_text``);
  ``lowered_from_text`` reads that dump back.

Errors follow the reference reader: a missing "values" or "nodes" key, or a
node naming an unknown value id, raises ValueError.
"""
from __future__ import annotations

import json
import re
from typing import Any, Dict, List

from .ir import IRGraph, IRNode, IRValue

Lowered = List[Dict[str, Any]]


# ---------------------------------------------------------------- JSON IR
def ir_to_dict(ir: IRGraph) -> Dict[str, Any]:
    values: Dict[str, Any] = {}
    for vid in sorted(ir.values):
        v = ir.values[vid]
        d: Dict[str, Any] = {"id": v.id, "name": v.name, "shape": list(v.shape), "dtype": v.dtype,
                             "device": v.device}
        if v.view_of is not None:
            d["view_of"] = [int(v.view_of[0]), int(v.view_of[1])]
        values[str(vid)] = d
    nodes = [{"op": n.op, "inputs": list(n.inputs), "outputs": list(n.outputs), "attrs": dict(n.attrs)}
             for n in ir.nodes]
    return {"graph": ir.name, "values": values, "nodes": nodes}


def ir_to_json(ir: IRGraph, **kw) -> str:
    return json.dumps(ir_to_dict(ir), **kw)


def ir_from_dict(root: Dict[str, Any]) -> IRGraph:
    """Rebuilds an IRGraph with the document's value ids (cuda_exec.py:320-371)."""
    if "values" not in root:
        raise ValueError("missing 'values'")
    if "nodes" not in root:
        raise ValueError("missing 'nodes'")
    ir = IRGraph(name=str(root.get("graph", "graph")))
    max_id = -1
    for v in root["values"].values():
        vid = int(v["id"])
        view = v.get("view_of")
        ir.values[vid] = IRValue(vid, str(v["name"]), tuple(int(s) for s in v["shape"]), str(v["dtype"]),
                                 str(v["device"]), (int(view[0]), int(view[1])) if view is not None else None)
        max_id = max(max_id, vid)
    ir._next_vid = max_id + 1
    for n in root["nodes"]:
        ins = [int(x) for x in n.get("inputs", [])]
        outs = [int(x) for x in n.get("outputs", [])]
        for vid in ins:
            if vid not in ir.values:
                raise ValueError(f"invalid input vid={vid}")
        for vid in outs:
            if vid not in ir.values:
                raise ValueError(f"invalid output vid={vid}")
        ir.nodes.append(IRNode(str(n["op"]), ins, outs, dict(n.get("attrs", {}) or {})))
    return ir


def ir_from_json(text: str) -> IRGraph:
    return ir_from_dict(json.loads(text))


# ---------------------------------------------------------------- lowered list
_LINE = re.compile(r"^\s*#(\d+)\s+(\S+)\s+\(([^)]*)\)\s+->\s+\(([^)]*)\)(?:\s+\{(.*)\})?(?:\s+kid=(\S+))?\s*$")


def _attr_value(s: str) -> Any:
    if s in ("True", "False"):
        return s == "True"
    if s.startswith("["):  # a list attribute (grad_group jobs): Python literal of ints
        return json.loads(s)
    for cast in (int, float):
        try:
            return cast(s)
        except ValueError:
            pass
    return s


def _split_top(s: str) -> List[str]:
    """Splits `k=v, k=v` at the commas outside brackets."""
    parts, depth, cur = [], 0, ""
    for i, ch in enumerate(s):
        depth += ch == "["
        depth -= ch == "]"
        if depth == 0 and s.startswith(", ", i):
            parts.append(cur)
            cur = ""
            continue
        if depth == 0 and ch == " " and cur == "":
            continue
        cur += ch
    parts.append(cur)
    return parts


def lowered_from_text(text: str) -> Lowered:
    """Parses a lowered-ops dump (the 30_lowered.txt layout) into lowered dicts."""
    out: Lowered = []
    for line in text.splitlines():
        if not line.strip().startswith("#"):
            continue
        m = _LINE.match(line)
        if not m:
            raise ValueError(f"unparsable lowered-op line: {line!r}")
        _, op, ins, outs, attrs, kid = m.groups()
        item: Dict[str, Any] = {
            "op": op.strip().lower(),
            "inputs": [int(x) for x in ins.split(",") if x.strip()],
            "outputs": [int(x) for x in outs.split(",") if x.strip()],
            "attrs": {},
        }
        if attrs:
            for kv in _split_top(attrs):
                k, v = kv.split("=", 1)
                item["attrs"][k.strip()] = _attr_value(v.strip())
        if kid:
            item["kernel_id"] = kid
        out.append(item)
    return out


def lowered_to_json(lowered: Lowered, **kw) -> str:
    return json.dumps([dict(it) for it in lowered], **kw)


def lowered_from_json(text: str) -> Lowered:
    items = json.loads(text)
    out: Lowered = []
    for it in items:
        item = {"op": str(it["op"]).strip().lower(), "inputs": [int(x) for x in it.get("inputs", [])],
                "outputs": [int(x) for x in it.get("outputs", [])], "attrs": dict(it.get("attrs", {}) or {})}
        if it.get("kernel_id"):
            item["kernel_id"] = str(it["kernel_id"])
        out.append(item)
    return out
