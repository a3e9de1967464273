"""Symbolic IR: values (id, name, shape, dtype, device) and nodes
(op, input ids, output ids, attrs).

Same data model as the reference's core_v2/ir.py:7-46 so that graphs and
their text dumps line up one to one.  A value may be declared as a view of
another value (`view_of=(base_vid, element_offset)`); the binding plan then
allocates only the base and hands out views, which is how flat parameter /
gradient / optimizer-state buffers are laid out in HBM.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Tuple


@dataclass(frozen=True)
class IRValue:
    id: int
    name: str
    shape: Tuple[int, ...]
    dtype: str
    device: str
    view_of: Optional[Tuple[int, int]] = None  # (base vid, element offset)


@dataclass
class IRNode:
    op: str
    inputs: List[int]
    outputs: List[int]
    attrs: Dict[str, Any] = field(default_factory=dict)


@dataclass
class IRGraph:
    name: str = "graph"
    values: Dict[int, IRValue] = field(default_factory=dict)
    nodes: List[IRNode] = field(default_factory=list)
    _next_vid: int = 0

    def new_value(self, *, name: str, shape, dtype: str, device: str = "cuda:0",
                  view_of: Optional[Tuple[int, int]] = None) -> IRValue:
        v = IRValue(self._next_vid, str(name), tuple(int(s) for s in shape), str(dtype),
                    str(device), view_of)
        self.values[v.id] = v
        self._next_vid += 1
        return v

    def emit(self, *, op: str, inputs: List[IRValue], outputs: List[IRValue],
             attrs: Optional[Dict[str, Any]] = None) -> IRNode:
        n = IRNode(str(op), [int(v.id) for v in inputs], [int(v.id) for v in outputs],
                   dict(attrs or {}))
        self.nodes.append(n)
        return n

    def by_name(self, name: str) -> IRValue:
        for v in self.values.values():
            if v.name == name:
                return v
        raise KeyError(name)

    def dump(self) -> str:
        """Text dump in the layout of the reference's 20_ir.txt artifact."""
        lines = [f"=== IRGraph: {self.name} ===",
                 f"values: {len(self.values)}, nodes: {len(self.nodes)}", "", "[values]"]
        for vid in sorted(self.values):
            v = self.values[vid]
            lines.append(f"  v{vid:03d}  {v.name:<12} shape={v.shape} dtype={v.dtype} device={v.device}")
        lines += ["", "[nodes]"]
        for i, n in enumerate(self.nodes):
            ins = ", ".join(f"v{x:03d}" for x in n.inputs)
            outs = ", ".join(f"v{x:03d}" for x in n.outputs)
            a = ""
            if n.attrs:
                a = "  {" + ", ".join(f"{k}={v}" for k, v in n.attrs.items()) + "}"
            lines.append(f"  #{i:03d} {n.op:<10} ({ins}) -> ({outs}){a}")
        return "\n".join(lines)
