"""Binding plan: which IR values the caller provides and which the runtime
allocates once, before any capture.

Role rules (reference core_v2/plan.py:49-137):
  input  - name in {"x", "t"}
  static - name starts with "d_", "grad", "dY" or "opt."
  param  - name matches ^\\d+\\.(W|b)$
  static - everything else
Allocation (plan.py:160-209): statics are allocated up front; "opt.step*",
"opt.m.*" and "opt.v.*" start at zero, the rest are uninitialised.  Values
declared as views of another value are bound as views of its buffer.
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Set, Tuple

import torch

from .ir import IRGraph

ROLE_INPUT, ROLE_PARAM, ROLE_STATIC = "input", "param", "static"


@dataclass
class BindSpec:
    vid: int
    role: str
    name: str
    shape: Tuple[int, ...]
    dtype: str
    device: str


@dataclass
class BindingPlan:
    name: str
    specs: Dict[int, BindSpec] = field(default_factory=dict)
    inputs: List[int] = field(default_factory=list)
    params: List[int] = field(default_factory=list)
    statics: List[int] = field(default_factory=list)

    def role_of(self, vid: int) -> str:
        s = self.specs.get(int(vid))
        return s.role if s is not None else "unknown"

    def dump(self) -> str:
        """Text dump in the layout of the reference's 40_plan.txt artifact."""
        lines = [f"=== BindingPlan({self.name.split(':')[0]}) ===", f"name: {self.name}",
                 f"inputs: {len(self.inputs)}, params: {len(self.params)}, statics: {len(self.statics)}"]
        for title, vids in (("inputs", self.inputs), ("params", self.params), ("statics", self.statics)):
            lines += ["", f"[{title}]"]
            for vid in vids:
                s = self.specs[vid]
                lines.append(f"  v{vid:03d}  {s.name:<12} role={s.role:<6} shape={s.shape} "
                             f"dtype={s.dtype} device={s.device}")
        return "\n".join(lines)


@dataclass
class PlanOptions:
    input_names: Set[str] = field(default_factory=lambda: {"x", "t"})
    param_regex: str = r"^\d+\.(W|b)$"
    static_prefixes: Tuple[str, ...] = ("d_", "grad", "dY", "opt.")
    # extra names bound by the caller as params (e.g. a flat parameter buffer
    # whose per-layer views carry the "<i>.W" / "<i>.b" names)
    param_names: Set[str] = field(default_factory=set)


def build_binding_plan(ir: IRGraph, *, opts: Optional[PlanOptions] = None) -> BindingPlan:
    opts = opts or PlanOptions()
    pre = re.compile(opts.param_regex)
    plan = BindingPlan(name=f"{ir.name}:binding_plan")
    for vid in sorted(ir.values):
        v = ir.values[vid]
        nm = v.name
        if nm in opts.input_names:
            role = ROLE_INPUT
        elif nm in opts.param_names:
            role = ROLE_PARAM
        elif any(nm.startswith(p) for p in opts.static_prefixes):
            role = ROLE_STATIC
        elif pre.match(nm):
            role = ROLE_PARAM
        else:
            role = ROLE_STATIC
        plan.specs[vid] = BindSpec(vid, role, nm, tuple(v.shape), v.dtype, v.device)
        {ROLE_INPUT: plan.inputs, ROLE_PARAM: plan.params}.get(role, plan.statics).append(vid)
    return plan


def torch_dtype(ds: str) -> torch.dtype:
    for key, dt in (("bfloat16", torch.bfloat16), ("float16", torch.float16),
                    ("float32", torch.float32), ("float64", torch.float64),
                    ("int64", torch.int64), ("int32", torch.int32)):
        if key in str(ds):
            return dt
    return torch.float32


def _zero_init(name: str) -> bool:
    return name.startswith("opt.step") or name.startswith("opt.m.") or name.startswith("opt.v.")


def allocate_static_env(ir: IRGraph, plan: BindingPlan, *,
                        device: Optional[torch.device] = None) -> Dict[int, torch.Tensor]:
    """Allocates every static value (views after their bases)."""
    if device is None:
        dev0 = next((ir.values[v].device for v in plan.statics), "cuda")
        device = torch.device(dev0 if "cuda" in dev0 else "cuda")
    env: Dict[int, torch.Tensor] = {}
    for vid in sorted(plan.statics, key=lambda v: ir.values[v].view_of is not None):
        v = ir.values[vid]
        if v.view_of is not None:
            continue
        dt = torch_dtype(v.dtype)
        env[vid] = (torch.zeros if _zero_init(v.name) else torch.empty)(v.shape, device=device, dtype=dt)
    bind_views(ir, env, set(plan.statics))
    return env


def bind_views(ir: IRGraph, env: Dict[int, torch.Tensor], vids: Optional[set] = None) -> None:
    """Creates env entries for values declared as views of bound bases."""
    for vid, v in ir.values.items():
        if v.view_of is None or (vids is not None and vid not in vids):
            continue
        base, off = v.view_of
        if base not in env:
            continue
        n = 1
        for d in v.shape:
            n *= int(d)
        env[vid] = env[base].view(-1)[off:off + n].view(v.shape)
