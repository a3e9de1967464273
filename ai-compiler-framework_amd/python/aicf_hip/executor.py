"""Planned executor: runs a lowered op list through aicf_cuda._C, or
captures it once as a hipGraph and replays it.

Follows the reference's PlannedExecutor (core_v2/exec.py:302-497):
  * build_env allocates statics and binds caller inputs/params by name
    (exact name, then name without a "d_" prefix, then suffix match) with
    shape/dtype/device checks (exec.py:60-174,337-390);
  * _execute_lowered calls _C.launch_by_id when an op carries a kernel_id,
    else _C.op_call, unless require_kernel_id forbids runtime dispatch
    (exec.py:393-453);
  * AICF_WARMUP=1 turns step_inc into a copy and runs Adam with lr 0
    (exec.py:396,423-431);
  * capture = graph_begin, the same op loop on the capture stream,
    graph_end; replay = n x graph_launch (exec.py:467-497).
With own_graph=True the executor captures into a graph handle of its own
(_C.graph_create) instead of the process-wide graph, so several executors
stay instantiated side by side; capturing again on that handle (recapture,
e.g. after binding other input tensors) updates the executable in place.
Attributes are packed for every op that has any (the reference packs only
gemm, gemm_epilogue and adam_step, exec.py:263-277, so e.g. sgd_step ran
with its default lr).
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple

import torch

from aicf_cuda import _C

from .ir import IRGraph
from .lower import EPILOGUE_KINDS, epilogue_kind  # noqa: F401 (re-exported)
from .plan import BindingPlan, allocate_static_env, bind_views


@dataclass
class ExecOptions:
    debug: bool = False
    debug_limit: int = 50
    check_shapes: bool = True
    check_device: bool = True
    check_dtype: bool = True
    require_kernel_id: bool = False


OPNAME_TO_KIND: Dict[str, int] = {
    "add": int(_C.OpKind.EltwiseAdd), "relu": int(_C.OpKind.EltwiseRelu),
    "gemm": int(_C.OpKind.Gemm), "bias_add": int(_C.OpKind.BiasAdd),
    "reduce_sum": int(_C.OpKind.ReduceSum), "mse_grad": int(_C.OpKind.MseGrad),
    "mse_loss": int(_C.OpKind.MseGrad), "relu_bwd": int(_C.OpKind.ReluBwd),
    "sgd_step": int(_C.OpKind.SgdStep), "copy": int(_C.OpKind.Copy),
    "copy_saved": int(_C.OpKind.Copy), "copy_aux": int(_C.OpKind.Copy),
    "grad_zero": int(_C.OpKind.GradZero), "adam_step": int(_C.OpKind.AdamStep),
    "adamw_step": int(_C.OpKind.AdamStep), "step_inc": int(_C.OpKind.StepInc),
    "bias_corr": int(_C.OpKind.BiasCorr), "layernorm_fwd": int(_C.OpKind.LayerNormFwd),
    "layernorm_bwd": int(_C.OpKind.LayerNormBwd), "batchnorm_fwd": int(_C.OpKind.BatchNormFwd),
    "batchnorm_bwd": int(_C.OpKind.BatchNormBwd), "gemm_epilogue": int(_C.OpKind.GemmEpilogue),
    "row_softmax": int(_C.OpKind.RowSoftmax), "row_reduce": int(_C.OpKind.RowReduce),
    "softmax_xent": int(_C.OpKind.SoftmaxXent), "gelu_bwd": int(_C.OpKind.GeluBwd),
    "gelu": int(_C.OpKind.EltwiseGelu), "transpose": int(_C.OpKind.Transpose),
    "gemm_adamw": int(_C.OpKind.GemmAdamW), "xent_head": int(_C.OpKind.XentHead),
    "grad_group": int(_C.OpKind.GradGroup), "adamw_multi": int(_C.OpKind.AdamWMulti),
    "mse_colsum": int(_C.OpKind.MseColsum), "colsum_adamw": int(_C.OpKind.ColsumAdamW),
    "grad_group_adamw": int(_C.OpKind.GradGroup), "gemm_epilogue_bcopy": int(_C.OpKind.GemmEpilogue),
}


def _fourcc_le(tag: bytes) -> int:
    return int.from_bytes(tag, "little")


SCHEMA_ADAM = _fourcc_le(b"ADAM")
SCHEMA_GGRA = _fourcc_le(b"GGRA")
SCHEMA_XHST = _fourcc_le(b"XHST")
SCHEMA_GEPI = _fourcc_le(b"GEPI")
SCHEMA_BCOR = _fourcc_le(b"BCOR")
SCHEMA_SGDS = _fourcc_le(b"SGDS")
SCHEMA_MSEG = _fourcc_le(b"MSEG")
SCHEMA_RRED = _fourcc_le(b"RRED")
SCHEMA_GADW = _fourcc_le(b"GADW")
SCHEMA_GGRP = _fourcc_le(b"GGRP")
SCHEMA_MSCS = _fourcc_le(b"MSCS")
SCHEMA_CADW = _fourcc_le(b"CADW")
SCHEMA_GEMM = int.from_bytes(b"GEMM", "big")
SCHEMA_RSUM = int.from_bytes(b"RSUM", "big")



def warmup_attrs(op: str, attrs: Dict[str, Any]) -> Dict[str, Any]:
    """Attributes of an op under AICF_WARMUP=1 (exec.py:423-431): every Adam
    update runs with lr 0, and a grad_group's step_inc job and the step
    increments of mse_colsum and xent_head add 0 (the copy the warmup makes
    of step_inc)."""
    if op in ("adam_step", "adamw_step", "gemm_adamw", "adamw_multi", "colsum_adamw", "grad_group_adamw"):
        return dict(attrs, lr=0.0)
    if op == "mse_colsum":  # its step_inc part adds 0
        return dict(attrs, step_inc=0)
    if op == "xent_head" and "step_inc" in attrs:  # adds 0; the bias corrections it writes carry lr 0
        return dict(attrs, step_inc=0, **({"lr": 0.0} if "lr" in attrs else {}))
    if op == "grad_group":
        return dict(attrs, jobs=[[j[0], j[1], j[2], j[3], 0 if j[0] == 3 else j[4], j[5]]
                                 for j in attrs.get("jobs", [])])
    return attrs


def pack_attrs(op: str, attrs: Dict[str, Any]) -> Tuple[int, bytes]:
    op = str(op).strip().lower()
    a = dict(attrs or {})
    if op == "gemm":
        return 0, struct.pack("<ii", int(bool(a.get("transA", False))), int(bool(a.get("transB", False))))
    if op in ("gemm_epilogue", "gemm_epilogue_bcopy"):
        return SCHEMA_GEPI, struct.pack("<iii", int(bool(a.get("transA", False))),
                                        int(bool(a.get("transB", False))), epilogue_kind(a))
    if op == "gemm_adamw":
        return SCHEMA_GADW, struct.pack("<iifffff", int(bool(a.get("transA", False))),
                                        int(bool(a.get("transB", False))), float(a.get("lr", 1e-3)),
                                        float(a.get("beta1", 0.9)), float(a.get("beta2", 0.999)),
                                        float(a.get("eps", 1e-8)), float(a.get("weight_decay", 0.0)))
    if op == "mse_colsum":
        return SCHEMA_MSCS, struct.pack("<fi", float(a.get("scale", 0.0)), int(a.get("step_inc", 1)))
    if op == "colsum_adamw":
        return SCHEMA_CADW, struct.pack("<ifffff", int(a["tensors"]), float(a.get("lr", 1e-3)),
                                        float(a.get("beta1", 0.9)), float(a.get("beta2", 0.999)),
                                        float(a.get("eps", 1e-8)), float(a.get("weight_decay", 0.0)))
    if op == "grad_group":
        jobs = [tuple(int(x) for x in j) for j in a.get("jobs", [])]
        return SCHEMA_GGRP, struct.pack("<i", len(jobs)) + b"".join(struct.pack("<iiiiii", *j) for j in jobs)
    if op == "grad_group_adamw":
        jobs = [tuple(int(x) for x in j) for j in a.get("jobs", [])]
        head = struct.pack("<ifffffi", len(jobs), float(a.get("lr", 1e-3)), float(a.get("beta1", 0.9)),
                           float(a.get("beta2", 0.999)), float(a.get("eps", 1e-8)),
                           float(a.get("weight_decay", 0.0)), int(a["scalars_input"]))
        return SCHEMA_GGRA, head + b"".join(struct.pack("<" + "i" * 12, *j) for j in jobs)
    if op == "xent_head" and "step_inc" in a:
        pay = struct.pack("<i", int(a["step_inc"]))
        if "lr" in a:  # the step's AdamW bias corrections too
            pay += struct.pack("<fff", float(a["lr"]), float(a.get("beta1", 0.9)), float(a.get("beta2", 0.999)))
        return SCHEMA_XHST, pay
    if op in ("adam_step", "adamw_step", "adamw_multi"):
        vals = [float(a.get("lr", 1e-3)), float(a.get("beta1", 0.9)), float(a.get("beta2", 0.999)),
                float(a.get("eps", 1e-8))]
        if op in ("adamw_step", "adamw_multi"):
            vals.append(float(a.get("weight_decay", 0.0)))
        return SCHEMA_ADAM, struct.pack("<" + "f" * len(vals), *vals)
    if op == "bias_corr":
        return SCHEMA_BCOR, struct.pack("<ff", float(a.get("beta1", 0.9)), float(a.get("beta2", 0.999)))
    if op == "sgd_step" and "lr" in a:
        return SCHEMA_SGDS, struct.pack("<f", float(a["lr"]))
    if op in ("mse_grad", "mse_loss") and "scale" in a:
        return SCHEMA_MSEG, struct.pack("<f", float(a["scale"]))
    if op == "reduce_sum" and "axis" in a:
        return SCHEMA_RSUM, struct.pack("<q", int(a["axis"]))
    if op == "row_reduce":
        return SCHEMA_RRED, struct.pack("<i", 1 if str(a.get("op", "sum")) == "max" else 0)
    return 0, b""


def _unwrap(x):
    return x.data if hasattr(x, "data") and not isinstance(x, torch.Tensor) else x


def _canon(s: str) -> str:
    return s[2:] if s.startswith("d_") else s


class PlannedExecutor:
    def __init__(self, *, ir: IRGraph, lowered: List[Dict[str, Any]], plan: BindingPlan,
                 device: Optional[torch.device] = None, opts: Optional[ExecOptions] = None,
                 own_graph: bool = False):
        self.ir = ir
        self.lowered = lowered
        self.plan = plan
        self.device = device
        self.opts = opts or ExecOptions()
        self.env: Dict[int, torch.Tensor] = {}
        self._captured = False
        self._steps = 1  # passes over the ops per captured graph (capture(steps=...))
        self._own_graph = bool(own_graph)
        self._handle: Optional[int] = None
        # resolve kinds and pack attributes once; the per-op host work in the
        # loop is then only the tensor list lookup and the binding call
        self._ops = []
        for it in lowered:
            op = str(it["op"]).strip().lower()
            if op not in OPNAME_TO_KIND:
                raise RuntimeError(f"[exec] unsupported lowered op '{op}' (no OpKind mapping)")
            self._ops.append((op, OPNAME_TO_KIND[op], it.get("kernel_id"),
                              [int(x) for x in it.get("inputs", [])],
                              [int(y) for y in it.get("outputs", [])], dict(it.get("attrs", {}) or {})))

    # ---- trace passthrough (exec.py:318-334)
    def trace_enable(self, flag: bool = True) -> None:
        _C.trace_enable(bool(flag))

    def trace_reset(self) -> None:
        _C.trace_reset()

    def trace_get(self) -> List[str]:
        return list(_C.trace_get())

    # ---- binding
    def _check(self, vid: int, t: torch.Tensor) -> None:
        spec = self.plan.specs[vid]
        o = self.opts
        if o.check_shapes and tuple(t.shape) != tuple(spec.shape):
            raise RuntimeError(f"[plan] shape mismatch for vid{vid}({spec.name}): "
                               f"{tuple(t.shape)} != {tuple(spec.shape)}")
        if o.check_dtype:
            want = spec.dtype.replace("torch.", "")
            if str(t.dtype).replace("torch.", "") != want:
                raise RuntimeError(f"[plan] dtype mismatch for vid{vid}({spec.name}): {t.dtype} vs {spec.dtype}")
        if o.check_device and "cuda" in spec.device and not t.is_cuda:
            raise RuntimeError(f"[plan] device mismatch for vid{vid}({spec.name}): expected cuda, got {t.device}")

    def _candidates(self, key: str) -> List[int]:
        specs = self.plan.specs
        exact = [v for v, s in specs.items() if s.name == key]
        if exact:
            return exact
        canon = [v for v, s in specs.items() if _canon(s.name) == _canon(key)]
        if canon:
            return canon
        suffix = [v for v, s in specs.items() if s.name.endswith(key)]
        if suffix:
            return suffix
        return [v for v, s in specs.items() if _canon(s.name).endswith(_canon(key))]

    def build_env(self, *, inputs: Dict[str, Any], params: Dict[str, Any],
                  reuse_static: bool = False) -> Dict[int, torch.Tensor]:
        if not reuse_static or not self.env:
            self.env = allocate_static_env(self.ir, self.plan, device=self.device)
        for kind, src in (("input", inputs), ("param", params)):
            for name, obj in src.items():
                t = _unwrap(obj)
                if not isinstance(t, torch.Tensor):
                    raise TypeError(f"[plan] {kind} '{name}' must be torch.Tensor-like, got {type(obj)}")
                cands = self._candidates(str(name))
                pref = [v for v in cands if self.plan.specs[v].role == kind] or cands
                chosen = None
                for v in pref:
                    try:
                        self._check(v, t)
                        chosen = v
                        break
                    except RuntimeError:
                        continue
                if chosen is None:
                    raise KeyError(f"[plan] unknown or ambiguous {kind} name='{name}'. candidates={cands}")
                self.env[chosen] = t
        bind_views(self.ir, self.env)
        for vid in self.plan.inputs + self.plan.params + self.plan.statics:
            if vid not in self.env:
                s = self.plan.specs[vid]
                raise RuntimeError(f"[plan] env missing vid{vid} ({s.name}) role={s.role}")
        return self.env

    # ---- execution
    @torch.no_grad()
    def _execute_lowered(self, *, stream: int) -> None:
        warmup = os.getenv("AICF_WARMUP", "0") == "1"
        for i in range(len(self._ops)):
            self.launch_op(i, stream=stream, warmup=warmup)

    @property
    def ops(self) -> List[Tuple[str, int, Optional[str], List[int], List[int], Dict[str, Any]]]:
        """The lowered ops as (op, kind, kernel_id, input vids, output vids, attrs)."""
        return list(self._ops)

    def launch_op(self, i: int, *, stream: int = 0, warmup: bool = False) -> None:
        """Launches lowered op i on the bound tensors (one step of run())."""
        op, kind, kid, ins, outs, attrs = self._ops[i]
        env = self.env
        ins_t = [env[v] for v in ins]
        outs_t = [env[v] for v in outs]
        if self.opts.debug and i < self.opts.debug_limit:
            print(f"[exec][#{i:03d}] {op} kind={kind} kernel_id={kid} attrs={attrs}")
        if warmup and op == "step_inc":
            outs_t[0].copy_(ins_t[0])
            return
        if warmup:
            attrs = warmup_attrs(op, attrs)
        schema, payload = pack_attrs(op, attrs)
        if kid is not None:
            _C.launch_by_id(str(kid), _C.OpKind(kind), ins_t, outs_t, schema, payload, int(stream))
        else:
            if self.opts.require_kernel_id:
                raise RuntimeError(f"[exec] require_kernel_id=True but lowered op #{i} '{op}' has no kernel_id")
            _C.op_call(kind, ins_t, outs_t, schema, payload, int(stream))

    @torch.no_grad()
    def run(self, *, inputs: Dict[str, Any], params: Dict[str, Any],
            reuse_static: bool = True) -> Dict[int, torch.Tensor]:
        self.build_env(inputs=inputs, params=params, reuse_static=reuse_static)
        self._execute_lowered(stream=0)
        return self.env

    @torch.no_grad()
    def capture(self, *, inputs: Dict[str, Any], params: Dict[str, Any],
                reuse_static: bool = True, steps: int = 1) -> Dict[int, torch.Tensor]:
        """Binds and captures the lowered ops into the graph.  steps > 1
        (not in the reference executor): the graph holds that many
        consecutive passes over the ops, and one replay advances as many
        steps (for steps of a few microseconds, where a graph launch's own
        cost is a large part of a replay)."""
        if int(steps) < 1:
            raise ValueError("[exec] capture: steps must be >= 1")
        self._steps = int(steps)
        self.build_env(inputs=inputs, params=params, reuse_static=reuse_static)
        self._capture_env()
        return self.env

    @torch.no_grad()
    def recapture(self, *, inputs: Optional[Dict[str, Any]] = None,
                  params: Optional[Dict[str, Any]] = None) -> Dict[int, torch.Tensor]:
        """Binds the given tensors over the current environment (statics are
        kept) and captures again.  On an own graph handle the executable is
        updated in place when the op sequence is unchanged."""
        if not self.env:
            raise RuntimeError("[exec] recapture called before capture()")
        self.build_env(inputs=dict(inputs or {}), params=dict(params or {}), reuse_static=True)
        self._capture_env()
        return self.env

    def _capture_env(self) -> None:
        # work queued on torch's stream (initialisation of the bound tensors)
        # must be complete before the first replay reads them
        torch.cuda.synchronize()
        self._captured = False
        if self._own_graph:
            if self._handle is None:
                self._handle = int(_C.graph_create())
            s = int(_C.graph_begin_h(self._handle))
            try:
                for _ in range(self._steps):
                    self._execute_lowered(stream=s)
            finally:
                _C.graph_end_h(self._handle)
        else:
            s = int(_C.graph_begin())
            try:
                for _ in range(self._steps):
                    self._execute_lowered(stream=s)
            finally:
                _C.graph_end()
        self._captured = True

    @torch.no_grad()
    def replay(self, n: int = 1) -> None:
        if n <= 0:
            return
        if not self._captured:
            raise RuntimeError("[exec] replay called before capture()")
        if self._handle is not None:
            _C.graph_launch_h_n(self._handle, int(n))
        else:
            for _ in range(int(n)):
                _C.graph_launch()

    @property
    def steps_per_replay(self) -> int:
        """Steps one replay advances (capture(steps=...))."""
        return self._steps

    @property
    def graph_handle(self) -> Optional[int]:
        return self._handle

    @property
    def graph_updates(self) -> int:
        """Captures applied to this executor's own graph by in-place update."""
        return int(_C.graph_updates_h(self._handle)) if self._handle is not None else 0

    def graph_stream(self) -> int:
        return int(_C.graph_stream_h(self._handle)) if self._handle is not None else int(_C.graph_stream())

    def reset_graph(self) -> None:
        if self._handle is not None:
            _C.graph_reset_h(self._handle)
        else:
            _C.graph_reset()
        self._captured = False

    def close(self) -> None:
        """Releases the own graph handle (its graph, stream and event)."""
        if self._handle is not None:
            h, self._handle = self._handle, None
            _C.graph_destroy(h)
        self._captured = False

    def value(self, name: str) -> torch.Tensor:
        return self.env[self.ir.by_name(name).id]
