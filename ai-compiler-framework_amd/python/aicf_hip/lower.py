"""Lowering of the IR to the backend's primitive ops, plus the two
compile-time rewrites of the reference pipeline:

* StageA  lower_to_backend_ops  (reference core_v2/lower.py:24-147)
    Linear    -> gemm(transB=True) + in-place bias_add
    LinearBwd -> gemm dX = dY.W, gemm dW = dY^T.X, reduce_sum(axis 0) for db
    Save      -> copy_saved;  other ops map one to one
  and the ops this backend appends (GELU, softmax cross-entropy, fused MSE
  loss, AdamW with in-kernel bias correction, row softmax / reduce).
* StageC  fuse_gemm_epilogue    (reference rewrites/stageC_fuse_epilogue.py:5-76)
    gemm [-> bias_add in place] -> relu  ==> gemm_epilogue (bias_relu/relu)
  extended with gemm -> bias_add -> gelu (==> bias_gelu, keeping the
  pre-activation when a later gelu_bwd needs it) and gemm -> gelu_bwd
  (==> dgelu epilogue).
* StageC' fuse_colsum_into_dgelu (not in the reference; opt-in): the column
  sum (bias gradient) of a dGELU GEMM's output is taken in that GEMM's
  epilogue (GEPI kind 6) instead of by a reduce_sum over the stored tensor.
* StageE  fuse_optimizer_into_gemms (not in the reference; opt-in): a
  weight-gradient GEMM whose output only feeds the flat AdamW step becomes
  gemm_adamw (AdamW applied in the GEMM's epilogue, no fp32 gradient in
  memory); the flat step keeps the remaining ranges.
* StageF  fuse_small_step (not in the reference; opt-in): for steps whose
  tensors are too small to fill the GPU, so that every launch costs its
  dispatch time rather than its work: copy_saved of a value nothing writes
  again is dropped (readers take the source); the classifier head
  gemm -> bias_add -> softmax_xent with its backward gemm (dY.W) and the
  relu_bwd behind it becomes one xent_head op (one wave per row); runs of
  independent small jobs (fp32 GEMMs with few tiles, column sums, the loss
  mean, step_inc) become one grad_group launch; consecutive adamw_step ops
  sharing step and hyperparameters become one adamw_multi launch.
* StageG  fuse_step_tail (not in the reference; opt-in, after StageC' and
  StageE): the loss and bias tail of a large MSE step in two launches: the
  MSE loss, the last bias's column sums (as partials) and step_inc become one
  mse_colsum op; the dGELU GEMMs keep their column sums as partials (GEPI
  kind 7); the bias AdamW step finishes all of them (colsum_adamw).
* StageB  apply_kernel_selection (reference kernel_select.py:22-142 and the
  vec2/half2 upgrades of plan.py:371-444): pins a kernel_id on every op.

A lowered op is a dict {op, inputs, outputs, attrs[, kernel_id]} - the
format the reference executor consumes (lower.py:9-21, exec.py:393-453).
"""
from __future__ import annotations

from typing import Any, Dict, Iterable, List, Optional

from .ir import IRGraph

Lowered = List[Dict[str, Any]]

_PRIMITIVES = {
    "gemm", "gemm_epilogue", "bias_add", "add", "relu", "reduce_sum", "mse_grad", "relu_bwd",
    "copy", "copy_saved", "copy_aux", "grad_zero", "adam_step", "step_inc", "bias_corr",
    "sgd_step", "gelu", "gelu_bwd", "softmax_xent", "row_softmax", "row_reduce", "mse_loss",
    "adamw_step", "layernorm_fwd", "layernorm_bwd", "batchnorm_fwd", "batchnorm_bwd",
    "transpose", "gemm_adamw", "xent_head", "grad_group", "adamw_multi", "mse_colsum",
    "colsum_adamw", "grad_group_adamw", "gemm_epilogue_bcopy",
}

_ALIASES = {"adamstep": "adam_step", "stepinc": "step_inc", "biascorr": "bias_corr",
            "msegrad": "mse_grad", "relubwd": "relu_bwd", "sgdstep": "sgd_step",
            "linearbwd": "linear_bwd", "gelubwd": "gelu_bwd", "softmaxxent": "softmax_xent",
            "mseloss": "mse_loss", "adamwstep": "adamw_step", "rowsoftmax": "row_softmax",
            "rowreduce": "row_reduce"}


EPILOGUE_KINDS = {"bias_relu": 0, "bias": 1, "relu": 2, "bias_gelu": 3, "gelu": 4, "dgelu": 5}


def epilogue_kind(attrs: Dict[str, Any]) -> int:
    """GEPI kind from either the executor's `epilogue` attr (exec.py:223-252)
    or StageC's epilogue_act / epilogue_bias pair."""
    if "epilogue" in attrs:
        e = str(attrs["epilogue"]).strip().lower().replace("+", "_")
        e = {"biasrelu": "bias_relu", "bias_only": "bias", "biasonly": "bias",
             "relu_only": "relu", "reluonly": "relu"}.get(e, e)
        return EPILOGUE_KINDS.get(e, 0)
    act = str(attrs.get("epilogue_act", "relu")).lower()
    bias = bool(attrs.get("epilogue_bias", True))
    if act == "dgelu":
        cs = attrs.get("epilogue_colsum", False)
        return 7 if cs == "partials" else 6 if cs else 5
    if act == "gelu":
        return 3 if bias else 4
    if act in ("none", ""):
        return 1
    return 0 if bias else 2


def _item(op: str, inputs, outputs, attrs=None) -> Dict[str, Any]:
    return {"op": str(op).strip().lower(), "inputs": [int(x) for x in inputs],
            "outputs": [int(y) for y in outputs], "attrs": dict(attrs or {})}


def lower_to_backend_ops(ir: IRGraph) -> Lowered:
    """StageA: semantics-preserving lowering; no kernel ids yet."""
    out: Lowered = []
    for n in ir.nodes:
        op = str(n.op).strip().lower()
        op = _ALIASES.get(op, op)
        ins, outs, attrs = list(n.inputs), list(n.outputs), dict(n.attrs)
        if op == "linear":
            x, w, y = ins[0], ins[1], outs[0]
            out.append(_item("gemm", [x, w], [y], {"transB": True}))
            if attrs.get("bias", False) and len(ins) >= 3:
                out.append(_item("bias_add", [y, ins[2]], [y]))
        elif op == "linear_bwd":
            x, w, dy = ins[0], ins[1], ins[2]
            dx, dw = outs[0], outs[1]
            if attrs.get("need_dx", True):
                out.append(_item("gemm", [dy, w], [dx], {"transA": False, "transB": False}))
            out.append(_item("gemm", [dy, x], [dw], {"transA": True, "transB": False}))
            if attrs.get("bias", False) and len(outs) >= 3:
                rs_outs = [outs[2]] + ([int(attrs["db_workspace"])] if "db_workspace" in attrs else [])
                out.append(_item("reduce_sum", [dy], rs_outs, {"axis": 0, "keepdim": False}))
        elif op == "save":
            out.append(_item("copy_saved", [ins[0]], [outs[0]]))
        elif op in ("relu", "mse_grad", "relu_bwd", "sgd_step") or op in _PRIMITIVES:
            out.append(_item(op, ins, outs, attrs))
        else:
            raise RuntimeError(f"[lower] unsupported IR op '{n.op}' (normalized='{op}')")
    return out


def _refs(it: Dict[str, Any], vid: int) -> bool:
    return vid in it.get("inputs", []) or vid in it.get("outputs", [])


def fuse_gemm_epilogue(ir: IRGraph, lowered: Lowered, *, fuse_bias: bool = False) -> Lowered:
    """StageC: fold the activation (and an in-place bias add) that consumes a
    GEMM output into the GEMM.  As in the reference rewrite, the bias add and
    relu must follow the GEMM directly; a gelu_bwd may come later as long as
    nothing in between touches the GEMM output."""
    out: Lowered = []
    lowered = list(lowered)
    consumed = set()
    i = 0
    kind = lambda it: str(it.get("op", "")).strip().lower()  # noqa: E731
    while i < len(lowered):
        if i in consumed:
            i += 1
            continue
        g = lowered[i]
        if kind(g) != "gemm" or len(g["outputs"]) != 1:
            out.append(g)
            i += 1
            continue
        y = int(g["outputs"][0])
        j = i + 1
        bias = None
        if j < len(lowered) and kind(lowered[j]) == "bias_add":
            b = lowered[j]
            if len(b["inputs"]) == 2 and int(b["inputs"][0]) == y and b["outputs"] == [y]:
                bias = b
                j += 1
        act = lowered[j] if j < len(lowered) else None
        if bias is None and act is not None and not _refs(act, y):
            # first later op touching y may be a gelu_bwd(y, z)
            k = j
            while k < len(lowered) and not _refs(lowered[k], y):
                k += 1
            if k < len(lowered) and kind(lowered[k]) == "gelu_bwd" and lowered[k]["inputs"][0] == y \
                    and not any(_refs(lowered[q], y) for q in range(k + 1, len(lowered))):
                attrs = dict(g.get("attrs", {}))
                attrs["epilogue_act"] = "dgelu"
                attrs["epilogue_bias"] = False
                out.append({"op": "gemm_epilogue", "inputs": list(g["inputs"]) + [int(lowered[k]["inputs"][1])],
                            "outputs": list(lowered[k]["outputs"]), "attrs": attrs})
                consumed.add(k)
                i += 1
                continue
        attrs = dict(g.get("attrs", {}))
        if act is not None and kind(act) == "relu" and act["inputs"] == [y]:
            attrs["epilogue_act"] = "relu"
            attrs["epilogue_bias"] = bias is not None
            ins = list(g["inputs"]) + ([int(bias["inputs"][1])] if bias else [])
            out.append({"op": "gemm_epilogue", "inputs": ins, "outputs": list(act["outputs"]),
                        "attrs": attrs})
            i = j + 1
        elif act is not None and kind(act) == "gelu" and act["inputs"] == [y]:
            attrs["epilogue_act"] = "gelu"
            attrs["epilogue_bias"] = bias is not None
            ins = list(g["inputs"]) + ([int(bias["inputs"][1])] if bias else [])
            outs = list(act["outputs"])
            if act.get("attrs", {}).get("save_preact", False):
                outs.append(y)  # keep the pre-activation for gelu_bwd
            out.append({"op": "gemm_epilogue", "inputs": ins, "outputs": outs, "attrs": attrs})
            i = j + 1
        elif (bias is None and act is not None and kind(act) == "gelu_bwd"
              and act["inputs"][0] == y):
            attrs["epilogue_act"] = "dgelu"
            attrs["epilogue_bias"] = False
            ins = list(g["inputs"]) + [int(act["inputs"][1])]
            out.append({"op": "gemm_epilogue", "inputs": ins, "outputs": list(act["outputs"]),
                        "attrs": attrs})
            i = j + 1
        elif bias is not None and fuse_bias:
            # bias only (off by default: the reference fuses only with relu)
            attrs["epilogue_act"] = "none"
            attrs["epilogue_bias"] = True
            out.append({"op": "gemm_epilogue", "inputs": list(g["inputs"]) + [int(bias["inputs"][1])],
                        "outputs": [y], "attrs": attrs})
            i = j
        else:
            out.append(g)
            i += 1
    return out


# ---------------------------------------------------------------- StageD
def _writes(it: Dict[str, Any], vid: int) -> bool:
    return vid in it.get("outputs", [])


# Cost model of StageD's "cost" policy (MI355X measurements): a 2-D
# transpose streams its bytes twice at ~5.5 TB/s; reading an M/N-contiguous
# operand in place (transposing LDS loads) costs the GEMM nothing measurable
# against the K-contiguous form (dX GEMM 8192x4096x4096 with dGELU, W in place
# vs W^T: 256.4 vs 256.6 us in the same process), so "cost" transposes
# nothing at that penalty; "all" still normalizes every operand.
TRANSPOSE_BYTES_PER_S = 5.5e12
GEMM_FLOPS_PER_S = 1.2e15
MN_OPERAND_PENALTY = 0.0


def normalize_gemm_layout(ir: IRGraph, lowered: Lowered, *, min_flops: float = 2.0 ** 30,
                          policy: str = "all") -> Lowered:
    """StageD (not in the reference): rewrite 16-bit GEMMs whose operands are
    M/N-contiguous (transA=True on A, transB=False on B) into explicit 2-D
    transposes plus the K-contiguous form (transA=False, transB=True).  The
    GEMM kernel also reads M/N-contiguous operands in place, somewhat slower,
    so the policy decides per operand: "all" transposes every such operand,
    "cost" only those whose transpose is cheaper than the in-place penalty
    (TRANSPOSE_BYTES_PER_S, GEMM_FLOPS_PER_S, MN_OPERAND_PENALTY).  The
    transposed copies become new IR values; a copy is reused while its source
    is not written in between.  Small GEMMs (< min_flops) are left alone."""
    if policy not in ("all", "cost"):
        raise ValueError(f"normalize_gemm_layout: unknown policy {policy!r}")
    out: Lowered = []
    cache: Dict[int, int] = {}  # source vid -> transposed vid (valid until the source is written)
    kind = lambda it: str(it.get("op", "")).strip().lower()  # noqa: E731

    def transposed(src: int) -> int:
        if src in cache:
            return cache[src]
        v = ir.values[src]
        tv = ir.new_value(name=f"{v.name}^T", shape=(v.shape[1], v.shape[0]), dtype=v.dtype,
                          device=v.device)
        out.append(_item("transpose", [src], [tv.id]))
        cache[src] = tv.id
        return tv.id

    def pays(vid: int, flops: float) -> bool:
        if policy == "all" or vid in cache:
            return True
        nbytes = 2.0 * _numel(ir, vid)
        return 2.0 * nbytes / TRANSPOSE_BYTES_PER_S < MN_OPERAND_PENALTY * flops / GEMM_FLOPS_PER_S

    for it in lowered:
        op = kind(it)
        if op in ("gemm", "gemm_epilogue"):
            a, b = int(it["inputs"][0]), int(it["inputs"][1])
            attrs = dict(it.get("attrs", {}) or {})
            ta, tb = bool(attrs.get("transA", False)), bool(attrs.get("transB", False))
            dts = str(ir.values[a].dtype)
            sa, sb = ir.values[a].shape, ir.values[b].shape
            M = sa[1] if ta else sa[0]
            K = sa[0] if ta else sa[1]
            N = sb[0] if tb else sb[1]
            flops = 2.0 * M * N * K
            if ("float16" in dts or "bfloat16" in dts) and flops >= min_flops and (ta or not tb):
                do_a = ta and pays(a, flops)
                do_b = (not tb) and pays(b, flops)
                if do_a or do_b:
                    it = dict(it)
                    ins = list(it["inputs"])
                    if do_a:
                        ins[0] = transposed(a)
                        attrs["transA"] = False
                    if do_b:
                        ins[1] = transposed(b)
                        attrs["transB"] = True
                    it["inputs"], it["attrs"] = ins, attrs
                    it.pop("kernel_id", None)
        for o in it.get("outputs", []):
            for src in [s for s in cache if s == int(o)]:
                del cache[src]
        out.append(it)
    return out


# ---------------------------------------------------------------- StageB
def _dt(ir: IRGraph, vid: int) -> str:
    return str(ir.values[int(vid)].dtype)


def _is(ds: str, kind: str) -> bool:
    if kind == "f16":
        return "float16" in ds and "bfloat16" not in ds
    return kind in ds


def _numel(ir: IRGraph, vid: int) -> int:
    n = 1
    for d in ir.values[int(vid)].shape:
        n *= int(d)
    return n


def pick_kernel_id(ir: IRGraph, it: Dict[str, Any]) -> Optional[str]:
    op = str(it["op"]).strip().lower()
    ins, outs = it.get("inputs", []), it.get("outputs", [])
    attrs = it.get("attrs", {}) or {}
    in0 = _dt(ir, ins[0]) if ins else ""
    out0 = _dt(ir, outs[0]) if outs else ""
    f16 = _is(in0, "f16") or _is(out0, "f16")
    bf16 = _is(in0, "bfloat16") or _is(out0, "bfloat16")
    last = ir.values[int(outs[0])].shape[-1] if outs and ir.values[int(outs[0])].shape else 1
    even_last = int(last) % 2 == 0
    if op == "gemm_epilogue":
        if f16:
            return "gemm_bias_relu_f16_tc_wmma_out_f16_v0"
        if bf16:
            return "gemm_epilogue_bf16_mfma_f32out_v0" if _is(out0, "float32") else \
                "gemm_epilogue_bf16_mfma_v0"
        act = str(attrs.get("epilogue_act", "relu"))
        return "gemm_bias_relu_f32_naive_v0" if act == "relu" else "gemm_epilogue_f32_mfma_v0"
    if op == "gemm":
        if f16:
            return "gemm_f16_tc_wmma_out_f16_v0"
        if bf16:
            return "gemm_bf16_mfma_f32out_v0" if _is(out0, "float32") else "gemm_bf16_mfma_v0"
        return "gemm_f32_naive_v0"
    if op == "bias_add":
        return ("bias_add_f16_vec2_v0" if even_last else "bias_add_f16_v0") if f16 else "bias_add_f32_v0"
    if op == "add":
        return ("add_f16_vec2_v0" if even_last else "add_f16_v0") if f16 else "add_f32_v0"
    if op == "relu":
        return ("relu_f16_vec2_v0" if even_last else "relu_f16_v0") if f16 else "relu_f32_v0"
    if op == "relu_bwd":
        return ("relu_bwd_f16_vec2_v0" if even_last else "relu_bwd_f16_v0") if f16 else "relu_bwd_f32_v0"
    if op == "mse_grad":
        return "mse_grad_f16_v0" if f16 else "mse_grad_f32_v0"
    if op == "mse_loss":
        return "mse_loss_grad_v0"
    if op == "reduce_sum":
        if _is(out0, "f16"):
            return "reduce_sum_keep_lastdim_f16_v0"
        if _is(in0, "f16"):
            return "reduce_sum_keep_lastdim_f16_to_f32_v0"
        if _is(in0, "bfloat16"):
            return "reduce_sum_keep_lastdim_bf16_to_f32_v0"
        return "reduce_sum_keep_lastdim_f32_v0"
    if op == "sgd_step":
        if f16:
            return "sgd_step_f16_half2_v0" if _numel(ir, outs[0]) % 2 == 0 else "sgd_step_f16_v0"
        return "sgd_step_f32_v0"
    if op in ("copy", "copy_saved", "copy_aux"):
        return "copy_f16_v0" if f16 else ("copy_bf16_v0" if bf16 else "copy_f32_v0")
    if op == "grad_zero":
        return "grad_zero_v0"
    if op == "adam_step":
        return "adam_step_f32_v0"
    if op == "adamw_step":
        return "adamw_step_f32_v1"
    if op == "gemm_adamw":
        return "gemm_adamw_bf16_v0"
    if op == "step_inc":
        return "step_inc_v0"
    if op == "bias_corr":
        return "bias_corr_v0"
    if op == "gelu":
        return "gelu_bf16_v0" if bf16 else "gelu_f32_v0"
    if op == "gelu_bwd":
        return "gelu_bwd_bf16_v0" if bf16 else "gelu_bwd_f32_v0"
    if op == "softmax_xent":
        return "softmax_xent_f32_v0"
    if op == "row_softmax":
        return "row_softmax_f32_v0"
    if op == "row_reduce":
        return "row_reduce_f32_v0"
    if op == "transpose":
        return "transpose2d_v0"
    if op == "xent_head":
        return "xent_head_step_f32_v0" if len(ins) == 6 else "xent_head_f32_v0"
    if op == "grad_group":
        return "grad_group_f32_v0"
    if op == "grad_group_adamw":
        return "grad_group_adamw_f32_v0"
    if op == "gemm_epilogue_bcopy":
        return "gemm_small_bcopy_f32_v0"
    if op == "adamw_multi":
        return "adamw_multi_f32_v0"
    if op == "mse_colsum":
        return "mse_colsum_v0"
    if op == "colsum_adamw":
        return "colsum_adamw_f32_v0"
    if op in ("layernorm_fwd", "layernorm_bwd"):
        return f"{op}_{'f16' if f16 else 'f32'}_v0"
    if op in ("batchnorm_fwd", "batchnorm_bwd"):
        return f"{op}_f16_v0"
    return None


def apply_kernel_selection(ir: IRGraph, lowered: Lowered) -> Lowered:
    """StageB: attach a kernel_id to every op that lacks one."""
    out: Lowered = []
    for it in lowered:
        it = dict(it)
        if it.get("kernel_id") is None:
            kid = pick_kernel_id(ir, it)
            if kid is not None:
                it["kernel_id"] = kid
        out.append(it)
    return out


def _base_and_offset(ir: IRGraph, vid: int):
    v = ir.values[vid]
    return (v.view_of[0], v.view_of[1]) if v.view_of else (vid, 0)


def _view(ir: IRGraph, base: int, off: int, shape, dtype: str) -> int:
    """A view of `base` at element offset `off` with this shape and dtype:
    an existing IR value if one matches, else a new one."""
    shape = tuple(int(s) for s in shape)
    for v in ir.values.values():
        if v.view_of == (base, off) and v.shape == shape and v.dtype == dtype:
            return v.id
    b = ir.values[base]
    return ir.new_value(name=f"{b.name}[{off}:{off + _numel_shape(shape)}]", shape=shape, dtype=dtype,
                        device=b.device, view_of=(base, off)).id


def _numel_shape(shape) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n


def gemm_adamw_eligible(M: int, N: int, K: int) -> bool:
    """Shapes the fused kernel (256 x 256 tiles) covers."""
    return M % 256 == 0 and N % 256 == 0 and K % 64 == 0 and M > 0 and N > 0 and K > 0


def fuse_optimizer_into_gemms(ir: IRGraph, lowered: Lowered) -> Lowered:
    """StageE (not in the reference): for the flat AdamW step
    adamw_step(P, G, M, V, step) -> (P, M, V, Wb), every bf16 GEMM that writes
    a 2-D view of G read by no other op becomes
        gemm_adamw(A, B, P', M', V', step) -> (P', M', V', Wb')
    with P', M', V', Wb' the views of P, M, V, Wb at the same offset: AdamW
    runs in the GEMM's epilogue and the fp32 gradient never goes to memory.
    The flat step is replaced by steps over the ranges no GEMM covered (one
    per contiguous range), and step_inc moves in front of the first fused GEMM
    (the fused kernels read the incremented counter, as the flat step does).
    The updates are bit-identical to the unfused plan: the epilogue applies
    the same AdamW expression to the same fp32 accumulators the GEMM would
    have stored."""
    kind = lambda it: str(it.get("op", "")).strip().lower()  # noqa: E731
    ad = [i for i, it in enumerate(lowered) if kind(it) == "adamw_step"]
    if len(ad) != 1 or len(lowered[ad[0]]["outputs"]) != 4:
        return lowered
    adam = lowered[ad[0]]
    P, G, M, V, step = (int(x) for x in adam["inputs"])
    Wb = int(adam["outputs"][3])
    if any(ir.values[x].view_of for x in (P, G, M, V, Wb)):
        return lowered
    hyper = {k: adam.get("attrs", {}).get(k) for k in ("lr", "beta1", "beta2", "eps", "weight_decay")}
    hyper = {k: v for k, v in hyper.items() if v is not None}

    def readers(vid: int) -> int:
        return sum(1 for it in lowered if vid in it.get("inputs", []))

    def touched_later(idx: int, lo: int, hi: int) -> bool:
        """Whether an item after `idx` (before the flat step) reads or writes
        P, M, V or Wb in [lo, hi): the fused kernel updates that range where
        the GEMM stood, the unfused plan only at the flat step."""
        for it in lowered[idx + 1:ad[0]]:
            for x in list(it.get("inputs", [])) + list(it.get("outputs", [])):
                b, o = _base_and_offset(ir, int(x))
                if b in (P, M, V, Wb) and o < hi and lo < o + _numel(ir, int(x)):
                    return True
        return False

    out: Lowered = []
    covered = []
    first_fused = None
    for idx, it in enumerate(lowered):
        if kind(it) == "gemm" and len(it["outputs"]) == 1 and idx < ad[0]:
            o = int(it["outputs"][0])
            base, off = _base_and_offset(ir, o)
            a, b = (int(x) for x in it["inputs"])
            attrs = dict(it.get("attrs", {}))
            ta, tb = bool(attrs.get("transA", False)), bool(attrs.get("transB", False))
            sa, sb = ir.values[a].shape, ir.values[b].shape
            if base == G and len(ir.values[o].shape) == 2 and readers(o) == 0 \
                    and "bfloat16" in str(ir.values[a].dtype) and "bfloat16" in str(ir.values[b].dtype) \
                    and len(sa) == 2 and len(sb) == 2:
                Mg = sa[1] if ta else sa[0]
                Kg = sa[0] if ta else sa[1]
                Ng = sb[0] if tb else sb[1]
                if tuple(ir.values[o].shape) == (Mg, Ng) and gemm_adamw_eligible(Mg, Ng, Kg) \
                        and not touched_later(idx, off, off + Mg * Ng):
                    shp = ir.values[o].shape
                    pv = _view(ir, P, off, shp, ir.values[P].dtype)
                    mv = _view(ir, M, off, shp, ir.values[M].dtype)
                    vv = _view(ir, V, off, shp, ir.values[V].dtype)
                    wv = _view(ir, Wb, off, shp, ir.values[Wb].dtype)
                    if first_fused is None:
                        first_fused = len(out)
                    out.append(_item("gemm_adamw", [a, b, pv, mv, vv, step], [pv, mv, vv, wv],
                                     dict(transA=ta, transB=tb, **hyper)))
                    covered.append((off, off + _numel(ir, o)))
                    continue
        if idx == ad[0] and covered:
            total = _numel(ir, P)
            gaps, pos = [], 0
            for s, e in sorted(covered):
                if s > pos:
                    gaps.append((pos, s))
                pos = max(pos, e)
            if pos < total:
                gaps.append((pos, total))
            for s, e in gaps:
                views = [_view(ir, x, s, (e - s,), ir.values[x].dtype) for x in (P, G, M, V, Wb)]
                out.append(_item("adamw_step", [views[0], views[1], views[2], views[3], step],
                                 [views[0], views[2], views[3], views[4]], dict(adam.get("attrs", {}))))
            continue
        out.append(it)
    if first_fused is not None:
        si = [i for i, it in enumerate(out) if kind(it) == "step_inc" and int(it["inputs"][0]) == step]
        if len(si) == 1 and si[0] > first_fused:
            inc = out.pop(si[0])
            out.insert(first_fused, inc)
    return out


def fuse_colsum_into_dgelu(ir: IRGraph, lowered: Lowered) -> Lowered:
    """StageC' (not in the reference): reduce_sum(dz) -> (db, workspace) over
    the output of a bf16 dGELU gemm_epilogue becomes part of that GEMM (GEPI
    kind 6: outputs dz, db, workspace).  Only where the GEMM runs on the
    256 x 256 tiles that carry the column sums (bf16 2-D operands, M and N
    multiples of 256, K of 64) and the reduce_sum has a [P >= M/256, N] fp32
    workspace; db then sums one partial per 256-row tile instead of the
    two-pass column sum's order (equal to fp32 rounding)."""
    kind = lambda it: str(it.get("op", "")).strip().lower()  # noqa: E731
    producer = {}
    for i, it in enumerate(lowered):
        if kind(it) == "gemm_epilogue" and len(it["outputs"]) == 1 and \
                str(it.get("attrs", {}).get("epilogue_act", "")).lower() == "dgelu":
            producer[int(it["outputs"][0])] = i
    out = [dict(it, inputs=list(it["inputs"]), outputs=list(it["outputs"]), attrs=dict(it.get("attrs", {})))
           for it in lowered]
    drop = set()
    for j, it in enumerate(out):
        if kind(it) != "reduce_sum" or len(it["inputs"]) != 1 or len(it["outputs"]) != 2:
            continue
        if int(it.get("attrs", {}).get("axis", 0)) != 0:
            continue
        dz = int(it["inputs"][0])
        i = producer.get(dz)
        if i is None or i > j:
            continue
        g = out[i]
        a, b = (int(x) for x in g["inputs"][:2])
        ta, tb = bool(g["attrs"].get("transA", False)), bool(g["attrs"].get("transB", False))
        sa, sb = ir.values[a].shape, ir.values[b].shape
        if len(sa) != 2 or len(sb) != 2 or not all("bfloat16" in str(ir.values[v].dtype) for v in (a, b, dz)):
            continue
        M, K = (sa[1], sa[0]) if ta else (sa[0], sa[1])
        N = sb[0] if tb else sb[1]
        db, ws = (int(x) for x in it["outputs"])
        wsh = ir.values[ws].shape
        if M % 256 or N % 256 or K % 64 or len(wsh) != 2 or wsh[1] != N or wsh[0] < M // 256:
            continue
        if tuple(ir.values[db].shape) != (N,) or "float32" not in str(ir.values[db].dtype):
            continue
        g["outputs"] = [dz, db, ws]
        g["attrs"]["epilogue_colsum"] = True
        drop.add(j)
    return [it for j, it in enumerate(out) if j not in drop]


# ---------------------------------------------------------------- StageG
MAX_COLSUM_ADAMW = 8


# bf16 columns per lane of the mse_colsum kernel (kMseColsumVecBf16 in
# csrc/kernels/eltwise.hip)
MSE_COLSUM_VEC_BF16 = 8


def fuse_step_tail(ir: IRGraph, lowered: Lowered) -> Lowered:
    """StageG (not in the reference): for a step with
        mse_loss(y, t) -> (dY, loss, ws);  reduce_sum(dY) -> (db_L, P_ws)
        gemm_epilogue dGELU + column sums (dz, db_l, ws_l) for the hidden biases
        step_inc(step);  adamw_step over the range the db's tile
    the tail becomes
        mse_colsum(y, t, step) -> (dY, loss, ws, C_L, step)   at the loss
        gemm_epilogue dGELU + partials (dz, C_l)               (GEPI kind 7)
        colsum_adamw(C_1 .. C_L, P, M, V, step) -> (G, P, M, V, Wb)
    with C_* new fp32 partial values: C_L [P, N] (the reduce_sum's workspace
    rows, so its column sums are that op's bits), C_l [M / 256, N] (the
    GEMM's 256-row tiles, finished in the order of the finish kernel, so db_l
    and the updates are the unfused tail's bits).  The step counter is
    incremented by the loss op, before every reader of it.  Anything that
    does not match leaves the list unchanged."""
    k = _kind
    low = [dict(it, inputs=list(it["inputs"]), outputs=list(it["outputs"]), attrs=dict(it.get("attrs", {})))
           for it in lowered]
    ml = [i for i, it in enumerate(low) if k(it) == "mse_loss" and len(it["outputs"]) == 3]
    ad = [i for i, it in enumerate(low) if k(it) == "adamw_step" and len(it["outputs"]) == 4]
    si = [i for i, it in enumerate(low) if k(it) == "step_inc"]
    if len(ml) != 1 or len(ad) != 1 or len(si) != 1:
        return lowered
    im, ia, iss = ml[0], ad[0], si[0]
    dY = int(low[im]["outputs"][0])
    step = int(low[iss]["inputs"][0])
    adam = low[ia]
    if int(adam["inputs"][4]) != step or int(low[iss]["outputs"][0]) != step or not im < iss < ia:
        return lowered
    sY = ir.values[dY].shape
    if len(sY) != 2:
        return lowered
    Mrows, N = int(sY[0]), int(sY[1])
    # the last bias: reduce_sum(dY) with a [P, N] workspace
    rs = [i for i, it in enumerate(low) if k(it) == "reduce_sum" and it["inputs"] == [dY]
          and len(it["outputs"]) == 2 and int(it["attrs"].get("axis", 0)) == 0]
    if len(rs) != 1:
        return lowered
    ir_ = rs[0]
    dbL, wsL = (int(x) for x in low[ir_]["outputs"])
    P = int(ir.values[wsL].shape[0]) if len(ir.values[wsL].shape) == 2 else 0
    # bf16 gradients: the partition of the two-pass bf16 column sum (its bits)
    if P < 1 or Mrows % P or Mrows < 2 * P or N % 8 or not _is(_dt(ir, dY), "bfloat16"):
        return lowered
    # nothing between the loss and step_inc touches the step counter, and
    # nothing between the loss and the reduce_sum writes dY
    for it in low[im + 1:iss]:
        if step in it["inputs"] or step in it["outputs"]:
            return lowered
    for it in low[im + 1:ir_]:
        if any(_base(ir, int(o)) == _base(ir, dY) for o in it["outputs"]):
            return lowered
    # the hidden biases: dGELU GEMMs with column sums
    dg = [i for i, it in enumerate(low) if k(it) == "gemm_epilogue" and it["attrs"].get("epilogue_colsum") is True
          and len(it["outputs"]) == 3]
    db_of = {dbL: None}
    for i in dg:
        db_of[int(low[i]["outputs"][1])] = i
    # the bias step's range is tiled by the db values, in order
    Pv, Gv, Mv, Vv, _ = (int(x) for x in adam["inputs"])
    Wv = int(adam["outputs"][3])
    gb, s = _base_and_offset(ir, Gv)
    n = _numel(ir, Gv)
    spans = sorted((_base_and_offset(ir, d)[1], d) for d in db_of)
    if len(spans) > MAX_COLSUM_ADAMW or any(_base(ir, d) != gb for d in db_of):
        return lowered
    pos = s
    for off, d in spans:
        if off != pos or len(ir.values[d].shape) != 1:
            return lowered
        pos += _numel(ir, d)
    if pos != s + n:
        return lowered
    # the db values are read by nothing but the bias step this replaces (it
    # reads G, which is the one db value itself when there is one layer)
    for i, it in enumerate(low):
        if i != ia and any(int(x) in db_of for x in it["inputs"]):
            return lowered
    dev = ir.values[dY].device
    part = {}
    part[dbL] = ir.new_value(name=f"{ir.values[dbL].name}.partials", shape=(P, N), dtype="torch.float32",
                             device=dev).id
    for d, i in db_of.items():
        if i is None:
            continue
        dz = int(low[i]["outputs"][0])
        rows, cols = (int(x) for x in ir.values[dz].shape)
        if rows % 256 or cols != _numel(ir, d):
            return lowered
        part[d] = ir.new_value(name=f"{ir.values[d].name}.partials", shape=(rows // 256, cols),
                               dtype="torch.float32", device=dev).id
    y, t = (int(x) for x in low[im]["inputs"])
    loss, ws = int(low[im]["outputs"][1]), int(low[im]["outputs"][2])
    # mse_colsum writes one loss partial per workgroup: ceil(N / (64 lanes x
    # MSE_COLSUM_VEC_BF16 columns)) x P; mse_loss's buffer may be smaller
    need = -(-N // (64 * MSE_COLSUM_VEC_BF16)) * P
    if _numel(ir, ws) < need or not _f32(ir, ws):
        ws = ir.new_value(name=f"{ir.values[loss].name}.colsum_partials", shape=(need,), dtype="torch.float32",
                          device=dev).id
    msc = _item("mse_colsum", [y, t, step], [dY, loss, ws, part[dbL], step], dict(low[im]["attrs"]))
    for d, i in db_of.items():
        if i is not None:
            low[i]["outputs"] = [int(low[i]["outputs"][0]), part[d]]
            low[i]["attrs"]["epilogue_colsum"] = "partials"
    hyper = {kk: adam["attrs"][kk] for kk in ("lr", "beta1", "beta2", "eps", "weight_decay") if kk in adam["attrs"]}
    cad = _item("colsum_adamw", [part[d] for _, d in spans] + [Pv, Mv, Vv, step], [Gv, Pv, Mv, Vv, Wv],
                dict(hyper, tensors=len(spans)))
    out: Lowered = []
    for i, it in enumerate(low):
        if i == im:
            out.append(msc)
        elif i in (ir_, iss):
            continue
        elif i == ia:
            out.append(cad)
        else:
            out.append(it)
    return out


# ---------------------------------------------------------------- StageF
GJ_GEMM, GJ_COLSUM, GJ_MEAN, GJ_STEP = 0, 1, 2, 3
MAX_GROUP_JOBS = 8
# fp32 GEMMs with fewer 64 x 64 output tiles than this run on the small-GEMM
# kernel (kSmallGemmMaxTiles64 in csrc/common/smallstep.hpp, which the GEMM
# dispatcher uses); only those are grouped as gradient-group jobs
SMALL_GEMM_MAX_TILES64 = 128
MAX_ADAMW_TENSORS = 8


def _kind(it: Dict[str, Any]) -> str:
    return str(it.get("op", "")).strip().lower()


def _f32(ir: IRGraph, vid: int) -> bool:
    return "float32" in _dt(ir, vid)


def _base(ir: IRGraph, vid: int) -> int:
    return _base_and_offset(ir, int(vid))[0]


def _aligned16(ir: IRGraph, vid: int) -> bool:
    """The value starts 16 bytes into a 16-byte boundary of its buffer: base
    allocations do; a view (IR views are contiguous, row-major slices of
    their base) when its element offset, in the base's element size, is a
    multiple of 16 bytes."""
    base, off = _base_and_offset(ir, int(vid))
    es = 2 if "float16" in _dt(ir, base) else 4  # bf16/f16 are 2 bytes, f32/i32 4
    return (int(off) * es) % 16 == 0


def drop_dead_saves(ir: IRGraph, lowered: Lowered, keep: Iterable[int] = ()) -> Lowered:
    """copy_saved(src) -> dst where nothing after the copy writes src (or its
    base buffer): the readers of dst read src instead and the copy goes.
    Once the copy is gone dst is never written, so the copy stays when
    anything else could read dst: an op before the copy (it reads the
    previous step's save), or the caller after the step (dst in `keep`, or
    bound by the caller as an input or a parameter)."""
    from .plan import ROLE_STATIC, build_binding_plan

    keep = {int(v) for v in keep}
    plan = build_binding_plan(ir)
    out = [dict(it, inputs=list(it["inputs"]), outputs=list(it["outputs"])) for it in lowered]
    drop = set()
    for i, it in enumerate(out):
        if _kind(it) != "copy_saved" or len(it["inputs"]) != 1 or len(it["outputs"]) != 1:
            continue
        src, dst = int(it["inputs"][0]), int(it["outputs"][0])
        if ir.values[src].view_of or ir.values[dst].view_of:
            continue
        if dst in keep or plan.role_of(dst) != ROLE_STATIC:
            continue
        if any(int(v) == dst for x in out[:i] for v in x["inputs"]):
            continue
        later = out[i + 1:]
        if any(_base(ir, o) == src for x in later for o in x["outputs"]):
            continue
        if any(int(o) == dst for x in later for o in x["outputs"]):
            continue
        for x in later:
            x["inputs"] = [src if int(v) == dst else int(v) for v in x["inputs"]]
        drop.add(i)
    return [it for i, it in enumerate(out) if i not in drop]


def _head_shapes_ok(ir: IRGraph, H: int, W: int, b: int, t: int, L: int, S: int) -> bool:
    sh = lambda v: tuple(int(d) for d in ir.values[int(v)].shape)  # noqa: E731
    if len(sh(H)) != 2 or len(sh(W)) != 2:
        return False
    B, K = sh(H)
    C = sh(W)[0]
    return (sh(W) == (C, K) and sh(b) == (C,) and sh(t) == (B,) and sh(L) == (B, C) and sh(S) == (B, K)
            and K % 4 == 0 and 4 <= K <= 2048 and 1 <= C <= 32 and "int32" in _dt(ir, t)
            and all(_f32(ir, v) for v in (H, W, b, L, S))
            # xent_head reads H, W and S with 16-byte loads (K % 4 keeps every row aligned)
            and all(_aligned16(ir, v) for v in (H, W, S)))


def fuse_xent_head(ir: IRGraph, lowered: Lowered) -> Lowered:
    """gemm(H, W^T) -> L; bias_add(L, b) in place; softmax_xent(L, t) ->
    (loss, dY, pred, row_loss); later gemm(dY, W) -> dH and relu_bwd(dH, S)
    -> dX  ==>  xent_head(H, W, b, t, S) -> (L, dY, pred, row_loss, dH, dX)
    followed by loss_mean(row_loss) -> loss (a grad_group job).  The
    backward gemm and relu_bwd move up to the head: allowed when nothing in
    between writes W, S, H or dY or reads dH or dX."""
    out = list(lowered)
    i = 0
    while i + 2 < len(out):
        g, ba, sx = out[i], out[i + 1], out[i + 2]
        if not (_kind(g) == "gemm" and _kind(ba) == "bias_add" and _kind(sx) == "softmax_xent"):
            i += 1
            continue
        ga = g.get("attrs", {}) or {}
        if bool(ga.get("transA", False)) or not bool(ga.get("transB", False)) or len(g["inputs"]) != 2:
            i += 1
            continue
        H, W = (int(x) for x in g["inputs"])
        L = int(g["outputs"][0])
        if [int(x) for x in ba["inputs"]][:1] != [L] or [int(x) for x in ba["outputs"]] != [L] \
                or [int(x) for x in sx["inputs"]][:1] != [L] or len(sx["outputs"]) != 4:
            i += 1
            continue
        b, t = int(ba["inputs"][1]), int(sx["inputs"][1])
        loss, dY, pred, rl = (int(x) for x in sx["outputs"])
        d = r = None
        for j in range(i + 3, len(out)):
            it = out[j]
            if d is None and _kind(it) == "gemm" and [int(x) for x in it["inputs"]] == [dY, W] and \
                    not bool((it.get("attrs") or {}).get("transA", False)) and \
                    not bool((it.get("attrs") or {}).get("transB", False)):
                d = j
            elif d is not None and _kind(it) == "relu_bwd" and \
                    int(it["inputs"][0]) == int(out[d]["outputs"][0]):
                r = j
                break
        if d is None or r is None:
            i += 1
            continue
        dH, S, dX = int(out[d]["outputs"][0]), int(out[r]["inputs"][1]), int(out[r]["outputs"][0])
        if not _head_shapes_ok(ir, H, W, b, t, L, S) or not (_aligned16(ir, dH) and _aligned16(ir, dX)):
            i += 1
            continue
        bases_fixed = {_base(ir, v) for v in (W, S, H, dY, b, t)}
        moved_reads = {_base(ir, v) for v in (dH, dX)}
        ok = True
        for j in range(i + 3, r):
            if j == d:
                continue
            it = out[j]
            if any(_base(ir, o) in (bases_fixed | moved_reads) for o in it["outputs"]) or \
                    any(_base(ir, v) in moved_reads for v in it["inputs"]):
                ok = False
                break
        if not ok or any(int(v) == dH for k, it in enumerate(out) if k not in (d, r) for v in it["inputs"]):
            i += 1
            continue
        head = _item("xent_head", [H, W, b, t, S], [L, dY, pred, rl, dH, dX])
        mean = _item("loss_mean", [rl], [loss])
        out = out[:i] + [head, mean] + [it for k, it in enumerate(out[i + 3:], start=i + 3) if k not in (d, r)]
        i += 2
    return out


def _job_of(ir: IRGraph, it: Dict[str, Any]) -> Optional[tuple]:
    """(type, inputs, outputs, f0, f1) when the op can run as a grad_group job.
    The jobs read any offset (the small GEMM falls back to 4-byte loads off a
    16-byte boundary) and need unit column strides, which IR values (base
    buffers and contiguous views of them) always have."""
    k = _kind(it)
    ins, outs = [int(x) for x in it["inputs"]], [int(x) for x in it["outputs"]]
    attrs = it.get("attrs", {}) or {}
    if k == "gemm" and len(ins) == 2 and len(outs) == 1 and all(_f32(ir, v) for v in ins + outs):
        sa, sb = ir.values[ins[0]].shape, ir.values[ins[1]].shape
        if len(sa) != 2 or len(sb) != 2:
            return None
        ta, tb = bool(attrs.get("transA", False)), bool(attrs.get("transB", False))
        M = sa[1] if ta else sa[0]
        N = sb[0] if tb else sb[1]
        if ((M + 63) // 64) * ((N + 63) // 64) >= SMALL_GEMM_MAX_TILES64 or not _small_gemm_ranges_ok(ir, ins):
            return None
        return (GJ_GEMM, ins, outs, int(ta), int(tb))
    if k == "reduce_sum" and len(ins) == 1 and len(outs) == 1 and int(attrs.get("axis", 0)) == 0 \
            and len(ir.values[ins[0]].shape) == 2 and _f32(ir, ins[0]) and _f32(ir, outs[0]):
        return (GJ_COLSUM, ins, outs, 0, 0)
    if k == "loss_mean":
        return (GJ_MEAN, ins, outs, 0, 0)
    if k == "step_inc" and len(ins) == 1 and len(outs) == 1 and ins == outs:
        return (GJ_STEP, ins, outs, 1, 0)
    return None


def _small_gemm_ranges_ok(ir: IRGraph, operands) -> bool:
    """The small GEMM reads its operands through buffer loads with 32-bit
    byte offsets: each operand (contiguous, fp32) spans fewer than 2^31
    bytes."""
    return all(4 * _numel(ir, int(v)) < 2 ** 31 for v in operands)


def _group_item(jobs: List[tuple]) -> Dict[str, Any]:
    ins: List[int] = []
    outs: List[int] = []
    recs = []
    for typ, ji, jo, f0, f1 in jobs:
        for v in ji:
            if v not in ins:
                ins.append(v)
        for v in jo:
            if v not in outs:
                outs.append(v)
        recs.append([typ, ins.index(ji[0]), ins.index(ji[1]) if len(ji) > 1 else 0, outs.index(jo[0]), f0, f1])
    return _item("grad_group", ins, outs, {"jobs": recs})


def group_small_jobs(ir: IRGraph, lowered: Lowered) -> Lowered:
    """Runs of consecutive ops that can run as grad_group jobs and are
    independent (no job reads or writes a buffer another job of the run
    writes) become one grad_group; a run of one op stays as it is, except
    loss_mean, which has no kernel of its own."""
    out: Lowered = []
    run: List[tuple] = []
    run_items: Lowered = []

    def flush():
        if len(run) >= 2 or any(j[0] == GJ_MEAN for j in run):
            out.append(_group_item(run))
        else:
            out.extend(run_items)
        run.clear()
        run_items.clear()

    for it in lowered:
        job = _job_of(ir, it)
        if job is None:
            flush()
            out.append(it)
            continue
        _, ji, jo, _, _ = job
        rb = {_base(ir, v) for j in run for v in j[1]}
        wb = {_base(ir, v) for j in run for v in j[2]}
        jr, jw = {_base(ir, v) for v in ji}, {_base(ir, v) for v in jo}
        if len(run) >= MAX_GROUP_JOBS or (jr & wb) or (jw & (rb | wb)):
            flush()
        run.append(job)
        run_items.append(it)
    flush()
    return out


def fuse_adamw_multi(ir: IRGraph, lowered: Lowered) -> Lowered:
    """Consecutive adamw_step(P, G, M, V, step) -> (P, M, V) ops (fp32, in
    place, same step and hyperparameters, distinct buffers) become
    adamw_multi((P, G, M, V) x T, step) -> (P, M, V) x T."""
    out: Lowered = []
    run: Lowered = []

    def key(it):
        return (int(it["inputs"][4]), tuple(sorted((it.get("attrs") or {}).items())))

    def flush():
        if len(run) >= 2:
            ins: List[int] = []
            outs: List[int] = []
            for it in run:
                ins += [int(x) for x in it["inputs"][:4]]
                outs += [int(x) for x in it["outputs"]]
            ins.append(int(run[0]["inputs"][4]))
            out.append(_item("adamw_multi", ins, outs, dict(run[0].get("attrs") or {})))
        else:
            out.extend(run)
        run.clear()

    for it in lowered:
        ok = (_kind(it) == "adamw_step" and len(it["inputs"]) == 5 and len(it["outputs"]) == 3
              and [int(x) for x in it["outputs"]] == [int(it["inputs"][k]) for k in (0, 2, 3)]
              and all(_f32(ir, int(v)) for v in it["inputs"][:4])
              # adamw_multi moves whole 16-byte vectors (adamw_step has an unaligned fallback)
              and all(_aligned16(ir, int(v)) for v in it["inputs"][:4]))
        if ok and run:
            used = {_base(ir, int(v)) for r in run for v in r["inputs"][:4]}
            if key(it) != key(run[0]) or len(run) >= MAX_ADAMW_TENSORS or \
                    any(_base(ir, int(v)) in used for v in it["inputs"][:4]):
                flush()
        if ok:
            run.append(it)
        else:
            flush()
            out.append(it)
    flush()
    return out


def _bcopy_source(ir: IRGraph, lowered: Lowered, gi: int, P: int) -> Optional[int]:
    """Index of the last op before lowered[gi] that can write a copy of P as
    it reads it: a small fp32 gemm_epilogue (bias+ReLU, bias or ReLU) with
    P as its B operand read K-contiguously (transB) in 16-byte vectors, and
    nothing between it and lowered[gi] writes P."""
    for k in range(gi - 1, -1, -1):
        it = lowered[k]
        if any(_base(ir, o) == P for o in it["outputs"]):
            return None
        if _kind(it) != "gemm_epilogue" or len(it["inputs"]) != 3 or len(it["outputs"]) != 1 or \
                int(it["inputs"][1]) != P:
            continue
        a = it.get("attrs") or {}
        if not bool(a.get("transB", False)) or epilogue_kind(a) not in (0, 1, 2):
            continue
        A, C = int(it["inputs"][0]), int(it["outputs"][0])
        if not all(_f32(ir, v) for v in (A, P, C)) or _base(ir, C) == P or _base(ir, A) == P:
            continue
        N, K = (int(d) for d in ir.values[P].shape)
        sa = ir.values[A].shape
        M = int(sa[1] if bool(a.get("transA", False)) else sa[0])
        if K % 4 or not _aligned16(ir, P) or ((M + 63) // 64) * ((N + 63) // 64) >= SMALL_GEMM_MAX_TILES64 \
                or not _small_gemm_ranges_ok(ir, (A, P)):
            continue
        return k
    return None


def _adamw_ok(ir: IRGraph, it: Dict[str, Any]) -> bool:
    return (_kind(it) == "adamw_step" and len(it["inputs"]) == 5 and len(it["outputs"]) == 3
            and [int(x) for x in it["outputs"]] == [int(it["inputs"][k]) for k in (0, 2, 3)]
            and all(_f32(ir, int(v)) for v in it["inputs"][:4]))


def fuse_adamw_into_group(ir: IRGraph, lowered: Lowered) -> Lowered:
    """grad_group followed by adamw_step(P, G, M, V, step) -> (P, M, V) ops
    whose G is the output of one of the group's GEMM or column-sum jobs ==>
    grad_group_adamw: each update applied where its gradient is stored (the
    bits of adamw_step).  Of the adamw_steps that follow the group directly,
    those whose gradient the group computes move into it; the others stay
    after it.  Conditions:
      * same step and hyperparameters, distinct fp32 P, M, V buffers, G the
        whole output of its job;
      * the group's step_inc job leaves the group for the xent_head right
        before it, which advances the counter and writes the advanced step's
        bias corrections {lr / bc1, 1 / bc2} once (a new 2-float value the
        updates read, the values adamw_step derives from the counter);
      * no job reads P, M or V, except a GEMM job with P as its B operand:
        that job reads a copy of P written by an earlier small gemm_epilogue
        that reads P K-contiguously (gemm_epilogue_bcopy), when nothing in
        between writes P."""
    out = list(lowered)
    gi = 0
    while gi < len(out):
        g = out[gi]
        if _kind(g) != "grad_group":
            gi += 1
            continue
        run = []
        for it in out[gi + 1:]:
            if not _adamw_ok(ir, it):
                break
            run.append(it)
        res = _group_adamw(ir, out, gi, run) if run else None
        if res is None:
            gi += 1
            continue
        out = res
        gi += 1
    return out


def _group_adamw(ir: IRGraph, lowered: Lowered, gi: int, run: Lowered) -> Optional[Lowered]:
    g = lowered[gi]
    gins, gouts = [int(v) for v in g["inputs"]], [int(v) for v in g["outputs"]]
    jobs = [list(j) for j in g["attrs"]["jobs"]]
    key = lambda it: tuple(sorted((it.get("attrs") or {}).items()))  # noqa: E731
    step = int(run[0]["inputs"][4])
    if any(int(it["inputs"][4]) != step or key(it) != key(run[0]) for it in run):
        return None
    # jobs as (type, [inputs], [output], f0, f1); the step job goes
    jtup = []
    step_job = None
    for j in jobs:
        typ = int(j[0])
        ji = [gins[j[1]]] + ([gins[j[2]]] if typ == GJ_GEMM else [])
        if typ == GJ_STEP:
            if step_job is not None or gins[j[1]] != step or gouts[j[3]] != step:
                return None
            step_job = j
            continue
        if any(_base(ir, v) == _base(ir, step) for v in ji + [gouts[j[3]]]):
            return None
        jtup.append([typ, ji, gouts[j[3]], int(j[4]), int(j[5]), None])
    # the step counter: advanced by the xent_head right before the group,
    # which also derives the step's bias corrections once (a launch of its
    # own would cost what the fusion saves)
    h = lowered[gi - 1] if gi > 0 else None
    if step_job is None or h is None or _kind(h) != "xent_head" or len(h["inputs"]) != 5 or \
            any(_base(ir, v) == _base(ir, step) for v in list(h["inputs"]) + list(h["outputs"])):
        return None
    # the updates whose gradient is a GEMM or column-sum job's whole output
    fused, rest = [], []
    for it in run:
        P, G, M, V = (int(v) for v in it["inputs"][:4])
        hit = [t for t in jtup if t[2] == G and t[0] in (GJ_GEMM, GJ_COLSUM) and t[5] is None]
        if len(hit) != 1 or tuple(ir.values[P].shape) != tuple(ir.values[G].shape) or \
                any(_numel(ir, v) != _numel(ir, G) for v in (M, V)):
            rest.append(it)
            continue
        hit[0][5] = (P, M, V)
        fused.append(it)
    out = list(lowered)
    # a job that reads a moved update's P, M or V: a GEMM's B operand P can
    # read a copy of P; otherwise that update stays behind
    copies: Dict[int, tuple] = {}  # P -> (index of the op that copies it, the jobs that read it)
    for it in list(fused):
        P, M, V = (int(it["inputs"][k]) for k in (0, 2, 3))
        bases = {_base(ir, v) for v in (P, M, V)}
        readers = [(t, pos) for t in jtup for pos, v in enumerate(t[1]) if _base(ir, v) in bases]
        ok = not any(_base(ir, t[2]) in bases for t in jtup)
        ok = ok and all(t[0] == GJ_GEMM and pos == 1 and t[1][1] == P and _base(ir, P) == P
                        for t, pos in readers)
        k = _bcopy_source(ir, out, gi, P) if ok and readers else None
        if not ok or (readers and k is None):
            fused.remove(it)
            rest.append(it)
            for t in jtup:
                if t[5] is not None and t[5][0] == P:
                    t[5] = None
            continue
        if readers:
            copies[P] = (k, readers)
    rest = [it for it in run if it in rest]  # in their original order
    pmv_bases = [_base(ir, int(it["inputs"][k])) for it in fused for k in (0, 2, 3)]
    if not fused or len(set(pmv_bases)) != len(pmv_bases) or _base(ir, step) in pmv_bases:
        return None
    # the updates that stay behind touch none of the moved ones' buffers
    if any(_base(ir, v) in pmv_bases for it in rest for v in it["inputs"]):
        return None
    if len({k for k, _ in copies.values()}) != len(copies):
        return None
    for P, (k, readers) in copies.items():
        src = ir.values[P]
        cv = ir.new_value(name=f"{src.name}.copy", shape=tuple(src.shape), dtype=src.dtype, device=src.device)
        g0 = out[k]
        out[k] = _item("gemm_epilogue_bcopy", list(g0["inputs"]), [int(g0["outputs"][0]), cv.id],
                       dict(g0.get("attrs") or {}))
        for t, pos in readers:
            t[1][pos] = cv.id
    # the head advances the counter and writes the step's bias corrections
    # once ({lr / bc1, 1 / bc2}), which the group's updates read
    hp = dict(run[0].get("attrs") or {})
    sv = ir.values[step]
    scal = ir.new_value(name=f"{sv.name}.adamw_scalars", shape=(2,), dtype="torch.float32", device=sv.device)
    h = out[gi - 1]
    out[gi - 1] = _item("xent_head", list(h["inputs"]) + [step], list(h["outputs"]) + [step, scal.id],
                        dict(h.get("attrs") or {}, step_inc=int(step_job[4]), lr=float(hp.get("lr", 1e-3)),
                             beta1=float(hp.get("beta1", 0.9)), beta2=float(hp.get("beta2", 0.999))))
    item = _group_adamw_item(jtup, scal.id, hp)
    n = len(run)
    return out[:gi] + [item] + rest + out[gi + 1 + n:]


def _group_adamw_item(jtup, scal: int, hp: Dict[str, Any]) -> Dict[str, Any]:
    ins: List[int] = []
    outs: List[int] = []

    def idx(lst, v):
        if v not in lst:
            lst.append(v)
        return lst.index(v)

    recs = []
    for typ, ji, jo, f0, f1, pmv in jtup:
        r = [typ, idx(ins, ji[0]), idx(ins, ji[1]) if len(ji) > 1 else 0, idx(outs, jo), f0, f1]
        if pmv is None:
            r += [-1] * 6
        else:
            r += [idx(ins, v) for v in pmv] + [idx(outs, v) for v in pmv]
        recs.append(r)
    si = idx(ins, scal)
    attrs = {"jobs": recs, "scalars_input": si, "lr": float(hp.get("lr", 1e-3)),
             "beta1": float(hp.get("beta1", 0.9)), "beta2": float(hp.get("beta2", 0.999)),
             "eps": float(hp.get("eps", 1e-8)), "weight_decay": float(hp.get("weight_decay", 0.0))}
    return _item("grad_group_adamw", ins, outs, attrs)


def fuse_small_step(ir: IRGraph, lowered: Lowered, keep: Iterable[int] = (), *,
                    adamw_into_group: bool = True) -> Lowered:
    """StageF: drop_dead_saves -> fuse_xent_head -> group_small_jobs ->
    fuse_adamw_into_group (adamw_into_group) -> fuse_adamw_multi.  keep:
    values the caller reads after the step."""
    low = drop_dead_saves(ir, lowered, keep)
    low = fuse_xent_head(ir, low)
    low = group_small_jobs(ir, low)
    if adamw_into_group:
        low = fuse_adamw_into_group(ir, low)
    low = fuse_adamw_multi(ir, low)
    assert not any(_kind(it) == "loss_mean" for it in low)
    return low


def compile_lowered(ir: IRGraph, *, fuse: bool = True, fuse_bias: bool = False,
                    nt_layout: Any = False, nt_min_flops: float = 2.0 ** 30,
                    fuse_optimizer: bool = False, fuse_colsum: bool = False,
                    fuse_small: Any = False, fuse_tail: bool = False,
                    keep_values: Iterable[int] = ()) -> Lowered:
    """StageA -> StageC -> (StageC') -> (StageD) -> (StageE) -> (StageF) -> (StageG) -> StageB.
    nt_layout: False (no StageD), True / "all" (transpose every M/N-contiguous
    16-bit operand) or "cost" (transpose only where that is cheaper than
    reading it in place); fuse_colsum: StageC'; fuse_optimizer: StageE;
    fuse_small: StageF (True; "four" leaves its AdamW updates in their own
    launch); fuse_tail: StageG.  keep_values: value ids the caller reads
    after a step, which the rewrites must keep writing."""
    low = lower_to_backend_ops(ir)
    if fuse:
        low = fuse_gemm_epilogue(ir, low, fuse_bias=fuse_bias)
    if fuse and fuse_colsum:
        low = fuse_colsum_into_dgelu(ir, low)
    if nt_layout:
        policy = "all" if nt_layout is True else str(nt_layout)
        low = normalize_gemm_layout(ir, low, min_flops=nt_min_flops, policy=policy)
    if fuse_optimizer:
        low = fuse_optimizer_into_gemms(ir, low)
    if fuse_small:
        low = fuse_small_step(ir, low, keep_values, adamw_into_group=fuse_small != "four")
    if fuse_tail:
        low = fuse_step_tail(ir, low)
    return apply_kernel_selection(ir, low)


def _fmt_attr(v: Any) -> str:
    return str(v)


def lowered_to_text(lowered: Lowered, name: str) -> str:
    """Text dump in the layout of the reference's 30_lowered.txt artifact."""
    lines = [f"=== LoweredOps({name}) ===", f"ops: {len(lowered)}", ""]
    for i, it in enumerate(lowered):
        ins = ", ".join(str(x) for x in it["inputs"])
        outs = ", ".join(str(y) for y in it["outputs"])
        ins = f"({ins})" if len(it["inputs"]) != 1 else f"({ins})"
        s = f"  #{i:03d} {it['op']:<10} {ins} -> ({outs})"
        attrs = it.get("attrs") or {}
        if attrs:
            s += "  {" + ", ".join(f"{k}={_fmt_attr(attrs[k])}" for k in sorted(attrs)) + "}"
        if it.get("kernel_id"):
            s += f"  kid={it['kernel_id']}"
        lines.append(s)
    return "\n".join(lines)
