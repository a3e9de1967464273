"""Benchmark of the gfx950 hot path (one JSON line on stdout).

Headline (`value`): steps/s of the bf16 MLP train step replayed as ONE
hipGraph - batch 8192, 4 x Linear 4096->4096 (bf16 weights, fp32 master
copy in one flat buffer), GELU, MSE loss, fused AdamW - inputs resident in
HBM.  `components` carries the other metrics of the benchmark measured in
the same run: bf16 GEMM TFLOP/s at 8192^3, row softmax (+row max/sum) GB/s
and fused Adam GB/s over 2^28 parameters.  `roofline` is for the dominant
kernel of the step (the bf16 GEMM at 8192x4096x4096), timed with HIP
events on the stream it runs on.  `cpu_baseline` is the CPU oracle
(oracle/aicf_oracle.c, the reference kernels' arithmetic restated) timed on
a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import struct
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for p in (REPO / "ai-compiler-framework_amd" / "python", REPO / "oracle", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

METRIC = "GEMM TFLOP/s + softmax/Adam HBM GB/s; MLP train-steps/s (hipGraph)"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

GEPI = int.from_bytes(b"GEPI", "little")
ADAM = int.from_bytes(b"ADAM", "little")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _cs() -> int:
    """torch's current stream as the launch stream argument."""
    import torch

    return torch.cuda.current_stream().cuda_stream


WARM_S = 0.05  # seconds of back-to-back work before a timed region
# The step's clock ramp spans ~50 replays (~150 ms): the headline warms longer.
STEP_WARM_S = 0.25


def _warm(launch, warm_s: float) -> None:
    """Keep the GPU busy with `launch` for warm_s seconds: after an idle gap
    the clock takes tens of milliseconds to return to its loaded steady state,
    and a few warmup calls of a sub-millisecond kernel time the ramp."""
    import torch

    t0 = time.perf_counter()
    while True:
        for _ in range(4):
            launch()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= warm_s:
            return


def time_launches(fn, iters: int, warmup: int, stream=None, graph: bool = False, warm_s: float = WARM_S) -> float:
    """Average milliseconds per call of fn(), HIP events on `stream`
    (torch's current stream by default), after `warmup` calls and then at
    least warm_s seconds of calls.  graph: the `iters` calls are captured into
    one graph (fn launches on torch's current stream) and the graph is timed,
    so that kernels of a few microseconds are timed back to back on the device
    rather than at the rate the host issues them."""
    import torch

    if graph:
        gs = torch.cuda.Stream()
        with torch.cuda.stream(gs):
            for _ in range(warmup):
                fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=gs):
            for _ in range(iters):
                fn()
        g.replay()
        torch.cuda.synchronize()
        _warm(g.replay, warm_s)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        rs = torch.cuda.current_stream()  # replay() launches on torch's current stream
        e0.record(rs)
        g.replay()
        e1.record(rs)
        torch.cuda.synchronize()
        del g
        return e0.elapsed_time(e1) / iters
    s = stream or torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    _warm(fn, warm_s)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(iters):
        fn()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


# ------------------------------------------------------------------ GEMM
def bench_gemm(C, M, N, K, act_kind=None, iters=20, warmup=5, save_preact=False):
    """bf16 X[M,K] . W[N,K]^T (+bias, act) -> bf16, fp32 accumulate.  With
    save_preact the bias+GELU epilogue also writes the pre-activation Z, as
    the forward GEMMs of the train step do."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    s = 1.0 / math.sqrt(K)
    X = ((torch.rand((M, K), device="cuda", generator=g) * 2 - 1) * s).to(torch.bfloat16)
    W = ((torch.rand((N, K), device="cuda", generator=g) * 2 - 1) * s).to(torch.bfloat16)
    b = ((torch.rand(N, device="cuda", generator=g) * 2 - 1) * s)
    Y = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
    if act_kind is None:
        fn = lambda: C.launch_by_id("gemm_bf16_mfma_v0", C.OpKind.Gemm, [X, W], [Y], 0,  # noqa: E731
                                    struct.pack("<ii", 0, 1))
    else:
        outs = [Y, torch.empty_like(Y)] if save_preact else [Y]
        fn = lambda: C.launch_by_id("gemm_epilogue_bf16_mfma_v0", C.OpKind.GemmEpilogue,  # noqa: E731
                                    [X, W, b], outs, GEPI, struct.pack("<iii", 0, 1, act_kind))
    ms = time_launches(fn, iters, warmup)
    return {"ms": ms, "tflops": 2.0 * M * N * K / (ms * 1e-3) / 1e12}


# C4: GEMM + bias + activation over the configured shapes (GEPI kinds:
# 1 bias only, 0 bias+ReLU, 3 bias+GELU)
C4_SHAPES = [(1024, 1024, 1024), (4096, 4096, 4096), (8192, 8192, 8192),
             (8192, 4096, 256), (8192, 4096, 11008)]
C4_ACTS = {"none": 1, "relu": 0, "gelu": 3}


def bench_layouts(C, n=4096, iters=10):
    """Plain GEMM C[n,n] = op(A) . op(B) at n^3 in the four operand layouts of
    the reference's gemm op (transA, transB), bf16 and fp32: every layout is
    read in place, none is transposed first."""
    import torch

    out = {}
    for dt, kid in (("bf16", "gemm_bf16_mfma_v0"), ("fp32", "gemm_f32_naive_v0")):
        tdt = torch.bfloat16 if dt == "bf16" else torch.float32
        g = torch.Generator(device="cuda")
        g.manual_seed(n + 5)
        A = ((torch.rand((n, n), device="cuda", generator=g) * 2 - 1) / math.sqrt(n)).to(tdt)
        B = ((torch.rand((n, n), device="cuda", generator=g) * 2 - 1) / math.sqrt(n)).to(tdt)
        Y = torch.empty((n, n), device="cuda", dtype=tdt)
        peak = PEAK_BF16_TFLOPS if dt == "bf16" else PEAK_FP32_TFLOPS
        for ta in (0, 1):
            for tb in (0, 1):
                pay = struct.pack("<ii", ta, tb)
                fn = lambda: C.launch_by_id(kid, C.OpKind.Gemm, [A, B], [Y], 0, pay, _cs())  # noqa: E731
                ms = time_launches(fn, iters, 2)
                tf = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
                out[f"gemm_{dt}_{n}^3_{'T' if ta else 'N'}{'T' if tb else 'N'}"] = {
                    "value": round(tf, 2), "unit": "TFLOP/s", "frac": round(tf / peak, 4), "ms": round(ms, 4)}
    return out


def bench_c4(C, dtype="bf16", shapes=C4_SHAPES, acts=("none", "relu", "gelu"), iters=10):
    """X~U(-1,1)/sqrt(K) [M,K], W [N,K], b [N]; act(X.W^T + b).  bf16: bf16 in,
    fp32 accumulate, bf16 out; fp32: fp32 throughout."""
    import torch

    out = {}
    for (M, N, K) in shapes:
        g = torch.Generator(device="cuda")
        g.manual_seed(M + N + K)
        s = 1.0 / math.sqrt(K)
        tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
        X = ((torch.rand((M, K), device="cuda", generator=g) * 2 - 1) * s).to(tdt)
        W = ((torch.rand((N, K), device="cuda", generator=g) * 2 - 1) * s).to(tdt)
        b = ((torch.rand(N, device="cuda", generator=g) * 2 - 1) * s)
        Y = torch.empty((M, N), device="cuda", dtype=tdt)
        kid = "gemm_epilogue_bf16_mfma_v0" if dtype == "bf16" else "gemm_epilogue_f32_mfma_v0"
        flops = 2.0 * M * N * K
        for act in acts:
            pay = struct.pack("<iii", 0, 1, C4_ACTS[act])
            fn = lambda: C.launch_by_id(kid, C.OpKind.GemmEpilogue, [X, W, b], [Y], GEPI, pay,  # noqa: E731
                                        _cs())
            n = iters if flops < 1e12 else max(3, iters // 2)
            # small shapes run for a few microseconds: time them from a captured graph
            ms = time_launches(fn, n, 2, graph=flops < 1e11)
            tf = flops / (ms * 1e-3) / 1e12
            peak = PEAK_BF16_TFLOPS if dtype == "bf16" else PEAK_FP32_TFLOPS
            out[f"c4_{dtype}_{M}x{N}x{K}_{act}"] = {"value": round(tf, 2), "unit": "TFLOP/s",
                                                    "frac": round(tf / peak, 4), "ms": round(ms, 4)}
    return out


# C1: the reference MLP (fp32, B=64, 784->256(ReLU)->10, softmax-xent, Adam)
# lowering (fuse_small) and steps per captured graph
C1_VARIANTS = {"three_launch": (True, 1), "four_launch": ("four", 1), "reference_lowering": (False, 1),
               "three_launch_10_steps_per_replay": (True, 10)}


def bench_c1(rounds=10, chunk=100, warm_s=STEP_WARM_S):
    """Replayed-graph time of one C1 train step for each lowering (True: the
    three-launch StageF plan, "four": its four-launch form, False: the
    reference pipeline's 17 ops), each on a graph handle of its own, warmed
    together for warm_s, then timed in `rounds` rounds of `chunk` steps
    with the lowerings alternated (order reversed every other round), so
    that clock and box state are shared.  The last variant captures ten
    consecutive steps per graph: a graph launch costs ~4 us of GPU time of
    its own, a fifth of this step."""
    import torch

    from aicf_hip import mlp

    data = mlp.init_mlp_xent()
    exs = {}
    for k, (fs, per) in C1_VARIANTS.items():
        ir, lowered, plan = mlp.build_mlp_xent(fuse_small=fs)
        params = {n: torch.from_numpy(v.copy()).cuda() for n, v in data.items() if "." in n}
        inputs = {"x": torch.from_numpy(data["x"]).cuda(), "t": torch.from_numpy(data["t"]).cuda()}
        ex = mlp.make_executor(ir, lowered, plan, own_graph=True)
        ex.build_env(inputs=inputs, params=params, reuse_static=False)
        ex.capture(inputs=inputs, params=params, reuse_static=True, steps=per)
        exs[k] = (ex, lowered)
    s = torch.cuda.current_stream()  # graph_launch replays on the caller's stream
    for ex, _ in exs.values():
        ex.replay(3)
    torch.cuda.synchronize()
    _warm(lambda: [ex.replay(max(1, 10 // ex.steps_per_replay)) for ex, _ in exs.values()], warm_s)
    tot = {k: 0.0 for k in exs}
    names = list(exs)
    for r in range(rounds):
        for k in (names if r % 2 == 0 else names[::-1]):
            ex = exs[k][0]
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            ex.replay(max(1, chunk // ex.steps_per_replay))
            e1.record(s)
            torch.cuda.synchronize()
            tot[k] += e0.elapsed_time(e1) / (max(1, chunk // ex.steps_per_replay) * ex.steps_per_replay)
    out = {}
    for k, (ex, lowered) in exs.items():
        us = tot[k] * 1e3 / rounds
        out[k] = {"value": round(us, 2), "unit": "us/step", "steps_per_s": round(1e6 / us, 1),
                  "ops_per_step": len(lowered), "steps_per_replay": ex.steps_per_replay,
                  "loss_after": float(ex.value("loss").item())}
        ex.close()
    return out


# ------------------------------------------------------------------ softmax
def bench_softmax(C, rows, cols, iters=20, warmup=3):
    """Row softmax + row max + row sum, fp32; rotates buffer sets so the
    working set exceeds the 256 MB MALL."""
    import torch

    per_set = rows * cols * 4 * 2
    nsets = max(1, min(64, math.ceil(512e6 / per_set)))
    g = torch.Generator(device="cuda")
    g.manual_seed(2)
    sets = []
    for _ in range(nsets):
        x = torch.randn((rows, cols), device="cuda", generator=g) * 2.0
        x[-1].fill_(-1e4)
        sets.append((x, torch.empty_like(x), torch.empty(rows, device="cuda"),
                     torch.empty(rows, device="cuda")))
    k = [0]

    def fn():
        x, y, mx, sm = sets[k[0] % nsets]
        k[0] += 1
        C.op_call(int(C.OpKind.RowSoftmax), [x, ], [y, mx, sm], 0, b"", _cs())

    ms = time_launches(fn, iters, warmup, graph=True)
    nbytes = 8 * rows * cols + 8 * rows
    return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes, "buffer_sets": nsets}


# ------------------------------------------------------------------ row reductions / losses
RRED = int.from_bytes(b"RRED", "little")


def _rotating_sets(make, per_set_bytes):
    """Enough buffer sets that one pass over them exceeds the 256 MB MALL."""
    nsets = max(1, min(64, math.ceil(512e6 / per_set_bytes)))
    return [make() for _ in range(nsets)]


def bench_rowreduce(C, rows, cols, op, iters=20, warmup=3):
    """Row max (op 1) or row sum (op 0) of X [rows, cols] fp32: one read of X."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    sets = _rotating_sets(lambda: (torch.randn((rows, cols), device="cuda", generator=g) * 2.0,
                                   torch.empty(rows, device="cuda")), rows * cols * 4)
    k = [0]
    pay = struct.pack("<i", op)

    def fn():
        x, o = sets[k[0] % len(sets)]
        k[0] += 1
        C.op_call(int(C.OpKind.RowReduce), [x], [o], RRED, pay, _cs())

    ms = time_launches(fn, iters, warmup, graph=True)
    nbytes = 4 * rows * cols + 4 * rows
    return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "buffer_sets": len(sets)}


def bench_xent(C, rows, cols, iters=20, warmup=3):
    """Fused softmax cross-entropy forward + backward: logits [rows, cols] fp32
    and int32 labels -> mean loss, dlogits, argmax, per-row loss."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(5)

    def make():
        z = torch.randn((rows, cols), device="cuda", generator=g) * 3.0
        lab = torch.randint(0, cols, (rows,), device="cuda", generator=g, dtype=torch.int32)
        return (z, lab, torch.empty((), device="cuda"), torch.empty_like(z),
                torch.empty(rows, dtype=torch.int32, device="cuda"), torch.empty(rows, device="cuda"))

    sets = _rotating_sets(make, rows * cols * 8)
    k = [0]

    def fn():
        z, lab, loss, dz, am, rl = sets[k[0] % len(sets)]
        k[0] += 1
        C.op_call(int(C.OpKind.SoftmaxXent), [z, lab], [loss, dz, am, rl], 0, b"", _cs())

    ms = time_launches(fn, iters, warmup, graph=True)
    nbytes = 8 * rows * cols + 16 * rows  # logits in, dlogits out, labels, argmax, row loss (r+w)
    return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "buffer_sets": len(sets)}


def bench_mse(C, rows, cols, iters=20, warmup=3):
    """Fused MSE loss + gradient of the train step: bf16 prediction, fp32
    target -> bf16 gradient and the mean loss (8 bytes per element)."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(6)

    def make():
        p = torch.randn((rows, cols), device="cuda", generator=g).to(torch.bfloat16)
        t = torch.randn((rows, cols), device="cuda", generator=g)
        return (p, t, torch.empty_like(p), torch.empty((), device="cuda"),
                torch.empty(max(1024, -(-rows * cols // 2048)), device="cuda"))  # as the step sizes it

    sets = _rotating_sets(make, rows * cols * 8)
    k = [0]

    def fn():
        p, t, d, loss, part = sets[k[0] % len(sets)]
        k[0] += 1
        C.launch_by_id("mse_loss_grad_v0", C.OpKind.MseGrad, [p, t], [d, loss, part], 0, b"", _cs())

    ms = time_launches(fn, iters, warmup, graph=True)
    nbytes = 8 * rows * cols
    return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "buffer_sets": len(sets)}


def bench_colsum(C, rows, cols, iters=20, warmup=3, partials=True):
    """Bias gradient of the train step: column sum of dY [rows, cols] bf16 ->
    fp32 [cols] (2 bytes per element read), with the [64, cols] partials
    buffer the lowered step passes (two passes: 64 row slices, then their
    fixed-order sum), or, partials=False, with the reference's one output
    (one pass over narrow column blocks)."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    sets = _rotating_sets(lambda: (torch.randn((rows, cols), device="cuda", generator=g).to(torch.bfloat16),
                                   torch.empty(cols, device="cuda"), torch.empty((64, cols), device="cuda")),
                          rows * cols * 2)
    k = [0]

    def fn():
        x, o, part = sets[k[0] % len(sets)]
        k[0] += 1
        C.launch_by_id("reduce_sum_keep_lastdim_bf16_to_f32_v0", C.OpKind.ReduceSum, [x],
                       [o, part] if partials else [o], 0, b"", _cs())

    ms = time_launches(fn, iters, warmup, graph=True)
    nbytes = 2 * rows * cols + 4 * cols
    return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "buffer_sets": len(sets)}


def bench_torch_matmul(M, N, K, iters=20, warmup=5):
    """The vendor library on the same box (torch.matmul -> hipBLASLt), bf16
    X[M,K] . W[N,K]^T, as a reference line for the GEMM kernel."""
    import torch

    X = torch.randn((M, K), device="cuda").to(torch.bfloat16)
    W = torch.randn((N, K), device="cuda").to(torch.bfloat16)
    Y = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
    ms = time_launches(lambda: torch.matmul(X, W.t(), out=Y), iters, warmup)
    return {"ms": ms, "tflops": 2.0 * M * N * K / (ms * 1e-3) / 1e12}


# ------------------------------------------------------------------ Adam
def bench_adam(C, n=1 << 28, steps=10):
    """Fused AdamW over a flat fp32 buffer, t = 1..steps, in place."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    P = torch.randn(n, device="cuda", generator=g) * 0.02
    G = torch.randn(n, device="cuda", generator=g) * 1e-3
    M = torch.zeros(n, device="cuda")
    V = torch.zeros(n, device="cuda")
    step = torch.zeros((), dtype=torch.int32, device="cuda")
    pay = struct.pack("<fffff", 1e-3, 0.9, 0.999, 1e-8, 0.01)

    def fn():
        C.launch_by_id("step_inc_v0", C.OpKind.StepInc, [step], [step])
        C.launch_by_id("adamw_step_f32_v1", C.OpKind.AdamStep, [P, G, M, V, step], [P, M, V], ADAM, pay)

    # step_inc is a 1-thread kernel (~2 us); it is part of the step.  A
    # 12 ms window read 5.9-6.5 TB/s from run to run: the median of five
    # windows after a longer warm-up
    wins = [time_launches(fn, steps, 1, warm_s=STEP_WARM_S if w == 0 else 0.0) for w in range(5)]
    ms = sorted(wins)[len(wins) // 2]
    nbytes = 28 * n
    return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes_per_step": nbytes,
            "windows_gbs": [round(nbytes / (w * 1e-3) / 1e9, 1) for w in wins], "final_step": int(step.item())}


# ------------------------------------------------------------------ MLP
def _make_step(B, D, L, own_graph=False, **plan_kw):
    """The bf16 MLP step built, initialised (seed 0) and captured."""
    from aicf_hip import mlp

    ir, lowered, plan = mlp.build_mlp_mse(B, D, L, **plan_kw)
    ex = mlp.make_executor(ir, lowered, plan, own_graph=own_graph)
    inputs, params = mlp.init_mlp_mse(B, D, L)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    mlp.refresh_shadow(ex)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    return ex, lowered


def bench_mlp(B, D, L, steps, warmup, warm_s=STEP_WARM_S, **plan_kw):
    """`warmup` untimed replays, then at least warm_s seconds of back-to-back
    replays (the clock's loaded steady state, as every component gets), then
    exactly `steps` replays timed with HIP events on the replay stream,
    synchronised on both sides."""
    import torch

    ex, lowered = _make_step(B, D, L, **plan_kw)
    gs = torch.cuda.current_stream()  # graph_launch replays on the caller's stream
    losses = []
    for _ in range(warmup):
        ex.replay(1)
    torch.cuda.synchronize()
    losses.append(float(ex.value("loss").item()))
    tw = time.perf_counter()
    _warm(lambda: ex.replay(1), warm_s)
    warm_ms = (time.perf_counter() - tw) * 1e3
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(gs)
    ex.replay(steps)
    e1.record(gs)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / steps
    losses.append(float(ex.value("loss").item()))
    finite = all(math.isfinite(v) for v in losses)
    ngemm = sum(1 for it in lowered if it["op"] in ("gemm", "gemm_epilogue", "gemm_adamw"))
    ex.reset_graph()
    return {"ms": ms, "wall_ms": wall * 1e3 / steps, "steps_per_s": 1e3 / ms, "losses": losses,
            "finite": finite, "ops": len(lowered), "gemms": ngemm, "warm_ms": warm_ms}


# The step in the headline's plan and the plans it is compared with.
STEP_VARIANTS = {
    "headline": dict(fuse_optimizer=True, fuse_colsum=True, fuse_tail=True),
    "without_tail_fusion": dict(fuse_optimizer=True, fuse_colsum=True),
    "without_dead_input_dx": dict(dead_dx=False, fuse_optimizer=True, fuse_colsum=True, fuse_tail=True),
    "reference_op_split": dict(),
}


def bench_mlp_alternated(B, D, L, rounds=10, chunk=10, warm_s=STEP_WARM_S):
    """Every step variant captured on a graph handle of its own, warmed
    together, then timed in `rounds` rounds of `chunk` replays each,
    variants alternated (order reversed every other round), so that clock
    and box state are shared and the plans compare like for like."""
    import torch

    exs = {k: _make_step(B, D, L, own_graph=True, **kw) for k, kw in STEP_VARIANTS.items()}
    for ex, _ in exs.values():
        ex.replay(3)
    torch.cuda.synchronize()
    _warm(lambda: [ex.replay(1) for ex, _ in exs.values()], warm_s)
    s = torch.cuda.current_stream()
    tot = {k: 0.0 for k in exs}
    names = list(exs)
    for r in range(rounds):
        for k in (names if r % 2 == 0 else names[::-1]):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            exs[k][0].replay(chunk)
            e1.record(s)
            torch.cuda.synchronize()
            tot[k] += e0.elapsed_time(e1)
    out = {}
    for k, (ex, lowered) in exs.items():
        ms = tot[k] / (rounds * chunk)
        out[k] = {"ms": ms, "steps_per_s": 1e3 / ms, "ops": len(lowered),
                  "gemms": sum(1 for it in lowered if it["op"] in ("gemm", "gemm_epilogue", "gemm_adamw")),
                  "loss_after": float(ex.value("loss").item())}
        ex.close()
    return out


STEP_GEMM_OPS = ("gemm", "gemm_epilogue", "gemm_adamw")
# The step's GEMM launches by kernel instantiation (the template arguments in
# the kernel name): role, launches per step (B=8192, D=4096, L=4) and
# algorithmic MiB moved per launch.
STEP_GEMM_ROLES = [
    ("<2, 2, 2, 256, 256, 2, 4, true, true, 2>", "fwd bias+GELU (+Z)", 3, 64 + 32 + 64 + 64),
    ("<2, 2, 0, 256, 256, 2, 2, true, true, 2>", "fwd bias (last layer)", 1, 64 + 32 + 64),
    ("<2, 2, 3, 256, 256, 2, 4, true, false, 2>", "dX with dGELU", 3, 64 + 32 + 64 + 64),
    ("<2, 2, 0, 256, 256, 2, 4, true, false, 2>", "dX (first layer)", 1, 64 + 32 + 64),
    ("<2, 0, 4, 256, 256, 2, 4, false, false, 2>", "dW + AdamW", 4, 64 + 64 + 3 * 64 * 2 + 32),
]


def gemm_role(op, attrs, n_out):
    from aicf_hip.executor import epilogue_kind

    if op == "gemm_adamw":
        return "dW + AdamW"
    if op == "gemm":
        return "dX (first layer)"
    kind = epilogue_kind(attrs)  # GEPI: 5 dGELU, 6/7 dGELU + column sums / partials, 3 bias+GELU, 1 bias
    return {5: "dX with dGELU", 6: "dX with dGELU", 7: "dX with dGELU",
            3: "fwd bias+GELU (+Z)"}.get(kind, "fwd bias (last layer)")


def build_step(B, D, L, fuse_optimizer=True, fuse_colsum=True, fuse_tail=True):
    from aicf_hip import mlp

    ir, lowered, plan = mlp.build_mlp_mse(B, D, L, fuse_optimizer=fuse_optimizer, fuse_colsum=fuse_colsum,
                                          fuse_tail=fuse_tail)
    ex = mlp.make_executor(ir, lowered, plan)
    inputs, params = mlp.init_mlp_mse(B, D, L)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    mlp.refresh_shadow(ex)
    return ex


def step_gemm_times(ex, iters, warmup=2, graph=True, warm_s=WARM_S):
    """Average ms per launch of each GEMM op of the step, HIP events on
    torch's current stream around a captured graph of `iters` launches of the
    op on the step's own tensors (back to back on the device, as in the
    step's own graph, rather than at the rate the host issues eager
    launches), after one eager pass over the step (so every activation holds
    this step's values; the AdamW over the biases, which no GEMM reads, is
    left out).  graph=False: eager launches instead (the counter runs, which
    count dispatches)."""
    import torch

    s = torch.cuda.current_stream()
    for i, o in enumerate(ex.ops):
        if o[0] not in ("adamw_step", "colsum_adamw"):
            ex.launch_op(i, stream=s.cuda_stream)
    torch.cuda.synchronize()
    res = []
    for i, (op, _kind, kid, _ins, outs, attrs) in enumerate(ex.ops):
        if op not in STEP_GEMM_OPS:
            continue
        ms = time_launches(lambda i=i: ex.launch_op(i, stream=torch.cuda.current_stream().cuda_stream),
                           iters, warmup, graph=graph, warm_s=warm_s)
        res.append({"op": i, "kernel_id": kid, "role": gemm_role(op, attrs, len(outs)), "ms": ms})
    return res


def bench_copy_ceiling(C, elems=1 << 29, iters=10, warmup=2):
    """HBM read+write ceiling of this part for a plain stream: copy_bf16_v0
    (16-byte nontemporal vector per lane) over 1 GiB, 2 bytes read and 2
    written per element; the reference point for the kernels that read and
    write a stream (softmax, xent, MSE, AdamW)."""
    import torch

    x = torch.ones(elems, device="cuda", dtype=torch.bfloat16)
    y = torch.empty_like(x)
    fn = lambda: C.launch_by_id("copy_bf16_v0", C.OpKind.Copy, [x], [y], 0, b"")  # noqa: E731
    wins = [time_launches(fn, iters, warmup, warm_s=STEP_WARM_S if w == 0 else 0.0) for w in range(5)]
    ms = sorted(wins)[len(wins) // 2]  # the median of five windows, as the AdamW line
    return {"gbs": 4.0 * elems / (ms * 1e-3) / 1e9, "ms": ms}


def bench_copy_sized(C, read_bytes, iters=20, warmup=3):
    """The copy kernel (copy_bf16_v0) moving `read_bytes` in and out, timed
    like the row kernels: a captured graph of back-to-back launches over
    rotated buffer sets whose working set exceeds the 256 MB MALL.  At sizes
    where a launch's fixed cost (dispatch, first-load latency, drain) is a
    large part of its time, this is the practical ceiling of a kernel that
    reads and writes that many bytes."""
    import torch

    elems = read_bytes // 2
    sets = _rotating_sets(lambda: (torch.ones(elems, device="cuda", dtype=torch.bfloat16),
                                   torch.empty(elems, device="cuda", dtype=torch.bfloat16)), 2 * read_bytes)
    k = [0]

    def fn():
        x, y = sets[k[0] % len(sets)]
        k[0] += 1
        C.launch_by_id("copy_bf16_v0", C.OpKind.Copy, [x], [y], 0, b"", _cs())

    ms = time_launches(fn, iters, warmup, graph=True)
    return {"ms": ms, "gbs": 2.0 * read_bytes / (ms * 1e-3) / 1e9}


def bench_mfma_ceiling(form=16, waves_per_simd=4, iters=20000, launches=8, warm=4):
    """Sustained rate of the register-only MFMA loop (aicf_diag_mfma_loop_form
    on random operands, no memory traffic): form 16 is v_mfma_f32_16x16x32_bf16,
    the instruction the bf16 GEMM kernels issue, form 32 is
    v_mfma_f32_32x32x16_bf16.  The higher of the two is the power-limited MFMA
    ceiling of this part, the practical upper bound of any bf16 GEMM on it.
    `warm` launches (~14 ms each) bring the board to its power-limited steady
    state before the timed ones."""
    import ctypes

    import torch

    from aicf_cuda import abi

    lib = abi.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks = cus * waves_per_simd  # 4 waves per workgroup, one per SIMD
    out = torch.zeros(1, device="cuda")
    s = torch.cuda.current_stream()
    flops = blocks * 4.0 * iters * (1 << 18)  # 2^18 flop per wave and round in either form
    times = []
    for k in range(warm + launches):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        st = lib.aicf_diag_mfma_loop_form(ctypes.c_void_p(out.data_ptr()), blocks, iters, k + 1, form,
                                          ctypes.c_void_p(s.cuda_stream))
        e1.record(s)
        torch.cuda.synchronize()
        if st != 0:
            raise RuntimeError(f"aicf_diag_mfma_loop_form failed: status {st}")
        if k >= warm:
            times.append(e0.elapsed_time(e1))
    ms = sum(times) / len(times)
    return {"tflops": flops / (ms * 1e-3) / 1e12, "ms": ms, "form": form}


# ------------------------------------------------------------------ CPU baseline
def cpu_baseline_mlp(B, D, L, sample_rows):
    """Oracle timing of one MLP step on `sample_rows` rows (every GEMM of the
    step with the reference's per-output sequential-k algorithm, GELU, MSE,
    column sums), scaled to the full batch, plus AdamW over all parameters."""
    import numpy as np

    import oracle as orc

    r = np.random.default_rng(0)
    b = sample_rows
    W = [orc.bf16_round(r.uniform(-0.03, 0.03, (D, D)).astype(np.float32)) for _ in range(L)]
    x = orc.bf16_round(r.standard_normal((b, D)).astype(np.float32))
    t_ = r.standard_normal((b, D)).astype(np.float32)
    t0 = time.perf_counter()
    hs, zs = [x], []
    for i in range(L):
        z = orc.gemm_ref_f32(hs[-1], W[i], False, True)
        zs.append(z)
        hs.append(orc.gelu_f64(z.astype(np.float64)).astype(np.float32) if i < L - 1 else z)
    dy = orc.mse_grad_f32(hs[-1], t_).reshape(b, D)
    for i in range(L - 1, -1, -1):
        orc.gemm_ref_f32(dy, hs[i], True, False)          # dW
        orc.colsum_f64(dy)                                 # db
        dx = orc.gemm_ref_f32(dy, W[i], False, False)      # dX
        if i > 0:
            dy = (dx * orc.gelu_grad_f64(zs[i - 1].astype(np.float64))).astype(np.float32)
    t_batch = time.perf_counter() - t0
    n = L * (D * D + D)
    # separate P, G, M, V: the update reads four streams and writes three
    P = np.full(n, 0.01, np.float32)
    G = np.full(n, 1e-3, np.float32)
    M = np.zeros(n, np.float32)
    V = np.zeros(n, np.float32)
    t1 = time.perf_counter()
    orc.adamw(P, G, M, V, 1, wd=0.01)
    t_adam = time.perf_counter() - t1
    per_step = t_batch * (B / b) + t_adam
    return {"value": 1.0 / per_step, "unit": "steps/s", "cores": orc.threads(), "kind": "port",
            "sample": f"{b} of {B} rows of one step (12 GEMMs with the reference's sequential-k "
                      f"fp32 algorithm + GELU/MSE/colsum) scaled by {B // b}, plus AdamW over all "
                      f"{n} parameters; measured {t_batch:.2f}s + {t_adam:.2f}s",
            "modelled_seconds_per_step": per_step}


def _cpu(value, unit, sample, **extra):
    import oracle as orc

    d = {"value": value, "unit": unit, "cores": orc.threads(), "kind": "port", "sample": sample}
    d.update(extra)
    return d


def cpu_baseline_c1(iters=20):
    """C1 on the host: the whole fp32 step of the reference MLP (64 x 784 ->
    256 ReLU -> 10, softmax cross-entropy, Adam) through the oracle: the six
    GEMMs of the reference lowering with its per-output sequential-k
    algorithm (gemm/launcher.cu:155-172), bias add, ReLU and its backward,
    the loss and its gradient, the column sums and the AdamW update of every
    parameter; microseconds per step."""
    import numpy as np

    import oracle as orc
    from aicf_hip import mlp

    d = mlp.init_mlp_xent()
    x, lab = d["x"], d["t"]
    P = {k: d[k].copy() for k in ("0.W", "0.b", "2.W", "2.b")}
    Ms = {k: np.zeros(v.size, np.float32) for k, v in P.items()}
    Vs = {k: np.zeros(v.size, np.float32) for k, v in P.items()}
    t0 = time.perf_counter()
    for it in range(iters):
        z = orc.gemm_ref_f32(x, P["0.W"], False, True) + P["0.b"][None, :]
        h = orc.relu_f32(z).reshape(z.shape)
        logits = orc.gemm_ref_f32(h, P["2.W"], False, True) + P["2.b"][None, :]
        _, dz, _, _ = orc.softmax_xent_f64(logits, lab)
        dz = dz.astype(np.float32)
        g = {"2.W": orc.gemm_ref_f32(dz, h, True, False), "2.b": orc.colsum_f64(dz).astype(np.float32)}
        dh = orc.gemm_ref_f32(dz, P["2.W"], False, False)
        dzz = orc.relu_bwd_f32(dh, h).reshape(dh.shape)
        g["0.W"] = orc.gemm_ref_f32(dzz, x, True, False)
        g["0.b"] = orc.colsum_f64(dzz).astype(np.float32)
        orc.gemm_ref_f32(dzz, P["0.W"], False, False)  # the input gradient the lowering emits
        for k in P:
            p, Ms[k], Vs[k] = orc.adamw(P[k], g[k], Ms[k], Vs[k], it + 1)
            P[k] = p.reshape(P[k].shape)
    us = (time.perf_counter() - t0) / iters * 1e6
    return _cpu(round(us, 1), "us/step", f"{iters} full steps at the configuration's own size")


def cpu_baseline_c2(rows=1024):
    """C2 on the host: row softmax with row max and row sum (the oracle's
    per-row pass, fp64 accumulation and output, OpenMP over rows) on the
    first `rows` rows of each width; GB/s at the GPU metric's algorithmic
    bytes (fp32 in and out, 8 B per element + 8 B per row)."""
    import numpy as np

    import oracle as orc

    out = {}
    r = np.random.default_rng(2)
    for cols in (128, 1024, 8192, 32768):
        x = (r.standard_normal((rows, cols)) * 2.0).astype(np.float32)
        orc.softmax_rows_f64(x[:8])
        t0 = time.perf_counter()
        orc.softmax_rows_f64(x)
        dt = time.perf_counter() - t0
        nbytes = 8.0 * rows * cols + 8.0 * rows
        out[cols] = _cpu(round(nbytes / dt / 1e9, 2), "GB/s",
                         f"{rows} of 16384 rows x {cols}; fp64 accumulation and output")
    return out


def cpu_baseline_c3(n=1 << 26):
    """C3 on the host: the oracle's AdamW (OpenMP over elements) over `n`
    parameters with separate P, G, M, V arrays, one step; GB/s at 28 B per
    parameter (4 streams read, 3 written)."""
    import numpy as np

    import oracle as orc

    r = np.random.default_rng(3)
    P = (r.standard_normal(n, dtype=np.float32) * 0.02)
    G = (r.standard_normal(n, dtype=np.float32) * 1e-3)
    M = np.zeros(n, np.float32)
    V = np.zeros(n, np.float32)
    orc.adamw(P[:1024], G[:1024], M[:1024], V[:1024], 1, wd=0.01)
    t0 = time.perf_counter()
    orc.adamw(P, G, M, V, 1, wd=0.01)
    dt = time.perf_counter() - t0
    return _cpu(round(28.0 * n / dt / 1e9, 2), "GB/s", f"2^{int(math.log2(n))} of 2^28 parameters, one step")


def cpu_baseline_c4(rows=8):
    """C4 on the host: the reference's fp32 GEMM algorithm (one sequential-k
    dot per output, gemm/launcher.cu:155-172; OpenMP over outputs) on the
    first `rows` rows of X at each shape, extrapolated to TFLOP/s (the
    epilogue is not timed: it is negligible beside the dots)."""
    import numpy as np

    import oracle as orc

    out = {}
    for (M, N, K) in C4_SHAPES:
        x = np.linspace(-1.0, 1.0, rows * K, dtype=np.float32).reshape(rows, K) / math.sqrt(K)
        w = np.linspace(-1.0, 1.0, N * K, dtype=np.float32).reshape(N, K)[:, ::-1].copy() / math.sqrt(K)
        orc.gemm_ref_f32(x[:1, :64], w[:8, :64], False, True)
        t0 = time.perf_counter()
        orc.gemm_ref_f32(x, w, False, True)
        dt = time.perf_counter() - t0
        out[(M, N, K)] = _cpu(round(2.0 * rows * N * K / dt / 1e12, 6), "TFLOP/s",
                              f"{rows} of {M} rows, fp32 sequential-k dots, extrapolated by rate")
    return out


# ------------------------------------------------------------------ main
# ------------------------------------------------------------------ HBM traffic (rocprofv3 --pmc)
TRAFFIC_FILE = REPO / "profiles" / "step_gemms_8192x4096x4096_traffic.md"
CALIB_ELEMS = 1 << 27          # calibration copy: 2^27 bf16 = 256 MiB read + 256 MiB written
CALIB_KIB = CALIB_ELEMS * 2 / 1024


def roofline_only(C, B, D, L, launches):
    """The roofline kernel family alone: one eager pass over the step, then
    4 warm-up and `launches` timed launches of each of the step's GEMM ops on
    its own tensors, then 3 calibration copies of known size; the program
    profiled by the FETCH_SIZE / WRITE_SIZE passes."""
    import torch

    ex = build_step(B, D, L)
    t = step_gemm_times(ex, iters=launches, warmup=0, graph=False, warm_s=0.0)
    x = torch.ones(CALIB_ELEMS, device="cuda", dtype=torch.bfloat16)
    y = torch.empty_like(x)
    for _ in range(3):
        C.launch_by_id("copy_bf16_v0", C.OpKind.Copy, [x], [y], 0, b"")
    torch.cuda.synchronize()
    log(f"[bench] roofline-only: {len(t)} GEMM ops x ({launches} + 1) launches, 3 calibration copies; {t}")


def mfma_report(counter_csv, trace_csv, pattern):
    """MFMA utilisation and effective clock of the dispatches whose kernel
    name contains `pattern`, from one rocprofv3 run with --pmc
    SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_BF16 and
    --kernel-trace.  SQ_VALU_MFMA_BUSY_CYCLES is summed over the 1024 SIMDs,
    GRBM_GUI_ACTIVE over the 8 XCDs (cycles of each XCD's clock)."""
    import csv
    from collections import defaultdict

    cnt = defaultdict(lambda: defaultdict(float))
    names = {}
    with open(counter_csv, newline="") as f:
        for row in csv.DictReader(f):
            d = int(row["Dispatch_Id"])
            cnt[d][row["Counter_Name"]] += float(row["Counter_Value"])
            names[d] = row.get("Kernel_Name", "")
    dur = {}
    with open(trace_csv, newline="") as f:
        for row in csv.DictReader(f):
            dur[int(row["Dispatch_Id"])] = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) * 1e-9
    rows = []
    for d in sorted(cnt):
        if pattern not in names[d] or d not in dur:
            continue
        c = cnt[d]
        gui = c["GRBM_GUI_ACTIVE"] / 8.0
        flop = c["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512.0
        rows.append((d, dur[d], gui / dur[d] / 1e9, c["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui * 1024.0),
                     flop / dur[d] / 1e12))
    lines = [f"| dispatch | us | clock GHz | MFMA busy | TFLOP/s |", "|---:|---:|---:|---:|---:|"]
    for d, t, clk, util, tf in rows:
        lines.append(f"| {d} | {t * 1e6:.1f} | {clk:.2f} | {util * 100:.1f}% | {tf:.0f} |")
    if rows:
        n = len(rows)
        lines.append(f"| mean | {sum(r[1] for r in rows) / n * 1e6:.1f} | {sum(r[2] for r in rows) / n:.2f} | "
                     f"{sum(r[3] for r in rows) / n * 100:.1f}% | {sum(r[4] for r in rows) / n:.0f} |")
    return lines


# Shape sets of --vendor-compare: (M, N, K) NT shapes, launches per group,
# whether the step's dW layout follows, and the report's description.
VENDOR_SETS = {
    "large": {"shapes": ((8192, 8192, 8192), (8192, 4096, 4096)), "group": 5, "dw": True,
              "desc": "8192^3 NT, 8192x4096x4096 NT (the step's forward layout), dW = dZ^T.H with K = 8192 "
                      "(fp32 out for ours, bf16 for hipBLASLt)"},
    "small": {"shapes": ((1024, 1024, 1024), (8192, 4096, 256), (8192, 4096, 512)), "group": 100, "dw": False,
              "desc": "the C4 shapes with few tiles or short K: 1024^3, 8192x4096x256 and 8192x4096x512 NT, "
                      "plain bf16 out (no bias)"},
}


def vendor_compare(C, shape_set="large"):
    """Our bf16 GEMM and torch.matmul (hipBLASLt) on the same operands, over
    the shapes of VENDOR_SETS[shape_set] (the large set adds the step's dW
    layout, dZ^T . H with K = 8192; ours writes fp32, hipBLASLt bf16).  Per
    shape, four alternating groups of launches (ours, vendor, ours, vendor),
    so that neither library always runs on a cooler or hotter part.  The
    program profiled for the counter comparisons."""
    import torch

    vs = VENDOR_SETS[shape_set]
    g = torch.Generator(device="cuda")
    g.manual_seed(9)

    def alternate(ours, vendor):
        for _ in range(2):
            for fn in (ours, vendor):
                for _ in range(vs["group"]):
                    fn()

    for (M, N, K) in vs["shapes"]:
        X = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
        W = torch.randn((N, K), device="cuda", generator=g).to(torch.bfloat16)
        Y = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
        alternate(lambda: C.launch_by_id("gemm_bf16_mfma_v0", C.OpKind.Gemm, [X, W], [Y], 0,
                                         struct.pack("<ii", 0, 1)),
                  lambda: torch.matmul(X, W.t(), out=Y))
    if not vs["dw"]:
        torch.cuda.synchronize()
        log(f"[bench] vendor-compare ({shape_set}): {len(vs['shapes'])} shapes x 2 x ({vs['group']} ours, "
            f"{vs['group']} torch.matmul) launches")
        return
    dZ = torch.randn((8192, 4096), device="cuda", generator=g).to(torch.bfloat16)
    H = torch.randn((8192, 4096), device="cuda", generator=g).to(torch.bfloat16)
    dW = torch.empty((4096, 4096), device="cuda")
    dWb = torch.empty((4096, 4096), device="cuda", dtype=torch.bfloat16)
    alternate(lambda: C.launch_by_id("gemm_bf16_mfma_f32out_v0", C.OpKind.Gemm, [dZ, H], [dW], 0,
                                     struct.pack("<ii", 1, 0)),
              lambda: torch.matmul(dZ.t(), H, out=dWb))
    torch.cuda.synchronize()
    log("[bench] vendor-compare: 3 shapes x 2 x (5 ours, 5 torch.matmul) launches")


def pmc_mfma_compare_report(counter_csv, trace_csv):
    """MFMA utilisation and clock per (kernel, shape) of a --vendor-compare
    run (rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE
    SQ_INSTS_VALU_MFMA_MOPS_BF16 --kernel-trace); the first launch of each
    group is dropped."""
    import csv
    from collections import OrderedDict, defaultdict

    cnt = defaultdict(lambda: defaultdict(float))
    names = {}
    with open(counter_csv, newline="") as f:
        for row in csv.DictReader(f):
            d = int(row["Dispatch_Id"])
            cnt[d][row["Counter_Name"]] += float(row["Counter_Value"])
            names[d] = row.get("Kernel_Name", "")
    dur = {}
    with open(trace_csv, newline="") as f:
        for row in csv.DictReader(f):
            dur[int(row["Dispatch_Id"])] = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) * 1e-9
    groups = OrderedDict()
    for d in sorted(cnt):
        n = names[d]
        if not ("gemm_nt" in n or "Cijk" in n) or d not in dur:
            continue
        flop = cnt[d]["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512.0
        short = n.replace("void aicf::hip::(anonymous namespace)::", "").split("(")[0][:72]
        key = ("ours " if "gemm_nt" in n else "hipBLASLt ") + short + f" | {flop / 1e9:.0f} GFLOP"
        groups.setdefault(key, []).append(d)
    lines = [
        "# bf16 GEMM on MI355X: our kernel vs hipBLASLt, MFMA utilisation and clock",
        "",
        "Commands (GPU box, repo root):",
        "```",
        "rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_BF16 --kernel-trace "
        "--output-format csv -d gpurun_out/pmc_vendor -o run -- python3 bench.py --vendor-compare",
        "python3 bench.py --pmc-mfma-compare-report gpurun_out/pmc_vendor/run_counter_collection.csv "
        "gpurun_out/pmc_vendor/run_kernel_trace.csv",
        "```",
        "",
        "MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x 1024 SIMDs) = achieved / peak at "
        "the clock the part actually ran; clock = GRBM_GUI_ACTIVE per XCD / kernel duration.  Shapes: "
        "8192^3 NT (1100 GFLOP), 8192x4096x4096 NT (275), dW = dZ^T.H with K = 8192 (275, second "
        "group of that size).",
        "",
        "| kernel | GFLOP | launches | us | clock GHz | MFMA busy | TFLOP/s | % of 2.5 PF |",
        "|---|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for key, ds in groups.items():
        ds = ds[1:] if len(ds) > 4 else ds  # the first launch of each kernel warms it up
        t = sum(dur[d] for d in ds) / len(ds)
        gui = sum(cnt[d]["GRBM_GUI_ACTIVE"] for d in ds) / len(ds) / 8.0
        busy = sum(cnt[d]["SQ_VALU_MFMA_BUSY_CYCLES"] for d in ds) / len(ds)
        flop = sum(cnt[d]["SQ_INSTS_VALU_MFMA_MOPS_BF16"] for d in ds) / len(ds) * 512.0
        name, gf = key.split(" | ")
        lines.append(f"| `{name}` | {gf.split()[0]} | {len(ds)} | {t * 1e6:.1f} | {gui / t / 1e9:.2f} | "
                     f"{busy / (gui * 1024.0) * 100:.1f}% | {flop / t / 1e12:.0f} | "
                     f"{flop / t / 1e12 / PEAK_BF16_TFLOPS * 100:.1f}% |")
    lines.append("")
    print("\n".join(lines))


VENDOR_PASSES = [
    "SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT "
    "SQ_LDS_IDX_ACTIVE SQ_INSTS_VMEM_RD SQ_INSTS_VMEM_WR SQ_INSTS_SALU",
    "TA_TA_BUSY_sum TD_TD_BUSY_sum TCP_TOTAL_CACHE_ACCESSES_sum TCP_TCC_READ_REQ_sum SQ_WAIT_INST_LDS "
    "SQ_WAIT_ANY SQ_WAVE_CYCLES SQ_INSTS_VALU GRBM_GUI_ACTIVE",
]


def pmc_compare_report(*paths, shape_set="large"):
    """Per-flop counter comparison of our bf16 GEMM and hipBLASLt on the same
    operands, from the two rocprofv3 --pmc passes of --vendor-compare
    (VENDOR_PASSES, each with --kernel-trace): arguments are counter_csv,
    trace_csv of pass 1, then of pass 2.  Launches are grouped by library,
    kernel and grid (the shape); the first launch of a group is dropped."""
    import csv
    from collections import OrderedDict, defaultdict

    def load(counter_csv, trace_csv):
        cnt = defaultdict(lambda: defaultdict(float))
        meta = {}
        with open(counter_csv, newline="") as f:
            for row in csv.DictReader(f):
                d = int(row["Dispatch_Id"])
                cnt[d][row["Counter_Name"]] += float(row["Counter_Value"])
                meta[d] = (row.get("Kernel_Name", ""), row.get("Grid_Size", ""))
        dur = {}
        with open(trace_csv, newline="") as f:
            for row in csv.DictReader(f):
                dur[int(row["Dispatch_Id"])] = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) * 1e-9
        groups = OrderedDict()
        per_shape = 4 * VENDOR_SETS[shape_set]["group"]  # GEMM launches per shape, both libraries
        i = 0
        for d in sorted(cnt):
            n, grid = meta[d]
            if not ("gemm_nt" in n or "Cijk" in n) or d not in dur:
                continue
            short = n.replace("void aicf::hip::(anonymous namespace)::", "").split("(")[0][:64]
            lib = ("ours " if "gemm_nt" in n else "hipBLASLt ") + short
            groups.setdefault((lib, grid, i // per_shape), []).append(d)
            i += 1
        out = OrderedDict()
        for key, ds in groups.items():
            ds = ds[1:] if len(ds) > 4 else ds
            m = defaultdict(float)
            for d in ds:
                for k, v in cnt[d].items():
                    m[k] += v / len(ds)
            m["_us"] = sum(dur[d] for d in ds) / len(ds) * 1e6
            m["_n"] = len(ds)
            out[key] = m
        return out

    p1 = load(paths[0], paths[1])
    p2 = load(paths[2], paths[3]) if len(paths) >= 4 else {}
    lines = [
        "# bf16 GEMM on MI355X: our kernel vs hipBLASLt, per-flop counters",
        "",
        "Commands (GPU box, repo root; one rocprofv3 run per counter pass):",
        "```",
    ]
    flag = "" if shape_set == "large" else f" --vendor-set {shape_set}"
    for i, pas in enumerate(VENDOR_PASSES):
        lines.append(f"rocprofv3 --pmc {pas} --kernel-trace --output-format csv -d gpurun_out/pmc_v{i + 1} -o run "
                     f"-- python3 bench.py --vendor-compare{flag}")
    lines += [
        "python3 bench.py --pmc-compare-report gpurun_out/pmc_v1/run_counter_collection.csv "
        "gpurun_out/pmc_v1/run_kernel_trace.csv gpurun_out/pmc_v2/run_counter_collection.csv "
        f"gpurun_out/pmc_v2/run_kernel_trace.csv{flag}",
        "```",
        "",
        f"Shapes: {VENDOR_SETS[shape_set]['desc']}.  clock = GRBM_GUI_ACTIVE per XCD / duration; MFMA busy = "
        "SQ_VALU_MFMA_BUSY_CYCLES / (GUI cycles per XCD x 1024 SIMDs); per-GFLOP columns divide by the "
        "flops the MFMA counter saw (SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512).  LDS conflict = "
        "SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE; TA / TD busy = busy cycles summed over the 256 CUs' units "
        "/ (GUI cycles per XCD x 256); waits = SQ_WAIT_* / SQ_WAVE_CYCLES.",
        "",
        "| kernel | grid | n | us | GHz | MFMA busy | TF/s | LDS instr /GF | LDS conflict | VMEM rd /GF | "
        "VMEM wr /GF | SALU /GF | VALU /GF | TA busy | TD busy | TCP acc /GF | TCC rd req /GF | wait LDS | "
        "wait any |",
        "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for key, m in p1.items():
        name, grid, _shape = key
        gui = m["GRBM_GUI_ACTIVE"] / 8.0
        us = m["_us"]
        gf = m["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512.0 / 1e9
        q = p2.get(key, {})
        gui2 = q.get("GRBM_GUI_ACTIVE", 0.0) / 8.0
        wave = q.get("SQ_WAVE_CYCLES", 0.0)

        def per(v):
            return f"{v / gf:.0f}" if gf else "-"

        def frac(v, den):
            return f"{v / den * 100:.1f}%" if den else "-"

        lines.append(
            f"| `{name}` | {grid} | {m['_n']} | {us:.1f} | {gui / (us * 1e-6) / 1e9:.2f} | "
            f"{frac(m['SQ_VALU_MFMA_BUSY_CYCLES'], gui * 1024.0)} | {gf * 1e9 / (us * 1e-6) / 1e12:.0f} | "
            f"{per(m['SQ_INSTS_LDS'])} | {frac(m['SQ_LDS_BANK_CONFLICT'], m['SQ_LDS_IDX_ACTIVE'])} | "
            f"{per(m['SQ_INSTS_VMEM_RD'])} | {per(m['SQ_INSTS_VMEM_WR'])} | {per(m['SQ_INSTS_SALU'])} | "
            f"{per(q.get('SQ_INSTS_VALU', 0.0)) if q else '-'} | "
            f"{frac(q.get('TA_TA_BUSY_sum', 0.0), gui2 * 256.0)} | {frac(q.get('TD_TD_BUSY_sum', 0.0), gui2 * 256.0)} | "
            f"{per(q.get('TCP_TOTAL_CACHE_ACCESSES_sum', 0.0)) if q else '-'} | "
            f"{per(q.get('TCP_TCC_READ_REQ_sum', 0.0)) if q else '-'} | "
            f"{frac(q.get('SQ_WAIT_INST_LDS', 0.0), wave)} | {frac(q.get('SQ_WAIT_ANY', 0.0), wave)} |")
    lines.append("")
    print("\n".join(lines))


def pmc_report(fetch_csv, write_csv, mfma_csv=None, trace_csv=None):
    """Markdown summary of two rocprofv3 --pmc runs of --roofline-only
    (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), per GEMM role of the step
    and weighted by the role's launches per step.  Each counter is scaled by
    the calibration copy's expected/measured ratio.  With the MFMA counter run
    and its kernel trace, also the MFMA utilisation and clock per dispatch."""
    import csv
    from statistics import mean

    def per_kernel(path, counter):
        vals = {"copy": []}
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                name = row.get("Kernel_Name", "")
                if "map1" in name:
                    vals["copy"].append(float(row["Counter_Value"]))
                    continue
                for sig, role, _n, _mib in STEP_GEMM_ROLES:
                    if "gemm_nt_kernel" in name and sig in name:
                        vals.setdefault(role, []).append(float(row["Counter_Value"]))
        return vals

    fe, wr = per_kernel(fetch_csv, "FETCH_SIZE"), per_kernel(write_csv, "WRITE_SIZE")
    f_r = CALIB_KIB / mean(fe["copy"])
    f_w = CALIB_KIB / mean(wr["copy"])
    lines = [
        "# HBM traffic of the step's GEMM launches (bf16, B=8192, D=4096, L=4)",
        "",
        "Commands (GPU box, repo root):",
        "```",
        "rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/pmc_fetch -o run -- "
        "python3 bench.py --roofline-only",
        "rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/pmc_write -o run -- "
        "python3 bench.py --roofline-only",
        "python3 bench.py --pmc-report <fetch counter_collection.csv> <write counter_collection.csv> "
        "<mfma counter_collection.csv> <mfma kernel_trace.csv>",
        "```",
        "",
        "`--roofline-only` builds the step, runs it once eagerly, launches each of its 12 GEMM ops 9 "
        "more times on the step's own tensors (4 warm-up launches, then 5 timed), then 3 calibration copies.",
        "",
        f"calibration copy (copy_bf16_v0, {CALIB_KIB:.0f} KiB read + written): "
        f"FETCH_SIZE {mean(fe['copy']):.0f} KiB -> factor {f_r:.4f}; "
        f"WRITE_SIZE {mean(wr['copy']):.0f} KiB -> factor {f_w:.4f}",
        "",
        "| role | launches/step | dispatches (fetch, write) | HBM read MB | HBM write MB | "
        "algorithmic MB | ratio |",
        "|---|---:|---:|---:|---:|---:|---:|",
    ]
    tot_b = tot_alg = 0.0
    n_step = 0
    for _sig, role, n, mib in STEP_GEMM_ROLES:
        if role not in fe or role not in wr:
            continue
        rb = mean(fe[role]) * f_r * 1024
        wb = mean(wr[role]) * f_w * 1024
        alg = mib * 2.0 ** 20
        lines.append(f"| {role} | {n} | {len(fe[role])}, {len(wr[role])} | {rb / 1e6:.1f} | {wb / 1e6:.1f} | "
                     f"{alg / 1e6:.1f} | {(rb + wb) / alg:.3f} |")
        tot_b += n * (rb + wb)
        tot_alg += n * alg
        n_step += n
    lines += [
        "",
        "Algorithmic bytes per launch: operands read once and outputs written once (bf16 activations "
        "64 MiB, weights 32 MiB; dW+AdamW: dY and h 64 MiB each, P/M/V fp32 64 MiB each read and "
        "written, bf16 shadow 32 MiB).",
        "",
        f"step mean over {n_step} launches: {tot_b / n_step / 1e6:.1f} MB measured, "
        f"{tot_alg / n_step / 1e6:.1f} MB algorithmic",
        "",
        f"traffic_bytes_per_launch: {int(round(tot_b / max(n_step, 1)))}",
        "",
    ]
    if mfma_csv and trace_csv:
        lines += [
            "## MFMA utilisation and clock of the same GEMM launches",
            "",
            "```",
            "rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_BF16 "
            "--kernel-trace --output-format csv -d gpurun_out/pmc_mfma -o run -- python3 bench.py "
            "--roofline-only",
            "```",
            "",
            "MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x 1024 SIMDs); clock = "
            "GRBM_GUI_ACTIVE per XCD / kernel duration; TFLOP/s from SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512.",
            "",
        ]
        for sig, role, _n, _mib in STEP_GEMM_ROLES:
            lines += [f"### {role}", ""] + mfma_report(mfma_csv, trace_csv, sig) + [""]
    print("\n".join(lines))


# Streaming kernels profiled by --streaming-only: (label, kernel-name pattern,
# algorithmic bytes per dispatch).  Shapes follow the benchmark configs.
SR, SC = 16384, 32768
STREAMING = [
    ("row softmax (+max, +sum) 16384x128 f32", "row_reg_kernel<16, 2, 0>", 8 * SR * 128 + 8 * SR),
    ("row softmax (+max, +sum) 16384x1024 f32", "row_reg_kernel<128, 2, 0>", 8 * SR * 1024 + 8 * SR),
    ("row sum 16384x128 f32", "row_reg_kernel<16, 2, 1>", 4 * SR * 128 + 4 * SR),
    ("row max 16384x128 f32", "row_reg_kernel<16, 2, 2>", 4 * SR * 128 + 4 * SR),
    ("row sum 16384x1024 f32", "row_reg_kernel<128, 2, 1>", 4 * SR * 1024 + 4 * SR),
    ("row max 16384x1024 f32", "row_reg_kernel<128, 2, 2>", 4 * SR * 1024 + 4 * SR),
    ("row softmax (+max, +sum) 16384x8192 f32", "row_reg_kernel<128, 16, 0>", 8 * SR * 8192 + 8 * SR),
    ("row softmax (+max, +sum) 16384x32768 f32", "row_reg_kernel<512, 16, 0>", 8 * SR * SC + 8 * SR),
    ("row sum 16384x32768 f32", "row_reg_kernel<512, 16, 1>", 4 * SR * SC + 4 * SR),
    ("row max 16384x32768 f32", "row_reg_kernel<512, 16, 2>", 4 * SR * SC + 4 * SR),
    ("softmax xent fwd+bwd 16384x8192 f32", "row_reg_kernel<128, 16, 3>", 8 * SR * 8192 + 16 * SR),
    ("mse loss+grad 8192x4096 (bf16 p, f32 t, bf16 grad)", "mse_loss_grad_oneshot", 8 * 8192 * 4096),
    ("bias grad colsum 8192x4096 bf16 -> f32", "colsum_vec_kernel", 2 * 8192 * 4096 + 4 * 4096),
    ("column sum, one output 8192x4096 bf16 -> f32", "colsum_narrow_kernel", 2 * 8192 * 4096 + 4 * 4096),
    ("AdamW 2^28 f32 (P,G,M,V in; P,M,V out)", "adamw_vec4_kernel", 28 * (1 << 28)),
]


def streaming_only(C):
    """Each streaming kernel of the benchmark three times at its benchmark
    shape, then three calibration copies; the program profiled by the
    FETCH_SIZE / WRITE_SIZE passes of the streaming traffic summary."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(8)
    for cols in (128, 1024, 8192):
        xs = torch.randn((SR, cols), device="cuda", generator=g) * 2.0
        ys = torch.empty_like(xs)
        mxs, sms = torch.empty(SR, device="cuda"), torch.empty(SR, device="cuda")
        for _ in range(3):
            C.op_call(int(C.OpKind.RowSoftmax), [xs], [ys, mxs, sms], 0, b"", 0)
        if cols <= 1024:
            for op in (0, 1):
                for _ in range(3):
                    C.op_call(int(C.OpKind.RowReduce), [xs], [mxs], RRED, struct.pack("<i", op), 0)
        del xs, ys
    x = torch.randn((SR, SC), device="cuda", generator=g) * 2.0
    y = torch.empty_like(x)
    mx, sm = torch.empty(SR, device="cuda"), torch.empty(SR, device="cuda")
    for _ in range(3):
        C.op_call(int(C.OpKind.RowSoftmax), [x], [y, mx, sm], 0, b"", 0)
    for op in (0, 1):
        for _ in range(3):
            C.op_call(int(C.OpKind.RowReduce), [x], [mx], RRED, struct.pack("<i", op), 0)
    del x, y
    z = torch.randn((SR, 8192), device="cuda", generator=g) * 3.0
    lab = torch.randint(0, 8192, (SR,), device="cuda", generator=g, dtype=torch.int32)
    loss, dz = torch.empty((), device="cuda"), torch.empty_like(z)
    am, rl = torch.empty(SR, dtype=torch.int32, device="cuda"), torch.empty(SR, device="cuda")
    for _ in range(3):
        C.op_call(int(C.OpKind.SoftmaxXent), [z, lab], [loss, dz, am, rl], 0, b"", 0)
    del z, dz
    pb = torch.randn((8192, 4096), device="cuda", generator=g).to(torch.bfloat16)
    t = torch.randn((8192, 4096), device="cuda", generator=g)
    d, part = torch.empty_like(pb), torch.empty(8192 * 4096 // 2048, device="cuda")
    for _ in range(3):
        C.launch_by_id("mse_loss_grad_v0", C.OpKind.MseGrad, [pb, t], [d, loss, part])
    o, opart = torch.empty(4096, device="cuda"), torch.empty((64, 4096), device="cuda")
    for _ in range(3):
        C.launch_by_id("reduce_sum_keep_lastdim_bf16_to_f32_v0", C.OpKind.ReduceSum, [d], [o, opart])
    for _ in range(3):
        C.launch_by_id("reduce_sum_keep_lastdim_bf16_to_f32_v0", C.OpKind.ReduceSum, [d], [o])
    del pb, t, d
    n = 1 << 28
    P = torch.randn(n, device="cuda", generator=g) * 0.02
    G = torch.randn(n, device="cuda", generator=g) * 1e-3
    M, V = torch.zeros(n, device="cuda"), torch.zeros(n, device="cuda")
    step = torch.zeros((), dtype=torch.int32, device="cuda")
    pay = struct.pack("<fffff", 1e-3, 0.9, 0.999, 1e-8, 0.01)
    for _ in range(3):
        C.launch_by_id("step_inc_v0", C.OpKind.StepInc, [step], [step])
        C.launch_by_id("adamw_step_f32_v1", C.OpKind.AdamStep, [P, G, M, V, step], [P, M, V], ADAM, pay)
    del P, G, M, V
    xc = torch.ones(CALIB_ELEMS, device="cuda", dtype=torch.bfloat16)
    yc = torch.empty_like(xc)
    for _ in range(3):
        C.launch_by_id("copy_bf16_v0", C.OpKind.Copy, [xc], [yc], 0, b"")
    torch.cuda.synchronize()
    log(f"[bench] streaming-only: {len(STREAMING)} kernels x 3 dispatches, 3 calibration copies")


def pmc_streaming_report(fetch_csv, write_csv):
    """Markdown summary of two rocprofv3 --pmc runs of --streaming-only:
    HBM bytes per dispatch of each streaming kernel (calibrated like the GEMM
    summary) against its algorithmic bytes."""
    import csv
    from collections import defaultdict
    from statistics import mean

    def per_kernel(path, counter):
        vals = defaultdict(list)
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                name = row.get("Kernel_Name", "")
                for label, pat, _ in STREAMING:
                    if pat in name:
                        vals[label].append(float(row["Counter_Value"]))
                if "map1" in name:
                    vals["copy"].append(float(row["Counter_Value"]))
        return vals

    fe, wr = per_kernel(fetch_csv, "FETCH_SIZE"), per_kernel(write_csv, "WRITE_SIZE")
    f_r = CALIB_KIB / mean(fe["copy"])
    f_w = CALIB_KIB / mean(wr["copy"])
    lines = [
        "# HBM traffic of the streaming kernels (one dispatch each, benchmark shapes)",
        "",
        "Commands (GPU box, repo root):",
        "```",
        "rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/pmc_sfetch -o run -- "
        "python3 bench.py --streaming-only",
        "rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/pmc_swrite -o run -- "
        "python3 bench.py --streaming-only",
        "python3 bench.py --pmc-streaming-report <fetch counter_collection.csv> "
        "<write counter_collection.csv>",
        "```",
        "",
        f"calibration copy (copy_bf16_v0, {CALIB_KIB:.0f} KiB read + written): FETCH_SIZE "
        f"{mean(fe['copy']):.0f} KiB -> factor {f_r:.4f}; WRITE_SIZE {mean(wr['copy']):.0f} KiB -> "
        f"factor {f_w:.4f}",
        "",
        "| kernel | algorithmic MB | HBM read MB | HBM write MB | HBM / algorithmic |",
        "|---|---:|---:|---:|---:|",
    ]
    for label, _, alg in STREAMING:
        if not fe.get(label) or not wr.get(label):
            lines.append(f"| {label} | {alg / 1e6:.1f} | n/a | n/a | n/a |")
            continue
        rb = mean(fe[label]) * f_r * 1024
        wb = mean(wr[label]) * f_w * 1024
        lines.append(f"| {label} | {alg / 1e6:.1f} | {rb / 1e6:.1f} | {wb / 1e6:.1f} | "
                     f"{(rb + wb) / alg:.3f} |")
    lines.append("")
    print("\n".join(lines))


def stats_report(stats_csv, trace_csv, steps):
    """Markdown summary of `rocprofv3 --kernel-trace --stats` over
    `bench.py --steps N --no-cpu --no-components`: per-kernel totals, and the
    launches of the replayed step (those between the first and the last
    replay) grouped per step."""
    import csv

    with open(stats_csv, newline="") as f:
        stats = list(csv.DictReader(f))
    with open(trace_csv, newline="") as f:
        trace = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    short = lambda n: n.replace("aicf::hip::(anonymous namespace)::", "").split("(")[0][:80]  # noqa: E731
    lines = [
        "# Kernel time summary: bf16 MLP train step (hipGraph replay) + roofline GEMM",
        "",
        "Command (repo root, one MI355X):",
        "",
        "```",
        f"rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/prof -o bench -- "
        f"python3 -u bench.py --steps {steps} --no-cpu --no-components",
        "python3 bench.py --stats-report gpurun_out/prof/bench_kernel_stats.csv "
        f"gpurun_out/prof/bench_kernel_trace.csv {steps}",
        "```",
        "",
        f"Process contents: warmup + {steps} timed replays of the captured step (batch 8192, 4 x 4096^2, "
        "GELU, MSE, AdamW in the dW GEMMs' epilogue, the loss and bias tail in mse_colsum and "
        "colsum_adamw), then the roofline measurement: one eager pass over the step and 12 launches of "
        "each of its 12 GEMM ops.",
        "`gemm_nt_kernel<IN, OUT, ACT, BM, BN, WM, WN, AKC, BKC, S>`: IN 2 = bf16; OUT 2 = bf16, 0 = fp32; "
        "ACT 0 none, 2 GELU (+ pre-activation store), 3 dGELU, 4 AdamW; WM x WN waves; AKC/BKC operand "
        "K-contiguous (false: M/N-contiguous, read in place through transposing LDS reads); S LDS stages.",
        "",
        "| kernel | calls | avg us | % time |",
        "|---|---:|---:|---:|",
    ]
    for r in stats[:16]:
        lines.append(f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                     f"{float(r['Percentage']):.2f} |")
    # one replayed step = the kernels between two adamw launches (AdamW ends the step)
    ends = [i for i, r in enumerate(trace) if "adamw" in r["Kernel_Name"]]
    if len(ends) >= 3:
        a, b = ends[-2] + 1, ends[-1] + 1
        step = trace[a:b]
        t0 = int(step[0]["Start_Timestamp"])
        t1 = int(step[-1]["End_Timestamp"])
        busy = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in step)
        lines += ["", f"Last replayed step, launch by launch ({len(step)} kernels, first start to last end "
                  f"{(t1 - t0) / 1e3:.1f} us, kernels busy {busy / 1e3:.1f} us):", "",
                  "| # | kernel | us |", "|---:|---|---:|"]
        for i, r in enumerate(step):
            lines.append(f"| {i} | `{short(r['Kernel_Name'])}` | "
                         f"{(int(r['End_Timestamp']) - int(r['Start_Timestamp'])) / 1e3:.1f} |")
        dur = lambda rs: [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3  # noqa: E731
                          for rs_ in [rs] for r in rs_ if "gemm_nt_kernel" in r["Kernel_Name"]]
        g_step, g_roof = dur(step), dur(trace[b:])
        if g_step:
            lines += ["", f"GEMM launches of the last replayed step: {len(g_step)}, mean "
                      f"{sum(g_step) / len(g_step):.1f} us (the roofline's avg_ms is the same mean over "
                      "graphs of 10 launches of each GEMM op)."]
        if g_roof:
            lines.append(f"GEMM launches after the replays (roofline measurement): {len(g_roof)}, mean "
                         f"{sum(g_roof) / len(g_roof):.1f} us.")
    lines.append("")
    print("\n".join(lines))


def c1_trace_report(stats_csv, trace_csv):
    """Markdown summary of `rocprofv3 --kernel-trace --stats` over
    `bench.py --c1-only`: per-kernel totals, then the last replayed step of
    the three-launch lowering, of the four-launch one and of the reference's
    17-op lowering, launch by launch."""
    import csv

    with open(stats_csv, newline="") as f:
        stats = list(csv.DictReader(f))
    with open(trace_csv, newline="") as f:
        trace = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    short = lambda n: n.replace("aicf::hip::(anonymous namespace)::", "").split("(")[0][:80]  # noqa: E731
    us = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3  # noqa: E731
    lines = [
        "# Kernel time summary: C1, the reference MLP step (batch 64, 784 -> 256 ReLU -> 10, softmax "
        "cross-entropy, Adam), hipGraph replay",
        "",
        "Command (repo root, one MI355X):",
        "",
        "```",
        "rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/c1prof -o c1 -- python3 -u bench.py "
        "--c1-only",
        "python3 bench.py --c1-trace-report gpurun_out/c1prof/c1_kernel_stats.csv "
        "gpurun_out/c1prof/c1_kernel_trace.csv",
        "```",
        "",
        "Process contents: the three-launch step (StageF), its four-launch form (AdamW in a launch of its "
        "own) and the reference pipeline's 17-op lowering, each captured on a graph handle of its own; "
        "warmed together, then 5 rounds of 20 steps each, alternated.",
        "",
        "| kernel | calls | avg us | % time |",
        "|---|---:|---:|---:|",
    ]
    for r in stats[:20]:
        lines.append(f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{float(r['Percentage']):.2f} |")
    # the last step of each lowering in the kernel sequence (the lowerings
    # are replayed alternated): three-launch = gemm, head, group not
    # followed by adamw_multi; four-launch = the same followed by it
    ktr = [r for r in trace if "copyBuffer" not in r["Kernel_Name"]]
    nm = [r["Kernel_Name"] for r in ktr]
    three = four = None
    for i in range(len(nm) - 2):
        if "gemm_small" in nm[i] and "xent_head" in nm[i + 1] and "grad_group" in nm[i + 2]:
            if i + 3 < len(nm) and "adamw_multi" in nm[i + 3]:
                four = ktr[i:i + 4]
            else:
                three = ktr[i:i + 3]
    # the reference lowering's step ends with its four adamw_step launches
    ad = [i for i, r in enumerate(ktr) if "adamw_vec4" in r["Kernel_Name"]
          and (i + 1 == len(ktr) or "adamw_vec4" not in ktr[i + 1]["Kernel_Name"])]
    ref_step = ktr[ad[-1] - 17:ad[-1] + 1] if ad and ad[-1] >= 17 else []
    for title, step in (("three-launch lowering", three or []), ("four-launch lowering", four or []),
                        ("reference 17-op lowering", ref_step)):
        if not step:
            continue
        t0, t1 = int(step[0]["Start_Timestamp"]), int(step[-1]["End_Timestamp"])
        lines += ["", f"Last replayed step of the {title} ({len(step)} kernels, first start to last end "
                  f"{(t1 - t0) / 1e3:.1f} us, kernels busy {sum(us(r) for r in step):.1f} us):", "",
                  "| # | kernel | us |", "|---:|---|---:|"]
        for i, r in enumerate(step):
            lines.append(f"| {i} | `{short(r['Kernel_Name'])}` | {us(r):.2f} |")
    lines.append("")
    print("\n".join(lines))


def read_traffic():
    """HBM bytes per launch of the roofline kernel from the committed PMC summary."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 50 warmup replays: the part's clocks ramp over the first ~50 steps
    # (3.23 ms for the first 10, 2.95 ms from the 50th on, flat over 400).
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--batch", type=int, default=8192)
    ap.add_argument("--hidden", type=int, default=4096)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--no-components", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=8)
    ap.add_argument("--roofline-only", action="store_true",
                    help="run only the roofline GEMM and a calibration copy (for rocprofv3 --pmc)")
    ap.add_argument("--pmc-report", nargs="+", metavar="CSV",
                    help="summarise rocprofv3 --pmc CSVs of --roofline-only (FETCH, WRITE "
                         "[, MFMA counters, kernel trace]) and exit")
    ap.add_argument("--stats-report", nargs=3, metavar=("STATS_CSV", "TRACE_CSV", "STEPS"),
                    help="summarise a rocprofv3 --kernel-trace --stats run of the step and exit")
    ap.add_argument("--vendor-set", choices=sorted(VENDOR_SETS), default="large",
                    help="shape set of --vendor-compare and --pmc-compare-report")
    ap.add_argument("--vendor-compare", action="store_true",
                    help="our GEMM and torch.matmul on the same shapes (for rocprofv3 --pmc)")
    ap.add_argument("--pmc-compare-report", nargs=4, metavar="CSV",
                    help="per-flop counter comparison of --vendor-compare (two passes: counter, trace each)")
    ap.add_argument("--pmc-mfma-compare-report", nargs=2, metavar=("COUNTER_CSV", "TRACE_CSV"),
                    help="summarise a rocprofv3 MFMA-counter run of --vendor-compare and exit")
    ap.add_argument("--c1-trace-report", nargs=2, metavar=("STATS_CSV", "TRACE_CSV"))
    ap.add_argument("--c1-only", action="store_true",
                    help="the C1 step (reference MLP) replayed, both lowerings; the program of the C1 trace")
    ap.add_argument("--streaming-only", action="store_true",
                    help="run each streaming kernel at its benchmark shape (for rocprofv3 --pmc)")
    ap.add_argument("--pmc-streaming-report", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarise two rocprofv3 --pmc CSVs of --streaming-only and exit")
    args = ap.parse_args()
    if args.pmc_report:
        pmc_report(*args.pmc_report)
        return
    if args.pmc_mfma_compare_report:
        pmc_mfma_compare_report(*args.pmc_mfma_compare_report)
        return
    if args.pmc_compare_report:
        pmc_compare_report(*args.pmc_compare_report, shape_set=args.vendor_set)
        return
    if args.c1_trace_report:
        c1_trace_report(*args.c1_trace_report)
        return
    if args.stats_report:
        stats_report(args.stats_report[0], args.stats_report[1], int(args.stats_report[2]))
        return
    if args.pmc_streaming_report:
        pmc_streaming_report(*args.pmc_streaming_report)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); multi-GPU runs are not "
              f"part of this build", file=sys.stderr)
        sys.exit(2)

    import torch

    from aicf_cuda import _C as C

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    B, D, L = args.batch, args.hidden, args.layers
    log(f"[bench] device={torch.cuda.get_device_name(0)} mlp B={B} D={D} L={L}")
    if args.roofline_only:
        roofline_only(C, B, D, L, 5)
        return
    if args.streaming_only:
        streaming_only(C)
        return
    if args.c1_only:
        print(json.dumps(bench_c1(rounds=5, chunk=20, warm_s=0.05)))
        return
    if args.vendor_compare:
        vendor_compare(C, args.vendor_set)
        return

    res = bench_mlp(B, D, L, args.steps, args.warmup, **STEP_VARIANTS["headline"])
    log(f"[bench] mlp {res}")

    # dominant kernel: gemm_nt_kernel, the step's 12 GEMM launches (~88% of
    # the step), each 2*B*D*D flop; timed on the step's own tensors
    ex = build_step(B, D, L)
    times = step_gemm_times(ex, iters=10)
    del ex
    avg_ms = sum(t["ms"] for t in times) / len(times)
    flops = 2.0 * B * D * D
    achieved = flops / (avg_ms * 1e-3) / 1e12
    per_role = {}
    for t in times:
        per_role.setdefault(t["role"], []).append(t["ms"])
    traffic = read_traffic() if (B, D, L) == (8192, 4096, 4) else None
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "traffic": traffic, "traffic_unit": "bytes/launch (mean over the step's GEMM launches)",
                "kernel": f"gemm_nt_kernel: the step's {len(times)} GEMM launches "
                          "(bias+GELU+Z, bias, dX+dGELU, dX, dW+AdamW epilogues)",
                "shape": [B, D, D], "flops_per_launch": flops, "avg_ms": round(avg_ms, 4),
                "per_role_avg_ms": {k: round(sum(v) / len(v), 4) for k, v in per_role.items()},
                "measured": "HIP events (torch's current stream) around a captured graph of 10 launches of "
                            "each GEMM op of the step on the step's own tensors, after the timed replays"}
    log(f"[bench] roofline step gemms {times}")
    ceils = {f: bench_mfma_ceiling(form=f) for f in (16, 32)}
    ceil = max(ceils.values(), key=lambda c: c["tflops"])
    roofline["power_limited_mfma_ceiling"] = round(ceil["tflops"], 1)
    roofline["frac_of_ceiling"] = round(achieved / ceil["tflops"], 4)
    log(f"[bench] register-only MFMA loops {ceils}")

    comps = {"mfma_register_loop_bf16": {
        "value": round(ceil["tflops"], 1), "unit": "TFLOP/s", "frac": round(ceil["tflops"] / PEAK_BF16_TFLOPS, 4),
        "by_form": {f"{f}x{f}x{512 // f}": round(c["tflops"], 1) for f, c in ceils.items()},
        "note": "the faster of v_mfma_f32_16x16x32_bf16 (the GEMMs' instruction) and "
                "v_mfma_f32_32x32x16_bf16 on random register operands, no memory traffic: the "
                "power-limited MFMA ceiling of this part, measured in this run"}}
    if not args.no_components:
        gg = bench_gemm(C, 8192, 8192, 8192)
        comps["gemm_bf16_8192^3"] = {"value": round(gg["tflops"], 2), "unit": "TFLOP/s",
                                     "frac": round(gg["tflops"] / PEAK_BF16_TFLOPS, 4),
                                     "ms": round(gg["ms"], 4)}
        log(f"[bench] gemm 8192^3 {gg}")
        for cols in (128, 1024, 8192, 32768):
            sm = bench_softmax(C, 16384, cols)
            cs_ = bench_copy_sized(C, 16384 * cols * 4)
            comps[f"softmax_16384x{cols}"] = {"value": round(sm["gbs"], 1), "unit": "GB/s",
                                              "frac": round(sm["gbs"] / PEAK_HBM_GBS, 4),
                                              "ms": round(sm["ms"], 5),
                                              "buffer_sets": sm["buffer_sets"],
                                              "copy_same_bytes_gbs": round(cs_["gbs"], 1),
                                              "frac_of_copy_same_bytes": round(sm["gbs"] / cs_["gbs"], 4)}
            log(f"[bench] softmax {cols} {sm} copy of the same bytes {cs_}")
        for cols in (128, 1024, 8192, 32768):
            for name, op in (("rowmax", 1), ("rowsum", 0)):
                rr = bench_rowreduce(C, 16384, cols, op)
                comps[f"{name}_16384x{cols}"] = {"value": round(rr["gbs"], 1), "unit": "GB/s",
                                                 "frac": round(rr["gbs"] / PEAK_HBM_GBS, 4),
                                                 "ms": round(rr["ms"], 5), "buffer_sets": rr["buffer_sets"]}
                log(f"[bench] {name} {cols} {rr}")
        cp = bench_copy_ceiling(C)
        comps["hbm_copy_1GiB"] = {"value": round(cp["gbs"], 1), "unit": "GB/s",
                                  "frac": round(cp["gbs"] / PEAK_HBM_GBS, 4), "ms": round(cp["ms"], 4),
                                  "note": "plain read+write stream (copy_bf16_v0): the ceiling of the "
                                          "read-and-write kernels on this part, measured in this run"}
        log(f"[bench] copy ceiling {cp}")
        xe = bench_xent(C, 16384, 8192)
        comps["softmax_xent_fwd_bwd_16384x8192"] = {"value": round(xe["gbs"], 1), "unit": "GB/s",
                                                    "frac": round(xe["gbs"] / PEAK_HBM_GBS, 4),
                                                    "ms": round(xe["ms"], 5)}
        log(f"[bench] xent {xe}")
        ms_ = bench_mse(C, B, D)
        comps[f"mse_loss_grad_bf16_{B}x{D}"] = {"value": round(ms_["gbs"], 1), "unit": "GB/s",
                                                "frac": round(ms_["gbs"] / PEAK_HBM_GBS, 4),
                                                "ms": round(ms_["ms"], 5)}
        log(f"[bench] mse {ms_}")
        cs = bench_colsum(C, B, D)
        comps[f"colsum_bf16_f32_{B}x{D}"] = {"value": round(cs["gbs"], 1), "unit": "GB/s",
                                             "frac": round(cs["gbs"] / PEAK_HBM_GBS, 4),
                                             "ms": round(cs["ms"], 5)}
        log(f"[bench] colsum {cs}")
        cs1 = bench_colsum(C, B, D, partials=False)
        comps[f"colsum_bf16_f32_{B}x{D}_one_output"] = {"value": round(cs1["gbs"], 1), "unit": "GB/s",
                                                        "frac": round(cs1["gbs"] / PEAK_HBM_GBS, 4),
                                                        "ms": round(cs1["ms"], 5)}
        log(f"[bench] colsum one output {cs1}")
        ad = bench_adam(C)
        comps["adamw_2^28"] = {"value": round(ad["gbs"], 1), "unit": "GB/s",
                               "frac": round(ad["gbs"] / PEAK_HBM_GBS, 4), "ms": round(ad["ms"], 4)}
        log(f"[bench] adam {ad}")
        for (M_, N_, K_) in ((8192, 8192, 8192), (B, D, D)):
            tm = bench_torch_matmul(M_, N_, K_)
            comps[f"vendor_hipblaslt_bf16_{M_}x{N_}x{K_}"] = {
                "value": round(tm["tflops"], 2), "unit": "TFLOP/s",
                "frac": round(tm["tflops"] / PEAK_BF16_TFLOPS, 4), "ms": round(tm["ms"], 4),
                "note": "torch.matmul (hipBLASLt) in the same process, reference line only"}
            log(f"[bench] torch.matmul {M_}x{N_}x{K_} {tm}")
        alt = bench_mlp_alternated(B, D, L)
        notes = {
            "reference_op_split": "same step with the reference's op split: dW GEMMs write the fp32 gradient, one "
                                  "streaming AdamW over all parameters, bias gradients by separate column sums",
            "without_dead_input_dx": "same step with the first layer's input gradient (never consumed) removed; "
                                     "the headline keeps it, as the reference's lowering emits it",
            "without_tail_fusion": "the headline plan with the loss and bias tail unfused (mse_loss, reduce_sum, "
                                   "step_inc, column-sum finishes and the bias AdamW as separate launches); same "
                                   "parameters bit for bit",
        }
        for k, note in notes.items():
            comps[f"mlp_step_{k}"] = {
                "value": round(alt[k]["steps_per_s"], 3), "unit": "steps/s", "ms": round(alt[k]["ms"], 4),
                "ops": alt[k]["ops"], "gemms_per_step": alt[k]["gemms"],
                "headline_plan_in_the_same_loop_ms": round(alt["headline"]["ms"], 4), "note": note}
        comps["mlp_step_variants_alternated"] = {
            "value": round(alt["headline"]["steps_per_s"], 3), "unit": "steps/s",
            "ms": {k: round(v["ms"], 4) for k, v in alt.items()},
            "note": "the headline plan and each variant on graph handles of their own, warmed together, then "
                    "10 rounds of 10 replays each with the variants alternated (order reversed every other round)"}
        log(f"[bench] mlp variants alternated {alt}")
        c1v = bench_c1()
        c1 = dict(c1v["three_launch"], four_launch=c1v["four_launch"],
                  reference_lowering=c1v["reference_lowering"],
                  ten_steps_per_replay=c1v["three_launch_10_steps_per_replay"],
                  note="each lowering on a graph handle of its own, warmed together, then 10 rounds of 100 "
                       "steps with the lowerings alternated; value: one step per graph replay")
        comps["c1_mlp_fp32_64x784x256x10_step"] = c1
        log(f"[bench] c1 {c1}")
        for dt, shapes in (("bf16", C4_SHAPES), ("fp32", C4_SHAPES)):
            c4 = bench_c4(C, dt, shapes)
            comps.update(c4)
            log(f"[bench] c4 {dt} {c4}")
        lay = bench_layouts(C)
        comps.update(lay)
        log(f"[bench] layouts {lay}")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_mlp(B, D, L, args.cpu_rows)
        log(f"[bench] cpu {cpu}")
        if not args.no_components:
            # the oracle on the host beside each configuration's GPU line
            comps["c1_mlp_fp32_64x784x256x10_step"]["cpu_baseline"] = cpu_baseline_c1()
            for cols, v in cpu_baseline_c2().items():
                comps[f"softmax_16384x{cols}"]["cpu_baseline"] = v
            comps["adamw_2^28"]["cpu_baseline"] = cpu_baseline_c3()
            for (M_, N_, K_), v in cpu_baseline_c4().items():
                for key in [k for k in comps if k.startswith("c4_") and k.split("_")[2] == f"{M_}x{N_}x{K_}"]:
                    comps[key]["cpu_baseline"] = v
            log(f"[bench] cpu per config: c1 {comps['c1_mlp_fp32_64x784x256x10_step']['cpu_baseline']}, "
                f"c3 {comps['adamw_2^28']['cpu_baseline']}")

    out = {
        "metric": METRIC,
        "value": round(res["steps_per_s"], 3),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch generator: x,t ~ N(0,1); Kaiming-uniform weights)",
        "config": {"workload": "mlp_mse_bf16_train_step_hipgraph", "global_batch": B,
                   "hidden": D, "layers": L, "activation": "gelu_tanh", "loss": "mse",
                   "optimizer": "adamw(lr=1e-3, b=(0.9,0.999), eps=1e-8)",
                   "optimizer_in_dw_gemm_epilogue": True,
                   "bias_grads_in_dgelu_gemm_epilogue": True,
                   "gemms_per_step": res["gemms"], "ops_per_step": res["ops"],
                   "parallelism": "single_gpu"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "components": comps,
        "loss_first_last": res["losses"],
        "warm_ms": round(res["warm_ms"], 1),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
