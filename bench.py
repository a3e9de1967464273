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


def time_launches(fn, iters: int, warmup: int, stream=None) -> float:
    """Average milliseconds per call of fn(), HIP events on `stream`
    (torch's current stream by default)."""
    import torch

    s = stream or torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
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
            fn = lambda: C.launch_by_id(kid, C.OpKind.GemmEpilogue, [X, W, b], [Y], GEPI, pay)  # noqa: E731
            n = iters if flops < 1e12 else max(3, iters // 2)
            ms = time_launches(fn, n, 2)
            tf = flops / (ms * 1e-3) / 1e12
            peak = PEAK_BF16_TFLOPS if dtype == "bf16" else PEAK_FP32_TFLOPS
            out[f"c4_{dtype}_{M}x{N}x{K}_{act}"] = {"value": round(tf, 2), "unit": "TFLOP/s",
                                                    "frac": round(tf / peak, 4), "ms": round(ms, 4)}
    return out


# C1: the reference MLP (fp32, B=64, 784->256(ReLU)->10, softmax-xent, Adam)
def bench_c1(steps=200, warmup=5):
    """Replayed-graph time of one C1 train step."""
    import torch

    from aicf_cuda import _C
    from aicf_hip import mlp

    ir, lowered, plan = mlp.build_mlp_xent()
    data = mlp.init_mlp_xent()
    params = {k: torch.from_numpy(v.copy()).cuda() for k, v in data.items() if "." in k}
    inputs = {"x": torch.from_numpy(data["x"]).cuda(), "t": torch.from_numpy(data["t"]).cuda()}
    ex = mlp.make_executor(ir, lowered, plan)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    gs = torch.cuda.ExternalStream(int(_C.graph_stream()))
    ex.replay(warmup)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(gs)
    ex.replay(steps)
    e1.record(gs)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    loss = float(ex.value("loss").item())
    ex.reset_graph()
    return {"value": round(us, 2), "unit": "us/step", "steps_per_s": round(1e6 / us, 1),
            "ops_per_step": len(lowered), "loss_after": loss}


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
        C.op_call(int(C.OpKind.RowSoftmax), [x, ], [y, mx, sm], 0, b"", 0)

    ms = time_launches(fn, iters, warmup)
    nbytes = 8 * rows * cols + 8 * rows
    return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes, "buffer_sets": nsets}


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

    # step_inc is a 1-thread kernel (~2 us); it is part of the step
    ms = time_launches(fn, steps, 1)
    nbytes = 28 * n
    return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes_per_step": nbytes,
            "final_step": int(step.item())}


# ------------------------------------------------------------------ MLP
def bench_mlp(B, D, L, steps, warmup, dead_dx=True):
    import torch

    from aicf_hip import mlp

    ir, lowered, plan = mlp.build_mlp_mse(B, D, L, dead_dx=dead_dx)
    ex = mlp.make_executor(ir, lowered, plan)
    inputs, params = mlp.init_mlp_mse(B, D, L)
    ex.build_env(inputs=inputs, params=params, reuse_static=False)
    mlp.refresh_shadow(ex)
    ex.capture(inputs=inputs, params=params, reuse_static=True)
    gs = torch.cuda.ExternalStream(int(ex_stream()))
    losses = []
    for _ in range(warmup):
        ex.replay(1)
    torch.cuda.synchronize()
    losses.append(float(ex.value("loss").item()))
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
    ngemm = sum(1 for it in lowered if it["op"] in ("gemm", "gemm_epilogue"))
    ex.reset_graph()
    return {"ms": ms, "wall_ms": wall * 1e3 / steps, "steps_per_s": 1e3 / ms, "losses": losses,
            "finite": finite, "ops": len(lowered), "gemms": ngemm}


def ex_stream():
    from aicf_cuda import _C

    return _C.graph_stream()


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
    P = np.zeros(n, np.float32)
    G = np.full(n, 1e-3, np.float32)
    t1 = time.perf_counter()
    orc.adamw(P, G, P, P, 1, wd=0.01)
    t_adam = time.perf_counter() - t1
    per_step = t_batch * (B / b) + t_adam
    return {"value": 1.0 / per_step, "unit": "steps/s", "cores": orc.threads(), "kind": "port",
            "sample": f"{b} of {B} rows of one step (12 GEMMs with the reference's sequential-k "
                      f"fp32 algorithm + GELU/MSE/colsum) scaled by {B // b}, plus AdamW over all "
                      f"{n} parameters; measured {t_batch:.2f}s + {t_adam:.2f}s",
            "modelled_seconds_per_step": per_step}


# ------------------------------------------------------------------ main
# ------------------------------------------------------------------ HBM traffic (rocprofv3 --pmc)
TRAFFIC_FILE = REPO / "profiles" / "gemm_bias_gelu_8192x4096x4096_traffic.md"
CALIB_ELEMS = 1 << 27          # calibration copy: 2^27 bf16 = 256 MiB read + 256 MiB written
CALIB_KIB = CALIB_ELEMS * 2 / 1024


def roofline_only(C, B, D, launches):
    """The roofline kernel alone (launches x the step's bias+GELU GEMM with
    saved pre-activation), then 3 calibration copies of known size; the
    program profiled by the FETCH_SIZE / WRITE_SIZE passes."""
    import torch

    g = bench_gemm(C, B, D, D, act_kind=3, iters=launches, warmup=1, save_preact=True)
    x = torch.ones(CALIB_ELEMS, device="cuda", dtype=torch.bfloat16)
    y = torch.empty_like(x)
    for _ in range(3):
        C.launch_by_id("copy_bf16_v0", C.OpKind.Copy, [x], [y], 0, b"")
    torch.cuda.synchronize()
    log(f"[bench] roofline-only: {launches + 1} gemm launches, 3 calibration copies; {g}")


def pmc_report(fetch_csv, write_csv):
    """Markdown summary of two rocprofv3 --pmc runs of --roofline-only
    (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch).  Each counter is scaled
    by calibration copy's expected/measured ratio."""
    import csv
    from statistics import mean

    def per_kernel(path, counter):
        vals = {"gemm": [], "copy": []}
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                name = row.get("Kernel_Name", "")
                key = "gemm" if "gemm_nt" in name else "copy" if "map1" in name else None
                if key:
                    vals[key].append(float(row["Counter_Value"]))
        return vals

    fe, wr = per_kernel(fetch_csv, "FETCH_SIZE"), per_kernel(write_csv, "WRITE_SIZE")
    f_r = CALIB_KIB / mean(fe["copy"])
    f_w = CALIB_KIB / mean(wr["copy"])
    fetch_b = mean(fe["gemm"]) * f_r * 1024
    write_b = mean(wr["gemm"]) * f_w * 1024
    lines = [
        "# HBM traffic of the step's bias+GELU GEMM (8192x4096x4096, bf16, Z saved)",
        "",
        "Commands (GPU box, repo root):",
        "```",
        "rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/pmc_fetch -o run -- "
        "python3 bench.py --roofline-only",
        "rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/pmc_write -o run -- "
        "python3 bench.py --roofline-only",
        "python3 bench.py --pmc-report <fetch counter_collection.csv> <write counter_collection.csv>",
        "```",
        "",
        f"calibration copy (copy_bf16_v0, {CALIB_KIB:.0f} KiB read + written): "
        f"FETCH_SIZE {mean(fe['copy']):.0f} KiB -> factor {f_r:.4f}; "
        f"WRITE_SIZE {mean(wr['copy']):.0f} KiB -> factor {f_w:.4f}",
        f"gemm dispatches: {len(fe['gemm'])} (fetch run), {len(wr['gemm'])} (write run)",
        f"gemm FETCH_SIZE {mean(fe['gemm']):.0f} KiB/dispatch -> {fetch_b / 1e6:.1f} MB",
        f"gemm WRITE_SIZE {mean(wr['gemm']):.0f} KiB/dispatch -> {write_b / 1e6:.1f} MB",
        "algorithmic bytes: X 64 MiB + W 32 MiB read, Y 64 MiB + Z 64 MiB written = 224 MiB",
        "",
        f"traffic_bytes_per_launch: {int(round(fetch_b + write_b))}",
        "",
    ]
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
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=8192)
    ap.add_argument("--hidden", type=int, default=4096)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--no-components", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=8)
    ap.add_argument("--roofline-only", action="store_true",
                    help="run only the roofline GEMM and a calibration copy (for rocprofv3 --pmc)")
    ap.add_argument("--pmc-report", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarise two rocprofv3 --pmc CSVs of --roofline-only and exit")
    args = ap.parse_args()
    if args.pmc_report:
        pmc_report(*args.pmc_report)
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
        roofline_only(C, B, D, 5)
        return

    res = bench_mlp(B, D, L, args.steps, args.warmup)
    log(f"[bench] mlp {res}")

    # dominant kernel: forward GEMM of the step (bias + GELU epilogue)
    g = bench_gemm(C, B, D, D, act_kind=3, iters=20, warmup=3, save_preact=True)
    flops = 2.0 * B * D * D
    traffic = read_traffic() if (B, D) == (8192, 4096) else None
    roofline = {"bound": "mfma", "achieved": round(g["tflops"], 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(g["tflops"] / PEAK_BF16_TFLOPS, 4),
                "traffic": traffic, "traffic_unit": "bytes/launch",
                "kernel": "gemm_epilogue_bf16_mfma_v0 (bias+gelu, pre-activation saved)",
                "shape": [B, D, D], "flops_per_launch": flops, "avg_ms": round(g["ms"], 4)}
    log(f"[bench] roofline gemm {g}")

    comps = {}
    if not args.no_components:
        gg = bench_gemm(C, 8192, 8192, 8192)
        comps["gemm_bf16_8192^3"] = {"value": round(gg["tflops"], 2), "unit": "TFLOP/s",
                                     "frac": round(gg["tflops"] / PEAK_BF16_TFLOPS, 4),
                                     "ms": round(gg["ms"], 4)}
        log(f"[bench] gemm 8192^3 {gg}")
        for cols in (128, 1024, 8192, 32768):
            sm = bench_softmax(C, 16384, cols)
            comps[f"softmax_16384x{cols}"] = {"value": round(sm["gbs"], 1), "unit": "GB/s",
                                              "frac": round(sm["gbs"] / PEAK_HBM_GBS, 4),
                                              "ms": round(sm["ms"], 5),
                                              "buffer_sets": sm["buffer_sets"]}
            log(f"[bench] softmax {cols} {sm}")
        ad = bench_adam(C)
        comps["adamw_2^28"] = {"value": round(ad["gbs"], 1), "unit": "GB/s",
                               "frac": round(ad["gbs"] / PEAK_HBM_GBS, 4), "ms": round(ad["ms"], 4)}
        log(f"[bench] adam {ad}")
        c1 = bench_c1()
        comps["c1_mlp_fp32_64x784x256x10_step"] = c1
        log(f"[bench] c1 {c1}")
        for dt, shapes in (("bf16", C4_SHAPES), ("fp32", C4_SHAPES[:3])):
            c4 = bench_c4(C, dt, shapes)
            comps.update(c4)
            log(f"[bench] c4 {dt} {c4}")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_mlp(B, D, L, args.cpu_rows)
        log(f"[bench] cpu {cpu}")

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
                   "gemms_per_step": res["gemms"], "ops_per_step": res["ops"],
                   "parallelism": "single_gpu"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "components": comps,
        "loss_first_last": res["losses"],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
