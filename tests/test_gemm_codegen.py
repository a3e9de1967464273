"""Code-generation guard for the GEMM kernel's main loop (CPU only: hipcc
cross-compiles gfx950 assembly here).

The K loop must wait for its direct-to-LDS loads once per K-step (at the
barrier) and never in front of a fragment read: a compiler-inserted
`s_waitcnt vmcnt(0)` there exposes the full global-load latency every
sub-step and halves the kernel's rate, while every result stays bit-exact,
so no parity test notices.  Two ways this has happened: the compiler cannot
separate transposing LDS reads from in-flight LDS-DMA writes, and a second
LDS object written by LDS-DMA makes it give up on the first one."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
SRC = REPO / "ai-compiler-framework_amd" / "csrc" / "kernels" / "gemm.hip"

# bf16 in; OUT 2 bf16 / 0 fp32; ACT 0 none, 2 GELU, 3 dGELU, 4 AdamW; waves; AKC, BKC
KERNELS = [
    "gemm_nt_kernelILi2ELi2ELi0ELi256ELi256ELi2ELi2ELb1ELb1E",  # 4-wave, K-contiguous (8192^3)
    "gemm_nt_kernelILi2ELi2ELi2ELi256ELi256ELi2ELi4ELb1ELb1E",  # forward bias+GELU(+Z)
    "gemm_nt_kernelILi2ELi2ELi3ELi256ELi256ELi2ELi4ELb1ELb0E",  # dX dGELU, W read in place
    "gemm_nt_kernelILi2ELi0ELi0ELi256ELi256ELi2ELi4ELb0ELb0E",  # dW, both M/N-contiguous, fp32 out
    "gemm_nt_kernelILi2ELi0ELi4ELi256ELi256ELi2ELi4ELb0ELb0E",  # dW with the AdamW epilogue
]


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("gemm_asm") / "gemm.s"
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", f"-I{REPO / 'include'}", "--cuda-device-only", "-S", str(SRC), "-o", str(out)]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-4000:]
    return out.read_text()


def kernel_body(asm: str, mangled_part: str) -> list[str]:
    m = re.search(r"^(_ZN\S*" + re.escape(mangled_part) + r"\S*):", asm, re.M)
    assert m, f"kernel {mangled_part} not found"
    start = m.end()
    end = asm.index("s_endpgm", start)
    return asm[start:end].splitlines()


def k_loop(lines: list[str]) -> list[str]:
    """The innermost loop: from its header label to the backward branch to it.
    The assembler annotates a loop header as `; =>This Loop Header: Depth=d`
    or `; =>  This Inner Loop Header: Depth=d`, on the label's line or on the
    line after it."""
    depth_of = {}
    for i, ln in enumerate(lines):
        m = re.search(r"Loop Header: Depth=(\d+)", ln)
        if m:
            j = i
            while j >= 0 and not lines[j].startswith(".LBB"):
                j -= 1
            depth_of[j] = int(m.group(1))
    assert depth_of, "no loop in the kernel"
    i = max(depth_of, key=lambda k: (depth_of[k], -k))
    label = lines[i].split(":")[0]
    for j in range(i + 1, len(lines)):
        if re.search(r"s_cbranch_\w+\s+" + re.escape(label) + r"\b", lines[j]):
            return lines[i:j + 1]
    raise AssertionError(f"no backward branch to {label}")


@pytest.mark.parametrize("kernel", KERNELS)
def test_k_loop_waits_for_its_loads_once_per_k_step(asm, kernel):
    loop = k_loop(kernel_body(asm, kernel))
    waits = [l.strip() for l in loop if "s_waitcnt" in l and "vmcnt" in l]
    assert len(waits) == 1, waits
    assert any("s_barrier" in l for l in loop)
    loads = [l for l in loop if re.search(r"(buffer|global)_load\w*.*\blds\b", l)]
    assert loads, "the K loop issues the next stage's direct-to-LDS loads"


# The 8-wave kernels: no scratch (spill) traffic at all.  A spilled value
# reloaded in the epilogue comes with an `s_waitcnt vmcnt(0)` that also
# waits for the epilogue's own loads and stores, one at a time (the dGELU
# pre-activation load ran 16 round trips in series that way, +26 us per
# 8192x4096x4096 GEMM).
@pytest.mark.parametrize("kernel", [k for k in KERNELS if "ELi2ELi4E" in k])
def test_eight_wave_kernels_do_not_spill(asm, kernel):
    body = kernel_body(asm, kernel)
    spills = [l.strip() for l in body if "scratch_" in l]
    assert not spills, spills[:4]
