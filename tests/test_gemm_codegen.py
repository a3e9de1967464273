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


# The M/N-contiguous operand loads are inline asm (`buffer_load_dwordx4 v,
# s[..], s offen lds`), hidden from the compiler's hazard tracking: nothing
# stops it from reusing the lane-offset VGPR of such a load while the load
# is still in flight.  Every one of them must keep that VGPR unwritten until
# a `s_waitcnt vmcnt(0)`, on the fall-through path and, past a backward
# branch, from the loop header on.
_DST_OPS = re.compile(r"^(v_|ds_read|ds_load|buffer_load|global_load|flat_load|scratch_load)")
_REG = re.compile(r"^v(\d+)$|^v\[(\d+):(\d+)\]$")


def _vgprs(operand: str) -> set[int]:
    m = _REG.match(operand.strip())
    if not m:
        return set()
    if m.group(1) is not None:
        return {int(m.group(1))}
    return set(range(int(m.group(2)), int(m.group(3)) + 1))


def _instr(line: str):
    s = line.split(";")[0].strip()
    if not s or s.startswith(".") or s.endswith(":"):
        return None, []
    parts = s.split(None, 1)
    ops = [o.strip() for o in parts[1].split(",")] if len(parts) > 1 else []
    return parts[0], ops


def _written_vgprs(line: str) -> set[int]:
    mnem, ops = _instr(line)
    if not mnem or not ops or not _DST_OPS.match(mnem):
        return set()
    if mnem.startswith(("v_cmp", "v_readlane", "v_readfirstlane")):
        return set()
    if re.search(r"\blds\b", line.split(";")[0]) and "_load" in mnem:
        return set()  # a direct-to-LDS load writes LDS; its first VGPR is the lane offset it reads
    return _vgprs(ops[0])


def _is_vm_drain(line: str) -> bool:
    s = line.split(";")[0]
    return "s_waitcnt" in s and ("vmcnt(0)" in s or re.search(r"s_waitcnt\s+0\b", s) is not None)


def asm_lds_loads(body: list[str]) -> list[tuple[int, int]]:
    """(line index after the asm block, voffset VGPR) of each inline-asm
    direct-to-LDS buffer load."""
    out = []
    in_asm = False
    pending = []
    for i, ln in enumerate(body):
        if "ASMSTART" in ln:
            in_asm, pending = True, []
            continue
        if "ASMEND" in ln:
            out += [(i + 1, r) for r in pending]
            in_asm = False
            continue
        m = re.search(r"buffer_load_dwordx4\s+v(\d+),\s*s\[\d+:\d+\],\s*s\d+\s+offen\s+lds", ln)
        if in_asm and m:
            pending.append(int(m.group(1)))
    return out


def _first_write_before_drain(body, start, reg, labels):
    seen = set()
    todo = [start]
    while todo:
        i = todo.pop()
        while i < len(body):
            if i in seen:
                break
            seen.add(i)
            ln = body[i]
            if _is_vm_drain(ln):
                break
            if reg in _written_vgprs(ln):
                return i
            m = re.search(r"s_(?:cbranch_\w+|branch)\s+(\.LBB\w+)", ln.split(";")[0])
            if m and m.group(1) in labels and labels[m.group(1)] < i:
                todo.append(labels[m.group(1)] + 1)
                if "s_branch" in ln:
                    break
            i += 1
    return None


def test_asm_lds_loads_keep_their_offset_vgpr_until_drained(asm):
    names = re.findall(r"^(_Z\S*gemm_nt_kernel\S*):", asm, re.M)
    assert names
    checked = 0
    for name in names:
        body = kernel_body(asm, name[name.index("gemm_nt_kernel"):])
        labels = {ln.split(":")[0]: i for i, ln in enumerate(body) if ln.startswith(".LBB")}
        for start, reg in asm_lds_loads(body):
            hit = _first_write_before_drain(body, start, reg, labels)
            assert hit is None, f"{name}: v{reg} of the asm load before line {start} is written at " \
                                f"'{body[hit].strip()}' before a vmcnt(0) wait"
            checked += 1
    assert checked > 100, checked


def test_asm_offset_guard_flags_a_planted_write(asm):
    """The guard itself: a write of the offset VGPR planted (in the text)
    right after one asm load, or behind the loop's backward branch, is
    reported."""
    name = re.findall(r"^(_Z\S*gemm_nt_kernel\S*ELb0ELb0E\S*):", asm, re.M)[0]
    body = kernel_body(asm, name[name.index("gemm_nt_kernel"):])
    labels = {ln.split(":")[0]: i for i, ln in enumerate(body) if ln.startswith(".LBB")}
    start, reg = asm_lds_loads(body)[0]
    assert _first_write_before_drain(body, start, reg, labels) is None
    planted = body[:start] + [f"\tv_mov_b32_e32 v{reg}, 0"] + body[start:]
    labels2 = {ln.split(":")[0]: i for i, ln in enumerate(planted) if ln.startswith(".LBB")}
    assert _first_write_before_drain(planted, start, reg, labels2) == start
    assert _written_vgprs("\tds_read_b128 v[4:7], v1 offset:16") == {4, 5, 6, 7}
    assert _written_vgprs("\tbuffer_load_dwordx4 v3, s[0:3], s16 offen lds") == set()
    assert _written_vgprs("\tbuffer_load_dwordx4 v[4:7], v3, s[0:3], 0 offen") == {4, 5, 6, 7}
    assert _written_vgprs("\tds_write_b128 v1, v[4:7]") == set()
    assert _is_vm_drain("\ts_waitcnt vmcnt(0) lgkmcnt(0)") and not _is_vm_drain("\ts_waitcnt vmcnt(3)")


def test_no_nt_kernel_uses_scratch(asm):
    """Every gemm_nt_kernel instantiation (4- and 8-wave, every epilogue and
    operand layout) keeps its registers within the file: no private segment
    (spill) bytes in its kernel descriptor."""
    found = 0
    for m in re.finditer(r"\.amdhsa_kernel (\S+)\n(.*?)\.end_amdhsa_kernel", asm, re.S):
        if "gemm_nt_kernel" not in m.group(1):
            continue
        found += 1
        seg = re.search(r"\.amdhsa_private_segment_fixed_size\s+(\d+)", m.group(2))
        assert seg and int(seg.group(1)) == 0, (m.group(1), seg.group(1) if seg else None)
    assert found > 100, found


# Small-tile kernels with deeper pipelines (S LDS stages): the loop that
# issues loads waits once per K-step with vmcnt((S - 2) x loads per K-step),
# so S - 2 K-steps of loads stay in flight across the barrier, and no
# vmcnt(0) (from __syncthreads' fence or a compiler-inserted wait) drains them.
DEEP = [("gemm_nt_kernelILi2ELi2ELi0ELi64ELi64ELi2ELi2ELb1ELb1ELi8E", 24),   # 64x64, 8 stages, 4 loads
        ("gemm_nt_kernelILi2ELi2ELi3ELi64ELi64ELi2ELi2ELb1ELb1ELi8E", 24),   # with the GELU epilogue
        ("gemm_nt_kernelILi2ELi2ELi0ELi128ELi128ELi2ELi2ELb1ELb1ELi4E", 16)]  # 128x128, 4 stages, 8 loads


def loops(lines: list[str]) -> list[list[str]]:
    out = []
    for i, ln in enumerate(lines):
        if "Loop Header" not in ln:
            continue
        j = i
        while j >= 0 and not lines[j].startswith(".LBB"):
            j -= 1
        label = lines[j].split(":")[0]
        for k in range(j + 1, len(lines)):
            if re.search(r"s_cbranch_\w+\s+" + re.escape(label) + r"\b", lines[k]):
                out.append(lines[j:k + 1])
                break
    return out


@pytest.mark.parametrize("kernel,vm", DEEP)
def test_deep_pipeline_keeps_loads_in_flight(asm, kernel, vm):
    body = kernel_body(asm, kernel)
    main = [lp for lp in loops(body) if any("v_mfma" in l for l in lp)
            and any(re.search(r"(buffer|global)_load\w*.*\blds\b", l) for l in lp)]
    assert len(main) == 1, len(main)
    waits = [l.strip() for l in main[0] if "s_waitcnt" in l and "vmcnt" in l]
    assert waits == [f"s_waitcnt vmcnt({vm}) lgkmcnt(0)"], waits
    assert sum("s_barrier" in l for l in main[0]) == 1


# The inline-asm LDS loads also hide their scalar operands (buffer resource,
# scalar offset) from the hazard recognizer: a vector-memory read of an SGPR
# written by a VALU instruction (v_readfirstlane, v_readlane, a v_cmp into an
# SGPR pair) needs 5 wait states in between, which the compiler does not count
# for an asm block.  Every such load must have 5 wait states (its own s_nop
# included) after the last VALU write of an SGPR it reads.
VMEM_SGPR_WAIT_STATES = 5


def _sgprs(tok: str) -> set[int]:
    m = re.match(r"^s\[(\d+):(\d+)\]$", tok.strip())
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"^s(\d+)$", tok.strip())
    return {int(m.group(1))} if m else set()


def asm_load_sgpr_hazards(lines: list[str], need: int = VMEM_SGPR_WAIT_STATES) -> list[tuple[int, str, str]]:
    """(line, VALU instruction, asm load) for each asm direct-to-LDS load with
    fewer than `need` wait states after a VALU write of an SGPR it reads,
    looking back along the fall-through path.  A label reached before `need`
    wait states is reported too (other paths lead there), as ("label", load)."""
    out = []
    for i, ln in enumerate(lines):
        if "ASMSTART" not in ln:
            continue
        j, block = i + 1, []
        while j < len(lines) and "ASMEND" not in lines[j]:
            block.append(lines[j].split(";")[0].strip())
            j += 1
        load = [b for b in block if b.startswith("buffer_load") and re.search(r"\blds\b", b)]
        if not load:
            continue
        ops = [o.strip() for o in load[0].split(None, 1)[1].replace(" offen lds", "").split(",")]
        used = set().union(*(_sgprs(o) for o in ops[1:]))
        ws = 0
        for b in block:
            if b.startswith("buffer_load"):
                break
            ws += int(b.split()[1]) + 1 if b.startswith("s_nop") else (1 if b else 0)
        k = i - 1
        while ws < need and k >= 0:
            s = lines[k].split(";")[0].strip()
            k -= 1
            if not s or s.startswith("."):
                continue
            if s.endswith(":"):
                out.append((i, "label " + s, load[0]))
                break
            mnem = s.split()[0]
            if mnem.startswith("s_nop"):
                ws += int(s.split()[1]) + 1
                continue
            if mnem.startswith("v_") and len(s.split(None, 1)) > 1:
                if _sgprs(s.split(None, 1)[1].split(",")[0]) & used:
                    out.append((i, s, load[0]))
            ws += 1
    return out


def test_asm_lds_loads_wait_for_valu_written_sgprs(asm):
    lines = asm.splitlines()
    hazards = asm_load_sgpr_hazards(lines)
    assert not hazards, hazards[:4]
    n = sum(1 for ln in lines if re.search(r"buffer_load_dwordx4\s+v\d+,\s*s\[\d+:\d+\],\s*s\d+\s+offen\s+lds", ln))
    assert n > 100, n


def test_asm_sgpr_hazard_check_flags_a_planted_write():
    lines = ["\tv_readfirstlane_b32 s5, v3", "\t;;#ASMSTART", "\ts_nop 0",
             "\tbuffer_load_dwordx4 v182, s[4:7], s42 offen lds", "\t;;#ASMEND"]
    assert len(asm_load_sgpr_hazards(lines)) == 1
    lines[2] = "\ts_nop 4"
    assert asm_load_sgpr_hazards(lines) == []
    far = ["\tv_readfirstlane_b32 s42, v3", "\ts_add_i32 s1, s1, 1", "\ts_add_i32 s2, s2, 1",
           "\t;;#ASMSTART", "\ts_nop 1", "\tbuffer_load_dwordx4 v182, s[4:7], s42 offen lds", "\t;;#ASMEND"]
    assert len(asm_load_sgpr_hazards(far)) == 1  # 2 + 2 wait states < 5


def _stores(body: list[str]) -> tuple[int, int]:
    """(nontemporal, plain) 16-byte global stores of a kernel body."""
    st = [ln.split(";")[0].strip() for ln in body if ln.strip().startswith("global_store_dwordx4")]
    nt = sum(1 for s in st if re.search(r"\bnt\b", s))
    return nt, len(st) - nt


def test_epilogue_store_policy(asm):
    """Output stores carry the nontemporal hint on the tiles whose workgroups
    reach their epilogues at different times (here the 4-wave 256 x 256
    tiles), so the output does not evict operand lines other workgroups
    still stream through L2, and stay plain on the persistent 8-wave tiles,
    whose output the train step's next GEMM reads from the cache.  Both ways
    give the same bits; only the time changes (8192 x 4096 x 11008: 517 ->
    480 us; the step 1.2% slower with nontemporal stores everywhere)."""
    nt, plain = _stores(kernel_body(asm, KERNELS[0]))  # 4-wave, bias-free plain GEMM
    assert nt > 0 and plain == 0, (nt, plain)
    for k in KERNELS[1:4]:  # 8-wave persistent: GELU+Z, dGELU, fp32-out dW
        nt, plain = _stores(kernel_body(asm, k))
        assert nt == 0 and plain > 0, (k, nt, plain)
