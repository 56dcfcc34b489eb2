"""The row-tile kernels issue their weight and scale loads as plain instructions outside the compiler's wait
accounting and wait for them with counted vmcnt waits (unholy_amd/csrc/pipe.hpp vload16 / vlanded). That is only
safe while the compiled code neither reads nor overwrites a destination register of such a load before a wait has
retired it. This test compiles the kernels to gfx950 assembly and replays each kernel's instruction stream in layout
order against an in-order model of the vector-memory counter: loads retire oldest first, `s_waitcnt vmcnt(N)` leaves
the newest N outstanding. Any instruction that reads or writes a register still owned by an outstanding load fails."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _regs(spec):
    m = re.match(r"v\[(\d+):(\d+)\]", spec)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", spec)
    return {int(m.group(1))} if m else set()


def hazards(asm_lines):
    """Instructions touching a register whose load is still outstanding (straight-line, layout order)."""
    queue, bad = [], []
    for i, line in enumerate(asm_lines):
        t = line.strip()
        if not t or t.startswith((";", ".")):
            continue
        op = t.split()[0]
        if op == "s_waitcnt" and "vmcnt" in t:
            n = int(re.search(r"vmcnt\((\d+)\)", t).group(1))
            del queue[: max(0, len(queue) - n)]
            continue
        ops = re.findall(r"v\[\d+:\d+\]|v\d+\b", t)
        pending = set().union(*queue) if queue else set()
        if op.startswith(("global_load", "buffer_load", "scratch_load")):
            srcs = set().union(*(_regs(o) for o in ops[1:])) if len(ops) > 1 else set()
            if srcs & pending:
                bad.append((i, t))
            queue.append(set() if "lds" in op else _regs(ops[0]))
            continue
        store = op.startswith(("ds_write", "global_store", "buffer_store", "scratch_store", "global_atomic"))
        srcs = set().union(*(_regs(o) for o in (ops if store else ops[1:]))) if ops else set()
        dst = set() if store or not ops else _regs(ops[0])
        if (srcs | dst) & pending:
            bad.append((i, t))
        if op.startswith(("global_store", "buffer_store", "scratch_store", "global_atomic")):
            queue.append(set())
    return bad


def _kernel_asm(src, name_re, tmp_path):
    out = tmp_path / (os.path.basename(src) + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++20", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "unholy_amd", "csrc"),
           "--cuda-device-only", "-S", os.path.join(ROOT, "unholy_amd", "csrc", src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    lines = out.read_text().splitlines()
    kernels = {}
    for i, line in enumerate(lines):
        m = re.match(r"^(_Z\S*" + name_re + r"\S*):", line)
        if m:
            end = next(j for j in range(i, len(lines)) if lines[j].strip().startswith("s_endpgm"))
            kernels[m.group(1)] = lines[i:end + 1]
    return kernels


def test_hazard_model_catches_an_early_read():
    asm = ["global_load_dwordx4 v[4:7], v[0:1], off", "global_load_dword v8, v[2:3], off", "s_waitcnt vmcnt(1)",
           "v_add_f32 v9, v4, v5", "v_mov_b32 v10, v8"]
    assert hazards(asm) == [(4, "v_mov_b32 v10, v8")]
    assert hazards(asm[:4]) == []


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src,name,count", [("fp8_gemm.hip", "fp8_rows_kernel", 2),
                                            ("grouped_fp8w.hip", "grouped_fp8w_rows_kernel", 2)])
def test_counted_loads_have_no_early_use(src, name, count, tmp_path):
    kernels = _kernel_asm(src, name, tmp_path)
    assert len(kernels) == count, list(kernels)
    for k, lines in kernels.items():
        assert any("global_load_dwordx4" in l for l in lines), k
        assert hazards(lines) == [], k
