"""The row-tile kernels issue their weight and scale loads as plain instructions outside the compiler's wait
accounting and wait for them with counted vmcnt waits (unholy_amd/csrc/pipe.hpp vload16 / vlanded). That is only
safe while the compiled code neither reads nor overwrites a destination register of such a load before a wait has
retired it, on every path the code can take.

(fp8_tiled_kernel's next-stage activation scale is one such load, issued ahead of the stage's ring loads.) This test
compiles the kernels to gfx950 assembly, splits each kernel into basic blocks (labels, branches,
s_endpgm) and follows every path through them, loop back-edges included, against an in-order model of the
vector-memory counter: loads (and stores) retire oldest first, `s_waitcnt vmcnt(N)` leaves the newest N
outstanding. The set of queue states reaching each block is grown until it stops changing, so a path that waits
less (a vmcnt(16) branch beside a vmcnt(0) one) or comes round a loop with loads still in flight is seen. Any
instruction that reads or writes a register still owned by an outstanding load on some path fails the test. The
path set is exact for the kernels' own control flow: their chunk count is a template parameter, so no branch
selects a different wait."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

BRANCH = re.compile(r"s_(branch|cbranch_\w+)\s+(\S+)")
LOADS = ("global_load", "buffer_load", "scratch_load", "flat_load")
STORES = ("global_store", "buffer_store", "scratch_store", "flat_store", "global_atomic", "buffer_atomic",
          "flat_atomic")
QMAX = 64  # the counter's range: at most 63 outstanding, a longer queue keeps its newest entries


def _regs(spec):
    m = re.match(r"v\[(\d+):(\d+)\]", spec)
    if m:
        return frozenset(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", spec)
    return frozenset({int(m.group(1))}) if m else frozenset()


def _step(t, queue):
    """One instruction against the queue of outstanding loads (oldest first): (queue after it, touches a pending
    register)."""
    op = t.split()[0]
    if op == "s_waitcnt":
        m = re.search(r"vmcnt\((\d+)\)", t)
        if m:
            queue = queue[max(0, len(queue) - int(m.group(1))):]
        elif t.split()[1:2] == ["0"]:
            queue = ()
        return queue, False
    ops = re.findall(r"v\[\d+:\d+\]|v\d+\b", t)
    pending = frozenset().union(*queue) if queue else frozenset()
    if op.startswith(LOADS):
        srcs = frozenset().union(*(_regs(o) for o in ops[1:])) if len(ops) > 1 else frozenset()
        dst = frozenset() if "lds" in op else _regs(ops[0])
        return (queue + (dst,))[-QMAX:], bool((srcs | dst) & pending)
    store = op.startswith(STORES) or op.startswith("ds_write")
    srcs = frozenset().union(*(_regs(o) for o in (ops if store else ops[1:]))) if ops else frozenset()
    dst = frozenset() if store or not ops else _regs(ops[0])
    bad = bool((srcs | dst) & pending)
    if op.startswith(STORES):
        queue = (queue + (frozenset(),))[-QMAX:]
    return queue, bad


def hazards(asm_lines, max_states=200000):
    """(line, instruction) pairs that touch a register whose load may still be outstanding on some path."""
    insts, labels = [], {}
    for i, line in enumerate(asm_lines):
        t = line.split(";")[0].strip()
        if not t:
            continue
        m = re.match(r"^([.\w$]+):", t)
        if m:
            labels[m.group(1)] = len(insts)
            continue
        if t.startswith("."):
            continue
        insts.append((i, t))
    if not insts:
        return []
    enders = ("s_branch", "s_cbranch", "s_endpgm", "s_setpc")
    starts = sorted({0, *labels.values()} | {k + 1 for k, (_, t) in enumerate(insts) if t.startswith(enders)})
    starts = [s for s in starts if s < len(insts)]
    block_of = {s: b for b, s in enumerate(starts)}
    ends = starts[1:] + [len(insts)]
    succ = []
    for s, e in zip(starts, ends):
        last = insts[e - 1][1]
        nxt = [block_of[e]] if e in block_of else []
        m = BRANCH.match(last)
        if last.startswith("s_endpgm"):
            succ.append([])
        elif m:
            if m.group(2) not in labels:
                raise ValueError(f"branch to a label outside the kernel: {last}")
            tgt = block_of[labels[m.group(2)]]
            succ.append([tgt] if m.group(1) == "branch" else [tgt] + nxt)
        elif last.startswith("s_setpc"):
            raise ValueError(f"indirect branch: {last}")
        else:
            succ.append(nxt)
    seen = [set() for _ in starts]
    work, bad, states = [(0, ())], set(), 0
    while work:
        b, q = work.pop()
        if q in seen[b]:
            continue
        seen[b].add(q)
        states += 1
        if states > max_states:
            raise RuntimeError("too many queue states to follow")
        for k in range(starts[b], ends[b]):
            q, hit = _step(insts[k][1], q)
            if hit:
                bad.add(insts[k])
        work.extend((s, q) for s in succ[b] if q not in seen[s])
    return sorted(bad)


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
            end = next(j for j in range(i, len(lines)) if lines[j].startswith(".Lfunc_end"))
            kernels[m.group(1)] = lines[i:end]
    return kernels


def test_hazard_model_catches_an_early_read():
    asm = ["global_load_dwordx4 v[4:7], v[0:1], off", "global_load_dword v8, v[2:3], off", "s_waitcnt vmcnt(1)",
           "v_add_f32 v9, v4, v5", "v_mov_b32 v10, v8"]
    assert hazards(asm) == [(4, "v_mov_b32 v10, v8")]
    assert hazards(asm[:4]) == []


def test_hazard_model_follows_a_branch_chain_of_waits():
    # A switch over two counted waits: the vmcnt(0) case comes first in layout order, the vmcnt(1) case is the one
    # that leaves v8 pending. A layout-order replay would clear the queue at vmcnt(0) and see nothing.
    asm = ["global_load_dwordx4 v[4:7], v[0:1], off", "global_load_dword v8, v[2:3], off", "s_cmp_eq_u32 s0, 1",
           "s_cbranch_scc1 .LBB0_2", "s_waitcnt vmcnt(0)", "s_branch .LBB0_3", ".LBB0_2:", "s_waitcnt vmcnt(1)",
           ".LBB0_3:", "v_add_f32 v9, v4, v5", "v_mov_b32 v10, v8", "s_endpgm"]
    assert hazards(asm) == [(10, "v_mov_b32 v10, v8")]
    safe = list(asm)
    safe[7] = "s_waitcnt vmcnt(0)"
    assert hazards(safe) == []


def test_hazard_model_follows_a_loop_back_edge():
    # The load at the bottom of the loop is still in flight when the next iteration reads its register.
    asm = [".LBB0_1:", "v_add_f32 v9, v4, v5", "global_load_dwordx4 v[4:7], v[0:1], off", "s_cmp_lg_u32 s0, 0",
           "s_cbranch_scc1 .LBB0_1", "s_waitcnt vmcnt(0)", "s_endpgm"]
    # (the second iteration's load also overwrites the register of the one still in flight)
    assert hazards(asm) == [(1, "v_add_f32 v9, v4, v5"), (2, "global_load_dwordx4 v[4:7], v[0:1], off")]
    fixed = asm[:1] + ["s_waitcnt vmcnt(0)"] + asm[1:]
    assert hazards(fixed) == []


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src,name,count,load", [("fp8_gemm.hip", "fp8_rows_kernel", 8, "global_load_dwordx4"),
                                                 ("grouped_fp8w.hip", "grouped_fp8w_rows_kernel", 8, "global_load_dwordx4"),
                                                 ("fp8_tiled.hip", "fp8_tiled_kernel", 4, "global_load_dword ")])
def test_counted_loads_have_no_early_use(src, name, count, load, tmp_path):
    kernels = _kernel_asm(src, name, tmp_path)
    assert len(kernels) == count, list(kernels)
    for k, lines in kernels.items():
        assert any(load in l for l in lines) or "ILb0E" in k, k  # fp8_tiled_kernel<false>: no counted load
        assert any(BRANCH.match(l.strip()) for l in lines), k  # the model really walks branches here
        assert hazards(lines) == [], k
