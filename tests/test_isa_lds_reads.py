"""Static check of the device code: a register loaded by an inline-assembly LDS read (ds_read_*) is written when the
data returns, so no instruction may touch it before an s_waitcnt lgkmcnt that covers the read. The compiler waits for
its own loads, but not for these; a copy, spill or reuse of such a register before the wait reads or is overwritten
by stale data (a dead read whose register was reused for a store address has faulted the GPU).

Each HIP source is compiled for gfx950 to device assembly (same flags as kidi_amd/build.py) and every kernel is
scanned in order: LDS operations queue in issue order, lgkmcnt(N) retires all but the newest N."""

import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CSRC = os.path.join(ROOT, "kidi_amd", "csrc")
# sources that issue LDS reads or writes as inline assembly (the compiler tracks the others itself)
SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip") and
                 re.search(r"\bds_(read|write)", open(os.path.join(CSRC, f)).read()))
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S"]


def vgprs(text):
    out = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b", text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _scan(lines, state, in_asm, on_hazard, on_branch):
    """One pass over a block's instructions from pending-read state `state` (list of (line, instruction, registers) in
    issue order); returns the state at the end and whether control falls through to the next line."""
    for i, line in lines:
        if ";;#ASMSTART" in line:
            in_asm[0] = True
        if ";;#ASMEND" in line:
            in_asm[0] = False
        ins = line.split(";")[0].strip()
        if not ins or ins.startswith("."):
            continue
        op = ins.split()[0]
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", ins)
            if m:
                state = state[max(0, len(state) - int(m.group(1))):]
            continue
        args = ins[len(op):]
        used = vgprs(args)
        for _, read, dest in state:
            if dest & used:
                on_hazard(i, ins, read)
        if op.startswith(("ds_", "s_load", "s_buffer_load")):
            dest = vgprs(args.split(",")[0]) if in_asm[0] and op.startswith("ds_read") else set()
            state = state + [(i, ins, dest)]
        if op.startswith(("s_branch", "s_cbranch")):
            on_branch(args.strip().split()[0], state)
            if op == "s_branch":
                return state, False
    return state, True


def _merge(a, b):
    """Pending reads on either path, in issue order (entries of b missing from a appended)."""
    seen = {e[0] for e in a}
    return a + [e for e in b if e[0] not in seen]


def hazards(asm: str):
    """(kernel, line, instruction, pending read) for every touch of a register with an outstanding asm LDS read.

    Control flow is followed: each label's entry state is the merge of the states at every branch to it and, when the
    previous instruction falls through, of the state there; the scan repeats until no entry state changes (loops)."""
    found = []
    for func in re.split(r"\n(?=_Z\w+:)", asm):
        name = func.split(":", 1)[0]
        if not name.startswith("_Z") or ";;#ASMSTART" not in func:
            continue  # only inline-assembly LDS reads can be pending unseen
        lines = list(enumerate(func.split("s_endpgm")[0].split("\n")))
        # split into blocks at labels (the function's own label starts the first block)
        blocks, cur = [], ["", []]
        for i, line in lines[1:]:
            m = re.match(r"^(\.?[\w$.]+):", line)
            if m:
                blocks.append(cur)
                cur = [m.group(1), []]
            else:
                cur[1].append((i, line))
        blocks.append(cur)
        entry = {}
        hits = set()

        def on_branch(label, state):
            old = entry.get(label)
            new = state if old is None else _merge(old, state)
            if old is None or [e[0] for e in new] != [e[0] for e in old]:
                entry[label] = new
                changed[0] = True

        for _ in range(64):
            changed = [False]
            state, falls, in_asm = [], True, [False]
            for label, body in blocks:
                if label:
                    inc = entry.get(label)
                    state = (inc or []) if not falls else (state if inc is None else _merge(state, inc))
                    if falls:
                        on_branch(label, state)  # the fall-through is one more way in
                state, falls = _scan(body, state, in_asm, lambda i, ins, read: hits.add((i, ins, read)), on_branch)
            if not changed[0]:
                break
        found += [(name,) + h for h in sorted(hits)]
    return found


def test_checker_flags_a_read_reused_before_its_wait():
    asm = "\n".join([
        "_Zk:", ";;#ASMSTART", "ds_read_b128 v[4:7], v1 offset:0", ";;#ASMEND",
        "v_mov_b32_e32 v5, 0", "s_waitcnt lgkmcnt(0)", "v_mov_b32_e32 v6, 0", "s_endpgm"])
    assert [h[2] for h in hazards(asm)] == ["v_mov_b32_e32 v5, 0"]
    ordered = asm.replace("v_mov_b32_e32 v5, 0\n", "")
    assert hazards(ordered) == []


def test_checker_follows_branches():
    """A block entered only by a branch starts from the state at the branch (here: after the wait), not from the
    layout predecessor's; a read still pending on a back-edge is seen at the loop head."""
    rotated = "\n".join([
        "_Zk:", ";;#ASMSTART", "ds_read_b128 v[4:7], v1 offset:0", ";;#ASMEND", "s_branch .LBB0_2",
        ".LBB0_1:", "v_mov_b32_e32 v5, 0",
        ".LBB0_2:", "s_waitcnt lgkmcnt(0)", "v_add_u32_e32 v6, v4, v4", "s_cbranch_scc1 .LBB0_1", "s_endpgm"])
    assert hazards(rotated) == []
    pending_on_back_edge = "\n".join([
        "_Zk:", ".LBB0_1:", "v_mov_b32_e32 v5, 0", "s_waitcnt lgkmcnt(0)", ";;#ASMSTART", "ds_read_b128 v[4:7], v1 offset:0",
        ";;#ASMEND", "s_cbranch_scc1 .LBB0_1", "s_endpgm"])
    assert [h[2] for h in hazards(pending_on_back_edge)] == ["v_mov_b32_e32 v5, 0"]


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_no_register_of_a_pending_lds_read_is_touched():
    assert "kq_gemm.hip" in SOURCES, SOURCES  # the prefill GEMM's ring reads and writes are inline assembly
    with tempfile.TemporaryDirectory() as tmp:
        procs = []
        for src in SOURCES:
            out = os.path.join(tmp, src + ".s")
            cmd = [HIPCC, *FLAGS, "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "kidi_amd", "csrc", src), "-o", out]
            procs.append((src, out, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        bad = []
        for src, out, p in procs:
            log, _ = p.communicate()
            assert p.returncode == 0, log.decode(errors="replace")[-2000:]
            with open(out) as f:
                bad += [(src,) + h for h in hazards(f.read())]
    assert not bad, "\n".join(f"{s} {k[:70]} line {i}: {ins!r} before the wait for {r!r}" for s, k, i, ins, r in bad[:10])
