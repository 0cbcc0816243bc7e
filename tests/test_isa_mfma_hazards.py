"""Static check of the device code: an MFMA result may not be read by a VALU instruction until enough wait states have
passed, and an MFMA may not read a register that a VALU instruction wrote until enough wait states have passed.
The compiler inserts those wait states for the MFMA builtins, but its hazard recognizer does not look into inline
assembly, and the prefill GEMMs issue their MFMAs and epilogues as inline assembly (to pin their order). The
required distances are measured here, not assumed: probe kernels built from the builtins are compiled and the s_nop
the compiler puts between each MFMA and a dependent VALU read (and between a VALU write and an MFMA reading it) is
taken as the requirement. Every inline-assembly MFMA of the prefill kernels must then be followed by at least that
many wait states (instructions, s_nop n counting n + 1) before the first VALU instruction that reads one of its
destination registers, and preceded by at least that many after the last VALU write of one of its sources."""

import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = ["kq_gemm.hip", "kq_gemm_g.hip", "kq_gemm8.hip"]
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S"]
MFMAS = ("v_mfma_i32_16x16x32_i8", "v_mfma_i32_16x16x64_i8", "v_mfma_f32_4x4x1_16b_f32", "v_mfma_i32_32x32x32_i8")

PROBE = r"""
#include <hip/hip_runtime.h>
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
__global__ void p32(const long* a, const long* b, float* o) {
    v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[threadIdx.x], b[threadIdx.x], v4i{0, 0, 0, 0}, 0, 0, 0);
    o[threadIdx.x] = (float)c[0];
}
__global__ void p64(const v4i* a, const v4i* b, float* o) {
    v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[threadIdx.x], b[threadIdx.x], v4i{0, 0, 0, 0}, 0, 0, 0);
    o[threadIdx.x] = (float)c[0];
}
__global__ void pw(const v4i* a, const v4i* b, v4i* o) {
    v4i A = a[threadIdx.x], B = b[threadIdx.x];
    o[threadIdx.x] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, A ^ B, 0, 0, 0);
}
typedef int v16i __attribute__((ext_vector_type(16)));
__global__ void p32w(const v4i* a, const v4i* b, float* o) {
    v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[threadIdx.x], b[threadIdx.x], v16i{0}, 0, 0, 0);
    o[threadIdx.x] = (float)c[5];
}
__global__ void p4(const float* a, const float* b, float* o) {
    v4f c = __builtin_amdgcn_mfma_f32_4x4x1f32(a[threadIdx.x], b[threadIdx.x], v4f{0, 0, 0, 0}, 0, 0, 0);
    o[threadIdx.x] = c[0] * 2.f;
}
"""


def vgprs(text):
    out = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b", text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def instructions(func: str):
    """(opcode, operand text, inside inline assembly) of one kernel's body, in order."""
    out = []
    in_asm = False
    for line in func.split("s_endpgm")[0].split("\n"):
        if ";;#ASMSTART" in line:
            in_asm = True
        if ";;#ASMEND" in line:
            in_asm = False
        ins = line.split(";")[0].strip()
        if ins.endswith(":") and not ins.startswith("_Z"):
            out.append(("<label>", "", in_asm))
            continue
        if not ins or ins.startswith("."):
            continue
        op = ins.split()[0]
        out.append((op, ins[len(op):], in_asm))
    return out


def distances(asm: str, only_inline: bool):
    """(kernel, mfma opcode, wait states before the first dependent VALU read) for every MFMA whose result is read
    in the same straight-line run (a branch or the end of the kernel ends the scan)."""
    found = []
    for func in re.split(r"\n(?=_Z\w+:)", asm):
        name = func.split(":", 1)[0]
        if not name.startswith("_Z"):
            continue
        ins = instructions(func)
        for i, (op, args, in_asm) in enumerate(ins):
            if op not in MFMAS or (only_inline and not in_asm):
                continue
            dest = vgprs(args.split(",")[0])
            waits = 0
            for op2, args2, _ in ins[i + 1:]:
                if op2 == "<label>":
                    continue
                if op2.startswith("s_cbranch") or op2 in ("s_branch", "s_setpc_b64"):
                    waits = None
                    break
                srcs = args2.split(",", 1)[1] if "," in args2 else ""
                if op2.startswith("v_") and not op2.startswith("v_mfma") and vgprs(srcs) & dest:
                    break
                waits += int(args2.split()[0]) + 1 if op2 == "s_nop" else 1
            else:
                waits = None
            if waits is not None:
                found.append((name, op, waits))
    return found


def source_distances(asm: str, only_inline: bool):
    """(kernel, mfma opcode, wait states since the last VALU write of one of its source registers) for every MFMA
    with such a write earlier in its straight-line run (a label or branch ends the backward scan)."""
    found = []
    for func in re.split(r"\n(?=_Z\w+:)", asm):
        name = func.split(":", 1)[0]
        if not name.startswith("_Z"):
            continue
        ins = instructions(func)
        for i, (op, args, in_asm) in enumerate(ins):
            if op not in MFMAS or (only_inline and not in_asm):
                continue
            srcs = vgprs(args.split(",", 1)[1]) if "," in args else set()
            waits = 0
            for op2, args2, _ in reversed(ins[:i]):
                if op2 == "<label>" or op2.startswith("s_cbranch") or op2 in ("s_branch", "s_setpc_b64"):
                    waits = None
                    break
                if op2.startswith("v_") and not op2.startswith("v_mfma") and vgprs(args2.split(",")[0]) & srcs:
                    break
                waits += int(args2.split()[0]) + 1 if op2 == "s_nop" else 1
            else:
                waits = None
            if waits is not None:
                found.append((name, op, waits))
    return found


def compile_asm(src_path, out_path):
    cmd = [HIPCC, *FLAGS, "-I", os.path.join(ROOT, "include"), src_path, "-o", out_path]
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)


def test_checker_measures_distance():
    asm = "\n".join(["_Zk:", ";;#ASMSTART", "v_mfma_i32_16x16x32_i8 v[4:7], v[0:1], v[2:3], 0", ";;#ASMEND",
                     "v_mov_b32_e32 v9, v1", "s_nop 3", "v_cvt_f32_i32_e32 v8, v5", "s_endpgm"])
    assert distances(asm, True) == [("_Zk", "v_mfma_i32_16x16x32_i8", 5)]
    asm = "\n".join(["_Zk:", "v_mov_b32_e32 v9, 0", "v_xor_b32_e32 v2, v1, v0", "s_nop 0", ";;#ASMSTART",
                     "v_mfma_i32_16x16x64_i8 v[4:7], v[0:3], v[8:11], v[12:15]", ";;#ASMEND", "s_endpgm"])
    assert source_distances(asm, True) == [("_Zk", "v_mfma_i32_16x16x64_i8", 1)]
    assert source_distances(asm.replace("v_xor_b32_e32 v2", "v_xor_b32_e32 v20"), True) == [
        ("_Zk", "v_mfma_i32_16x16x64_i8", 2)]
    # a label ends the backward scan
    asm = asm.replace("v_xor_b32_e32 v2", "v_xor_b32_e32 v20").replace("v_mov_b32_e32 v9, 0", "v_mov_b32_e32 v9, 0\n.LBB0_1:")
    assert source_distances(asm, True) == []


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_inline_mfma_results_wait_as_long_as_the_compiler_requires():
    with tempfile.TemporaryDirectory() as tmp:
        probe = os.path.join(tmp, "probe.hip")
        with open(probe, "w") as f:
            f.write(PROBE)
        procs = [("probe", os.path.join(tmp, "probe.s"), compile_asm(probe, os.path.join(tmp, "probe.s")))]
        for src in SOURCES:
            out = os.path.join(tmp, src + ".s")
            procs.append((src, out, compile_asm(os.path.join(ROOT, "kidi_amd", "csrc", src), out)))
        texts = {}
        for src, out, p in procs:
            log, _ = p.communicate()
            assert p.returncode == 0, log.decode(errors="replace")[-2000:]
            with open(out) as f:
                texts[src] = f.read()
    need = {}
    for _, op, waits in distances(texts["probe"], False):
        need[op] = max(need.get(op, 0), waits)
    assert set(need) == set(MFMAS), need
    assert need["v_mfma_i32_16x16x32_i8"] >= 4 and need["v_mfma_f32_4x4x1_16b_f32"] >= 2, need
    bad, seen = [], 0
    for src in SOURCES:
        for name, op, waits in distances(texts[src], True):
            seen += 1
            if waits < need[op]:
                bad.append((src, name[:70], op, waits, need[op]))
    assert seen > 0
    assert not bad, "\n".join(f"{s} {k}: {op} read after {w} wait states (needs {n})" for s, k, op, w, n in bad[:10])
    # sources: a VALU write followed by an MFMA that reads the register
    need_src = min(w for k, op, w in source_distances(texts["probe"], False) if k.startswith("_Z2pw"))
    assert need_src >= 2, need_src
    bad = [(src, name[:70], op, waits) for src in SOURCES for name, op, waits in source_distances(texts[src], True)
           if waits < need_src]
    assert not bad, "\n".join(f"{s} {k}: {op} reads a VALU result after {w} wait states (needs {need_src})"
                               for s, k, op, w in bad[:10])
