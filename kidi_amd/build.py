"""Build recipe for the HIP library (lib/libkq_hip.so) — hipcc for gfx950, in-tree, no JIT cache.

All device code is compiled with packed FP32 instructions disabled and without floating-point contraction
(every a*b+c rounds twice, matching the reference C++); divisions stay IEEE correctly rounded.
"""

from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = ["csrc/kq_kernels.hip", "csrc/kq_skinny.hip", "csrc/kq_decode.hip", "csrc/kq_gemm.hip", "csrc/kq_gemm_g.hip", "csrc/kq_gemm8.hip", "csrc/kq_greedy.hip", "csrc/kq_norm.hip", "csrc/kq_pack.hip", "csrc/kq_noalloc.hip", "csrc/kq_api.cpp", "csrc/kq_layout_host.cpp"]
LIB = os.path.join(HERE, "lib", "libkq_hip.so")
# The C++ adapter over the C ABI (Kidi's PACKED_LINEAR plug-in, compiled against a restatement of its contract).
ADAPTER_SOURCES = ["adapter/kidi_runtime.cpp", "adapter/packed_linear.cpp"]
ADAPTER_LIB = os.path.join(HERE, "lib", "libkq_adapter.so")
# Per-source flags: the decode kernels take their first nine scalar arguments preloaded into SGPRs at wave launch
# (gfx950 kernel-argument preloading; on firmware without it the code object's preamble loads them as usual).
EXTRA = {"csrc/kq_decode.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=9"]}

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Compile every source and link lib/libkq_hip.so. With incremental=True, objects kept in lib/obj/ from an
    earlier incremental build are reused when they are newer than their source and every header."""
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    objdir = os.path.join(HERE, "lib", "obj") if incremental else os.path.join(HERE, "lib")
    os.makedirs(objdir, exist_ok=True)
    headers = [os.path.join(HERE, "csrc", f) for f in os.listdir(os.path.join(HERE, "csrc")) if f.endswith(".hpp")]
    headers.append(os.path.join(ROOT, "include", "kq.h"))
    newest_header = max(os.path.getmtime(h) for h in headers)
    objs = []
    procs = []
    for src in SOURCES:
        obj = os.path.join(objdir, os.path.basename(src) + ".o")
        objs.append(obj)
        if incremental and os.path.exists(obj) and os.path.getmtime(obj) > max(
                newest_header, os.path.getmtime(os.path.join(HERE, src))):
            continue
        cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), "-I", os.path.join(ROOT, "include"), "-c", os.path.join(HERE, src),
               "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT), src))
    for p, src in procs:
        out, _ = p.communicate()
        text = "\n".join(l for l in out.decode(errors="replace").splitlines() if "packed-fp32-ops" not in l)
        if p.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{text}")
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    if not incremental:
        for o in objs:
            os.remove(o)
    build_adapter(verbose)
    return LIB


def build_adapter(verbose: bool = False) -> str:
    """lib/libkq_adapter.so: the C++20 adapter, linked against lib/libkq_hip.so (found next to it at run time)."""
    tmp = ADAPTER_LIB + ".tmp"
    cmd = [HIPCC, "-std=c++20", "-O2", "-fPIC", "-shared", "-Wall", "-I", os.path.join(ROOT, "include"),
           *[os.path.join(HERE, s) for s in ADAPTER_SOURCES], "-L", os.path.dirname(LIB), "-lkq_hip",
           "-Wl,-rpath,$ORIGIN", "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if p.returncode != 0:
        raise RuntimeError("hipcc failed for the adapter:\n" + p.stdout.decode(errors="replace"))
    os.replace(tmp, ADAPTER_LIB)
    return ADAPTER_LIB


if __name__ == "__main__":
    import sys

    print(build(verbose=True, incremental="--incremental" in sys.argv))
