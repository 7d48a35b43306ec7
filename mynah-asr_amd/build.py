"""Build the gfx950 backend unit and the C11 host mirror, in-tree.

    python mynah-asr_amd/build.py          # both libraries
Outputs (git-ignored, shipped with the tree):
    mynah-asr_amd/lib/libmynah_asr_hip.so  C ABI of include/mynah_asr_hip.h
    mynah-asr_amd/lib/libmynah_asr.so      C11 mirror of qmat.h / backend.h
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
LIB = os.path.join(PKG, "lib")
INC = os.path.join(ROOT, "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_LIB = os.path.join(LIB, "libmynah_asr_hip.so")
HOST_LIB = os.path.join(LIB, "libmynah_asr.so")

# -packed-fp32-ops: no v_pk_*_f32 in generated code; -ffp-contract=off: every
# fused multiply-add in the kernels is an explicit fmaf, so all kernels that
# share a device function perform the same float operations.
# -amdgpu-mfma-vgpr-form (device pass only): MFMA results land in VGPRs, so the
# f32 epilogue that scales them reads them without v_accvgpr_read copies.
HIP_FLAGS = ["-O3", "-std=c++17", "--offload-arch=gfx950", "-fPIC", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Xarch_device", "-mllvm=-amdgpu-mfma-vgpr-form",
             "-Wall", "-Wno-unused-function", "-I", INC, "-I", CSRC]


def _check(cmd: list[str], returncode: int, stderr: str) -> list[str]:
    """One finished compiler command: raises on failure, echoes its warnings,
    returns the kernels that spill registers (from the kernel-resource-usage
    remarks, which are not echoed)."""
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless
    noise = "is not a recognized feature for this target"
    lines, spills, kernel, in_remark = [], [], "", False
    for l in stderr.splitlines():
        if "remark:" in l and "kernel-resource-usage" in l:
            in_remark = True
            body = l.split("remark:", 1)[1].strip()
            if body.startswith("Function Name:"):
                kernel = body.split(":", 1)[1].split("[")[0].strip()
            elif body.startswith("VGPRs Spill:") and body.split(":", 1)[1].split("[")[0].strip() != "0":
                spills.append(f"{kernel} ({body.split(':', 1)[1].split('[')[0].strip()} VGPRs)")
            continue
        if in_remark and (l.lstrip()[:1].isdigit() or l.strip().startswith(("|", "^"))):
            continue   # the source lines a remark quotes
        in_remark = False
        if noise not in l:
            lines.append(l)
    err = "\n".join(lines)
    if returncode != 0:
        sys.stderr.write(err + "\n")
        raise RuntimeError(f"build failed: {' '.join(cmd[:3])} ...")
    if err.strip():
        sys.stderr.write(err + "\n")
    return spills


def _run(cmd: list[str]) -> list[str]:
    r = subprocess.run(cmd, capture_output=True, text=True)
    return _check(cmd, r.returncode, r.stderr)


def build_hip() -> str:
    os.makedirs(LIB, exist_ok=True)
    srcs = [os.path.join(CSRC, f) for f in ("kernels.hip", "attention.hip", "decoder.hip", "encoder.hip", "backend.cpp", "repack.cpp")]
    objs = []
    # the units compile side by side (each hipcc runs one device pass)
    jobs = []
    for s in srcs:
        o = os.path.join(LIB, os.path.basename(s) + ".o")
        cmd = [HIPCC, *HIP_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-x", "hip", "-c", s, "-o", o]
        jobs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.PIPE, text=True)))
        objs.append(o)
    spills = []
    for cmd, pr in jobs:
        _, err = pr.communicate()
        spills += _check(cmd, pr.returncode, err)
    # a kernel that spills runs from scratch memory: say which, so a change
    # that pushes one over its register budget does not go unnoticed
    for k in spills:
        sys.stderr.write(f"build.py: register spill in {k}\n")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", HIP_LIB, *objs])
    for o in objs:
        os.remove(o)
    return HIP_LIB


def build_host() -> str:
    srcs = [os.path.join(HOST, f) for f in ("qmat.c", "backend.c", "synth.c", "gguf.c")]
    if not all(os.path.exists(s) for s in srcs):
        return ""
    _run(["gcc", "-std=c11", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", "-ffp-contract=off",
          "-I", INC, "-I", HOST, "-o", HOST_LIB, *srcs,
          "-L", LIB, "-lmynah_asr_hip", "-Wl,-rpath,$ORIGIN", "-lm", "-lpthread"])
    return HOST_LIB


def build() -> None:
    build_hip()
    build_host()


if __name__ == "__main__":
    build()
    print("built", HIP_LIB, HOST_LIB if os.path.exists(HOST_LIB) else "")
