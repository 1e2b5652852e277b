"""Builds libjacq_kivi.so (the gfx950 KIVI kernels + the C ABI of
include/jacq_kivi.h) in-tree with hipcc.

    python -m jacq_amd.build
"""
from __future__ import annotations

import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libjacq_kivi.so")
TORCH_LIB = os.path.join(HERE, "libjacq_kivi_torch.so")
SOURCES = ["kivi_api.hip", "kivi_writer.hip", "kivi_decode.hip", "kivi_decode_mfma.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-shared",
    "-Wall",
    # No packed-FP32 instructions (v_pk_{add,mul,fma}_f32) anywhere.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # IEEE fp32 division for the writer's scale / code arithmetic.
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # keep MFMA accumulators in VGPRs (no per-iteration AGPR <-> VGPR copies)
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.isabs(cand) and os.path.exists(cand) or not os.path.isabs(cand)):
            return cand
    raise RuntimeError("hipcc not found")


# Kernels that must not spill: a spill makes the kernel need scratch memory,
# which cost the decode about 17 us (13%) when a 12-byte spill crept in.
NO_SCRATCH = ("kivi_decode_stream_kernel", "kivi_append_kernel")


def kernel_resources(remarks: str) -> dict:
    """{kernel symbol: {"vgprs", "scratch", "occupancy"}} from the compiler's
    -Rpass-analysis=kernel-resource-usage remarks."""
    out, cur = {}, None
    for line in remarks.splitlines():
        m = re.search(r"remark:\s+Function Name: (\S+)", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+(VGPRs|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]): (\d+)",
                      line)
        if m and cur is not None:
            key = {"VGPRs": "vgprs", "ScratchSize [bytes/lane]": "scratch",
                   "Occupancy [waves/SIMD]": "occupancy"}[m.group(1)]
            cur[key] = int(m.group(2))
    return out


def build(verbose: bool = False) -> str:
    cmd = [hipcc(), *HIPCC_FLAGS, "-Rpass-analysis=kernel-resource-usage",
           *[os.path.join(CSRC, s) for s in SOURCES], "-o", LIB + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building libjacq_kivi.so")
    spills = {k: v for k, v in kernel_resources(res.stderr).items()
              if any(n in k for n in NO_SCRATCH) and v.get("scratch", 0) > 0}
    if spills:
        os.remove(LIB + ".tmp")
        raise RuntimeError(f"kernels spill to scratch: {spills}")
    os.replace(LIB + ".tmp", LIB)
    return LIB


def build_torch_ops(verbose: bool = False) -> str:
    """libjacq_kivi_torch.so: the torch custom ops (csrc/kivi_torch_ops.cpp)
    over libjacq_kivi.so, found next to it through the $ORIGIN run path."""
    import torch  # noqa: F401  (its headers and libraries)
    from torch.utils import cpp_extension as ce

    inc = [a for d in ce.include_paths(device_type="cuda") for a in ("-I", d)]
    libdirs = [a for d in ce.library_paths(device_type="cuda") for a in ("-L", d)]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [hipcc(), "-O2", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-shared", "-Wall", "-Wno-unused-function",
           "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", os.path.join(ROOT, "include"), *inc,
           os.path.join(CSRC, "kivi_torch_ops.cpp"), "-o", TORCH_LIB + ".tmp",
           "-L", HERE, "-ljacq_kivi", "-Wl,-rpath,$ORIGIN", *libdirs,
           "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-ltorch", "-lamdhip64"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building libjacq_kivi_torch.so")
    os.replace(TORCH_LIB + ".tmp", TORCH_LIB)
    return TORCH_LIB


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_torch_ops(verbose=True))
