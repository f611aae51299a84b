"""Builds the gfx950 shared library libk2t_hip.so in-tree with hipcc.

Every HIP source is compiled for gfx950 only, with fp contraction off (all fused
multiply-adds in the kernels are explicit fmaf calls matching the reference's
vfmaq) and packed-FP32 instructions disabled.

The compiler's per-kernel resource report (-Rpass-analysis=kernel-resource-usage) is
parsed after each compile and written to _build/resource_usage.txt.  The build fails
when a kernel in NO_SCRATCH reports scratch (private) memory: the persistent decode
kernel runs at the 256-VGPR limit, and a build of it that spilled to scratch (a
prefetch step compiled as a real call with 512 B of scratch per lane) is the only
build of this library that ever faulted on the GPU.
"""
import concurrent.futures as cf
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libk2t_hip.so")
OBJ = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    "-Rpass-analysis=kernel-resource-usage",
]

# Mangled-name prefixes of kernels that must compile without scratch memory.
NO_SCRATCH = ("_ZN3k2t12_GLOBAL__N_116decode_mk_kernel",)

_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|SGPRs Spill|"
                     r"VGPRs Spill|Occupancy \[waves/SIMD\]):\s*(\S+)")


def resource_usage(text):
    """[(kernel, {field: value})] from hipcc's kernel-resource-usage remarks."""
    out = []
    for m in _REMARK.finditer(text):
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            out.append((val, {}))
        elif out:
            out[-1][1][key.split(" [")[0]] = int(val) if val.isdigit() else val
    return out


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src):
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj, resource_usage(r.stderr)


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        res = list(ex.map(_compile, srcs))
    objs = [o for o, _ in res]
    usage = [u for _, us in res for u in us]
    with open(os.path.join(OBJ, "resource_usage.txt"), "w") as f:
        for name, u in usage:
            f.write(f"{name} " + " ".join(f"{k}={v}" for k, v in u.items()) + "\n")
    bad = [(n, u.get("ScratchSize")) for n, u in usage if n.startswith(NO_SCRATCH) and u.get("ScratchSize", 0) != 0]
    if bad:
        raise RuntimeError("kernels that must not use scratch memory report scratch: " +
                           ", ".join(f"{n} ({b} B/lane)" for n, b in bad))
    if not any(n.startswith(NO_SCRATCH) for n, _ in usage):
        raise RuntimeError("no resource report for the persistent decode kernel (remark format changed?)")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", OUT, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    if verbose:
        print("built", OUT)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
