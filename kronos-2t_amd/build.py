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

# Extra flags of single sources.  The MFMA kernel's results feed VALU epilogues: with
# the VGPR form its MFMAs write ordinary VGPRs (no accumulator-register reads).
FILE_FLAGS = {"k2t_gemm_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

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


def _compile(src, objdir=None, defines=()):
    obj = os.path.join(objdir or OBJ, os.path.basename(src) + ".o")
    extra = FILE_FLAGS.get(os.path.basename(src), [])
    cmd = [HIPCC, *FLAGS, *extra, *[f"-D{d}" for d in defines], "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj, resource_usage(r.stderr)


def check_m0(src, objdir=None, defines=()):
    """Checks of the generated device assembly.

    M0: sources that stage weights with inline-assembly LDS-DMA loads set M0 themselves
    right before each load.  The compiler does not know of that, so its own code must not
    use M0 (every M0 reference is an s_mov_b32 into M0 directly followed by a
    global_load_lds).

    No flat memory instructions: a flat access is issued where the compiler cannot tell
    whether a pointer addresses LDS or global memory (a pointer taken through an integer,
    or a select of an LDS and a global pointer).  It counts against both the vector-memory
    and the LDS counters, so its wait also waits for every global load and store the wave
    has in flight, the weight prefetches included."""
    asm = os.path.join(objdir or OBJ, os.path.basename(src) + ".s")
    cmd = [HIPCC, *[f for f in FLAGS if not f.startswith("-Rpass")], *FILE_FLAGS.get(os.path.basename(src), []),
           *[f"-D{d}" for d in defines], "--cuda-device-only", "-S", src, "-o", asm]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src}:\n{r.stderr}")
    lines = [ln.strip() for ln in open(asm) if not ln.lstrip().startswith((";", "."))]
    for i, ln in enumerate(lines):
        if re.match(r"flat_(load|store|atomic)", ln):
            raise RuntimeError(f"{src}: flat memory instruction in device code ({ln!r}); state the pointer's "
                               "address space (ld_global / ld_lds)")
        if re.search(r"\bm0\b", ln):
            ok = (re.fullmatch(r"s_mov_b32 m0, s\d+", ln) is not None and i + 1 < len(lines)
                  and lines[i + 1].startswith("global_load_lds"))
            if not ok:
                raise RuntimeError(f"{src}: compiler-generated code uses M0 ({ln!r}); the LDS-DMA loads "
                                   "assume it does not")


def build(verbose=False, out=None, defines=()):
    """Builds libk2t_hip.so; `out` and `defines` make a variant elsewhere (a measurement
    build with -DK2T_MK_TRACE, say) without touching the product library."""
    objdir = OBJ if not defines else os.path.join(OBJ, "variant_" + "_".join(defines))
    os.makedirs(objdir, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        res = list(ex.map(lambda src: _compile(src, objdir, defines), srcs))
    objs = [o for o, _ in res]
    with cf.ThreadPoolExecutor(max_workers=8) as ex:
        list(ex.map(lambda src: check_m0(src, objdir, defines), [src for src in srcs if src.endswith(".hip")]))
    usage = [u for _, us in res for u in us]
    with open(os.path.join(objdir, "resource_usage.txt"), "w") as f:
        for name, u in usage:
            f.write(f"{name} " + " ".join(f"{k}={v}" for k, v in u.items()) + "\n")
    # (measurement variants may spill: they are never the product)
    bad = [(n, u.get("ScratchSize")) for n, u in usage
           if not defines and n.startswith(NO_SCRATCH) and u.get("ScratchSize", 0) != 0]
    if bad:
        raise RuntimeError("kernels that must not use scratch memory report scratch: " +
                           ", ".join(f"{n} ({b} B/lane)" for n, b in bad))
    if not any(n.startswith(NO_SCRATCH) for n, _ in usage):
        raise RuntimeError("no resource report for the persistent decode kernel (remark format changed?)")
    out = out or OUT
    os.makedirs(os.path.dirname(os.path.abspath(out)), exist_ok=True)
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", out, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    if verbose:
        print("built", out)
    return out


if __name__ == "__main__":
    import argparse
    ap = argparse.ArgumentParser()
    ap.add_argument("--define", action="append", default=[], help="preprocessor define of a variant build")
    ap.add_argument("--out", default=None, help="output path of a variant build")
    a = ap.parse_args()
    build(verbose=True, out=a.out, defines=tuple(a.define))
    sys.exit(0)
