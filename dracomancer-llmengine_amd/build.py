"""Build libdraco_hip.so (gfx950) in-tree.

Every .hip / .cpp file under csrc/ is compiled by hipcc for gfx950 and linked
into lib/libdraco_hip.so.  Packed-FP32 instruction selection is disabled for
all device code (-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
OBJDIR = os.path.join(HERE, "_build")
LIB = os.path.join(LIBDIR, "libdraco_hip.so")
TIMELINE_LIB = os.path.join(LIBDIR, "libdraco_hip_timeline.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("DRACO_ARCH", "gfx950")

# Kernel-argument preloading: the dispatcher places the first 14 dwords of
# the arguments in SGPRs, so a kernel issues its first loads after fewer
# dependent scalar loads of its arguments (configs[2] 2327 -> 2376 tok/s,
# configs[3] 600 -> 614 same-box; configs[0] / [4] flat).
COMMON = ["-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}", "-ffp-contract=off",
          "-mllvm", "-amdgpu-kernarg-preload-count=16",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-fopenmp", "-Wno-unused-result", f"-I{CSRC}"]
# Contraction is off everywhere: kernels call fmaf where they want a fused op, and
# host code (rope table, encoders) must round every operation like the reference.
DEVICE_CONTRACT = ["-fno-gpu-flush-denormals-to-zero"]
# Per-file flags.  The prefill GEMM post-processes every MFMA result on the VALU;
# the VGPR form of the MFMA writes them where the VALU reads them, instead of to
# accumulation registers that each need a v_accvgpr_read first.
FILE_FLAGS = {"gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
              # the scan kernels' reader counters: one lane's atomic whose result is
              # used only at the kernel's end (the optimizer's wave-level rewrite
              # would wait for it where it is issued)
              "gdn.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]}


def _sources():
    out = []
    for f in sorted(os.listdir(CSRC)):
        if f.endswith((".hip", ".cpp")):
            out.append(os.path.join(CSRC, f))
    return out


def _compile(src, objdir=OBJDIR, extra=()):
    obj = os.path.join(objdir, os.path.basename(src) + ".o")
    cmd = ([HIPCC] + COMMON + DEVICE_CONTRACT + FILE_FLAGS.get(os.path.basename(src), []) + list(extra) +
           ["-c", src, "-o", obj])
    if src.endswith(".hip"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj


def build(verbose=False, timeline=False):
    """timeline: the profiling variant (-DDRACO_TIMELINE: per-wave stamps in
    the roofline GEMV launch, read by timeline.py) as lib/libdraco_hip_timeline.so,
    objects in _build_timeline/; the product library is not touched."""
    lib = TIMELINE_LIB if timeline else LIB
    objdir = OBJDIR + "_timeline" if timeline else OBJDIR
    extra = ["-DDRACO_TIMELINE"] if timeline else []
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(objdir, exist_ok=True)
    srcs = _sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda f: _compile(f, objdir, extra), srcs))
    tmp = lib + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-fopenmp", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, lib)
    if verbose:
        print(f"[build] {lib} ({os.path.getsize(lib)} bytes) from {len(srcs)} sources")
    return lib


if __name__ == "__main__":
    build(verbose=True, timeline="--timeline" in sys.argv[1:])
    sys.exit(0)
