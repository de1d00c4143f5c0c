"""Builds libditch_hip.so (gfx950) in-tree with hipcc.

Each .hip source under csrc/ is compiled to an object in csrc/_build/, then
linked into ditch_amd/libditch_hip.so. Run as `python -m ditch_amd.build`.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libditch_hip.so")
ARCH = "gfx950"

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed FP32 instructions stay off: some of their forms have given
    # wrong results on these GPUs, with no error
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # f32 subnormals are kept (decode of E8M0 byte 0 and tiny FP8 products)
    "-fno-gpu-flush-denormals-to-zero",
    # every fused multiply-add in the kernels is written out explicitly
    "-ffp-contract=off",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


# per-source additions: the tiled GEMM keeps its MFMA accumulators in the
# architectural VGPRs (with them in AGPRs the register allocator copies every
# accumulator between the two files once per k stage); the GEMV's register
# ring of in-flight units is unrolled whatever its size (indexed at run time
# it would live in scratch memory)
# -disable-machine-sink: the products end each pipeline stage with a wait for
# the next stage's loads and a barrier; machine sinking moves the stage's
# register-only MFMAs past them (into the block after the copier branch),
# which serialises the MFMAs with the memory latency.
EXTRA = {"gemm_tile.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-disable-machine-sink"],
         "gemv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-pragma-unroll-threshold=1000000"],
         "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
         "gemm_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


def _includes(path, seen):
    """The source and every local header it includes, directly or not."""
    path = os.path.normpath(path)
    if path in seen or not os.path.exists(path):
        return seen
    seen.add(path)
    with open(path) as f:
        for line in f:
            line = line.strip()
            if line.startswith("#include \""):
                name = line.split('"')[1]
                _includes(os.path.join(os.path.dirname(path), name), seen)
    return seen


def _stale(src, obj):
    """The object is older than its source or a local header it includes."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = _includes(os.path.join(CSRC, src), set())
    return any(os.path.getmtime(d) > t for d in deps)


def _compile(src, build_dir, incremental=False):
    obj = os.path.join(build_dir, src.replace(".hip", ".o"))
    if incremental and not _stale(src, obj):
        return obj
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def build(verbose=True, incremental=False):
    """Compiles every source (incremental=True: only those whose object is
    older than the source or a header) and links the library."""
    build_dir = os.path.join(CSRC, "_build")
    os.makedirs(build_dir, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, build_dir, incremental), srcs))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources")
    return OUT


if __name__ == "__main__":
    try:
        build(incremental="--incremental" in sys.argv)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
