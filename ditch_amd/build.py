"""Builds libditch_hip.so (gfx950) in-tree with hipcc.

Each .hip source under csrc/ is compiled to an object in csrc/_build/, then
linked into ditch_amd/libditch_hip.so. Run as `python -m ditch_amd.build`.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

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


# sources compiled more than once: (object name, extra flags) per object
# (gemv.hip: one object per tile format and activation term count, each
# with those kernels, plus one with the dispatch; they compile in parallel)
VARIANTS = {"gemv.hip": [("gemv", [])] + [(f"gemv_tf{tf}_x{xt}", [f"-DGEMV_TF={tf}", f"-DGEMV_XT={xt}"])
                                           for tf in range(7) for xt in (2, 3) if xt == 2 or tf not in (1, 2)]}


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


def jobs():
    """(source, object name, extra flags) for every object of the library."""
    out = []
    for src in sources():
        for name, flags in VARIANTS.get(src, [(src[:-len(".hip")], [])]):
            out.append((src, name, flags))
    return out


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


def _compile(job, build_dir, incremental=False):
    src, name, flags = job
    obj = os.path.join(build_dir, name + ".o")
    if incremental and not _stale(src, obj):
        return obj
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), *flags, "-c", os.path.join(CSRC, src), "-o", obj]
    started = time.time()
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    # the object is as new as the sources the compiler read: an edit made
    # while it ran leaves the object stale for the next incremental build
    os.utime(obj, (started, started))
    return obj


def build(verbose=True, incremental=False):
    """Compiles every source (incremental=True: only those whose object is
    older than the source or a header) and links the library."""
    build_dir = os.path.join(CSRC, "_build")
    os.makedirs(build_dir, exist_ok=True)
    todo = jobs()
    # the slowest objects first, so the long compiles overlap
    order = sorted(range(len(todo)), key=lambda i: not todo[i][1].startswith(("gemv_tf", "gemm_tile")))
    objs = [None] * len(todo)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(todo))) as ex:
        for i, obj in zip(order, ex.map(lambda i: _compile(todo[i], build_dir, incremental), order)):
            objs[i] = obj
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(sources())} sources ({len(todo)} objects)")
    return OUT


if __name__ == "__main__":
    try:
        build(incremental="--incremental" in sys.argv)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
