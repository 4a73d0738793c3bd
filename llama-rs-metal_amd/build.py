"""Build libmoe_hip.so (HIP kernels + C ABI) for gfx950 with hipcc.

Every translation unit under csrc/ is compiled in parallel into _build/ and
linked into llama-rs-metal_amd/libmoe_hip.so (in-tree, so it travels with the
repository snapshot to the GPU box); probe/ (the benchmark's measurement
and synthetic-weight helpers) becomes libmoe_probe.so.  Always rebuilds.

`--timeline` builds the measurement variant libmoe_hip_timeline.so instead:
the same sources with MOE_TIMELINE defined, so the decode kernels record
per-wave phase stamps (decode_timeline.py reads them).
"""
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmoe_hip.so")
TIMELINE_BUILD = os.path.join(HERE, "_build_timeline")
TIMELINE_LIB = os.path.join(HERE, "libmoe_hip_timeline.so")
PROBE = os.path.join(HERE, "probe")
PROBE_LIB = os.path.join(HERE, "libmoe_probe.so")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # packed FP32 instructions stay off (the compiler would otherwise form
    # v_pk_fma_f32 / v_pk_mul_f32 / v_pk_add_f32 from scalar code)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]


def _compile(src, out_dir=BUILD, extra=()):
    obj = os.path.join(out_dir, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, *extra, "-x", "hip", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msgs}")
    return obj, msgs


def _link(objs, lib):
    tmp = lib + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, lib)


def build(verbose=False):
    """Compiles csrc/ into libmoe_hip.so and probe/ (bench.py's measurement
    and synthetic-weight helpers, not the MoE ABI) into libmoe_probe.so."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    probe_srcs = sorted(glob.glob(os.path.join(PROBE, "*.hip")))
    jobs = min(len(srcs) + len(probe_srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(_compile, srcs + probe_srcs))
    if verbose:
        for obj, msgs in results:
            if msgs.strip():
                print(msgs)
    objs = [o for o, _ in results]
    _link(objs[:len(srcs)], LIB)
    _link(objs[len(srcs):], PROBE_LIB)
    return LIB


def build_timeline():
    """Compiles csrc/ with MOE_TIMELINE into libmoe_hip_timeline.so."""
    os.makedirs(TIMELINE_BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    with cf.ThreadPoolExecutor(max(1, min(8, os.cpu_count() or 1))) as ex:
        results = list(ex.map(lambda p: _compile(p, TIMELINE_BUILD, ("-DMOE_TIMELINE",)), srcs))
    _link([o for o, _ in results], TIMELINE_LIB)
    return TIMELINE_LIB


if __name__ == "__main__":
    if "--timeline" in sys.argv:
        print(build_timeline())
    else:
        print(build(verbose="-v" in sys.argv))
