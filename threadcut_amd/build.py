"""Build recipe of the threadcut HIP library (gfx950 only).

Compiles every ``csrc/*.hip`` source with hipcc (and the host-only
``csrc/*.cpp`` with g++) into ``_build/*.o`` in parallel, and links
``libthreadcut_hip.so`` next to this file, where
``threadcut_amd._lib`` loads it. The measurement kernels of ``csrc/bench/``
(not part of the decode ABI) link into ``libthreadcut_bench.so`` beside it, and
``libthreadcut_stamps.so`` is the whole library built with
``-DTC_DECODE_STAMPS=1 -DTC_PREFILL_STAMPS=1``: the decode partial kernel then
records a per-wave timeline and the prefill kernel per-tile phase stamps
(measurement only, ``bench.py --only decode-timeline`` and
``--only prefill-timeline``).
When the repository's ``tests/c_host/tc_host.c`` is present, it is built too
(gcc, C99): a host program that drives the library through the C ABI alone.
Run as ``python -m threadcut_amd.build``.
"""
import concurrent.futures
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libthreadcut_hip.so")
BENCH_LIB = os.path.join(HERE, "libthreadcut_bench.so")
STAMPS_LIB = os.path.join(HERE, "libthreadcut_stamps.so")
ARCH = "gfx950"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
C_HOST = os.path.join(os.path.dirname(HERE), "tests", "c_host", "tc_host.c")

# Packed-fp32 VALU forms stay off: the kernels are written for scalar fp32.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (needs ROCm)")
    return path


def _compile(src, obj, defines=()):
    if src.endswith(".cpp"):  # host-only C++
        cmd = ["g++", "-O3", "-std=c++17", "-fPIC", "-Wall", "-c", src, "-o", obj]
    else:
        cmd = [hipcc(), *COMMON_FLAGS, *defines, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass reports the device-only feature flag as unknown; drop that noise.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in r.stderr.splitlines() if noise not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{err}")
    return err


def _link(objs, lib):
    tmp = lib + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib)


def build(verbose=False):
    """Compile and link both libraries; returns the decode library's path. Always rebuilds."""
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    bench_sources = sorted(glob.glob(os.path.join(CSRC, "bench", "*.hip")))
    os.makedirs(os.path.join(BUILD, "stamps"), exist_ok=True)
    stamp_sources = [s for s in sources if s.endswith(".hip")]
    every = sources + bench_sources + stamp_sources
    objs = [os.path.join(BUILD, os.path.splitext(os.path.basename(s))[0] + ".o") for s in sources + bench_sources]
    stamp_objs = [os.path.join(BUILD, "stamps", os.path.splitext(os.path.basename(s))[0] + ".o")
                  for s in stamp_sources]
    defines = [()] * (len(sources) + len(bench_sources)) + [("-DTC_DECODE_STAMPS=1", "-DTC_PREFILL_STAMPS=1")] * len(stamp_sources)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(every))) as ex:
        for src, warn in zip(every, ex.map(_compile, every, objs + stamp_objs, defines)):
            if warn and verbose:
                print(f"[{os.path.basename(src)}]\n{warn}", file=sys.stderr)
    _link(objs[:len(sources)], LIB)
    _link(objs[len(sources):], BENCH_LIB)
    # The host-only objects are shared; only the HIP sources differ.
    host_objs = [o for s, o in zip(sources, objs) if s.endswith(".cpp")]
    _link(stamp_objs + host_objs, STAMPS_LIB)
    if os.path.exists(C_HOST):
        # The C host is a test program: a failure to build it is reported, and its tests then
        # fail, but the library stays usable.
        try:
            _build_c_host(C_HOST, os.path.splitext(C_HOST)[0])
        except (RuntimeError, OSError) as e:
            print(f"warning: {os.path.relpath(C_HOST, os.path.dirname(HERE))} not built: {e}", file=sys.stderr)
    return LIB


def _build_c_host(src, out):
    """A C99 program linked against the library and the HIP runtime, as a non-Python host
    (cgo, JNI, N-API) would link; it finds the library next to this file at run time."""
    rel = os.path.relpath(HERE, os.path.dirname(out))
    cmd = ["gcc", "-std=c99", "-O2", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{os.path.join(os.path.dirname(HERE), 'include')}", f"-I{ROCM}/include", src,
           f"-L{HERE}", "-lthreadcut_hip", f"-L{ROCM}/lib", "-lamdhip64",
           f"-Wl,-rpath,$ORIGIN/{rel}", f"-Wl,-rpath,{ROCM}/lib", "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"gcc failed on {os.path.basename(src)}:\n{r.stderr}")


if __name__ == "__main__":
    print(build(verbose=True))
