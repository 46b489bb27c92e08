"""Builds libulm_fm.so (the HIP/CDNA4 fast-memory library) in place.

    python unifiedlm.c_amd/build.py

Every source under csrc/ is compiled for gfx950 by hipcc into _build/ and
linked into unifiedlm.c_amd/libulm_fm.so, next to the Python modules that load
it; the layout probes (probe.hip) go into a test-only libulm_probe.so beside it. Packed fp32 VALU instructions are disabled (-packed-fp32-ops) and fp32
atomics use the hardware add (-munsafe-fp-atomics).
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libulm_fm.so")
PROBE_LIB = os.path.join(HERE, "libulm_probe.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")

SOURCES = ["status.hip", "elementwise.hip", "decode.hip", "address.hip", "fm_stats.hip", "fm_chunk.hip", "pair.hip",
           "fm_chunks.hip", "la_kgroup.hip", "fm_ops.hip", "block.hip", "wgrad.hip"]
PROBE_SOURCES = ["status.hip", "probe.hip"]   # the test-only probe library
ARCH = "gfx950"
FLAGS = [f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-munsafe-fp-atomics",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function", f"-I{INCLUDE}"]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the fast-memory library needs ROCm")
    return path


# per-source extra flags
EXTRA = {}


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc()] + FLAGS + EXTRA.get(src, []) + ["-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that line
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj, err


def _link(objs, lib):
    tmp = lib + ".tmp"
    # -z defs: an undefined symbol (a kernel whose host stub was not emitted, say)
    # fails the link instead of the first call
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", tmp] + objs
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {os.path.basename(lib)} failed:\n{res.stderr}")
    os.replace(tmp, lib)


def build(verbose=False):
    """Compile every source and link both shared libraries (always rebuilds)."""
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(set(SOURCES) | set(PROBE_SOURCES))
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        results = dict(zip(sources, ex.map(_compile, sources)))
    for obj, err in results.values():
        if err and verbose:
            print(err, file=sys.stderr)
    _link([results[src][0] for src in SOURCES], LIB)
    _link([results[src][0] for src in PROBE_SOURCES], PROBE_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
