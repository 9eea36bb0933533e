"""Builds arcinfer_amd/libqmatmul.so: every HIP source in csrc/ compiled for gfx950 with hipcc, then linked as one
shared library exporting the C ABI of include/qmatmul.h. Run `python -m arcinfer_amd.build` (or
__graft_entry__.build()). The library is built in-tree so it travels with the source tree to the GPU host."""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libqmatmul.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HOST_SOURCES = ["qm_gguf.cpp"]  # host-only C++ (g++)
SOURCES = ["qm_prep.hip", "qm_gemv.hip", "qm_gemv_q8.hip", "qm_gemv_k.hip", "qm_gemv_q6.hip", "qm_gemv_iq.hip", "qm_gemv_iq2.hip", "qm_gemv_iq2s.hip", "qm_gemv_q3.hip", "qm_gemv_iq1.hip", "qm_gemm.hip", "qm_gemm_f16.hip", "qm_moe.hip", "qm_moe_dec.hip", "qm_producers.hip", "qm_api.hip"]
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-fno-fast-math", "-fhip-fp32-correctly-rounded-divide-sqrt",
    # packed FP32 instructions stay off: every f32 op is a plain VALU op
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile_host(src):
    obj = os.path.join(BUILD, src.replace(".cpp", ".o"))
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-I", CSRC, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed on {src}:\n{r.stderr}")
    return obj


def _stale(src, obj):
    """True when obj is missing or older than src or any header in csrc/."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [os.path.join(CSRC, src)] + [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".h", ".inc"))]
    return any(os.path.getmtime(d) > t for d in deps)


def _compile(src, incremental=False):
    obj = os.path.join(BUILD, src.replace(".hip", ".o"))
    if incremental and not _stale(src, obj):
        return obj
    cmd = [HIPCC, *FLAGS, "-I", CSRC, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # (hipcc's host pass does not know the packed-fp32 feature name; that warning is expected)
    err = "\n".join(l for l in r.stderr.splitlines() if "not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose=True, incremental=False):
    """Compiles every source (incremental=True: only those whose object is older than the source or a header)."""
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda s: _compile(s, incremental), SOURCES)) + list(ex.map(_compile_host, HOST_SOURCES))
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(incremental="--incremental" in sys.argv)
