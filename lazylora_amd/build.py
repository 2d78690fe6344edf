"""Build the gfx950 HIP library in-tree: lazylora_amd/liblazylora_mxfp4.so.

hipcc cross-compiles for gfx950 without a GPU, so this runs on any host with ROCm. The
library is one shared object with a plain C ABI (include/lazylora_mxfp4.h); Python loads it
with ctypes and passes torch device pointers.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "liblazylora_mxfp4.so")
SOURCES = ["capi.hip", "mx_forward.hip", "mx_backward.hip", "mx_misc.hip", "mx_router.hip", "mx_lora.hip"]

# per-file flags: the transposed products keep their accumulators in VGPRs (the MFMA's VGPR
# form); with the default heuristics the compiler splits them over AGPRs and VGPRs and shuffles
# them with v_accvgpr moves inside the main loop
FILE_FLAGS = {"mx_backward.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # never emit packed-fp32 VALU ops (v_pk_add/mul/fma_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{os.path.join(ROOT, 'include')}",
]


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    return res.returncode, err


def build(verbose: bool = False) -> str:
    """Compile every source into LIB (always recompiles; the translation units in parallel,
    objects under _build/). Returns the library path."""
    from concurrent.futures import ThreadPoolExecutor
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    compile_flags = [f for f in FLAGS if f != "-shared"]
    jobs = []
    for src in SOURCES:
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        jobs.append(([HIPCC] + compile_flags + FILE_FLAGS.get(src, []) + ["-c", os.path.join(CSRC, src), "-o", obj],
                     obj))
    if verbose:
        for cmd, _ in jobs:
            print(" ".join(cmd), flush=True)
    with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1, 16)) as ex:
        results = list(ex.map(lambda j: _run(j[0]), jobs))
    for (cmd, _), (rc, err) in zip(jobs, results):
        if rc != 0:
            raise RuntimeError(f"hipcc failed ({rc}) on {cmd[-3]}:\n{err}")
        if verbose and err:
            print(err, file=sys.stderr)
    tmp = LIB + ".tmp"
    rc, err = _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC"] + [o for _, o in jobs] + ["-o", tmp])
    if rc != 0:
        raise RuntimeError(f"link failed ({rc}):\n{err}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
