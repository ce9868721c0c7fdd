"""Builds smallmind_amd/libsmx.so (HIP kernels + host runtime + C-ABI) for gfx950.

Every HIP source is compiled with hipcc for gfx950 only; objects are compiled in parallel
into smallmind_amd/_build/ and linked in-tree so the library travels with the repository.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libsmx.so")
BUILD = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# The matrix-core kernels keep MFMA results in ordinary VGPRs (gfx950 allows either register
# file): in the accumulation-register form every sub-block's results were copied out with one
# v_accvgpr_read per value, 20-30 % of the GEMM loop's VALU-slot instructions (configs[2]
# prefill 62.6-63.1K -> 66.1-66.4K tok/s, configs[4] +2.2 %; same results).
MFMA_VGPR = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]

# (source, object name, extra flags); the GEMV is built once per block format so its
# instantiations compile in parallel.
SOURCES = [("k_quant.hip", "k_quant", []), ("k_ops.hip", "k_ops", []), ("runtime.cpp", "runtime", []),
           ("gemv_dispatch.cpp", "gemv_dispatch", []), ("k_qgemm.hip", "k_qgemm", MFMA_VGPR),
           ("k_attn_prefill.hip", "k_attn_prefill", MFMA_VGPR), ("gguf.cpp", "gguf", []), ("smq.cpp", "smq", []), ("host_common.cpp", "host_common", []), ("k_sample.hip", "k_sample", [])] + [
           ("k_gemv.hip", f"k_gemv_f{f}", [f"-DSMX_GEMV_FMT={f}"]) for f in range(9)]

FLAGS = [
    "-O3", "-std=c++17", "--offload-arch=gfx950", "-fPIC", "-fvisibility=hidden",
    # Reference numerics: never fuse a*b+c unless the source calls fmaf.
    "-ffp-contract=off",
    # Keep the compiler from emitting packed fp32 arithmetic.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
]


# The fused GEMV keeps a row group's weight chunks in registers; an instance that spilled them
# to scratch memory once returned wrong sums (F32, 4 rows x 4 chunks; cause not established), so
# the build refuses any kernel instance with scratch memory, in every HIP source.
SPILL_CHECKED = tuple(sorted({src for src, _, _ in SOURCES if src.endswith(".hip")}))


def _spilling_kernels(remarks: str) -> list:
    """Kernels whose resource remark reports scratch memory (bytes per lane > 0)."""
    out, name = [], None
    for line in remarks.splitlines():
        if "Function Name:" in line:
            name = line.split("Function Name:", 1)[1].split()[0]
        elif "ScratchSize [bytes/lane]:" in line and name:
            if int(line.split("ScratchSize [bytes/lane]:", 1)[1].split()[0]) > 0:
                out.append(name)
    return out


def _compile(entry) -> str:
    src, name, extra = entry
    obj = os.path.join(BUILD, name + ".o")
    check = src in SPILL_CHECKED
    cmd = [HIPCC, *FLAGS, *extra, *(["-Rpass-analysis=kernel-resource-usage"] if check else []),
           "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    if check:
        bad = _spilling_kernels(r.stderr)
        if bad:
            os.remove(obj)
            raise RuntimeError(f"{src} ({' '.join(extra)}): kernel instances use scratch memory: {bad}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 8, 16)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    build_consumer()
    if verbose:
        print(f"built {OUT}")
    return OUT


ROOT = os.path.dirname(HERE)
CONSUMER = os.path.join(ROOT, "tests", "capi", "smx_consumer")


def build_consumer() -> str:
    """The C99 consumer of the C-ABI (tests/capi/smx_consumer.c), linked against libsmx.so with
    a relative run path so that it finds the in-tree library wherever the tree is copied."""
    cmd = ["gcc", "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
           CONSUMER + ".c", "-L", HERE, "-l:libsmx.so", "-Wl,-rpath,$ORIGIN/../../smallmind_amd",
           "-Wl,--allow-shlib-undefined", "-lm", "-o", CONSUMER]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"C consumer build failed:\n{r.stdout}\n{r.stderr}")
    return CONSUMER


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
