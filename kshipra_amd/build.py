"""Build the gfx950 C-ABI library ``libkshipra_quant.so`` in-tree with hipcc.

Usage: ``python -m kshipra_amd.build`` (also called by ``__graft_entry__.build``).
Every call recompiles.  Each ``csrc/*.hip`` file is compiled separately (in
parallel) and the objects are linked into one shared library next to this file.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libkshipra_quant.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = os.environ.get("KSHIPRA_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in device code.
# -fhip-fp32-correctly-rounded-divide-sqrt: IEEE division (quantize is bit-exact).
# -fno-gpu-flush-denormals-to-zero: fp32 subnormals are kept (tiny weights).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fno-fast-math",
    "-ffp-contract=fast",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build kshipra_amd)")


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False) -> str:
    hipcc = _hipcc()
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    with tempfile.TemporaryDirectory(prefix="kq_build_") as tmp:
        objs = [os.path.join(tmp, s[:-4] + ".o") for s in srcs]

        def compile_one(i):
            return _run([hipcc, *HIP_FLAGS, "-c", os.path.join(CSRC, srcs[i]), "-o", objs[i]])

        with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
            outs = list(ex.map(compile_one, range(len(srcs))))
        if verbose:
            for s, o in zip(srcs, outs):
                if o.strip():
                    print(f"[{s}]\n{o}")
        tmp_lib = LIB_PATH + ".tmp"
        _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp_lib, *objs])
        os.replace(tmp_lib, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
