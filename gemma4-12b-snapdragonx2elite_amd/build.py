"""Build recipe for libq4mi.so (gfx950) — plain hipcc, in-tree output.

``python build.py`` (or ``__graft_entry__.build()``) compiles every
``csrc/*.hip`` to an object in ``_build/`` and links
``libq4mi.so`` next to this file. No torch extension machinery: the library
depends only on the HIP runtime.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "libq4mi.so"
ARCH = os.environ.get("Q4MI_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # keep the reference's operation order where parity is bit-exact
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # no packed-fp32 VALU code generation on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# per-source extra flags: the small-M GEMV's MFMA results are read by VALU
# at once; in VGPRs (not AGPRs) that saves one v_accvgpr_read per value
FILE_FLAGS = {"gemv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
              # the online softmax rescales the attention accumulators every key tile: in AGPRs each
              # rescale moved them out and back (~20% of the loop's instructions)
              "prefill_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build libq4mi")


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = [l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l]
    return p.returncode, "\n".join(lines)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all sources (always) and link ``libq4mi.so``. Returns its path."""
    hipcc = _hipcc()
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    bdir = HERE / "_build"
    bdir.mkdir(exist_ok=True)
    objs = [bdir / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), 8)

    def compile_one(pair):
        s, o = pair
        return s, _run([hipcc, *HIPCC_FLAGS, *FILE_FLAGS.get(s.name, []), "-c", str(s), "-o", str(o)])

    with cf.ThreadPoolExecutor(jobs) as ex:
        for s, (rc, out) in ex.map(compile_one, zip(srcs, objs)):
            if rc != 0:
                raise RuntimeError(f"hipcc failed on {s.name}:\n{out}")
            if verbose and out.strip():
                print(out)
    tmp = OUT.with_suffix(".so.tmp")
    rc, out = _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    if rc != 0:
        raise RuntimeError(f"link failed:\n{out}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
