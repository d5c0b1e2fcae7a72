"""Build libtread_hip.so (gfx950) in-tree with hipcc.

Usage: python -m tread_amd.csrc.build   (or __graft_entry__.build())
Objects go to <repo>/_build/, the library to tread_amd/libtread_hip.so.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
ROOT = PKG.parent
SOURCES = ["runtime", "assemble", "deviation", "layer_ops", "attention", "skinny"]
LIB = PKG / "libtread_hip.so"
ARCH = os.environ.get("TREAD_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
          # packed-fp32 VALU forms stay off: ordinary float code only
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


# per-source extra flags: the attention kernel's online softmax takes maxima of finite or -inf
# scores only, so NaN-preserving min/max (and the canonicalising moves they need) are dropped
EXTRA = {"attention": ["-fno-honor-nans"]}


def _run(cmd):
    p = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in p.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(verbose=False):
    out = ROOT / "_build"
    out.mkdir(exist_ok=True)
    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8")))

    def one(name):
        obj = out / f"{name}.o"
        return _run([HIPCC, *CFLAGS, *EXTRA.get(name, []), "-c", str(HERE / f"{name}.hip"), "-o", str(obj)])

    with ThreadPoolExecutor(jobs) as ex:
        msgs = list(ex.map(one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *[str(out / f"{n}.o") for n in SOURCES]])
    os.replace(tmp, LIB)
    if verbose:
        for m in msgs:
            if m:
                print(m, file=sys.stderr)
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
