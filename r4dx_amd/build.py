"""Builds libr4d_mi355x.so (every HIP source under csrc/, gfx950 only) in-tree with hipcc.

python -m r4dx_amd.build  (or __graft_entry__.build()).  Compiles every time it is called."""
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libr4d_mi355x.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: every product is its own rounding (the bit-exact dequant and transform depend
# on it). -packed-fp32-ops off: no v_pk_*_f32 in generated code.
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I" + CSRC, "-I" + os.path.join(ROOT, "include"), "-Wall", "-Wno-unused-function"]

# Per-source extra flags. trellis_i8.hip: the int8 MFMA accumulators stay in VGPRs (the AGPR form of the int8 MFMA
# does not tie its destination to srcC, and the allocator then rotates 128 accumulators through copies).
EXTRA = {"trellis_i8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]}


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def build(verbose=False, jobs=8):
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs, procs = [], []
    for src in sources():
        obj = os.path.join(objdir, os.path.basename(src) + ".o")
        objs.append(obj)
        cmd = [HIPCC] + FLAGS + EXTRA.get(os.path.basename(src), []) + ["-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        if len(procs) >= jobs:
            _wait(procs.pop(0))
    for p in procs:
        _wait(p)
    tmp = LIB + ".tmp"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs, check=True)
    os.replace(tmp, LIB)
    return LIB


def _wait(item):
    src, p = item
    out, _ = p.communicate()
    text = out.decode(errors="replace")
    lines = [ln for ln in text.splitlines() if "packed-fp32-ops" not in ln]
    if p.returncode != 0:
        sys.stderr.write("\n".join(lines) + "\n")
        raise RuntimeError("hipcc failed on " + src)
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
