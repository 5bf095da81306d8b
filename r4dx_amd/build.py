"""Builds libr4d_mi355x.so (every HIP source under csrc/, gfx950 only) in-tree with hipcc.

python -m r4dx_amd.build  (or __graft_entry__.build()).  Compiles every time it is called."""
import glob
import json
import os
import re
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


# The resource gate (the reference fails its build the same way on a trellis instantiation that spills or exceeds its
# register budget, third_party/check_trellis_isa.cmake:1-40): every kernel's hipcc resource report
# (-Rpass-analysis=kernel-resource-usage) must show no scratch and no spills, and each kernel family keeps at least
# the occupancy (waves per SIMD) its design and measurements assume. The report goes to _build/resources.json.
REMARK = "-Rpass-analysis=kernel-resource-usage"
MIN_OCCUPANCY = [            # (demangled name prefix, waves per SIMD at least): every matching prefix applies
    ("tq_gemv_kernel<4, 1, 1, 4, true, 0, false>", 5),   # the decode GEMV at M = 1 (KB 4): VALU latency hiding
    ("tq_gemv_kernel<4, 1, 2, 4, true, 0, false>", 6),   # ... at M = 2..16
    ("tq_gemv_kernel<5, 1, 1, 4, true, 0, false>", 5),
    ("tq_gemv_kernel<", 2),
    ("tq_m256_kernel<", 2),      # 8 waves of 64, one workgroup per CU (96 KiB of LDS stages)
    ("tq_m256_finish", 4),
    ("ti8_gemm_kernel<", 2),     # 8 waves, one workgroup per CU
    ("w4_kernel<", 4),
    ("am_kernel<", 8),
]
# Kernels allowed a few SGPR spills (at most this many; they go to VGPR lanes by v_writelane, never to memory, and the
# gate still requires no scratch and no VGPR spill): the prefill GEMM keeps its launch arguments and the per-segment
# geometry of the balanced form in scalars across the whole kernel, outside the step loop.
SGPR_LANE_SPILLS = [("tq_m256_kernel<", 16)]


def parse_resources(text):
    """[{name, VGPRs, AGPRs, ScratchSize, Occupancy, VGPRsSpill, SGPRsSpill, LDS}] of one compile's remarks."""
    recs, cur = [], None
    for ln in text.splitlines():
        if "remark:" not in ln or REMARK not in ln:
            continue
        body = ln.split("remark:", 1)[1].replace("[" + REMARK + "]", "").strip()
        if body.startswith("Function Name:"):
            cur = {"mangled": body.split(":", 1)[1].strip()}
            recs.append(cur)
        elif cur is not None and ":" in body:
            k, v = body.rsplit(":", 1)
            k = k.split("[")[0].strip().replace(" ", "")
            try:
                cur[k] = int(v.strip())
            except ValueError:
                cur[k] = v.strip()
    if recs:
        out = subprocess.run(["c++filt"], input="\n".join(r["mangled"] for r in recs), capture_output=True,
                             text=True).stdout.splitlines()
        for r, n in zip(recs, out):
            r["name"] = n.replace("(anonymous namespace)::", "").replace("void ", "", 1)
    return recs


def gate(recs):
    """The gate's violations (empty: pass)."""
    bad = []
    for r in recs:
        name = r.get("name", r["mangled"])
        sgpr_ok = max([n for prefix, n in SGPR_LANE_SPILLS if name.startswith(prefix)] or [0])
        if r.get("ScratchSize", 0) or r.get("VGPRsSpill", 0) or r.get("SGPRsSpill", 0) > sgpr_ok:
            bad.append(f"{name}: scratch {r.get('ScratchSize')} B/lane, VGPR spill {r.get('VGPRsSpill')}, "
                       f"SGPR spill {r.get('SGPRsSpill')}")
        for prefix, occ in MIN_OCCUPANCY:
            if name.startswith(prefix) and r.get("Occupancy", 99) < occ:
                bad.append(f"{name}: occupancy {r.get('Occupancy')} waves/SIMD below {occ}")
    return bad


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def build(verbose=False, jobs=8):
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs, procs, recs_early = [], [], []
    for src in sources():
        obj = os.path.join(objdir, os.path.basename(src) + ".o")
        objs.append(obj)
        cmd = [HIPCC] + FLAGS + EXTRA.get(os.path.basename(src), []) + [REMARK, "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        if len(procs) >= jobs:
            recs_early.extend(_wait(procs.pop(0)))
    recs = recs_early
    for p in procs:
        recs += _wait(p)
    with open(os.path.join(objdir, "resources.json"), "w") as f:
        json.dump(recs, f, indent=0)
    bad = gate(recs)
    if bad:
        raise RuntimeError("resource gate (no scratch, no spills, per-family occupancy floors):\n  " + "\n  ".join(bad))
    tmp = LIB + ".tmp"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs, check=True)
    os.replace(tmp, LIB)
    return LIB


def _wait(item):
    src, p = item
    out, _ = p.communicate()
    text = out.decode(errors="replace")
    recs = parse_resources(text)
    for r in recs:
        r["source"] = os.path.basename(src)
    # the resource remarks (and the source lines clang echoes under them) are parsed, not shown
    lines = [ln for ln in text.splitlines() if "packed-fp32-ops" not in ln and REMARK not in ln]
    lines = [ln for ln in lines if not re.match(r"^\s*(\d+\s*\|.*|\|\s*\^.*)$", ln)]
    if p.returncode != 0:
        sys.stderr.write("\n".join(lines) + "\n")
        raise RuntimeError("hipcc failed on " + src)
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")
    return recs


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
