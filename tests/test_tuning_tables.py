"""The MI355X tuning rows in the engine's own formats (r4dx_amd/tables/*.inc, written by r4dx_amd/tuning_inc.py):
parsed as the engine's C++ would read them, and run through a restatement of the engine's planning rules
(src/model/linear.cpp) to show the engine, fed these rows unchanged, plans launches this library accepts:

* every row passes TrellisRowFits (linear.cpp:233-255), so BestRow (:272-296) can pick it;
* ResolveTuning's row-identity rule (:319-333: every M <= 16 chunk takes the M = 1 row) gives one (SK, SKG) to all
  M <= 16, and each band's pick is legal by r4d_gemm_trellis_nt_m64_check at every M it serves;
* PlanTrellisM256 (:680-724) yields a legal M = 256 plan for every config-2 shape and every table shape, one- and
  two-part, and the plan is r4dx_amd/plan.py's;
* PlanTrellisI8 (:726-767) finds a row for every class and the kernel's check accepts it;
* the committed files equal what the generator writes now (the tables follow the library's planners).
CPU only: the planners and checks launch nothing."""
import os
import re

import pytest

from r4dx_amd import plan, tuning_inc
from r4dx_amd.loader import lib

ROW = re.compile(r"\{Layout::kTrellis, (\d+), (\d+), (\d+), \{(\d+), (\d+), (\d+), (\d+), (\d+), (\d+), (\d+)\}, "
                 r"(\d+), (\d+)\},")
I8ROW = re.compile(r"^\s*\{(\d+), (\d+), (\d+), (\d+), (\d+)\},", re.M)


def _trellis_rows(name, path=None):
    text = open(path or os.path.join(tuning_inc.TABLES, name)).read()
    assert "static const GemmTuningRow kGemmTuningTable[] = {" in text and text.rstrip().endswith("};")
    rows = []
    for m in ROW.finditer(text):
        N, K, M, WV, SK, MB, NPW, NT, SKG, U, group, rate = (int(v) for v in m.groups())
        rows.append(dict(N=N, K=K, M=M, t=dict(WV=WV, SK=SK, MB=MB, NPW=NPW, NT=NT, SKG=SKG, U=U), group=group,
                         rate=rate))
    assert rows and len(rows) == len(re.findall(r"^\s+\{Layout::kTrellis", text, re.M))
    return rows


def _i8_rows(name, array):
    text = open(os.path.join(tuning_inc.TABLES, name)).read()
    assert f"const TrellisI8Row {array}[] = {{" in text
    return [tuple(int(v) for v in m.groups()) for m in I8ROW.finditer(text)]


# ---- restatement of the engine's rules (src/model/linear.cpp) ----------------------------------------------------
def trellis_max_mt(kb, np_, u):                      # linear.cpp:233-241
    if kb not in (3, 4, 5):
        return 0
    if np_ == 1:
        return 4 if u in (1, 2, 4) else 0
    if np_ == 2:
        return 4 if u == 1 else 3 if u == 2 else (3 if kb == 4 else 2) if u == 4 else 0
    if np_ == 4:
        return 2 if u == 1 else 1 if u == 2 else 0
    return 0


def trellis_row_fits(N, K, M, kb, t):                # linear.cpp:243-255
    def pow2_upto(v, hi):
        return 1 <= v <= hi and (v & (v - 1)) == 0
    if not (pow2_upto(t["WV"], 4) and pow2_upto(t["SK"], 16) and pow2_upto(t["SKG"], 8)):
        return False
    if t["NT"] not in (0, 1):
        return False
    if t["MB"] < 1 or t["MB"] > trellis_max_mt(kb, t["NPW"], t["U"]):
        return False
    wc = t["WV"] * t["NPW"] * 32
    if wc <= 0 or wc > 256 or N % wc:
        return False
    if t["WV"] * t["SK"] * 32 > 1024 or t["SK"] * wc * 32 > 64 * 1024:
        return False
    if (K // 16) % (t["SK"] * t["SKG"] * t["U"]):
        return False
    split = t["SKG"] > 1 or wc < 128
    return not split or (M + 15) // 16 <= t["MB"]


def best_row(rows, N, K, M, kb):                     # linear.cpp:272-296 (trellis branch)
    best = None
    for r in rows:
        if r["N"] != N or r["K"] != K or r["M"] < M or r["rate"] != kb:
            continue
        if not trellis_row_fits(N, K, M, kb, r["t"]):
            continue
        if best is None or r["M"] < best["M"]:
            best = r
    return best


def resolve(rows, N, K, M, kb):                      # linear.cpp:319-333, a trellis linear with its rows present
    if 1 < M <= 16:
        return resolve(rows, N, K, 1, kb)
    r = best_row(rows, N, K, M, kb)
    assert r is not None, ("no row", N, K, M, kb)    # (the engine would take FallbackTuning)
    return r["t"]


def plan_m256(rows, N, K, kb, parts=1, part_n0=None):   # linear.cpp:680-724
    t = resolve(rows, N, K, 64, kb)
    wc = t["WV"] * t["NPW"] * 32
    assert parts == 1 or part_n0 % wc == 0              # TrellisTuningFor keeps the row (linear.cpp:442-450)
    pref = 2 if t["SK"] <= 2 else (2 if (t["SK"] == 4 and kb == 4 and N == 34816) else 4)
    n_split = part_n0 if parts > 1 else N
    for skw in (pref, 4, 8, 2):
        if skw > t["SK"]:
            continue
        if lib().r4d_gemm_trellis_nt_m256_check(256, K, N, n_split, kb, t["SK"], 1, t["SKG"], 4, skw) is None:
            return t, skw
    return None, None


# ---- the tests ----------------------------------------------------------------------------------------------------
TABLES = [("gemm_tuning_table_trellis.inc", tuning_inc.TP1_SHAPES),
          ("gemm_tuning_table_trellis_tp2.inc", tuning_inc.TP2_SHAPES)]


def test_committed_tables_match_the_generator():
    want = tuning_inc.files()
    assert sorted(os.listdir(tuning_inc.TABLES)) == sorted(want)
    for name, text in want.items():
        assert open(os.path.join(tuning_inc.TABLES, name)).read() == text, name + ": run python -m r4dx_amd.tuning_inc"


@pytest.mark.parametrize("name,shapes", TABLES)
def test_every_row_fits_and_every_band_is_legal(name, shapes):
    rows = _trellis_rows(name)
    assert len(rows) == len(shapes) * len(tuning_inc.RATES) * len(tuning_inc.BANDS)
    L = lib()
    for r in rows:
        assert r["group"] == 0 and trellis_row_fits(r["N"], r["K"], r["M"], r["rate"], r["t"]), r
    for N, K, _ in shapes:
        for kb in tuning_inc.RATES:
            decode = {tuple(resolve(rows, N, K, M, kb).items()) for M in range(1, 17)}
            assert len(decode) == 1                      # row identity: one (SK, SKG) for every M <= 16
            for M in range(1, 65):
                t = resolve(rows, N, K, M, kb)
                p = plan.linear_tuning(N, K, kb, M)
                assert (t["SK"], t["SKG"]) == (p.SK, p.SKG), (N, K, kb, M)
                assert L.r4d_gemm_trellis_nt_m64_check(M, K, N, N, kb, t["SKG"], 1, 1, 1) is None, (N, K, kb, M)


@pytest.mark.parametrize("name,shapes", TABLES)
def test_plan_trellis_m256_takes_every_shape(name, shapes):
    rows = _trellis_rows(name)
    for N, K, _ in shapes:
        for kb in tuning_inc.RATES:
            t, skw = plan_m256(rows, N, K, kb)
            assert t is not None, (N, K, kb)
            p = plan.plan_trellis_m256(N, K, kb)
            assert p.ok and (t["SK"], t["SKG"], skw) == (p.SK, p.SKG, p.skw)
            # the M = 64 row is the order the M = 256 kernel reproduces: SK 1 or 2
            assert t["SK"] in (1, 2)


def test_plan_trellis_m256_config2_shapes_and_two_parts():
    rows = _trellis_rows("gemm_tuning_table_trellis.inc")
    from r4dx_amd import workloads as WL
    for _, K, N in WL.LAYER_SHAPES:
        for kb in tuning_inc.RATES:
            assert plan_m256(rows, N, K, kb)[0] is not None, (N, K, kb)
    for kb in tuning_inc.RATES:   # mlp gate | up as one two-part linear
        assert plan_m256(rows, 34816, 5120, kb, parts=2, part_n0=17408)[0] is not None


@pytest.mark.parametrize("coarse", [False, True])
@pytest.mark.parametrize("tp2", [False, True])
def test_i8_rows(coarse, tp2):
    c, t = ("c" if coarse else ""), ("_tp2" if tp2 else "")
    array = "kTrellisI8" + ("c" if coarse else "") + ("Tp2" if tp2 else "") + "Table"
    rows = _i8_rows(f"gemm_tuning_table_trellis_i8{c}{t}.inc", array)
    shapes = tuning_inc.TP2_SHAPES if tp2 else tuning_inc.TP1_SHAPES
    assert len(rows) == len(shapes) * len(tuning_inc.RATES)
    L = lib()
    for N, K, kb, skw, skg in rows:
        # PlanTrellisI8 (linear.cpp:726-767): the first row of the (N, K, KB), then the kernel's own check
        assert L.r4d_gemm_trellis_nt_i8_check(256, K, N, N, kb, skw, skg) is None, (N, K, kb, skw, skg)
        p = plan.plan_trellis_i8(N, K, kb, coarse=coarse)
        assert p.ok and (p.skw, p.SKG) == (skw, skg)
    for N, K, _ in shapes:
        for kb in tuning_inc.RATES:
            assert any(r[:3] == (N, K, kb) for r in rows)


REF_TABLE = "/root/reference/src/model/gemm_tuning_table_trellis.inc"


@pytest.mark.skipif(not os.path.exists(REF_TABLE), reason="the reference checkout is not here")
def test_reference_rdna4_rows_plan_the_m256_launch():
    """An engine still on the reference's own RDNA4 table (src/model/gemm_tuning_table_trellis.inc) plans the M = 256
    launch from the M = 64 row (linear.cpp:680-724). Every such row -- SK 1 or 2 (the one-wave-per-pair order) or SK
    4, 8, 16 (the 4-wave split order, r4d.h:406) -- passes the kernel's _check wherever its SKG divides the shape, and
    the planner returns a plan for it."""
    rows = _trellis_rows(None, REF_TABLE)
    ck = lib().r4d_gemm_trellis_nt_m256_check
    seen = {1: 0, 2: 0, 4: 0, 8: 0, 16: 0}
    for r in rows:
        if r["M"] != 64:
            continue
        t, kb, N, K = r["t"], r["rate"], r["N"], r["K"]
        seen[t["SK"]] += 1
        legal = ck(256, K, N, N, kb, t["SK"], 1, t["SKG"], 4, 2) is None
        if (K // 16) % (4 * t["SKG"]) == 0:
            assert legal, (N, K, kb, t)
        planned, _ = plan_m256(rows, N, K, kb)
        if legal:
            assert planned is not None, (N, K, kb, t)
    assert seen[4] + seen[8] + seen[16] > 0 and sum(seen.values()) > 0
