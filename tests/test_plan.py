"""The MI355X tuning plan (r4dx_amd/plan.py): refusals with a reason (the rules of src/model/linear.cpp:680-766),
the row-identity rule (every M <= 16 the same knobs), the M = 64 band on the M = 256 plan's (SK = 2, SKG), and
every accepted plan legal by the kernels' own _check. CPU only (the planners and checks launch nothing); the
GPU identity of an M = 256 launch with the M = 64 band's rows is tests/test_m256_gpu.py's."""
import pytest

from r4dx_amd import plan
from r4dx_amd import workloads as WL

SHAPES = [(N, K) for _, K, N in WL.LAYER_SHAPES] + [(34816, 5120)]


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("kb", [4, 5])
def test_plans_of_the_config1_shapes(N, K, kb):
    decode = [plan.linear_tuning(N, K, kb, M) for M in range(1, 17)]
    assert all(p.ok for p in decode) and len({(p.SK, p.SKG) for p in decode}) == 1
    band = [plan.linear_tuning(N, K, kb, M) for M in (17, 32, 33, 64)]
    m256 = plan.plan_trellis_m256(N, K, kb)
    assert m256.ok and all(p.ok and (p.SK, p.SKG) == (2, m256.SKG) for p in band)
    i8 = plan.plan_trellis_i8(N, K, kb)
    assert i8.ok and i8.skw in (2, 4, 8) and (K // 128) % (i8.skw * i8.SKG) == 0


def test_two_part_plans():
    assert plan.linear_tuning(34816, 5120, 4, 1, parts=2, part_n0=17408).ok
    assert plan.plan_trellis_m256(34816, 5120, 4, parts=2, part_n0=17408).ok
    assert plan.plan_trellis_i8(34816, 5120, 4, parts=2, part_n0=17408, coarse=True).kernel == "i8c"


@pytest.mark.parametrize("f,args,why", [
    (plan.plan_trellis_m256, (5120, 5120, 3), "KB"),
    (plan.plan_trellis_m256, (5120, 5100, 4), "128-blocks"),
    (plan.plan_trellis_m256, (5120, 5120, 4, 3, 128), "parts"),
    (plan.plan_trellis_m256, (5120, 5120, 4, 2, 5120), "part boundary"),
    (plan.plan_trellis_m256, (5120, 5120, 4, 2, 200), "part boundary"),
    (plan.plan_trellis_i8, (5120, 5120, 6), "KB"),
    (plan.linear_tuning, (5120, 5120, 4, 65), "M must be"),
    (plan.linear_tuning, (5120, 5120, 2, 1), "KB"),
])
def test_refusals_name_the_rule(f, args, why):
    p = f(*args)
    assert not p.ok and why in p.why


TP2_SHAPES = [(8704 * 2, 5120, 2, 8704), (5120, 5120, 1, None), (3072, 5120, 1, None), (512, 5120, 1, None),
              (5120, 8704, 1, None), (5120, 3072, 1, None)]


@pytest.mark.parametrize("N,K,parts,n0", TP2_SHAPES)
@pytest.mark.parametrize("kb", [4, 5])
def test_plans_of_the_tp2_rank_shapes(N, K, parts, n0, kb):
    """One TP = 2 rank's shapes (docs/trellis-kernel.md:197-203, rank K 8704 = 544 k-tiles = 2^5 17): every planner
    accepts them and every plan is legal by the kernels' own checks."""
    decode = [plan.linear_tuning(N, K, kb, M, parts=parts, part_n0=n0) for M in (1, 8, 16)]
    assert all(p.ok for p in decode) and len({(p.SK, p.SKG) for p in decode}) == 1
    assert (K // 16) % decode[0].SKG == 0
    m256 = plan.plan_trellis_m256(N, K, kb, parts=parts, part_n0=n0)
    assert m256.ok and (K // 16) % m256.SKG == 0
    i8 = plan.plan_trellis_i8(N, K, kb, parts=parts, part_n0=n0)
    assert i8.ok


@pytest.mark.parametrize("K,N", [(5120, 16384), (5120, 8192), (5120, 34816), (6144, 5120), (17408, 5120),
                                 (5120, 1024), (1024, 512), (8704, 5120), (3072, 5120), (5120, 6144), (5120, 10240),
                                 (5120, 5120)])
def test_gemv_split_planner_rules(K, N):
    """r4d_mi355x_trellis_gemv_skg: a power of two up to 8 dividing K/16 (whole k-tiles per slice; the engine's rows
    hold no other SKG), at least 10 k-tiles per wave of a slice when any split allows it, and the documented picks on
    the step's launch shapes."""
    from r4dx_amd import api
    skg = api.trellis_gemv_skg(K, N, 4)
    KT = K // 16
    assert KT % skg == 0 and skg in (1, 2, 4, 8)
    if skg > 1:
        assert KT / skg / 4 >= 10
    want = {(5120, 16384): 2, (5120, 8192): 2, (5120, 34816): 2, (6144, 5120): 8, (17408, 5120): 8,
            (5120, 1024): 8, (1024, 512): 1, (5120, 6144): 4, (5120, 10240): 4, (5120, 5120): 8}
    if (K, N) in want:
        assert skg == want[(K, N)]
