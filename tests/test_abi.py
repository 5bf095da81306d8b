"""CPU checks of the drop-in boundary: libr4d_mi355x.so loads without a GPU, exports every symbol
include/r4d_mi355x.h declares, and its host-side legality rules answer without launching."""
import ctypes as C
import os

import pytest

from r4dx_amd import loader

ROOT = os.path.dirname(loader.PKG)


@pytest.fixture(scope="module")
def L():
    return loader.lib()


def test_exports_every_declared_symbol(L):
    names = loader.header_symbols()
    assert len(names) >= 10
    for n in names:
        assert hasattr(L, n), n
        assert n in loader.SIGS, "no ctypes signature for " + n


def test_gemv_checks(L):
    ck = L.r4d_gemm_trellis_nt_m64_check
    assert ck(1, 5120, 5120, 5120, 4, 16, 1, 1, 1) is None
    assert b"M must be" in ck(65, 5120, 5120, 5120, 4, 1, 1, 1, 1)
    assert b"multiples of 128" in ck(1, 5100, 5120, 5120, 4, 1, 1, 1, 1)
    assert b"KB 6" in ck(1, 5120, 5120, 5120, 6, 1, 1, 1, 1)
    assert b"SKG" in ck(1, 5120, 5120, 5120, 4, 3, 1, 1, 1)
    assert b"ws and tickets" in ck(1, 5120, 5120, 5120, 4, 2, 1, 1, 0)
    assert b"svh" in ck(1, 5120, 5120, 5120, 4, 1, 1, 0, 1)
    assert b"n_split" in ck(1, 5120, 5120, 100, 4, 1, 1, 1, 1)
    assert ck(1, 5120, 5120, 5120, 4, 1, 0, 0, 0) is None      # _raw needs no svh
    # the finish addresses the partials with 32-bit offsets: SKG M N 4 must fit 2 GiB
    assert ck(64, 5120, 262144, 262144, 4, 32, 1, 1, 1) is None
    assert b"2 GiB" in ck(64, 5120, 262144 + 128, 262144 + 128, 4, 32, 1, 1, 1)


def test_xf_check_bounds_the_whole_lds():
    """r4dx_trellis_gemv_xf_check accepts exactly the launches whose A slice fits the fused transform's 96 KiB and
    whose LDS request -- the larger of the A slice and, reusing its bytes after the k loop, the split form's partial
    accumulators + the finish's buffers -- fits 160 KiB, so the entry never throws on a shape the check accepts.
    Every accepted (M, SKG) is reproduced by the same sizing rule here."""
    L = loader.lib()
    ck = L.r4dx_trellis_gemv_xf_check

    def lds(M, K, N, SKG, ws):
        split = ws or SKG > 1
        # at M = 1 a fused launch with N >= 8192 holds two pairs per workgroup
        npw, sk = (1 if M == 1 and N < 8192 else 2, 4) if split else (4, 1)
        mt = 1 if M <= 16 else 2 if M <= 32 else 4
        ktw = K // 16 // SKG
        steps = (ktw + 3) // 4
        pad = sk * ((steps + sk - 1) // sk) * 4
        tail = (sk - 1) * npw * 8 * mt * 64 * 4 + (M + 8 * min(M, 4)) * 128 * 4 + 16
        return max(pad * M * 32 + 32, tail), pad * M * 32

    for K in (1024, 5120, 6144, 17408):
        for SKG in (1, 2, 4, 8, 10, 16, 34, 40):
            if (K // 128) % SKG:
                continue
            for M in range(1, 65):
                for ws in (0, 1):
                    for N in (1024, 8192):
                        total, a_bytes = lds(M, K, N, SKG, ws)
                        ok = ck(M, K, N, N, 4, SKG, ws) is None
                        want = (ws or SKG == 1) and a_bytes <= 96 * 1024 and total <= 160 * 1024
                        assert ok == want, (K, N, SKG, M, ws)


def test_sizes_and_rates(L):
    assert L.r4d_gemm_trellis_nt_m64_ws_bytes(8, 5120, 4) == 4 * 8 * 5120 * 4
    assert L.r4d_gemm_trellis_nt_m64_tickets_bytes(5120) == 40 * 128   # one 128-byte line per group
    assert L.r4d_gemm_trellis_nt_m64_max_m() == 64
    assert [L.r4d_gemm_trellis_nt_m64_has_rate(k) for k in (2, 3, 4, 5, 6)] == [0, 1, 1, 1, 0]


@pytest.mark.parametrize("K,N", [(5120, 5120), (5120, 1024), (17408, 5120), (5120, 17408), (6144, 5120)])
def test_gemv_split_plan(L, K, N):
    skg = L.r4d_mi355x_trellis_gemv_skg(K, N, 4)
    assert skg >= 1 and (K // 16) % skg == 0 and (K // 16) // skg >= 8


def test_m256_checks(L):
    ck = L.r4d_gemm_trellis_nt_m256_check
    assert ck(256, 5120, 17408, 17408, 4, 0, 0, 4, 0, 0) is None
    assert ck(128, 5120, 5120, 5120, 5, 0, 0, 1, 0, 0) is None
    assert b"M must be" in ck(64, 5120, 5120, 5120, 4, 0, 0, 1, 0, 0)
    assert b"SKG" in ck(256, 5120, 5120, 5120, 4, 0, 0, 3, 0, 0)
    # SK 1 and 2 name the M = 64 one-wave-per-pair order, 4, 8 and 16 its 4-wave split order: both reproduced
    assert ck(256, 5120, 5120, 5120, 4, 2, 1, 2, 4, 2) is None and ck(256, 5120, 5120, 5120, 4, 1, 1, 2, 4, 0) is None
    for sk in (4, 8, 16):
        assert ck(256, 5120, 5120, 5120, 4, sk, 1, 2, 4, 4) is None
    for sk in (3, 32):
        assert b"SK must be 1, 2, 4, 8 or 16" in ck(256, 5120, 5120, 5120, 4, sk, 1, 2, 4, 4)
    # SKG slices, then (SKG > 1) the balanced form's hand-over area: M x 128 fp32 for each of min(units, CUs)
    # workgroups (no GPU here: 256 CUs assumed); SKG = 1 needs no more than the M x N floats
    assert L.r4d_gemm_trellis_nt_m256_ws_bytes(256, 5120, 2) == 2 * 256 * 5120 * 4 + 80 * 256 * 128 * 4
    assert L.r4d_gemm_trellis_nt_m256_ws_bytes(256, 5120, 8) == 8 * 256 * 5120 * 4 + 256 * 256 * 128 * 4
    assert L.r4d_gemm_trellis_nt_m256_ws_bytes(256, 34816, 1) == 256 * 34816 * 4
    for K, N in [(5120, 17408), (17408, 5120), (5120, 1024), (6144, 5120)]:
        skg = L.r4d_mi355x_trellis_m256_skg(K, N, 4)
        assert ck(256, K, N, N, 4, 0, 0, skg, 0, 0) is None
    # the kernel's stores and the split finish address the fp32 slices with 32-bit offsets: SKG M N 4 must fit 2 GiB
    assert ck(256, 2048, 262144, 262144, 4, 0, 0, 8, 0, 0) is None
    assert b"2 GiB" in ck(256, 2048, 262144 + 128, 262144 + 128, 4, 0, 0, 8, 0, 0)
    assert ck(128, 2048, 262144 + 128, 262144 + 128, 4, 0, 0, 8, 0, 0) is None


def test_trellis_i8_check_bounds_the_split_slices(L):
    """A split trellis-int8 launch sums its fp32 slices in the prefill GEMM's finish (32-bit offsets): skg 256 N 4
    bytes must fit 2 GiB; unsplit launches write no slices."""
    ck = L.r4d_gemm_trellis_nt_i8_check
    assert ck(256, 2048, 262144, 262144, 4, 2, 8) is None
    assert b"2 GiB" in ck(256, 2048, 262144 + 128, 262144 + 128, 4, 2, 8)
    assert ck(256, 2048, 262144 + 128, 262144 + 128, 4, 2, 1) is None


def test_w4a16_checks(L):
    ck = L.r4d_gemm_w4a16_nt_m64_check
    assert ck(32, 1, 5120, 248320) is None and ck(64, 8, 5120, 248320) is None
    assert b"group" in ck(128, 1, 5120, 248320)
    assert b"N must" in ck(64, 1, 5120, 248321)
    assert b"K must" in ck(64, 1, 5100, 256)
    assert ck(64, 64, 5120, 248320) is None            # A is staged in K chunks: any M up to 64
    assert [L.r4d_gemm_w4a16_nt_m64_has_group(g) for g in (16, 32, 64, 128)] == [0, 1, 1, 0]
    assert L.r4d_gemm_w4a16_nt_m64_group() == 64 and L.r4d_gemm_w4a16_nt_m64_max_m() == 64


def test_wq_guards_throw():
    """r4d.h:446-448: a null table or a bad group shift throws (std::runtime_error naming the rule) before any GPU
    work; run in a child process, since an exception cannot cross ctypes. The entries are reached with null
    device pointers, so nothing but the guard can run."""
    import subprocess
    import sys
    calls = [
        "L.r4d_gemm_trellis_nt_m64_wq(0, 0, 256, 0, 0, 0, 0, 0, 1, 1024, 256, 4, 0, 0, 0, 0, 1, 0, 0, 1.0, 0, 3, 0)",
        "L.r4d_gemm_trellis_nt_m64_raw_wq(0, 0, 256, 0, 0, 0, 0, 1, 1024, 256, 4, 0, 0, 0, 0, 1, 0, 0, 8, 4, 0)",
        "L.r4d_gemm_trellis_nt_m256_wq(0, 0, 256, 0, 0, 0, 0, 0, 256, 1024, 256, 4, 0, 0, 1, 0, 1.0, 0, 0, 0, 3)",
        "L.r4d_trellis_wscale_f32(8, 8, 1024, 256, 3, 3, 0)",
    ]
    rules = ["scale table", "gsh must be", "scale table", "KB must be"]
    for call, rule in zip(calls, rules):
        code = f"from r4dx_amd.loader import lib; L = lib(); {call}"
        p = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, cwd=ROOT, timeout=60)
        assert p.returncode != 0 and rule in p.stderr, (call, p.stderr[-400:])


def test_parts_check(L):
    def chk(n0, M=1, K=1024, N=1024, KB=4, SKG=1):
        a = (C.c_int * len(n0))(*n0)
        return L.r4dx_gemm_trellis_nt_m64_parts_check(len(n0), a, M, K, N, KB, SKG, 1)
    assert chk([0]) is None and chk([0, 256, 512, 768]) is None
    assert b"n0[0]" in chk([128, 256])
    assert b"rise" in chk([0, 512, 256]) and b"rise" in chk([0, 100]) and b"rise" in chk([0, 1024])
    assert b"parts" in L.r4dx_gemm_trellis_nt_m64_parts_check(5, (C.c_int * 5)(0, 128, 256, 384, 512), 1, 1024,
                                                              1024, 4, 1, 1)
    assert b"M must be" in chk([0, 256], M=65)


def test_parts_wrappers_refuse_before_launch():
    """api.trellis_gemm_m64_parts / _m256_parts apply the entries' rules first: a bad column start raises
    ValueError in Python (CPU tensors: nothing reaches a device)."""
    torch = pytest.importorskip("torch")
    from r4dx_amd import api
    a = [torch.zeros((1, 1024), dtype=torch.float16) for _ in range(2)]
    w = torch.zeros(1024 * 512 * 4 // 32, dtype=torch.int32)
    svh = torch.ones(512)
    with pytest.raises(ValueError, match="n0"):
        api.trellis_gemm_m64_parts(a, [0, 100], w, svh, 1024, 512, 4, skg=1)
    a256 = [torch.zeros((256, 1024), dtype=torch.float16) for _ in range(2)]
    with pytest.raises(ValueError, match="n0"):
        api.trellis_gemm_m256_parts(a256, [0, 512], w, svh, 1024, 512, 4, skg=1)
    with pytest.raises(ValueError, match="gsh"):
        api.trellis_gemm_m64(a[0], w, svh, 1024, 512, 4, skg=1, wq=(svh, 4))


def test_dense_i8_plan(L):
    """The dense int8 launch form: stream-K (0) for the per-128 modes, the K split of r4d_mi355x_i8_skg for row
    scales; every form passes the dense check."""
    for K, N in ((5120, 17408), (17408, 5120), (1024, 256)):
        assert L.r4d_mi355x_i8_dense_skg(K, N, 0) == L.r4d_mi355x_i8_skg(K, N)
        for mode in (1, 2):
            assert L.r4d_mi355x_i8_dense_skg(K, N, mode) == 0
        for mode in (0, 1, 2):
            assert not L.r4d_gemm_i8_dense_check(256, K, N, L.r4d_mi355x_i8_dense_skg(K, N, mode))
