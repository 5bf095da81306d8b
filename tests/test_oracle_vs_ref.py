"""The C restatement (oracle/_build/libr4o.so) against the reference's own header-only CPU references
compiled from the reference checkout into oracle/_ref (skipped when that checkout is absent, e.g. on
the GPU box).  Bit-exact everywhere: these are the same arithmetic."""
import numpy as np

import oracle_lib as O
from oracle_lib import ptr


def test_codebook_perm_state(olib, rlib):
    a = O.codebook()
    b = np.empty(65536, np.uint16)
    rlib.ref_codebook(ptr(b))
    assert np.array_equal(a, b)
    assert all(olib.r4o_tc_perm(p) == rlib.ref_tc_perm(p) for p in range(256))
    rng = np.random.default_rng(0)
    for KB in (3, 4, 5):
        ring = rng.integers(0, 2**32, 8 * KB, dtype=np.uint64).astype(np.uint32)
        for p in range(256):
            assert olib.r4o_trellis_state(ptr(ring), KB, p) == rlib.ref_trellis_state(ptr(ring), KB, p)


def test_decode_pair_grid(olib, rlib):
    rng = np.random.default_rng(1)
    for KB, K, N in [(4, 256, 384), (5, 128, 256), (3, 128, 128)]:
        words = rng.integers(0, 2**32, K * N * KB // 32, dtype=np.uint64).astype(np.uint32)
        g1 = np.empty_like(words)
        g2 = np.empty_like(words)
        olib.r4o_to_pair_grid(ptr(words), K, N, KB, ptr(g1))
        rlib.ref_to_pair_grid(ptr(words), K, N, KB, ptr(g2))
        assert np.array_equal(g1, g2)
        q1 = O.decode_pair_grid(g1, K, N, KB)
        q2 = np.empty((K, N), np.uint16)
        rlib.ref_decode_pair_grid(ptr(g1), K, N, KB, ptr(q2))
        assert np.array_equal(q1, q2)


def test_fwht_transform_epilogue_linear(olib, rlib):
    rng = np.random.default_rng(2)
    v = rng.standard_normal(128).astype(np.float32)
    a, b = v.copy(), v.copy()
    olib.r4o_fwht128_f32(ptr(a))
    rlib.ref_fwht_lds_f32(ptr(b))
    assert np.array_equal(a, b)
    M, K, N = 3, 384, 256
    x = O.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32) * 3)
    suh = np.where(rng.random(K) < 0.5, -1.0, 1.0).astype(np.float32)
    for s in (0, 3, -2):
        a1 = O.transform_input(x, True, suh, s)
        a2 = np.empty((M, K), np.uint16)
        rlib.ref_transform_input_bf16(ptr(x), M, K, ptr(suh), s, ptr(a2))
        assert np.array_equal(a1, a2)
    raw = (rng.standard_normal((M, N)) * 50).astype(np.float32)
    svh = rng.standard_normal(N).astype(np.float32)
    c1 = O.epilogue_from_raw(raw, svh, np.float32(0.0883883))
    c2 = np.empty((M, N), np.uint16)
    rlib.ref_epilogue_from_raw(ptr(raw), M, N, ptr(svh), np.float32(0.0883883), ptr(c2))
    assert np.array_equal(c1, c2)
    grid = rng.integers(0, 2**32, K * N * 4 // 32, dtype=np.uint64).astype(np.uint32)
    q = O.decode_pair_grid(grid, K, N, 4)
    af = rng.standard_normal((M, K)).astype(np.float16).view(np.uint16)
    a1f = rng.standard_normal((M, K)).astype(np.float16).view(np.uint16)
    y1 = O.linear_from_a(af, q, svh, prescale=1, a1=a1f, n_split=128)
    y2 = np.empty((M, N), np.float64)
    rlib.ref_linear_from_a(ptr(af), ptr(a1f), 128, M, K, N, ptr(q), ptr(svh), 1, ptr(y2))
    assert np.allclose(y1, y2, rtol=1e-12, atol=1e-12)


def test_int8_quantizers_and_gemm(olib, rlib):
    rng = np.random.default_rng(3)
    K, N = 256, 64
    grid = rng.integers(0, 2**32, K * N * 4 // 32, dtype=np.uint64).astype(np.uint32)
    q = O.decode_pair_grid(grid, K, N, 4)
    for fo, fr, ns in [("r4o_i8_quant_w_blk", "ref_i8_quant_w_blk", K // 128 * N),
                       ("r4o_i8_quant_w_col", "ref_i8_quant_w_col", N)]:
        s1, s2 = np.empty(ns, np.float32), np.empty(ns, np.float32)
        w1, w2 = np.empty((N, K), np.int8), np.empty((N, K), np.int8)
        getattr(olib, fo)(ptr(q), K, N, ptr(s1), ptr(w1))
        getattr(rlib, fr)(ptr(q), K, N, ptr(s2), ptr(w2))
        assert np.array_equal(s1, s2) and np.array_equal(w1, w2)
    M = 256
    x = (rng.standard_t(4, (M, K))).astype(np.float16)
    xf = x.astype(np.float32)
    for fo, fr, ns in [("r4o_i8_quant_act_blk", "ref_i8_quant_act_blk", K // 128 * M),
                       ("r4o_i8_quant_act_row", "ref_i8_quant_act_row", M)]:
        s1, s2 = np.empty(ns, np.float32), np.empty(ns, np.float32)
        a1, a2 = np.empty((M, K), np.int8), np.empty((M, K), np.int8)
        getattr(olib, fo)(ptr(x.view(np.uint16)), M, K, ptr(s1), ptr(a1))
        getattr(rlib, fr)(ptr(xf), K, ptr(s2), ptr(a2))
        assert np.array_equal(s1, s2) and np.array_equal(a1, a2)
    for r, k in [(0, 0), (17, 5), (200, 255), (63, 130)]:
        assert olib.r4o_a8_offset(r, k, K) == rlib.ref_a8_offset(r, k, K)
    for n in range(0, N, 7):
        for k in range(0, K, 5):
            assert olib.r4o_w8_offset(n, k, K) == rlib.ref_w8_offset(n, k, K)
    A = rng.integers(-127, 128, (16, K)).astype(np.int8)
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    sa = rng.random(K // 128 * 16).astype(np.float32)
    sw = rng.random(K // 128 * N).astype(np.float32)
    for mask in (0, 1, 2, 3):
        c1, c2 = np.empty((16, N)), np.empty((16, N))
        olib.r4o_i8_gemm_ref(ptr(A), ptr(sa), ptr(W), ptr(sw), 16, N, K, mask, ptr(c1), 1)
        rlib.ref_i8_gemm(ptr(A), ptr(sa), ptr(W), ptr(sw), 16, N, K, mask, ptr(c2))
        assert np.array_equal(c1, c2)


def test_w4a16_and_argmax(olib, rlib):
    rng = np.random.default_rng(4)
    N, K = 64, 512
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[3, :64] = 0.5          # a constant group
    w[4, 64:128] = 0.0       # an all-zero group
    for group in (32, 64):
        q = np.empty((N, K), np.uint8)
        sc = np.empty(N * K // group, np.float32)
        z = np.empty(N * K // group, np.uint8)
        olib.r4o_w4_quantize(ptr(w), N, K, group, ptr(q), ptr(sc), ptr(z))
        wq1, wsz1 = np.empty(N * K // 8, np.uint32), np.empty(N * K // group, np.uint32)
        olib.r4o_w4_pack(ptr(q), N, K, ptr(wq1))
        olib.r4o_w4_pack_scales(ptr(sc), ptr(z), N, K, group, ptr(wsz1))
        wq2, wsz2 = np.empty_like(wq1), np.empty_like(wsz1)
        rlib.ref_w4_quantize_pack(ptr(w), N, K, group, ptr(wq2), ptr(wsz2))
        assert np.array_equal(wq1, wq2) and np.array_equal(wsz1, wsz2)
    x = rng.standard_normal(10000).astype(np.float32)
    x[[5, 700]] = x.max() + 1
    x[::97] = np.nan
    import ctypes as C
    v1, v2 = C.c_float(), C.c_float()
    assert olib.r4o_argmax_f32(ptr(x), len(x), C.byref(v1)) == rlib.ref_argmax(ptr(x), len(x), C.byref(v2))
    assert v1.value == v2.value
    for f in rng.standard_normal(2000).astype(np.float32) * 1e3:
        assert olib.r4o_f32_to_f16(f) == rlib.ref_f32_to_f16(f)
        assert olib.r4o_f32_to_bf16(f) == rlib.ref_f32_to_bf16(f)


def test_weight_fake_quant(olib, rlib):
    """r4o_wq_table / r4o_wq_apply against src/model/fake_quant_w.h's FakeQuantWTableRef / FakeQuantWApplyRef
    (the reference's fp32 product rounded to f16 here, as its kernels do), on decoded trellis weights with an
    all-zero group planted, at the 32-k and 128-k group widths."""
    rng = np.random.default_rng(11)
    for KB, K, N in [(4, 256, 128), (5, 384, 64)]:
        words = rng.integers(0, 2**32, K * N * KB // 32, dtype=np.uint64).astype(np.uint32)
        q = O.decode_pair_grid(words, K, N, KB)
        q[32:64, 5] = 0
        for group in (32, 128):
            t = O.wq_table(q, group)
            tr = np.empty_like(t)
            rlib.ref_wq_table(ptr(q), K, N, group, ptr(tr))
            assert np.array_equal(t.view(np.uint32), tr.view(np.uint32))
            got = O.wq_apply(q, group, t)
            pr = np.empty((K, N), np.float32)
            rlib.ref_wq_apply(ptr(q), K, N, group, ptr(t), ptr(pr))
            want = np.array([rlib.ref_f32_to_f16(float(v)) for v in pr.ravel()], np.uint16).reshape(K, N)
            assert np.array_equal(got, want)
