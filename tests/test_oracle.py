"""The CPU oracle against the known answers the reference's tests hold, the committed golden byte
fixtures, and what the mathematics fixes (closed forms, invariants, brute force).  No GPU."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from oracle_lib import ptr


# ---- codebook: tests/reference/test_trellis_quant.py:81-101 ----------------------------------------
def test_codebook_known_answers(olib):
    cb = O.f16_bits_to_f32(O.codebook()).astype(np.float64)
    assert abs(cb.mean() - (-0.00193)) < 5e-6
    assert abs(cb.std() - 1.00031) < 5e-6
    assert abs(cb.min() - (-3.45312)) < 1e-5 and abs(cb.max() - 3.34766) < 1e-5
    assert len(np.unique(cb)) == 913
    assert cb[0] == -3.453125
    # the f16 constants the hash maps through (test_trellis_quant.py:92)
    assert olib.r4o_f16_to_f32(0x1EEE) == 0.00676727294921875
    assert olib.r4o_f16_to_f32(0xC931) == -10.3828125


def test_codebook_independent_derivation(olib):
    """Python integers + numpy's own f16 rounding, one state at a time (test_trellis_quant.py:93-100)."""
    cb = O.codebook()
    rng = np.random.default_rng(3)
    for s in [0, 1, 2, 255, 256, 4095, 65535] + rng.integers(0, 65536, 300).tolist():
        x = (int(s) * 0x83DCD12D) % (1 << 32)
        bs = sum((x >> (8 * i)) & 0xFF for i in range(4))
        v = np.float16((1024 + bs) * 0.00676727294921875 - 10.3828125)
        assert v.view(np.uint16) == cb[s], s


# ---- permutation: test_trellis_quant.py:104-110 ----------------------------------------------------
def test_tc_perm(olib):
    p = [olib.r4o_tc_perm(i) for i in range(256)]
    assert sorted(p) == list(range(256))
    assert p[:8] == [0, 16, 128, 144, 8, 24, 136, 152]
    assert p[40:48] == [33, 49, 161, 177, 41, 57, 169, 185]


# ---- ring state: brute force over a bit string -----------------------------------------------------
def _bitstring(words):
    return "".join(format(int(w), "032b") for w in words)   # stream bit 32w at bit 31 of word w


@pytest.mark.parametrize("KB", [3, 4, 5])
def test_trellis_state_bruteforce(olib, KB):
    rng = np.random.default_rng(KB)
    ring = rng.integers(0, 2**32, 8 * KB, dtype=np.uint64).astype(np.uint32)
    bits = _bitstring(ring)
    R = 256 * KB
    assert len(bits) == R
    for p in range(256):
        end = KB * (p + 1)
        s = "".join(bits[(end - 16 + i) % R] for i in range(16))
        assert olib.r4o_trellis_state(ptr(ring), KB, p) == int(s, 2), p
    # ring consistency: consecutive states overlap in 16 - KB bits (test_trellis_quant.py:317-322)
    st = [olib.r4o_trellis_state(ptr(ring), KB, p) for p in range(256)]
    m = (1 << (16 - KB)) - 1
    for p in range(256):
        assert (st[p] & m) == (st[(p + 1) % 256] >> KB)


# ---- pair grid + decode ------------------------------------------------------------------------------
def test_pair_grid_and_decode_closed_form(olib):
    K, N, KB = 64, 64, 4
    rng = np.random.default_rng(11)
    words = rng.integers(0, 2**32, K * N * KB // 32, dtype=np.uint64).astype(np.uint32)
    grid = np.empty_like(words)
    olib.r4o_to_pair_grid(ptr(words), K, N, KB, ptr(grid))
    # the pair grid is a permutation of whole tiles: tile (tn, tk) at the documented index
    nw = 8 * KB
    for tk in range(K // 16):
        for tn in range(N // 16):
            i = (((tn >> 1) * (K // 16) + tk) * 2 + (tn & 1)) * nw
            assert olib.r4o_pair_grid_index(K, KB, tn, tk) == i
            assert np.array_equal(grid[i:i + nw], words[(tk * (N // 16) + tn) * nw:][:nw])
    q = O.decode_pair_grid(grid, K, N, KB)
    cb = O.codebook()
    # element (16tk + r, 16tn + c) = cb[state(p)], p = perm^-1(16r + c), from the bit string
    for tk, tn in [(0, 0), (1, 3), (3, 2)]:
        ring = words[(tk * (N // 16) + tn) * nw:][:nw]
        bits = _bitstring(ring)
        for p in range(256):
            e = olib.r4o_tc_perm(p)
            end = KB * (p + 1)
            s = int("".join(bits[(end - 16 + i) % (256 * KB)] for i in range(16)), 2)
            assert q[16 * tk + e // 16, 16 * tn + e % 16] == cb[s]


# ---- FWHT ------------------------------------------------------------------------------------------------
def _hadamard(n):
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def test_fwht128(olib):
    H = _hadamard(128)
    rng = np.random.default_rng(5)
    v = rng.standard_normal(128)
    w = v.copy()
    olib.r4o_fwht128_f64(ptr(w))
    assert np.allclose(w, H @ v, atol=1e-12)
    olib.r4o_fwht128_f64(ptr(w))
    assert np.allclose(w, 128 * v, atol=1e-10)          # H H = 128 I
    # fp32 on integer inputs is exact
    x = rng.integers(-1000, 1000, 128).astype(np.float32)
    y = x.copy()
    olib.r4o_fwht128_f32(ptr(y))
    assert np.array_equal(y, (H @ x.astype(np.float64)).astype(np.float32))


# ---- transform / linear ---------------------------------------------------------------------------------
def test_transform_matches_fp64_within_f16(olib):
    rng = np.random.default_rng(9)
    M, K = 3, 512
    x = rng.standard_normal((M, K)).astype(np.float16)
    suh = np.where(rng.random(K) < 0.5, -1.0, 1.0).astype(np.float32)
    a = O.transform_input(x.view(np.uint16), False, suh, 0)
    t = x.astype(np.float64) * suh
    H = _hadamard(128)
    ref = np.concatenate([t[:, i:i + 128] @ H.T for i in range(0, K, 128)], axis=1) / np.sqrt(128)
    got = O.f16_bits_to_f32(a).astype(np.float64)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-10 + 2.0**-24)


def test_linear_one_hot_rows_return_q(olib):
    """A one-hot A row reads one row of Q (tests/kernels/test_trellis_decode.cpp:9-10): raw sums
    with A = e_k give Q[k] exactly."""
    K, N = 128, 256
    rng = np.random.default_rng(1)
    grid = rng.integers(0, 2**32, K * N * 4 // 32, dtype=np.uint64).astype(np.uint32)
    q = O.decode_pair_grid(grid, K, N, 4)
    a = np.zeros((4, K), np.uint16)
    ks = [0, 5, 77, 127]
    for m, k in enumerate(ks):
        a[m, k] = 0x3C00   # f16 1.0
    s = O.raw_sums(a, q)
    for m, k in enumerate(ks):
        assert np.array_equal(s[m].astype(np.float32), O.f16_bits_to_f32(q[k]))


def test_linear_from_a_matches_dense_math(olib):
    K, N, M = 256, 256, 2
    rng = np.random.default_rng(2)
    grid = rng.integers(0, 2**32, K * N * 4 // 32, dtype=np.uint64).astype(np.uint32)
    q = O.decode_pair_grid(grid, K, N, 4)
    a = rng.standard_normal((M, K)).astype(np.float16).view(np.uint16)
    svh = rng.standard_normal(N).astype(np.float32)
    y = O.linear_from_a(a, q, svh, prescale=2)
    H = _hadamard(128)
    qf = O.f16_bits_to_f32(q).astype(np.float64)
    s = O.f16_bits_to_f32(a).astype(np.float64) @ qf
    t = np.concatenate([s[:, i:i + 128] @ H.T for i in range(0, N, 128)], axis=1)
    ref = t * (2.0**-2 / np.sqrt(128)) * svh
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-9)


def test_epilogue_bf16_rounding(olib):
    rng = np.random.default_rng(4)
    s = rng.standard_normal((2, 256)).astype(np.float32)
    svh = rng.standard_normal(256).astype(np.float32)
    c = O.epilogue_from_raw(s, svh, np.float32(0.25))
    H = _hadamard(128)
    t = np.concatenate([s[:, i:i + 128].astype(np.float64) @ H.T for i in range(0, 256, 128)], axis=1)
    ref = t * svh * 0.25
    got = O.bf16_bits_to_f32(c).astype(np.float64)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-8 * 1.01 + 1e-30)


# ---- int8 -----------------------------------------------------------------------------------------------
def test_i8_quantizers_closed_form(olib):
    # QuantWTrick == rint(w * rs) for every f16 w with |w * rs| <= 127.07
    rng = np.random.default_rng(6)
    for _ in range(2000):
        w = np.float16(rng.standard_normal() * 3)
        amax = abs(float(w)) + abs(rng.standard_normal())
        rs = olib.r4o_i8_rs_half(np.float32(amax / 127.0))
        q = olib.r4o_i8_quant_w(int(w.view(np.uint16)), rs)
        exact = float(w) * float(np.uint16(rs).view(np.float16))
        assert q == int(np.rint(exact)), (w, rs)
    # QuantAct: clamp(rint(x/s)), s = amax/127 so the max maps to +-127
    M, K = 4, 256
    x = (rng.standard_t(4, (M, K)) * 2).astype(np.float16)
    sa = np.empty(M, np.float32)
    ap = np.empty((M, K), np.int8)
    olib.r4o_i8_quant_act_row(ptr(x.view(np.uint16)), M, K, ptr(sa), ptr(ap))
    xf = x.astype(np.float32)
    assert np.allclose(sa, np.abs(xf).max(1) / np.float32(127.0), rtol=0, atol=0)
    assert np.all(np.abs(ap).max(1) == 127)
    assert np.array_equal(ap, np.clip(np.rint(xf / sa[:, None]), -127, 127).astype(np.int8))


def test_i8_gemm_exact_integer(olib):
    rng = np.random.default_rng(8)
    M, N, K = 8, 16, 384
    a = rng.integers(-127, 128, (M, K)).astype(np.int8)
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    acc = np.empty((M, N), np.int32)
    olib.r4o_i8_gemm_i32(ptr(a), ptr(w), M, N, K, ptr(acc), 1)
    assert np.array_equal(acc, a.astype(np.int64) @ w.astype(np.int64).T)
    sa = rng.random(M).astype(np.float32)
    sw = rng.random(N).astype(np.float32)
    c = np.empty((M, N), np.float64)
    olib.r4o_i8_gemm_ref(ptr(a), ptr(sa), ptr(w), ptr(sw), M, N, K, 3, ptr(c), 1)
    assert np.allclose(c, sa[:, None].astype(np.float64) * sw[None, :] * acc, rtol=1e-13)


def test_a8_layout_is_permutation(olib):
    K = 256
    offs = np.array([olib.r4o_a8_offset(r, k, K) for r in range(256) for k in range(K)])
    assert np.array_equal(np.sort(offs), np.arange(256 * K))


def test_w8_layout_is_permutation(olib):
    K, N = 256, 128
    offs = np.array([olib.r4o_w8_offset(n, k, K) for n in range(N) for k in range(K)])
    assert np.array_equal(np.sort(offs), np.arange(N * K))
    # a lane's 16 bytes of fragment F are one column; its 8 bytes per half are 4 + 4 consecutive k
    assert olib.r4o_w8_offset(0, 0, K) == 0 and olib.r4o_w8_offset(0, 3, K) == 3
    assert olib.r4o_w8_offset(0, 8, K) == 4 and olib.r4o_w8_offset(0, 4, K) == 16 * 16
    assert olib.r4o_w8_offset(8, 0, K) == 8 and olib.r4o_w8_offset(16, 0, K) == 16 * 8
    assert olib.r4o_w8_offset(32, 0, K) == (K // 16) * 512 and olib.r4o_w8_offset(0, 16, K) == 512


# ---- w4a16: the reference's committed byte fixtures (tests/convert/test_pack_bytes.cpp:78-99) --------
def test_w4a16_pack_matches_reference_fixtures(olib):
    from safetensors.torch import load_file
    import os
    g = os.path.join(O.ROOT, "tests", "golden")
    w = load_file(os.path.join(g, "input.safetensors"))["w"].float().numpy()
    N, K, group = 32, 256, 64
    q = np.empty((N, K), np.uint8)
    sc = np.empty(N * K // group, np.float32)
    z = np.empty(N * K // group, np.uint8)
    olib.r4o_w4_quantize(ptr(w), N, K, group, ptr(q), ptr(sc), ptr(z))
    wq = np.empty(N * K // 8, np.uint32)
    wsz = np.empty(N * K // group, np.uint32)
    olib.r4o_w4_pack(ptr(q), N, K, ptr(wq))
    olib.r4o_w4_pack_scales(ptr(sc), ptr(z), N, K, group, ptr(wsz))
    assert wq.tobytes() == open(os.path.join(g, "w4a16_wq_g64.bin"), "rb").read()
    assert wsz.tobytes() == open(os.path.join(g, "w4a16_wsz_g64.bin"), "rb").read()
    # dequant of the packed form reproduces scale * (q - zero)
    deq = np.empty((N, K), np.float32)
    olib.r4o_w4_dequant(ptr(wq), ptr(wsz), N, K, group, ptr(deq))
    sc16 = sc.astype(np.float16).astype(np.float32).reshape(N, K // group)
    expect = np.repeat(sc16, group, 1) * (q.astype(np.float32) - np.repeat(z.reshape(N, -1), group, 1))
    assert np.array_equal(deq, expect)
    # the quantized weight is close to the original
    assert np.max(np.abs(deq - w)) <= np.max(sc) * 0.51 + 1e-3


# ---- argmax: argmax_ref.hpp order algebra ------------------------------------------------------------
def test_argmax_order(olib):
    def am(x):
        x = np.asarray(x, np.float32)
        v = C.c_float()
        return olib.r4o_argmax_f32(ptr(x), len(x), C.byref(v)), v.value
    assert am([1, 3, 3, 2]) == (1, 3.0)
    assert am([np.nan, 1, np.nan]) == (1, 1.0)
    i, v = am([-np.inf, np.nan, -np.inf])
    assert i == 0 and v == -np.inf
    assert am([np.nan, 5, 5, np.inf, np.inf])[0] == 3


# ---- the activation producers (r4o_silu_mul_bf16, r4o_attn_gate_mul_bf16) ---------------------------------
def _bf16(x):
    return O.f32_to_bf16_bits(np.asarray(x, np.float32))


def test_producers_closed_forms(olib):
    """sigmoid(0) = 1/2 exactly, sigmoid saturates to 1 at +100 (e^-100 is below an fp32 ulp of 1) and to 0
    at -100 (e^100 overflows): silu(g) u and a sigmoid(g) are then bf16(g u), +-0, bf16(a / 2), bf16(a)."""
    g = np.array([0.0, 100.0, -100.0, 0.0, 100.0, -100.0], np.float32)
    u = np.array([3.0, 1.5, 7.0, -2.0, -0.375, -5.0], np.float32)
    gu = np.concatenate([_bf16(g), _bf16(u)]).astype(np.uint16)
    out = np.empty(6, np.uint16)
    olib.r4o_silu_mul_bf16(ptr(gu), 1, 6, 12, ptr(out))
    got = O.bf16_bits_to_f32(out)
    want = np.array([0.0, 150.0, -0.0, -0.0, -37.5, 0.0], np.float32)
    assert np.array_equal(got, want) and np.array_equal(np.signbit(got), np.signbit(want))
    a = np.array([3.0, -1.25, 6.5, 1e-3], np.float32)
    gg = np.array([0.0, 0.0, 100.0, -100.0], np.float32)
    outg = np.empty(4, np.uint16)
    olib.r4o_attn_gate_mul_bf16(ptr(_bf16(a)), ptr(_bf16(gg)), 4, ptr(outg))
    assert np.array_equal(O.bf16_bits_to_f32(outg), O.bf16_bits_to_f32(_bf16([1.5, -0.625, 6.5, 0.0])))


def test_producers_match_float64(olib):
    """Random gate/up and attention values against a float64 restatement (g / (1 + e^-g) * u, a / (1 + e^-g)):
    within one bf16 ulp everywhere, and the rows, the [gate | up] split and the row stride are honoured."""
    rng = np.random.default_rng(7)
    rows, inter, stride = 3, 384, 2 * 384 + 64
    gu = _bf16(rng.normal(0, 3, (rows, stride)).astype(np.float32))
    out = np.empty((rows, inter), np.uint16)
    olib.r4o_silu_mul_bf16(ptr(gu), rows, inter, stride, ptr(out))
    g = O.bf16_bits_to_f32(gu[:, :inter]).astype(np.float64)
    u = O.bf16_bits_to_f32(gu[:, inter:2 * inter]).astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * u
    got = O.bf16_bits_to_f32(out).astype(np.float64)
    ulp = np.abs(O.bf16_bits_to_f32(_bf16(ref)).astype(np.float64)) * 2.0**-7 + 1e-30
    assert np.all(np.abs(got - ref) <= ulp)
    a = _bf16(rng.normal(0, 2, 1000).astype(np.float32))
    gg = _bf16(rng.normal(0, 4, 1000).astype(np.float32))
    outg = np.empty(1000, np.uint16)
    olib.r4o_attn_gate_mul_bf16(ptr(a), ptr(gg), 1000, ptr(outg))
    refg = O.bf16_bits_to_f32(a).astype(np.float64) / (1.0 + np.exp(-O.bf16_bits_to_f32(gg).astype(np.float64)))
    gotg = O.bf16_bits_to_f32(outg).astype(np.float64)
    assert np.all(np.abs(gotg - refg) <= np.abs(refg) * 2.0**-7 + 1e-30)


# ---- weight fake-quant: closed forms (src/model/fake_quant_w.h:96-140) ----------------------------------------
def _f16(x):
    return np.asarray(x, np.float16).view(np.uint16)


def test_wq_zero_group_and_grid_fixed_points():
    """An all-zero group takes scale 1 and stays zero; a group already on the int8 grid j / 16 with max 127 / 16
    has s = 1/16 exactly and every value is a fixed point (a dropped 1 / s or a wrong clamp moves them)."""
    K, N = 64, 4
    q = np.zeros((K, N), np.float32)
    j = np.arange(-127, 128)
    rng = np.random.default_rng(5)
    q[:, 1] = rng.choice(j, K) / 16.0
    q[7, 1] = 127 / 16.0
    q[:32, 2] = rng.choice(j, 32) / 16.0
    q[3, 2] = -127 / 16.0
    q[32:, 2] = rng.choice(j, 32) * 2.0 ** -8
    q[40, 2] = 127 * 2.0 ** -8
    bits = _f16(q)
    t = O.wq_table(bits, 32)
    assert t[0, 0] == 1.0 and t[1, 0] == 1.0
    assert t[0, 2] == np.float32(1 / 16) and t[1, 2] == np.float32(2.0 ** -8)
    out = O.wq_apply(bits, 32, t)
    assert np.array_equal(out[:, 0], bits[:, 0])
    assert np.array_equal(out[:, 2], bits[:, 2])
    t64 = O.wq_table(bits, 64)
    assert t64[0, 1] == np.float32(1 / 16)
    assert np.array_equal(O.wq_apply(bits, 64, t64)[:, 1], bits[:, 1])


def test_wq_ties_to_even_and_error_bound():
    """s = 1 (group max 127): halves go to the even integer (0.5 -> 0, 1.5 -> 2, 2.5 -> 2, -3.5 -> -4); on random
    decoded weights every value moves by at most s / 2 plus one f16 rounding and lands on the int8 grid."""
    col = np.zeros(32, np.float32)
    col[:6] = [127.0, 0.5, 1.5, 2.5, -3.5, -0.5]
    bits = _f16(col[:, None])
    out = O.f16_bits_to_f32(O.wq_apply(bits, 32))[:, 0]
    assert list(out[:6]) == [127.0, 0.0, 2.0, 2.0, -4.0, -0.0]
    rng = np.random.default_rng(6)
    K, N, KB = 256, 128, 4
    words = rng.integers(0, 2**32, K * N * KB // 32, dtype=np.uint64).astype(np.uint32)
    q = O.decode_pair_grid(words, K, N, KB)
    for g in (32, 64, 128):
        t = O.wq_table(q, g)
        qf = O.f16_bits_to_f32(q).astype(np.float64)
        amax = np.abs(qf).reshape(K // g, g, N).max(axis=1)
        assert np.allclose(t, amax / 127, rtol=2 ** -23, atol=0)
        o = O.f16_bits_to_f32(O.wq_apply(q, g, t)).astype(np.float64)
        s = np.repeat(t.astype(np.float64), g, axis=0)
        assert np.all(np.abs(o - qf) <= s / 2 + np.abs(o) * 2.0 ** -11 + 1e-30)
        # int8 grid: o / s within an f16 rounding of an integer in [-127, 127]
        r = o / s
        assert np.all(np.abs(r) <= 127 * (1 + 2.0 ** -10))
        assert np.all(np.abs(r - np.rint(r)) <= 127 * 2.0 ** -10)
