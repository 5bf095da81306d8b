"""GPU parity of the trellis path (r4d_trellis_reconstruct_f16, r4dx_trellis_input_*,
r4d_gemm_trellis_nt_m64 / _raw) against the CPU oracle, through the C ABI.

Bars: the decode and the transform are bit-exact; the bf16 linear is bit-exact against the oracle's
epilogue applied to the kernel's own fp32 sums; the fp32 sums are within 1e-3 relative error with a
1e-4 * rms(row) floor of the oracle's fp64 sums (fp32 accumulation, f16 x f16 products exact)."""
import numpy as np
import pytest

import oracle_lib as O
from r4dx_amd import workloads as WL

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no GPU", allow_module_level=True)

from r4dx_amd import api  # noqa: E402
from gpu_util import banner, close_rel, dev, host_u16  # noqa: E402

RAW_REL, RAW_FLOOR = 1e-3, 1e-4


def _grid(K, N, KB, seed):
    return WL.trellis_words(K, N, KB, seed)


@pytest.mark.parametrize("KB,K,N", [(4, 128, 128), (4, 256, 384), (5, 256, 256), (3, 384, 128),
                                    (4, 5120, 5120), (5, 1024, 2048), (4, 1040, 64)])
def test_reconstruct_bit_exact(KB, K, N):
    banner("reconstruct", KB, K, N)
    g = _grid(K, N, KB, 100 + KB)
    q_ref = O.decode_pair_grid(g, K, N, KB)
    q = api.trellis_reconstruct(dev(g), K, N, KB)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(q), q_ref)


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("prescale", [0, 3, -5])
def test_input_transform_bit_exact(bf16, prescale):
    banner("input", bf16, prescale)
    M, K = 5, 5120
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((M, K)) * 4).astype(np.float32)
    xb = O.f32_to_bf16_bits(x) if bf16 else x.astype(np.float16).view(np.uint16)
    s1, s2 = WL.signs(K, 1), WL.signs(K, 2)
    outs = api.trellis_input(dev(xb), [dev(s1), dev(s2)], prescale, bf16)
    torch.cuda.synchronize()
    for s, o in zip((s1, s2), outs):
        ref = O.transform_input(xb, bf16, s, prescale)
        assert np.array_equal(host_u16(o), ref)


def test_fwht128_matches_oracle():
    banner("fwht128")
    rng = np.random.default_rng(3)
    x = rng.standard_normal((7, 128)).astype(np.float32)
    t = api.fwht128(dev(x.copy()))
    torch.cuda.synchronize()
    ref = x.copy()
    for r in ref:
        O.lib().r4o_fwht128_f32(O.ptr(r))
    assert np.array_equal(t.cpu().numpy(), ref)


def _linear_case(K, N, KB, M, seed, skg=None, two_part=False):
    words, suh, svh = WL.trellis_linear(K, N, KB, seed)
    a0 = WL.activations_f16(M, K, seed + 5).view(np.uint16)
    a1 = WL.activations_f16(M, K, seed + 6).view(np.uint16) if two_part else None
    n_split = (N // 256) * 128 if two_part else N
    return words, svh, a0, a1, n_split


@pytest.mark.parametrize("KB,K,N,M,skg", [
    (4, 128, 128, 1, 1), (4, 512, 256, 1, 4), (4, 512, 256, 3, 2), (5, 768, 384, 8, 3),
    (3, 512, 128, 2, 1), (4, 1024, 512, 16, 8), (4, 1024, 256, 17, 4), (4, 512, 256, 64, 2),
    (5, 512, 128, 40, 1), (4, 5120, 5120, 1, None), (5, 5120, 5120, 1, None), (4, 5120, 1024, 8, None),
    (4, 2048, 256, 3, 16), (5, 4096, 384, 9, 32),   # SKG > 8: several slices per run of the finish
])
def test_gemm_raw_and_full(KB, K, N, M, skg):
    banner("gemm", KB, K, N, M, skg)
    skg = api.trellis_gemv_skg(K, N, KB) if skg is None else skg
    words, svh, a0, _, _ = _linear_case(K, N, KB, M, 10 * KB + M)
    w_d, a_d, svh_d = dev(words), dev(a0), dev(svh)
    tickets = api.TicketBuffer(N).t
    raw = api.trellis_gemm_m64(a_d, w_d, None, K, N, KB, skg=skg, raw=True, tickets=tickets)
    out_scale = np.float32(1.0 / np.sqrt(128.0))
    full = api.trellis_gemm_m64(a_d, w_d, svh_d, K, N, KB, skg=skg, out_scale=out_scale, tickets=tickets)
    torch.cuda.synchronize()
    q = O.decode_pair_grid(words, K, N, KB)
    ref = O.raw_sums(a0, q)
    raw_h = raw.cpu().numpy()
    assert close_rel(raw_h, ref, RAW_REL, RAW_FLOOR) <= 1.0
    # the epilogue is bit-exact given the kernel's own sums
    c_ref = O.epilogue_from_raw(raw_h, svh, out_scale)
    assert np.array_equal(host_u16(full), c_ref)
    # tickets are left zero by complete launches
    assert int(tickets.abs().sum()) == 0
    # and the linear is within bf16 rounding of the fp64 reference
    y = O.linear_from_a(a0, q, svh, 0)
    got = O.bf16_bits_to_f32(host_u16(full))
    assert close_rel(got, y, 2.0**-8, 1e-3) <= 1.0


def test_one_hot_rows_return_q():
    """tests/kernels/test_trellis_decode.cpp:9-10: one-hot A rows read rows of Q bit for bit."""
    banner("one-hot")
    K, N, KB = 1024, 512, 4
    words = _grid(K, N, KB, 5)
    ks = [0, 1, 15, 16, 255, 511, 777, 1023]
    a = np.zeros((len(ks), K), np.uint16)
    for m, k in enumerate(ks):
        a[m, k] = 0x3C00
    raw = api.trellis_gemm_m64(dev(a), dev(words), None, K, N, KB, skg=4, raw=True)
    torch.cuda.synchronize()
    q = O.decode_pair_grid(words, K, N, KB)
    got = raw.cpu().numpy()
    for m, k in enumerate(ks):
        assert np.array_equal(got[m], O.f16_bits_to_f32(q[k]))


def test_raw_clock_probe():
    """The _raw entry's clk (third_party/libr4d/r4d.h:376-383): workgroup (0, 0)'s thread 0 writes the shader
    clock and the wall clock at entry and at the end of its own work; clk = 0 leaves the launch as it was."""
    banner("clk")
    K, N, KB = 5120, 6144, 4
    words = _grid(K, N, KB, 9)
    a = dev(WL.activations_f16(1, K, 10).view(np.uint16))
    clk = torch.zeros(4, dtype=torch.int64, device="cuda")
    raw = api.trellis_gemm_m64(a, dev(words), None, K, N, KB, skg=4, raw=True, clk=clk)
    ref = api.trellis_gemm_m64(a, dev(words), None, K, N, KB, skg=4, raw=True)
    torch.cuda.synchronize()
    c = [int(v) for v in clk.cpu()]
    assert c[2] > c[0] > 0 and c[3] > c[1] > 0, c
    ghz = (c[2] - c[0]) / (c[3] - c[1]) * 0.1          # wall clock: 100 MHz
    assert 0.3 < ghz < 4.0, ghz
    assert torch.equal(raw, ref)


def test_row_identity_and_determinism():
    """For M <= 16 a row's bits do not depend on M or on the other rows (the reference's row identity
    rule, src/model/linear.cpp:33-53, third_party/libr4d/r4d.h:370-371), and repeated launches are
    bit-identical."""
    banner("row-identity")
    K, N, KB = 2048, 1024, 4
    words, svh, a, _, _ = _linear_case(K, N, KB, 16, 77)
    w_d, svh_d = dev(words), dev(svh)
    skg = api.trellis_gemv_skg(K, N, KB)
    full = {}
    for M in (1, 2, 3, 4, 8, 13, 16):
        full[M] = host_u16(api.trellis_gemm_m64(dev(a[:M]), w_d, svh_d, K, N, KB, skg=skg, out_scale=0.5))
    torch.cuda.synchronize()
    for M, c in full.items():
        assert np.array_equal(c, full[16][:M]), M
    again = host_u16(api.trellis_gemm_m64(dev(a[:8]), w_d, svh_d, K, N, KB, skg=skg, out_scale=0.5))
    assert np.array_equal(again, full[8])


def test_two_part_split():
    banner("two-part")
    K, N, KB, M = 512, 512, 4, 4
    words, svh, a0, a1, n_split = _linear_case(K, N, KB, M, 31, two_part=True)
    raw = api.trellis_gemm_m64(dev(a0), dev(words), None, K, N, KB, skg=2, a1=dev(a1), n_split=n_split, raw=True)
    torch.cuda.synchronize()
    q = O.decode_pair_grid(words, K, N, KB)
    ref = O.raw_sums(a0, q, a1=a1, n_split=n_split)
    assert close_rel(raw.cpu().numpy(), ref, RAW_REL, RAW_FLOOR) <= 1.0


@pytest.mark.parametrize("name,K,N", WL.LAYER_SHAPES)
def test_config1_shapes_m1_to_m8(name, K, N):
    """Config 1: every projection of the 27B-class layer at KB 4 and 5, M 1, 2, 4 and 8 (the decode step and the
    verify batches), each against the oracle's sums."""
    for KB in (4, 5):
        banner("config1", name, K, N, KB)
        words, svh, a, _, _ = _linear_case(K, N, KB, 8, hash(name) % 1000)
        q = O.decode_pair_grid(words, K, N, KB)
        ref = O.raw_sums(a, q)
        w_d = dev(words)
        for M in (1, 2, 4, 8):
            raw = api.trellis_gemm_m64(dev(a[:M]), w_d, None, K, N, KB, raw=True)
            torch.cuda.synchronize()
            assert close_rel(raw.cpu().numpy(), ref[:M], RAW_REL, RAW_FLOOR) <= 1.0, (KB, M)


@pytest.mark.parametrize("KB,K,N,M,skg,bf16,prescale", [
    (4, 5120, 17408, 1, None, False, 0), (4, 17408, 5120, 1, None, True, 3), (5, 5120, 1024, 8, None, False, -2),
    (4, 6144, 5120, 4, 2, True, 0), (4, 1024, 512, 1, 1, False, 0), (3, 1024, 256, 2, 4, False, 1)])
def test_gemv_fused_transform_bit_identical(KB, K, N, M, skg, bf16, prescale):
    """r4dx_trellis_gemv_xf == r4dx_trellis_input_* + r4d_gemm_trellis_nt_m64, byte for byte (two parts)."""
    banner("gemv xf", KB, K, N, M, skg, bf16, prescale)
    rng = np.random.default_rng(K + N + M)
    words = dev(WL.trellis_words(K, N, KB, 7))
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to("cuda")
    xb = (x.to(torch.bfloat16) if bf16 else x.half()).view(torch.int16)
    suh0, suh1 = dev(WL.signs(K, 8)), dev(WL.signs(K, 9))
    svh = dev(WL.svh_scales(N, 10))
    if skg is None:
        skg = api.trellis_gemv_skg(K, N, KB)
        while (K // 128) % skg:
            skg -= 1
    n_split = N // 2 if N >= 256 else N
    a0, a1 = api.trellis_input(xb, [suh0, suh1], prescale, bf16=bf16)
    ref = api.trellis_gemm_m64(a0, words, svh, K, N, KB, skg=skg, a1=a1, n_split=n_split, out_scale=0.0883883)
    got = api.trellis_gemv_xf(xb, suh0, words, svh, K, N, KB, skg=skg, suh1=suh1, n_split=n_split,
                              prescale=prescale, bf16=bf16, out_scale=0.0883883)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("M,KB,widths", [(1, 4, (6144, 1024, 1024)), (8, 5, (10240, 6144)),
                                         (64, 4, (256, 128, 384, 256)), (3, 5, (1024, 512, 512))])
def test_parts_launch_equals_one_launch_per_projection(M, KB, widths):
    """r4dx_gemm_trellis_nt_m64_parts: projections that share one input, laid out as one linear, give every column
    exactly what the projection's own launch gives at the same SKG; and the whole against the fp64 oracle."""
    banner("parts", M, KB, widths)
    K = 5120 if widths[0] > 1024 else 1024
    N = sum(widths)
    n0 = [int(x) for x in np.concatenate([[0], np.cumsum(widths)[:-1]])]
    words, _, svh = WL.trellis_linear(K, N, KB, 11 * M + KB)
    a = [WL.activations_f16(M, K, 70 + p).view(np.uint16) for p in range(len(widths))]
    a_d = [dev(x) for x in a]
    skg = api.trellis_gemv_skg(K, N, KB)
    osc = float(np.float32(1.0 / np.sqrt(128.0)))
    whole = host_u16(api.trellis_gemm_m64_parts(a_d, n0, dev(words), dev(svh), K, N, KB, skg=skg, out_scale=osc))
    grid = words.reshape(N // 32, -1)
    q = O.decode_pair_grid(words, K, N, KB)
    for p, (c0, wdt) in enumerate(zip(n0, widths)):
        w_p = np.ascontiguousarray(grid[c0 // 32:(c0 + wdt) // 32]).ravel()
        one = host_u16(api.trellis_gemm_m64(a_d[p], dev(w_p), dev(svh[c0:c0 + wdt]), K, wdt, KB, skg=skg,
                                            out_scale=osc))
        torch.cuda.synchronize()
        assert np.array_equal(whole[:, c0:c0 + wdt], one), p
        ref = O.linear_from_a(a[p], np.ascontiguousarray(q[:, c0:c0 + wdt]), svh[c0:c0 + wdt])
        assert close_rel(O.bf16_bits_to_f32(whole[:, c0:c0 + wdt]), ref, 2.0**-8, 1e-3) <= 1.0


@pytest.mark.parametrize("M,KB,widths,bf16,prescale", [(1, 4, (6144, 1024, 1024), False, 0),
                                                        (1, 4, (10240, 6144), True, 0), (8, 5, (10240, 6144), False, 2),
                                                        (4, 4, (256, 128, 384, 256), True, -3),
                                                        (2, 3, (1024, 512, 512), False, 0)])
def test_xf_parts_equals_transform_then_parts(M, KB, widths, bf16, prescale):
    """r4dx_trellis_gemv_xf_parts (the transform fused into the parts launch) == r4dx_trellis_input_* with one output
    per part, then r4dx_gemm_trellis_nt_m64_parts at the same SKG, byte for byte."""
    banner("xf parts", M, KB, widths, bf16, prescale)
    K = 5120 if widths[0] > 1024 else 1024
    N = sum(widths)
    n0 = [int(v) for v in np.concatenate([[0], np.cumsum(widths)[:-1]])]
    rng = np.random.default_rng(N + M)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to("cuda")
    xb = (x.to(torch.bfloat16) if bf16 else x.half()).view(torch.int16)
    suh = [dev(WL.signs(K, 20 + p)) for p in range(len(widths))]
    words, svh = dev(WL.trellis_words(K, N, KB, 12)), dev(WL.svh_scales(N, 13))
    skg = api.trellis_gemv_skg(K, N, KB)
    while (K // 128) % skg:
        skg -= 1
    osc = float(np.float32(1.0 / np.sqrt(128.0)))
    a = [o for i in range(0, len(suh), 3) for o in api.trellis_input(xb, suh[i:i + 3], prescale, bf16=bf16)]
    ref = api.trellis_gemm_m64_parts(a, n0, words, svh, K, N, KB, skg=skg, out_scale=osc)
    got = api.trellis_gemv_xf_parts(xb, suh, n0, words, svh, K, N, KB, skg=skg, prescale=prescale, bf16=bf16,
                                    out_scale=osc)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
