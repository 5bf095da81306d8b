"""GPU parity of the int8 x int8 trellis prefill GEMM (r4d_gemm_trellis_nt_i8 / _i8c) and its producers, through
the C ABI, in the shape of the reference's own test (tests/kernels/test_trellis_i8_gemm.cpp:1-30):

A. the weight scale tables and the int8 weights (dump_w, block and plain layouts) bit-exact against the oracle's
   decode (trellis_ref.hpp) and weight quantizer (int8_gemm_proto_ref.h:57-77,124-176);
B. the GEMM against the exact integer reference (int32 sums, per-128 or coarse rescale, FWHT, svh, out_scale in
   fp64) within the reference's bench tolerance -- 0.85 % of the value + 1e-4 of the row's rms (one bf16
   rounding and the fp32 sum order) -- on three column groups (first, middle, last) x 256 rows;
C. an EXACT check: a single nonzero activation per row makes every int32 sum one product, so the output must
   equal the oracle's fp32 epilogue of those products byte for byte (a wrong weight, k, row or scale shows);
D. a two-part launch equals two one-part launches byte for byte; E. repeats are byte-identical;
G. the same rows in another order give the same output rows.
"""
import numpy as np
import pytest

import oracle_lib as O
from oracle_lib import ptr
from r4dx_amd import workloads as WL

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no GPU", allow_module_level=True)

from r4dx_amd import api  # noqa: E402
from gpu_util import banner, close_rel, dev  # noqa: E402

OUT_SCALE = float(np.float32(1.0 / np.sqrt(128.0)))


def _weights(K, N, KB, seed):
    words = WL.trellis_words(K, N, KB, seed)
    q = O.decode_pair_grid(words, K, N, KB)            # f16 bits [K][N]
    return words, q


def _oracle_w(q, K, N, coarse):
    sw = np.empty(N if coarse else (K // 128) * N, np.float32)
    wp = np.empty((N, K), np.int8)
    (O.lib().r4o_i8_quant_w_col if coarse else O.lib().r4o_i8_quant_w_blk)(ptr(q), K, N, ptr(sw), ptr(wp))
    return sw, wp


def _oracle_a(x, coarse):
    M, K = x.shape
    sa = np.empty(M if coarse else (K // 128) * M, np.float32)
    ap = np.empty((M, K), np.int8)
    (O.lib().r4o_i8_quant_act_row if coarse else O.lib().r4o_i8_quant_act_blk)(ptr(x.view(np.uint16)), M, K, ptr(sa),
                                                                               ptr(ap))
    return sa, ap


def _hadamard128():
    h = np.array([[1.0]])
    while h.shape[0] < 128:
        h = np.block([[h, h], [h, -h]])
    return h


def _reference(ap, sa, wp, sw, svh, groups, coarse):
    """fp64 C for the column groups listed: exact int32 sums per 128-k block (or over K), the rescale, FWHT-128,
    svh, out_scale."""
    M, K = ap.shape
    N = wp.shape[0]
    H = _hadamard128()
    out = {}
    for gidx in groups:
        cols = slice(128 * gidx, 128 * gidx + 128)
        w = np.ascontiguousarray(wp[cols])
        if coarse:
            acc = np.empty((M, 128), np.int32)
            O.lib().r4o_i8_gemm_i32(ptr(ap), ptr(w), M, 128, K, ptr(acc), 0)
            y = acc.astype(np.float64) * sa.astype(np.float64)[:, None] * sw[cols].astype(np.float64)[None, :]
        else:
            y = np.zeros((M, 128))
            for kb in range(K // 128):
                a_b = np.ascontiguousarray(ap[:, 128 * kb:128 * kb + 128])
                w_b = np.ascontiguousarray(w[:, 128 * kb:128 * kb + 128])
                acc = np.empty((M, 128), np.int32)
                O.lib().r4o_i8_gemm_i32(ptr(a_b), ptr(w_b), M, 128, 128, ptr(acc), 0)
                y += acc * (sa[kb * M:(kb + 1) * M].astype(np.float64)[:, None] *
                            sw[kb * N + 128 * gidx: kb * N + 128 * gidx + 128].astype(np.float64)[None, :])
        out[gidx] = (y @ H) * svh[cols].astype(np.float64)[None, :] * OUT_SCALE
    return out


def _gpu_a(x, coarse):
    return api.i8_quant(dev(x.view(np.uint16)), blk=not coarse, ref_layout=True)


@pytest.mark.parametrize("coarse", [False, True])
@pytest.mark.parametrize("KB", [4, 5])
def test_tables_and_dump_bit_exact(coarse, KB):
    banner("ti8 tables", coarse, KB)
    K, N = 512, 384
    words, q = _weights(K, N, KB, 3 + KB)
    w_d = dev(words)
    sw = api.trellis_i8_table(w_d, K, N, KB, coarse)
    w8, wp = api.trellis_i8_dump(w_d, sw, K, N, KB, coarse)
    torch.cuda.synchronize()
    sw_ref, wp_ref = _oracle_w(q, K, N, coarse)
    assert np.array_equal(sw.cpu().numpy().view(np.uint32), sw_ref.view(np.uint32))
    assert np.array_equal(wp.cpu().numpy(), wp_ref)
    w8_ref = np.empty(N * K, np.int8)
    O.lib().r4o_pack_w8(ptr(wp_ref), N, K, ptr(w8_ref))
    assert np.array_equal(w8.cpu().numpy(), w8_ref)


CASES = [  # (K, N, KB, skg)
    (512, 384, 4, 1), (1024, 256, 5, 2), (1024, 384, 4, 4), (5120, 17408, 4, 1), (17408, 5120, 4, 4),
    (5120, 17408, 5, 2), (17408, 5120, 5, 4), (8704, 5120, 4, 2),  # the last: a TP = 2 rank of mlp.down
]


@pytest.mark.parametrize("coarse", [False, True])
@pytest.mark.parametrize("K,N,KB,skg", CASES)
def test_gemm_vs_exact_integer_reference(coarse, K, N, KB, skg):
    banner("ti8 gemm", coarse, K, N, KB, skg)
    words, q = _weights(K, N, KB, 11)
    x = WL.activations_f16(256, K, 12, outlier_frac=0.01)
    svh = WL.svh_scales(N, 13)
    w_d = dev(words)
    sw = api.trellis_i8_table(w_d, K, N, KB, coarse)
    a8, sa = _gpu_a(x, coarse)
    c = api.trellis_gemm_i8(a8, sa, w_d, sw, dev(svh), K, N, KB, coarse=coarse, skg=skg, out_scale=OUT_SCALE)
    torch.cuda.synchronize()
    got = O.bf16_bits_to_f32(c.view(torch.int16).cpu().numpy().view(np.uint16))
    sw_ref, wp = _oracle_w(q, K, N, coarse)
    sa_ref, ap = _oracle_a(x, coarse)
    assert np.array_equal(sa.cpu().numpy(), sa_ref)
    G = N // 128
    ref = _reference(ap, sa_ref, wp, sw_ref, svh, [0, G // 2, G - 1], coarse)
    for gidx, y in ref.items():
        assert close_rel(got[:, 128 * gidx:128 * gidx + 128], y, 0.0085, 1e-4) <= 1.0, gidx


@pytest.mark.parametrize("coarse", [False, True])
@pytest.mark.parametrize("K,N,KB,skg", [(1024, 384, 4, 1), (1024, 384, 5, 2), (2048, 256, 4, 4)])
def test_single_nonzero_activation_exact(coarse, K, N, KB, skg):
    banner("ti8 exact", coarse, K, N, KB, skg)
    rng = np.random.default_rng(5)
    words, q = _weights(K, N, KB, 21)
    x = np.zeros((256, K), np.float16)
    ks = rng.integers(0, K, 256)
    x[np.arange(256), ks] = rng.standard_normal(256).astype(np.float16) * 3
    svh = WL.svh_scales(N, 22)
    w_d = dev(words)
    sw = api.trellis_i8_table(w_d, K, N, KB, coarse)
    a8, sa = _gpu_a(x, coarse)
    c = api.trellis_gemm_i8(a8, sa, w_d, sw, dev(svh), K, N, KB, coarse=coarse, skg=skg, out_scale=OUT_SCALE)
    torch.cuda.synchronize()
    sw_ref, wp = _oracle_w(q, K, N, coarse)
    sa_ref, ap = _oracle_a(x, coarse)
    # the one product per (row, column), scaled in fp32 as the kernel does: float(int32) * (sa * sw)
    rows = np.arange(256)
    prod = ap[rows, ks].astype(np.int32)[:, None] * wp[:, ks].T.astype(np.int32)          # [256][N]
    if coarse:
        scale = (sa_ref[:, None] * sw_ref[None, :]).astype(np.float32)
    else:
        kb = ks // 128
        scale = (sa_ref[kb * 256 + rows][:, None] * sw_ref.reshape(K // 128, N)[kb]).astype(np.float32)
    s = (prod.astype(np.float32) * scale).astype(np.float32)
    ref = O.epilogue_from_raw(s, svh, OUT_SCALE)
    assert np.array_equal(c.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("coarse", [False, True])
def test_two_part_repeat_and_row_order(coarse):
    banner("ti8 parts", coarse)
    K, N, KB = 1024, 512, 4
    words, _ = _weights(K, N, KB, 31)
    w_d = dev(words)
    sw = api.trellis_i8_table(w_d, K, N, KB, coarse)
    svh = dev(WL.svh_scales(N, 32))
    x0, x1 = WL.activations_f16(256, K, 33), WL.activations_f16(256, K, 34)
    a0, s0 = _gpu_a(x0, coarse)
    a1, s1 = _gpu_a(x1, coarse)
    run = lambda a, s, **kw: api.trellis_gemm_i8(a, s, w_d, sw, svh, K, N, KB, coarse=coarse, skg=2, **kw)
    c0, c1 = run(a0, s0), run(a1, s1)
    for n_split in (128, 256, 384):
        c = run(a0, s0, a8_1=a1, sa_1=s1, n_split=n_split)
        torch.cuda.synchronize()
        assert torch.equal(c[:, :n_split].view(torch.int16), c0[:, :n_split].view(torch.int16))
        assert torch.equal(c[:, n_split:].view(torch.int16), c1[:, n_split:].view(torch.int16))
    for _ in range(2):
        assert torch.equal(run(a0, s0).view(torch.int16), c0.view(torch.int16))
    perm = np.random.default_rng(35).permutation(256)
    ap, sp = _gpu_a(np.ascontiguousarray(x0[perm]), coarse)
    cp = run(ap, sp)
    torch.cuda.synchronize()
    assert torch.equal(cp.view(torch.int16), c0[torch.from_numpy(perm).to(c0.device)].view(torch.int16))
