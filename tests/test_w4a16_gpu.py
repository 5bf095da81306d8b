"""GPU parity of the w4a16 group-quantized GEMM (r4d_gemm_w4a16_nt_m64, _g, _f32) and the argmax entries
through the C ABI, against the CPU oracle.  The LM-head workload (config 3): N = 248 320 (vocab), K = 5120, groups of
32 and 64, M in {1, 8}.

Bars: fp32 logits within 1e-3 relative error with a 1e-4 * rms(row) floor of the oracle's fp64
dequantize-and-multiply; bf16 C bit-exact to the RNE rounding of the same kernel's fp32 logits; argmax
bit-exact (index and value) against the oracle's argmax order over the same logits, and equal to the
argmax of the fp64 reference logits."""
import ctypes as C
import os

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


def _ref(a_bits, wq, wsz, N, K, group, cols=None):
    """fp64 oracle logits [M][N] (or [M][len(cols)] for a column subset, re-packed per 16-row tile)."""
    M = a_bits.shape[0]
    if cols is None:
        y = np.empty((M, N), np.float64)
        O.lib().r4o_w4_gemm_ref(ptr(np.ascontiguousarray(a_bits)), ptr(wq), ptr(wsz), M, N, K, group, ptr(y), 0)
        return y
    # gather whole 16-row tiles holding the requested columns, then pick the columns
    tiles = np.unique(np.asarray(cols) // 16)
    kb = K // 64
    wq_t = wq.reshape(N // 16, kb * 2 * 16 * 4)[tiles].reshape(-1)
    wsz_t = wsz.reshape(N // 16, K // group * 16)[tiles].reshape(-1)
    ns = len(tiles) * 16
    y = np.empty((M, ns), np.float64)
    O.lib().r4o_w4_gemm_ref(ptr(np.ascontiguousarray(a_bits)), ptr(wq_t), ptr(wsz_t), M, ns, K, group, ptr(y), 0)
    pos = {t: i for i, t in enumerate(tiles)}
    idx = np.array([pos[c // 16] * 16 + c % 16 for c in cols])
    return y[:, idx]


def test_reference_fixture_g64():
    """The reference's committed packed bytes (tests/convert/fixtures/w4a16_*_g64.bin, N = 32, K = 256)."""
    banner("w4a16 fixture")
    g = os.path.join(O.ROOT, "tests", "golden")
    wq = np.fromfile(os.path.join(g, "w4a16_wq_g64.bin"), np.uint32)
    wsz = np.fromfile(os.path.join(g, "w4a16_wsz_g64.bin"), np.uint32)
    N, K = 32, 256
    a = WL.activations_f16(3, K, 1).view(np.uint16)
    c = api.w4a16_gemm(dev(a), dev(wq), dev(wsz), K, N, 64, f32=True)
    torch.cuda.synchronize()
    assert close_rel(c.cpu().numpy(), _ref(a, wq, wsz, N, K, 64), 1e-3, 1e-4) <= 1.0


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("M", [1, 3, 8, 16, 40])
def test_w4a16_random(group, M):
    banner("w4a16", group, M)
    N, K = 1024, 512
    wq, wsz = WL.w4a16_packed(N, K, group, 5 + M)
    a = WL.activations_f16(M, K, 6).view(np.uint16)
    a_d, wq_d, wsz_d = dev(a), dev(wq), dev(wsz)
    c32 = api.w4a16_gemm(a_d, wq_d, wsz_d, K, N, group, f32=True)
    cbf = api.w4a16_gemm(a_d, wq_d, wsz_d, K, N, group)
    torch.cuda.synchronize()
    got = c32.cpu().numpy()
    assert close_rel(got, _ref(a, wq, wsz, N, K, group), 1e-3, 1e-4) <= 1.0
    assert np.array_equal(cbf.view(torch.int16).cpu().numpy().view(np.uint16), O.f32_to_bf16_bits(got))


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("M,N,K", [(1, 16, 448), (5, 48, 320), (8, 512, 5120), (9, 80, 704), (33, 256, 5120),
                                   (64, 512, 5120), (64, 32, 8192)])
def test_w4a16_shapes(group, M, N, K):
    """Ragged shapes: one tile (spare waves), an odd tile count, K not a multiple of the prefetch depth,
    A staged in several LDS chunks (M = 8 and 64 at K = 5120 and 8192), both MFMA forms and both row-tile
    counts."""
    banner("w4a16 shape", group, M, N, K)
    wq, wsz = WL.w4a16_packed(N, K, group, 11 + M)
    a = WL.activations_f16(M, K, 12).view(np.uint16)
    c32 = api.w4a16_gemm(dev(a), dev(wq), dev(wsz), K, N, group, f32=True)
    torch.cuda.synchronize()
    assert close_rel(c32.cpu().numpy(), _ref(a, wq, wsz, N, K, group), 1e-3, 1e-4) <= 1.0


@pytest.mark.parametrize("group", [32, 64])
def test_config3_lm_head(group):
    """Full vocab: logits on a random subset of 4096 columns vs the fp64 oracle, argmax bit-exact vs the
    oracle's order over the kernel's logits."""
    N, K = 248320, 5120
    wq, wsz = WL.w4a16_packed(N, K, group, 77)
    a = WL.activations_f16(8, K, 78).view(np.uint16)
    wq_d, wsz_d = dev(wq), dev(wsz)
    cols = np.sort(np.random.default_rng(1).choice(N, 4096, replace=False))
    for M in (1, 8):
        banner("config3", group, M)
        c = api.w4a16_gemm(dev(a[:M]), wq_d, wsz_d, K, N, group, f32=True)
        idx, val = api.argmax_rows(c)
        torch.cuda.synchronize()
        logits = c.cpu().numpy()
        assert close_rel(logits[:, cols], _ref(a[:M], wq, wsz, N, K, group, cols), 1e-3, 1e-4) <= 1.0
        for m in range(M):
            v = C.c_float()
            i = O.lib().r4o_argmax_f32(ptr(logits[m]), N, C.byref(v))
            assert int(idx[m]) == i and float(val[m]) == v.value


@pytest.mark.parametrize("group", [32, 64])
def test_argmax_end_to_end(group):
    """A 16 384-entry vocab where the whole fp64 reference is affordable: the kernel's argmax equals the
    argmax of the fp64 reference logits (the top-2 gap is checked to exceed the error bound)."""
    banner("argmax e2e", group)
    N, K, M = 16384, 5120, 8
    wq, wsz = WL.w4a16_packed(N, K, group, 90)
    a = WL.activations_f16(M, K, 91).view(np.uint16)
    c = api.w4a16_gemm(dev(a), dev(wq), dev(wsz), K, N, group, f32=True)
    idx, _ = api.argmax_rows(c)
    torch.cuda.synchronize()
    ref = _ref(a, wq, wsz, N, K, group)
    for m in range(M):
        top2 = np.sort(ref[m])[-2:]
        bound = 2e-3 * np.abs(top2[1]) + 2e-4 * np.sqrt(np.mean(ref[m] ** 2))
        if top2[1] - top2[0] > bound:
            assert int(idx[m]) == int(np.argmax(ref[m]))


def test_argmax_order_cases():
    banner("argmax cases")
    rows = [
        [1, 3, 3, 2],
        [np.nan, 1, np.nan, 1],
        [-np.inf, np.nan, -np.inf, -np.inf],
        [np.nan, np.nan, np.nan, np.nan],
        [-0.0, 0.0, -1, -0.0],
        [np.inf, 5, np.inf, np.nan],
    ]
    x = np.array(rows, np.float32)
    idx, val = api.argmax_rows(dev(x))
    torch.cuda.synchronize()
    for m in range(len(rows)):
        v = C.c_float()
        i = O.lib().r4o_argmax_f32(ptr(np.ascontiguousarray(x[m])), x.shape[1], C.byref(v))
        assert int(idx[m]) == i, (m, rows[m])
        assert np.float32(val[m].item()).tobytes() == np.float32(v.value).tobytes() or (np.isinf(v.value) and val[m].item() == v.value)
    # large random rows with planted ties, and the bf16 entry
    rng = np.random.default_rng(4)
    big = rng.standard_normal((3, 300001)).astype(np.float32)
    big[0, [7, 250000]] = 9.0
    big[1, ::1000] = np.nan
    idx, val = api.argmax_rows(dev(big))
    torch.cuda.synchronize()
    for m in range(3):
        v = C.c_float()
        assert int(idx[m]) == O.lib().r4o_argmax_f32(ptr(big[m]), big.shape[1], C.byref(v))
    row = torch.from_numpy(big[2]).to(torch.bfloat16).cuda()
    i_b, v_b = api.argmax_rows(row.view(1, -1))
    torch.cuda.synchronize()
    wid = row.float().cpu().numpy()
    v = C.c_float()
    assert int(i_b[0]) == O.lib().r4o_argmax_f32(ptr(wid), wid.shape[0], C.byref(v))


def test_argmax_two_streams_and_long_rows():
    """Two argmax calls in flight on two streams of one device, on different rows, each against the oracle
    (every stream has its own partials and tickets); a vocab of 2 000 003 (more than one batch of 8 elements
    per thread in each of the 256 workgroups of a row) with its maximum in the last element, at 64 rows; and
    100 calls in a row on one stream (the tickets self-reset) giving the same answer each time."""
    banner("argmax streams")
    rng = np.random.default_rng(11)
    xa = rng.standard_normal((5, 248320)).astype(np.float32)
    xb = rng.standard_normal((7, 248320)).astype(np.float32)
    da, db = dev(xa), dev(xb)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for s in (s1, s2):   # the first call on each stream allocates its scratch
        with torch.cuda.stream(s):
            api.argmax_rows(da[:1])
    torch.cuda.synchronize()
    for _ in range(3):
        with torch.cuda.stream(s1):
            ia, va = api.argmax_rows(da)
        with torch.cuda.stream(s2):
            ib, vb = api.argmax_rows(db)
        torch.cuda.synchronize()
        for x, idx in ((xa, ia), (xb, ib)):
            for m in range(x.shape[0]):
                v = C.c_float()
                assert int(idx[m]) == O.lib().r4o_argmax_f32(ptr(x[m]), x.shape[1], C.byref(v))
    big = rng.standard_normal((64, 2000003)).astype(np.float32)
    big[:, -1] = 50.0
    big[3, 5] = 50.0   # a tie: the lower index wins
    idx, _ = api.argmax_rows(dev(big))
    torch.cuda.synchronize()
    want = np.full(64, 2000002)
    want[3] = 5
    assert np.array_equal(idx.cpu().numpy(), want)
    first = api.argmax_rows(da)[0].cpu().numpy()
    for _ in range(100):
        i, _v = api.argmax_rows(da)
    torch.cuda.synchronize()
    assert np.array_equal(i.cpu().numpy(), first)
