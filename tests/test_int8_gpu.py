"""GPU parity of the int8 path (activation quantizers, the dense int8 x int8 GEMM) through the C ABI.
The int8 prefill workload (config 4): M = 256, (K, N) = (5120, 17408) and (17408, 5120), Student-t activations.

Bars: quantized bytes and scales bit-exact; int32 accumulators exact; f16 outputs within 1e-3 relative
error with a 1e-4 * rms(row) floor of the oracle's fp64 RefGemmInt8 (int8_gemm_proto_ref.h:95-110)."""
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


def _oracle_quant(x, blk):
    M, K = x.shape
    sa = np.empty((K // 128) * M if blk else M, np.float32)
    ap = np.empty((M, K), np.int8)
    f = O.lib().r4o_i8_quant_act_blk if blk else O.lib().r4o_i8_quant_act_row
    f(ptr(x.view(np.uint16)), M, K, ptr(sa), ptr(ap))
    return sa, ap


@pytest.mark.parametrize("blk", [False, True])
@pytest.mark.parametrize("ref_layout", [False, True])
@pytest.mark.parametrize("K", [5120, 1152, 17408])   # 1152: a row shorter than one pass of the row kernel
def test_quantizers_bit_exact(blk, ref_layout, K):
    banner("i8 quant", blk, ref_layout, K)
    x, _, _ = WL.int8_case(K, 128, 1)
    x[3, :] = 0                      # an all-zero row: scale 1
    x[5, 256:384] = 0                # an all-zero block
    a8, sa = api.i8_quant(dev(x.view(np.uint16)), blk, ref_layout)
    torch.cuda.synchronize()
    sa_ref, ap = _oracle_quant(x, blk)
    assert np.array_equal(sa.cpu().numpy(), sa_ref)
    got = a8.cpu().numpy()
    if ref_layout:
        ref = np.empty(256 * K, np.int8)
        O.lib().r4o_pack_a8(ptr(ap), K, ptr(ref))
        assert np.array_equal(got, ref)
    else:
        assert np.array_equal(got.reshape(256, K), ap)


def _a8(ap):
    out = np.empty(ap.size, np.int8)
    O.lib().r4o_pack_a8(ptr(ap), ap.shape[1], ptr(out))
    return out


def test_pack_w_matches_oracle():
    banner("i8 pack_w")
    rng = np.random.default_rng(3)
    N, K = 96, 384
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    got = api.i8_pack_w(dev(w)).cpu().numpy()
    ref = np.empty(N * K, np.int8)
    O.lib().r4o_pack_w8(ptr(w), N, K, ptr(ref))
    assert np.array_equal(got, ref)


def _i32_ref(a, w):
    ref = np.empty((256, w.shape[0]), np.int32)
    O.lib().r4o_i8_gemm_i32(ptr(a), ptr(w), 256, w.shape[0], a.shape[1], ptr(ref), 0)
    return ref


@pytest.mark.parametrize("K,N,skg", [(128, 128, 1), (512, 256, 1), (1024, 384, 2), (2048, 128, 4), (640, 512, 5),
                                     (384, 256, 3), (128, 128, 0), (1024, 384, 0), (640, 512, 0), (5120, 1280, 0),
                                     (2048, 4352, 0)])
def test_dense_int32_exact(K, N, skg):
    """skg = 0 is stream-K: 256 workgroups share the (group, 128-k block) units, so groups split into pieces
    at any block and workgroups span group boundaries; the int32 sums stay exact."""
    banner("i8 raw", K, N, skg)
    rng = np.random.default_rng(K + N)
    a = rng.integers(-127, 128, (256, K)).astype(np.int8)
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    w8 = api.i8_pack_w(dev(w))
    work = api.I8Workspace(N, skg, w8.device)
    for _ in range(2):       # the tickets reset themselves: a second launch on the same workspace
        c = api.i8_dense_gemm(dev(_a8(a)), None, w8, None, K, N, skg=skg, raw=True, work=work)
        torch.cuda.synchronize()
        assert np.array_equal(c.cpu().numpy(), _i32_ref(a, w))
    assert int(work.tickets.abs().sum()) == 0


def test_dense_int32_extremes():
    """Saturated operands: |sum| up to K 127^2 (K = 17408: 2.8e8 < 2^31), every sign combination."""
    K, N = 17408, 128
    a = np.full((256, K), 127, np.int8)
    a[1::2] = -127
    w = np.full((N, K), 127, np.int8)
    w[::3] = -127
    w[5, ::2] = 0
    c = api.i8_dense_gemm(dev(_a8(a)), None, api.i8_pack_w(dev(w)), None, K, N, skg=4, raw=True)
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), _i32_ref(a, w))


def _oracle_mode(x, w8, sw, mode):
    """The oracle's f64 result for scale mode 0 (row x column), 1 (per-128 activation x column) or 2 (per-128
    both: sw is [K/128][N])."""
    blk = mode != 0
    sa_ref, ap = _oracle_quant(x, blk)
    ref = np.empty((256, w8.shape[0]), np.float64)
    mask = {0: 3, 1: 2, 2: 0}[mode]
    O.lib().r4o_i8_gemm_ref(ptr(ap), ptr(sa_ref), ptr(w8), ptr(sw), 256, w8.shape[0], x.shape[1], mask, ptr(ref), 0)
    return ref


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("K,N,skg", [(1024, 256, 1), (2048, 384, 2), (1536, 128, 3), (2048, 384, 0), (5120, 2176, 0)])
def test_dense_scaled(mode, K, N, skg):
    banner("i8 dense", mode, K, N, skg)
    x, w8, sw = WL.int8_case(K, N, 7)
    if mode == 2:
        sw = np.random.default_rng(8).lognormal(np.log(0.01), 0.3, (K // 128, N)).astype(np.float32)
    a8, sa = api.i8_quant(dev(x.view(np.uint16)), mode != 0)
    c = api.i8_dense_gemm(a8, sa, api.i8_pack_w(dev(w8)), dev(sw.reshape(-1)), K, N, scale_mode=mode, skg=skg)
    torch.cuda.synchronize()
    assert close_rel(c.float().cpu().numpy(), _oracle_mode(x, w8, sw, mode), 1e-3, 1e-4) <= 1.0


def test_dense_stream_repeat_identical():
    """Stream-K, per-128 scales (fp32 pieces): the pieces are added in a fixed order, so repeats are byte-identical."""
    K, N = 5120, 2176
    x, w8, sw = WL.int8_case(K, N, 9)
    a8, sa = api.i8_quant(dev(x.view(np.uint16)), True)
    w_d, sw_d = api.i8_pack_w(dev(w8)), dev(sw)
    work = api.I8Workspace(N, 0, w_d.device)
    c0 = api.i8_dense_gemm(a8, sa, w_d, sw_d, K, N, scale_mode=1, skg=0, work=work)
    for _ in range(3):
        c = api.i8_dense_gemm(a8, sa, w_d, sw_d, K, N, scale_mode=1, skg=0, work=work)
        torch.cuda.synchronize()
        assert torch.equal(c.view(torch.int16), c0.view(torch.int16))


@pytest.mark.parametrize("K,N", [(5120, 17408), (17408, 5120)])
def test_config4(K, N):
    """Both config-4 shapes at the planner's split: the quantized bytes exact, the int32 accumulators exact,
    the f16 outputs within tolerance for the row and the per-128 activation scales."""
    x, w8, sw = WL.int8_case(K, N, 11)
    w_d = api.i8_pack_w(dev(w8))
    x_d = dev(x.view(np.uint16))
    raw = api.i8_dense_gemm(api.i8_quant(x_d, False)[0], None, w_d, None, K, N, raw=True)
    torch.cuda.synchronize()
    _, ap = _oracle_quant(x, False)
    assert np.array_equal(raw.cpu().numpy(), _i32_ref(ap, w8))
    for mode in (0, 1):
        banner("config4", K, N, mode)
        a8, sa = api.i8_quant(x_d, mode != 0)
        c = api.i8_dense_gemm(a8, sa, w_d, dev(sw), K, N, scale_mode=mode)
        torch.cuda.synchronize()
        assert close_rel(c.float().cpu().numpy(), _oracle_mode(x, w8, sw, mode), 1e-3, 1e-4) <= 1.0


@pytest.mark.parametrize("row_scale", [False, True])
@pytest.mark.parametrize("K,nout,prescale", [(5120, 1, 0), (17408, 1, 3), (1024, 2, -4), (2048, 3, 0),
                                              (1152, 2, 1)])   # 9 blocks: a partial group of the per-128 form
def test_fused_transform_quantizer_bit_exact(row_scale, K, nout, prescale):
    """r4dx_trellis_input_i8(r) == r4dx_trellis_input_bf16 then r4d_trellis_i8_quant_act(_row), byte for byte."""
    banner("xq", row_scale, K, nout, prescale)
    rng = np.random.default_rng(K + nout)
    x = torch.from_numpy(rng.standard_t(4, (256, K)).astype(np.float32)).to("cuda").to(torch.bfloat16).view(torch.int16)
    suh = [dev(WL.signs(K, 40 + o)) for o in range(nout)]
    got = api.trellis_input_i8(x, suh, prescale, row_scale)
    outs = api.trellis_input(x, suh, prescale, bf16=True)
    torch.cuda.synchronize()
    for o in range(nout):
        a8, sa = api.i8_quant(outs[o], blk=not row_scale, ref_layout=True)
        torch.cuda.synchronize()
        assert torch.equal(got[o][1].view(torch.int32), sa.view(torch.int32)), \
            (o, int((got[o][1] != sa).sum()), got[o][1][:4].tolist(), sa[:4].tolist())
        assert torch.equal(got[o][0], a8), (o, int((got[o][0] != a8).sum()))
