"""GPU parity of the int8 path (activation quantizers, the dense int8 x int8 GEMM) through the C ABI.
M = 256, (K, N) = (5120, 17408) and (17408, 5120), Student-t activations.

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
def test_quantizers_bit_exact(blk, ref_layout):
    banner("i8 quant", blk, ref_layout)
    K = 5120
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


@pytest.mark.parametrize("K,N,skg", [(512, 256, 1), (1024, 384, 2), (2048, 128, 4), (640, 512, 5)])
def test_dense_int32_exact(K, N, skg):
    banner("i8 raw", K, N, skg)
    rng = np.random.default_rng(K + N)
    a = rng.integers(-127, 128, (256, K)).astype(np.int8)
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    c = api.i8_dense_gemm(dev(a), None, dev(w), None, K, N, skg=skg, raw=True)
    torch.cuda.synchronize()
    ref = np.empty((256, N), np.int32)
    O.lib().r4o_i8_gemm_i32(ptr(a), ptr(w), 256, N, K, ptr(ref), 0)
    assert np.array_equal(c.cpu().numpy(), ref)


@pytest.mark.parametrize("blk", [False, True])
@pytest.mark.parametrize("K,N,skg", [(1024, 256, 1), (2048, 384, 2)])
def test_dense_scaled(blk, K, N, skg):
    banner("i8 dense", blk, K, N, skg)
    x, w8, sw = WL.int8_case(K, N, 7)
    a8, sa = api.i8_quant(dev(x.view(np.uint16)), blk)
    c = api.i8_dense_gemm(a8, sa, dev(w8), dev(sw), K, N, scale_blk=blk, skg=skg)
    torch.cuda.synchronize()
    sa_ref, ap = _oracle_quant(x, blk)
    ref = np.empty((256, N), np.float64)
    O.lib().r4o_i8_gemm_ref(ptr(ap), ptr(sa_ref), ptr(w8), ptr(sw), 256, N, K, 2 if blk else 3, ptr(ref), 0)
    assert close_rel(c.float().cpu().numpy(), ref, 1e-3, 1e-4) <= 1.0


@pytest.mark.parametrize("K,N", [(5120, 17408), (17408, 5120)])
def test_config4(K, N):
    """Both config-4 shapes: int32 accumulators exact, f16 outputs within tolerance for both scale
    variants."""
    x, w8, sw = WL.int8_case(K, N, 11)
    w_d = dev(w8)
    for blk in (False, True):
        banner("config4", K, N, blk)
        a8, sa = api.i8_quant(dev(x.view(np.uint16)), blk)
        c = api.i8_dense_gemm(a8, sa, w_d, dev(sw), K, N, scale_blk=blk)
        raw = api.i8_dense_gemm(a8, None, w_d, None, K, N, raw=True) if not blk else None
        torch.cuda.synchronize()
        sa_ref, ap = _oracle_quant(x, blk)
        assert np.array_equal(a8.cpu().numpy().reshape(256, K), ap)
        if raw is not None:
            ref_i = np.empty((256, N), np.int32)
            O.lib().r4o_i8_gemm_i32(ptr(ap), ptr(w8), 256, N, K, ptr(ref_i), 0)
            assert np.array_equal(raw.cpu().numpy(), ref_i)
        ref = np.empty((256, N), np.float64)
        O.lib().r4o_i8_gemm_ref(ptr(ap), ptr(sa_ref), ptr(w8), ptr(sw), 256, N, K, 2 if blk else 3, ptr(ref), 0)
        assert close_rel(c.float().cpu().numpy(), ref, 1e-3, 1e-4) <= 1.0
