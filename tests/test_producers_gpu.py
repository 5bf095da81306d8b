"""GPU parity of the activation producers fused into the trellis input transform (kernels.h:130-179:
r4dx_silu_mul_trellis_bf16 / _i8 / _i8r, r4dx_attn_gate_mul_trellis_bf16 / _i8 / _i8r) and of the producers
alone (r4dx_silu_mul_wide_bf16, r4dx_model_attn_gate_mul_bf16), through the C ABI.

Bars, as the reference's tests/kernels/test_trellis_input.cpp:17-20 and test_trellis_input_i8.cpp: every fused
entry is byte-identical to its two-launch form (the producer, then r4dx_trellis_input_bf16 / _i8 / _i8r) --
the TP = 1 and TP = 2 widths, M up to 64, prescale 0 / 4 / -3, inputs that saturate the sigmoid. The producers
against the CPU oracle: within one bf16 ulp everywhere (the device library's expf and the host's may differ by an
ulp, which can flip a bf16 rounding); the fused entries' f16 A bit-identical to the oracle's transform of the
device producer's values."""
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
from gpu_util import banner, dev  # noqa: E402


def _bf16_case(shape, seed, scale=3.0):
    """bf16 bits ~ N(0, scale) with saturating values (+-100, +-1e4) sprinkled in."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0, scale, shape).astype(np.float32)
    flat = x.reshape(-1)
    idx = rng.choice(flat.size, max(1, flat.size // 200), replace=False)
    flat[idx] = rng.choice([100.0, -100.0, 1e4, -1e4], idx.size)
    return O.f32_to_bf16_bits(x)


def _u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("I,M", [(17408, 1), (8704, 5), (1024, 64)])
@pytest.mark.parametrize("prescale", [0, 4, -3])
def test_silu_mul_trellis_bytes(I, M, prescale):
    banner("silu trellis", I, M, prescale)
    gu = dev(_bf16_case((M, 2 * I), I + M))
    suh = dev(WL.signs(I, 3))
    fused = api.silu_mul_trellis(gu, I, suh, prescale)
    h = api.silu_mul(gu, I)
    two = api.trellis_input(h, [suh], prescale)[0]
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), two.view(torch.int16))


@pytest.mark.parametrize("K,M", [(6144, 1), (3072, 7), (6144, 64)])
@pytest.mark.parametrize("prescale", [0, 4, -3])
def test_attn_gate_mul_trellis_bytes(K, M, prescale):
    banner("gate trellis", K, M, prescale)
    a = dev(_bf16_case((M, K), K + M, 2.0))
    g = dev(_bf16_case((M, K), K + M + 1, 4.0))
    suh = dev(WL.signs(K, 4))
    fused = api.attn_gate_mul_trellis(a, g, suh, prescale)
    two = api.trellis_input(api.attn_gate_mul(a, g), [suh], prescale)[0]
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), two.view(torch.int16))


def test_silu_row_stride_and_empty():
    """gate_up rows padded past 2 I (the stride is honoured) and rows = 0 (nothing is written)."""
    banner("silu stride")
    I, M, stride = 1024, 3, 2 * 1024 + 256
    gu = dev(_bf16_case((M, stride), 11))
    suh = dev(WL.signs(I, 5))
    fused = api.silu_mul_trellis(gu, I, suh)
    h = api.silu_mul(gu, I)
    torch.cuda.synchronize()
    ref = np.empty((M, I), np.uint16)
    O.lib().r4o_silu_mul_bf16(ptr(_u16(gu)), M, I, stride, ptr(ref))
    assert np.array_equal(_u16(h), ref) or np.max(np.abs(_u16(h).astype(np.int32) - ref.astype(np.int32))) <= 1
    two = api.trellis_input(h, [suh])[0]
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), two.view(torch.int16))
    # rows = 0 with valid pointers is a no-op (a null gate_up throws even then, as in the reference)
    out = torch.full((1, I), 7, dtype=torch.int16, device="cuda")
    api.lib().r4dx_silu_mul_trellis_bf16(gu.data_ptr(), 0, I, stride, suh.data_ptr(), out.data_ptr(), 0,
                                         torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert bool((out == 7).all())


@pytest.mark.parametrize("quant", ["blk", "row"])
@pytest.mark.parametrize("I", [17408, 5120])
def test_silu_mul_trellis_i8_bytes(quant, I):
    banner("silu i8", quant, I)
    gu = dev(_bf16_case((256, 2 * I), I + 1))
    suh = dev(WL.signs(I, 6))
    a8, sa = api.silu_mul_trellis(gu, I, suh, 0, quant=quant)
    (a8r, sar), = api.trellis_input_i8(api.silu_mul(gu, I), [suh], 0, row_scale=quant == "row")
    torch.cuda.synchronize()
    assert torch.equal(a8, a8r) and torch.equal(sa.view(torch.int32), sar.view(torch.int32))


@pytest.mark.parametrize("quant", ["blk", "row"])
def test_attn_gate_mul_trellis_i8_bytes(quant):
    banner("gate i8", quant)
    K = 6144
    a = dev(_bf16_case((256, K), 21, 2.0))
    g = dev(_bf16_case((256, K), 22, 4.0))
    suh = dev(WL.signs(K, 7))
    a8, sa = api.attn_gate_mul_trellis(a, g, suh, 4, quant=quant)
    (a8r, sar), = api.trellis_input_i8(api.attn_gate_mul(a, g), [suh], 4, row_scale=quant == "row")
    torch.cuda.synchronize()
    assert torch.equal(a8, a8r) and torch.equal(sa.view(torch.int32), sar.view(torch.int32))


def test_producers_vs_oracle():
    """The producers alone against the CPU oracle (within one bf16 ulp, nearly all bit-equal), and the fused
    entries' f16 A against the oracle's transform of the device producer's values (bit for bit)."""
    banner("producers oracle")
    I, M = 5120, 4
    gu_h = _bf16_case((M, 2 * I), 31)
    h = api.silu_mul(dev(gu_h), I)
    a_h, g_h = _bf16_case((M, I), 32, 2.0), _bf16_case((M, I), 33, 4.0)
    hg = api.attn_gate_mul(dev(a_h), dev(g_h))
    suh = WL.signs(I, 8)
    fs = api.silu_mul_trellis(dev(gu_h), I, dev(suh), 0)
    fg = api.attn_gate_mul_trellis(dev(a_h), dev(g_h), dev(suh), 0)
    torch.cuda.synchronize()
    ref_s = np.empty((M, I), np.uint16)
    O.lib().r4o_silu_mul_bf16(ptr(gu_h), M, I, 2 * I, ptr(ref_s))
    ref_g = np.empty((M, I), np.uint16)
    O.lib().r4o_attn_gate_mul_bf16(ptr(a_h), ptr(g_h), M * I, ptr(ref_g))
    for got, ref in ((_u16(h), ref_s), (_u16(hg), ref_g)):
        d = np.abs(got.astype(np.int32) - ref.astype(np.int32))
        # one bf16 ulp apart at most (adjacent bit patterns of the same sign; +-0 compare equal)
        same_val = O.bf16_bits_to_f32(got) == O.bf16_bits_to_f32(ref)
        assert np.all(same_val | (d <= 1)), int(d.max())
        assert np.mean(same_val) > 0.999
    # the fused entries' f16 A is the oracle's transform of the device producer's bf16 values, bit for bit
    for fused, hdev in ((fs, h), (fg, hg)):
        assert np.array_equal(_u16(fused), O.transform_input(_u16(hdev), True, suh, 0))
