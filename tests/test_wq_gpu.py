"""GPU parity of the weight fake-quant entries (r4d.h:425-454): r4d_trellis_wscale_f32, r4d_gemm_trellis_nt_m64_wq /
_raw_wq and r4d_gemm_trellis_nt_m256_wq, through the C ABI, against the oracle's restatement of
src/model/fake_quant_w.h (itself pinned bit for bit to that header in tests/test_oracle_vs_ref.py).

The cases follow the reference's tests/kernels/test_fake_quant_w.cpp:
  A  the scale table bit for bit against the oracle's table of the oracle's decode;
  B  one-hot A rows through _raw_wq return rows of the rounded weight Q' bit for bit (a single non-zero product
     per fp32 sum), unsplit and split, one A part and two, K with an odd k-step count;
  C  the M = 256 form equals four 64-row M = 64 launches at SK = 1 and the same SKG byte for byte, and differs
     from the stock kernel (so the comparison sees the rounding);
  D  _wq's bf16 output equals the oracle epilogue of the _raw_wq sums bit for bit, and the sums agree with an fp64
     matmul against Q' within 1e-3 relative (1e-4 rms floor)."""
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

ONE_F16 = 0x3C00


@pytest.mark.parametrize("KB", [4, 5])
@pytest.mark.parametrize("K", [1024, 1152])
@pytest.mark.parametrize("gsh", [1, 2, 3])
def test_wscale_table_exact(KB, K, gsh):
    banner("wscale", KB, K, gsh)
    N = 512
    words = WL.trellis_words(K, N, KB, 100 * KB + K + gsh)
    t = api.trellis_wscale(dev(words), K, N, KB, gsh)
    torch.cuda.synchronize()
    q = O.decode_pair_grid(words, K, N, KB)
    want = O.wq_table(q, 16 << gsh)
    assert np.array_equal(t.cpu().numpy().view(np.uint32), want.ravel().view(np.uint32))


def _one_hot(M, K, ks):
    a = np.zeros((M, K), np.uint16)
    a[np.arange(M), ks] = ONE_F16
    return a


@pytest.mark.parametrize("KB,K,skg,sk,M,two", [
    (4, 1024, 1, 0, 64, False), (4, 1024, 2, 0, 16, True), (5, 1152, 1, 1, 64, True),
    (5, 1152, 3, 0, 32, False), (4, 1152, 2, 1, 64, False), (5, 1024, 4, 0, 1, True),
])
@pytest.mark.parametrize("gsh", [1, 3])
def test_raw_wq_one_hot_rows(KB, K, skg, sk, M, two, gsh):
    banner("raw_wq one-hot", KB, K, skg, sk, M, two, gsh)
    N = 512
    words = WL.trellis_words(K, N, KB, 7 * K + KB)
    w_d = dev(words)
    tab = api.trellis_wscale(w_d, K, N, KB, gsh)
    q = O.decode_pair_grid(words, K, N, KB)
    qq = O.wq_apply(q, 16 << gsh)
    qqf = O.f16_bits_to_f32(qq)
    ns = N // 2 if two else N
    ws = torch.empty(api.lib().r4d_gemm_trellis_nt_m64_ws_bytes(M, N, skg) // 4, dtype=torch.float32,
                     device="cuda") if skg > 1 else None
    tk = api.TicketBuffer(N).t
    step = M if M > 1 else 97
    for kb in range(0, K, step):
        k0 = (kb + np.arange(M)) % K
        k1 = (kb + np.arange(M) + K // 2 + 5) % K
        a0, a1 = dev(_one_hot(M, K, k0)), dev(_one_hot(M, K, k1))
        c = api.trellis_gemm_m64(a0, w_d, None, K, N, KB, skg=skg, a1=a1 if two else None, n_split=ns,
                                 raw=True, sk=sk, ws=ws, tickets=tk, wq=(tab, gsh))
        torch.cuda.synchronize()
        got = c.cpu().numpy()
        want = qqf[k0].copy()
        if two:
            want[:, ns:] = qqf[k1][:, ns:]
        assert np.array_equal(got, want), kb
    if skg > 1:
        assert not tk.any().item()


CLASSES = [  # (name, K, N, n_split): the model's trellis classes, N cut so the oracle stays quick where it is used
    ("attn.k/attn.v", 5120, 1024, 1024),
    ("mlp.gate_up (cut)", 5120, 2048, 1024),
    ("mlp.down (cut)", 17408, 256, 256),
]


@pytest.mark.parametrize("name,K,N,ns", CLASSES)
@pytest.mark.parametrize("KB", [4, 5])
@pytest.mark.parametrize("gsh", [1, 3])
def test_m256_wq_equals_m64_wq_rows(name, K, N, ns, KB, gsh):
    banner("m256_wq == m64_wq", name, K, N, KB, gsh)
    M = 256
    skg = api.trellis_m256_skg(K, N, KB)
    words, _, svh = WL.trellis_linear(K, N, KB, K + N + KB)
    a = WL.activations_f16(M, K, 21, outlier_frac=0.01).view(np.uint16)
    a1 = WL.activations_f16(M, K, 22).view(np.uint16)
    w_d, a_d, a1_d, s_d = dev(words), dev(a), dev(a1), dev(svh)
    two = ns < N
    osc = float(np.float32(1.0 / np.sqrt(128.0)))
    tab = api.trellis_wscale(w_d, K, N, KB, gsh)
    big = api.trellis_gemm_m256(a_d, w_d, s_d, K, N, KB, skg=skg, a1=a1_d if two else None, n_split=ns,
                                out_scale=osc, wq=(tab, gsh))
    big2 = api.trellis_gemm_m256(a_d, w_d, s_d, K, N, KB, skg=skg, a1=a1_d if two else None, n_split=ns,
                                 out_scale=osc, wq=(tab, gsh))
    stock = api.trellis_gemm_m256(a_d, w_d, s_d, K, N, KB, skg=skg, a1=a1_d if two else None, n_split=ns,
                                  out_scale=osc)
    torch.cuda.synchronize()
    assert torch.equal(big.view(torch.int16), big2.view(torch.int16))
    assert not torch.equal(big.view(torch.int16), stock.view(torch.int16))
    for r0 in range(0, M, 64):
        sl = slice(r0, r0 + 64)
        small = api.trellis_gemm_m64(a_d[sl].contiguous(), w_d, s_d, K, N, KB, skg=skg,
                                     a1=a1_d[sl].contiguous() if two else None, n_split=ns, out_scale=osc,
                                     sk=1, wq=(tab, gsh))
        torch.cuda.synchronize()
        assert torch.equal(big[sl].view(torch.int16), small.view(torch.int16)), r0


@pytest.mark.parametrize("M,K,N,KB,skg,gsh", [
    (1, 1024, 512, 4, None, 3), (8, 2048, 256, 5, 2, 1), (64, 1152, 384, 4, 1, 2), (33, 5120, 256, 5, None, 3),
])
def test_wq_linear_vs_oracle(M, K, N, KB, skg, gsh):
    banner("wq linear", M, K, N, KB, skg, gsh)
    skg = api.trellis_gemv_skg(K, N, KB) if skg is None else skg
    words, _, svh = WL.trellis_linear(K, N, KB, 5 * K + M)
    a = WL.activations_f16(M, K, 31, outlier_frac=0.01).view(np.uint16)
    w_d, a_d = dev(words), dev(a)
    tab = api.trellis_wscale(w_d, K, N, KB, gsh)
    osc = np.float32(1.0 / np.sqrt(128.0))
    raw = api.trellis_gemm_m64(a_d, w_d, None, K, N, KB, skg=skg, raw=True, wq=(tab, gsh))
    full = api.trellis_gemm_m64(a_d, w_d, dev(svh), K, N, KB, skg=skg, out_scale=float(osc), wq=(tab, gsh))
    torch.cuda.synchronize()
    qq = O.wq_apply(O.decode_pair_grid(words, K, N, KB), 16 << gsh)
    raw_h = raw.cpu().numpy()
    assert close_rel(raw_h, O.raw_sums(a, qq), 1e-3, 1e-4) <= 1.0
    assert np.array_equal(host_u16(full), O.epilogue_from_raw(raw_h, svh, osc))
