"""Robustness of the split GEMV's handoff and of its legality rules, on the GPU, through the C ABI.

* Ticket recovery (third_party/libr4d/r4d.h:365-371): a ticket buffer left non-zero (what a launch that never
  completed leaves) is reset by r4d_gemm_trellis_nt_m64_zero_tickets, after which a split launch is bit-exact
  with a launch on a fresh buffer. No launch ever runs on the poisoned buffer (the kernel never waits on a
  ticket, so nothing could hang either way).
* Long repeats (tests/kernels/test_trellis_gemm.cpp's determinism and "rows >= M untouched" checks): 100 launches
  in a row on one ticket buffer at a config-1 shape are bit-identical, the tickets end at zero, and the rows of C
  past M keep their sentinel.
* Config-1 shapes at the verify batches M = 2 and 4, against the fp64 oracle.
* The fused transform at M = 64 on a slice its _check accepts (the check now bounds the whole LDS request).
"""
import numpy as np
import pytest

import oracle_lib as O
from r4dx_amd import workloads as WL

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no GPU", allow_module_level=True)

from r4dx_amd import api  # noqa: E402
from r4dx_amd.loader import lib  # noqa: E402
from gpu_util import banner, close_rel, dev, host_u16  # noqa: E402

OSC = float(np.float32(1.0 / np.sqrt(128.0)))


@pytest.mark.parametrize("K,N,M,skg", [(5120, 6144, 1, 2), (17408, 5120, 8, 8), (6144, 5120, 4, 4)])
def test_zero_tickets_recovers_a_poisoned_buffer(K, N, M, skg):
    banner("zero_tickets", K, N, M, skg)
    words, _, svh = WL.trellis_linear(K, N, 4, 21)
    a = dev(WL.activations_f16(M, K, 22).view(np.uint16))
    w_d, svh_d = dev(words), dev(svh)
    ref = host_u16(api.trellis_gemm_m64(a, w_d, svh_d, K, N, 4, skg=skg, out_scale=OSC))
    tk = api.TicketBuffer(N).t
    nbytes = lib().r4d_gemm_trellis_nt_m64_tickets_bytes(N)
    assert tk.numel() * 4 == nbytes == (N // 128) * 128
    tk.copy_(torch.randint(1, 1 << 20, tk.shape, dtype=torch.int32, device="cuda"))
    lib().r4d_gemm_trellis_nt_m64_zero_tickets(tk.data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert int(tk.abs().sum()) == 0
    got = host_u16(api.trellis_gemm_m64(a, w_d, svh_d, K, N, 4, skg=skg, out_scale=OSC, tickets=tk))
    torch.cuda.synchronize()
    assert np.array_equal(got, ref)
    assert int(tk.abs().sum()) == 0


def test_hundred_repeats_bit_identical_rows_past_m_untouched():
    banner("repeat100")
    K, N, KB, M = 5120, 6144, 4, 4
    words, _, svh = WL.trellis_linear(K, N, KB, 31)
    a = dev(WL.activations_f16(M, K, 32).view(np.uint16))
    w_d, svh_d = dev(words), dev(svh)
    skg = api.trellis_gemv_skg(K, N, KB)
    tk = api.TicketBuffer(N).t
    ws = torch.empty(lib().r4d_gemm_trellis_nt_m64_ws_bytes(M, N, skg) // 4, dtype=torch.float32, device="cuda")
    big = torch.full((M + 3, N), 0x7F7B, dtype=torch.int16, device="cuda")   # a bf16 sentinel past row M
    out = big[:M].view(torch.bfloat16)
    first = None
    for i in range(100):
        api.trellis_gemm_m64(a, w_d, svh_d, K, N, KB, skg=skg, out_scale=OSC, out=out, ws=ws, tickets=tk)
        if i == 0:
            torch.cuda.synchronize()
            first = host_u16(out)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(out), first)
    assert int(tk.abs().sum()) == 0
    assert bool((big[M:] == 0x7F7B).all())


@pytest.mark.parametrize("name,K,N", WL.LAYER_SHAPES)
def test_config1_shapes_m2_m4(name, K, N):
    """Config 1's verify batches M = 2 and 4 at every projection, KB 4 and 5, against the fp64 oracle; the bf16
    output equals the oracle's epilogue of the kernel's own sums."""
    for KB in (4, 5):
        banner("config1 m2/m4", name, K, N, KB)
        words, _, svh = WL.trellis_linear(K, N, KB, (hash(name) + 3) % 1000)
        a = WL.activations_f16(4, K, 41).view(np.uint16)
        q = O.decode_pair_grid(words, K, N, KB)
        ref = O.raw_sums(a, q)
        w_d, svh_d = dev(words), dev(svh)
        for M in (2, 4):
            raw = api.trellis_gemm_m64(dev(a[:M]), w_d, None, K, N, KB, raw=True)
            full = api.trellis_gemm_m64(dev(a[:M]), w_d, svh_d, K, N, KB, out_scale=OSC)
            torch.cuda.synchronize()
            raw_h = raw.cpu().numpy()
            assert close_rel(raw_h, ref[:M], 1e-3, 1e-4) <= 1.0, (KB, M)
            assert np.array_equal(host_u16(full), O.epilogue_from_raw(raw_h, svh, OSC)), (KB, M)


def test_fused_transform_at_m64():
    """The largest M the fused-transform check accepts at K = 5120 runs and equals the two-launch path."""
    banner("xf m64")
    K, N, KB, M = 5120, 1024, 4, 64
    L = lib()
    skg = next(s for s in (1, 2, 4, 8, 16, 20, 40) if not L.r4dx_trellis_gemv_xf_check(M, K, N, N, KB, s, 1))
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to("cuda").half().view(torch.int16)
    suh = dev(WL.signs(K, 8))
    words, svh = dev(WL.trellis_words(K, N, KB, 7)), dev(WL.svh_scales(N, 10))
    (a0,) = api.trellis_input(x, [suh], 0, bf16=False)
    ref = api.trellis_gemm_m64(a0, words, svh, K, N, KB, skg=skg, out_scale=OSC)
    got = api.trellis_gemv_xf(x, suh, words, svh, K, N, KB, skg=skg, out_scale=OSC)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
