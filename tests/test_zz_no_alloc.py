"""r4dx_gemm_trellis_nt_m64_noalloc (the GEMV with its split-K partials and tickets in the library's own device
array) against r4d_gemm_trellis_nt_m64 with caller buffers, through the C ABI: two calls in a row, the second with
a smaller input, both byte-identical to the existing entry at the same (SK, SKG); its size rule refuses what the
array cannot hold; and a captured call replays byte-identically with eager calls between the replays."""
import ctypes as C

import numpy as np
import pytest

from r4dx_amd import workloads as WL

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no GPU", allow_module_level=True)

from r4dx_amd import api  # noqa: E402
from r4dx_amd.loader import lib  # noqa: E402
from gpu_util import banner, dev, host_u16  # noqa: E402

OSC = float(np.float32(1.0 / np.sqrt(128.0)))


def _entry():
    L = lib()
    return L, L.r4dx_gemm_trellis_nt_m64_noalloc, L.r4dx_gemm_trellis_nt_m64_noalloc_check


def _noalloc(f, ck, a, w, svh, K, N, KB, SK, SKG, out):
    M = a.shape[0]
    msg = ck(M, K, N, N, KB, SKG)
    assert msg is None, msg
    f(a.data_ptr(), 0, N, w.data_ptr(), svh.data_ptr(), out.data_ptr(), M, K, N, KB, SK, SKG, OSC,
      torch.cuda.current_stream().cuda_stream)


def test_noalloc_equals_caller_buffer_entry_two_calls():
    L, f, ck = _entry()
    # the last case fills the array: 8 slices x 64 rows x 8192 columns x 4 bytes = 16 MiB of partials
    cases = [(5120, 17408, 4, 8, 0, None), (5120, 6144, 5, 1, 0, None), (6144, 5120, 4, 4, 1, 4),
             (5120, 8192, 4, 64, 0, 8)]
    for K, N, KB, M, SK, skg in cases:
        banner("noalloc", K, N, KB, M, SK, skg)
        skg = api.trellis_gemv_skg(K, N, KB) if skg is None else skg
        words, _, svh = WL.trellis_linear(K, N, KB, K + N + M)
        a = WL.activations_f16(M, K, 3).view(np.uint16)
        w_d, svh_d = dev(words), dev(svh)
        first = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        _noalloc(f, ck, dev(a), w_d, svh_d, K, N, KB, SK, skg, first)
        # the second call: a smaller input (fewer rows, fewer columns: the first tile pairs only)
        M2, N2 = max(1, M // 2), N // 2
        w2 = dev(np.ascontiguousarray(words.reshape(N // 32, -1)[:N2 // 32]).ravel())
        second = torch.empty((M2, N2), dtype=torch.bfloat16, device="cuda")
        _noalloc(f, ck, dev(a[:M2]), w2, svh_d[:N2].contiguous(), K, N2, KB, SK, skg, second)
        ref1 = api.trellis_gemm_m64(dev(a), w_d, svh_d, K, N, KB, skg=skg, sk=SK, out_scale=OSC)
        ref2 = api.trellis_gemm_m64(dev(a[:M2]), w2, svh_d[:N2].contiguous(), K, N2, KB, skg=skg, sk=SK,
                                    out_scale=OSC)
        torch.cuda.synchronize()
        assert np.array_equal(host_u16(first), host_u16(ref1))
        assert np.array_equal(host_u16(second), host_u16(ref2))


def test_noalloc_size_rule():
    L, f, ck = _entry()
    cap = L.r4dx_gemm_trellis_nt_m64_noalloc_max_ws_bytes()
    assert cap == 16 << 20
    assert ck(8, 5120, 34816, 34816, 4, 2) is None                      # 2.2 MB of partials
    assert ck(64, 5120, 8192, 8192, 4, 8) is None                       # exactly 16 MiB
    assert b"exceed the scratch" in ck(64, 5120, 8192 + 128, 8192 + 128, 4, 8)
    assert b"exceed the scratch" in ck(64, 5120, 34816, 34816, 4, 8)    # 71 MB
    assert b"N must be at most" in ck(1, 5120, 262144 + 128, 262144 + 128, 4, 1)


def test_noalloc_graph_replays():
    """The callers this entry is for capture it: a graph of one call (split, SKG 4) replayed three times with eager
    calls of the entry on another input between the replays (the array's tickets must be back at zero every time),
    each replay byte-identical to the eager call."""
    L, f, ck = _entry()
    K, N, KB, M, SK, skg = 2048, 1024, 4, 2, 0, 4
    banner("noalloc graph", K, N, M, skg)
    words, _, svh = WL.trellis_linear(K, N, KB, 61)
    w_d, svh_d = dev(words), dev(svh)
    a = [dev(WL.activations_f16(M, K, 62 + v).view(np.uint16)) for v in (0, 1)]
    out = [torch.empty((M, N), dtype=torch.bfloat16, device="cuda") for _ in (0, 1)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _noalloc(f, ck, a[0], w_d, svh_d, K, N, KB, SK, skg, out[0])
        torch.cuda.synchronize()
        want = host_u16(out[0]).copy()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            _noalloc(f, ck, a[0], w_d, svh_d, K, N, KB, SK, skg, out[0])
    torch.cuda.synchronize()
    for r in range(3):
        out[0].zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host_u16(out[0]), want), r
        with torch.cuda.stream(s):
            _noalloc(f, ck, a[1], w_d, svh_d, K, N, KB, SK, skg, out[1])
        torch.cuda.synchronize()
