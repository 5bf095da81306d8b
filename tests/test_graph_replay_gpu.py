"""HIP-graph capture of the path's entries: each entry is captured once on a side stream, and the graph is replayed
three times with eager calls of the same entry between the replays -- on other inputs, through the same ws and
tickets, so every replay must find the self-resetting tickets, the balanced form's flags and the stream-K pieces
as a complete launch leaves them. Every replay's output must equal the eager output of the captured inputs bit for
bit. Nothing in these launches may record a memset (the graphs hold kernel nodes only)."""
import numpy as np
import pytest

from r4dx_amd import workloads as WL

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no GPU", allow_module_level=True)

from r4dx_amd import api  # noqa: E402
from gpu_util import banner, dev  # noqa: E402


def _bits(t):
    t = t.detach()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.view(torch.int16)
    elif t.dtype == torch.float32:
        t = t.view(torch.int32)
    return t.cpu().numpy()


def _replays(name, run, out_of):
    """run(variant) launches the entry on the current stream for input variant 0 or 1 and returns its outputs;
    out_of(variant) names the output tensors (preallocated per variant)."""
    banner("graph", name)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(0)                                   # eager, on the capture stream (first-call state set up there)
        torch.cuda.synchronize()
        want = [_bits(t) for t in out_of(0)]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            run(0)
    torch.cuda.synchronize()
    for r in range(3):
        for t in out_of(0):
            t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for j, (t, w) in enumerate(zip(out_of(0), want)):
            got = _bits(t)
            bad = np.flatnonzero(got.reshape(-1) != w.reshape(-1))
            assert bad.size == 0, (name, r, j, int(bad.size), bad[:8].tolist(), got.reshape(-1)[bad[:4]].tolist(),
                                   w.reshape(-1)[bad[:4]].tolist())
        with torch.cuda.stream(s):
            run(1)                               # eager work between the replays, the same ws and tickets
        torch.cuda.synchronize()


KB, OUT_SCALE = 4, float(np.float32(1.0 / np.sqrt(128.0)))


def test_graph_gemv_parts_and_fused():
    K, N, M, skg = 2048, 1024, 1, 4
    words, _, svh = WL.trellis_linear(K, N, KB, 11)
    w_d, svh_d = dev(words), dev(svh)
    n0 = [0, 512]
    suh = [dev(WL.signs(K, 12)), dev(WL.signs(K, 13))]
    x = [dev(WL.activations_f16(M, K, 14 + v)) for v in (0, 1)]
    a = [[torch.empty((M, K), dtype=torch.float16, device="cuda") for _ in n0] for _ in (0, 1)]
    out = [torch.empty((M, N), dtype=torch.bfloat16, device="cuda") for _ in (0, 1)]
    ws = torch.empty(api.lib().r4d_gemm_trellis_nt_m64_ws_bytes(M, N, skg) // 4, dtype=torch.float32, device="cuda")
    tickets = api.TicketBuffer(N).t

    def two(v):
        api.trellis_input(x[v], suh, 0, bf16=False, outs=a[v])
        api.trellis_gemm_m64_parts(a[v], n0, w_d, svh_d, K, N, KB, skg=skg, out=out[v], ws=ws, tickets=tickets,
                                   out_scale=OUT_SCALE)

    def fused(v):
        api.trellis_gemv_xf_parts(x[v], suh, n0, w_d, svh_d, K, N, KB, skg=skg, out=out[v], ws=ws, tickets=tickets,
                                  out_scale=OUT_SCALE)
    _replays("gemv parts (transform + GEMV)", two, lambda v: [a[v][0], a[v][1], out[v]])
    _replays("gemv xf parts", fused, lambda v: [out[v]])


@pytest.mark.parametrize("M,K,N,kb,skg,sk", [(256, 2048, 512, 4, 2, 0), (128, 1024, 33024, 5, 1, 0),
                                             (256, 1152, 512, 4, 2, 4)])
def test_graph_m256(M, K, N, kb, skg, sk):
    """A split launch (slices + the finish launch), a balanced one (cut units handed over through flags), and the 4-wave
    split order (SK 4: a launch and a finish per 128-row half)."""
    words, _, svh = WL.trellis_linear(K, N, kb, 21)
    w_d, svh_d = dev(words), dev(svh)
    a = [dev(WL.activations_f16(M, K, 22 + v)) for v in (0, 1)]
    out = [torch.empty((M, N), dtype=torch.bfloat16, device="cuda") for _ in (0, 1)]
    ws = torch.empty(api.lib().r4d_gemm_trellis_nt_m256_ws_bytes(M, N, skg) // 4, dtype=torch.float32, device="cuda")
    tickets = api.TicketBuffer(N).t

    def run(v):
        api.trellis_gemm_m256(a[v], w_d, svh_d, K, N, kb, skg=skg, out=out[v], ws=ws, tickets=tickets,
                              out_scale=OUT_SCALE, sk=sk)
    _replays(f"m256 M={M} N={N} skg={skg} sk={sk}", run, lambda v: [out[v]])


def test_graph_trellis_i8_and_dense_int8():
    K, N = 1024, 512
    words, suh, svh = WL.trellis_linear(K, N, KB, 31)
    w_d, svh_d = dev(words), dev(svh)
    sw = api.trellis_i8_table(w_d, K, N, KB)
    x = [dev(WL.activations_f16(256, K, 32 + v).view(np.uint16)) for v in (0, 1)]
    q = [api.i8_quant(x[v], blk=True, ref_layout=True) for v in (0, 1)]
    out = [torch.empty((256, N), dtype=torch.bfloat16, device="cuda") for _ in (0, 1)]
    ws = torch.empty(api.lib().r4d_gemm_trellis_nt_i8_ws_bytes(256, N, 2) // 4, dtype=torch.float32, device="cuda")

    def ti8(v):
        api.trellis_gemm_i8(q[v][0], q[v][1], w_d, sw, svh_d, K, N, KB, skg=2, out=out[v], ws=ws,
                            out_scale=OUT_SCALE)
    _replays("trellis int8 per-128 skg 2", ti8, lambda v: [out[v]])

    K2, N2 = 2048, 384
    xd, w8, swd = WL.int8_case(K2, N2, 33)
    w8_d, sw_d = api.i8_pack_w(dev(w8)), dev(swd)
    xs = [dev(xd.view(np.uint16)), dev(WL.int8_case(K2, N2, 34)[0].view(np.uint16))]
    q2 = [api.i8_quant(xs[v], blk=True) for v in (0, 1)]
    work = api.I8Workspace(N2, 0, w8_d.device)
    out2 = [torch.empty((256, N2), dtype=torch.float16, device="cuda") for _ in (0, 1)]

    def dense(v):
        api.i8_dense_gemm(q2[v][0], q2[v][1], w8_d, sw_d, K2, N2, scale_mode=1, skg=0, out=out2[v], work=work)
    _replays("dense int8 stream-K per-128", dense, lambda v: [out2[v]])


def test_graph_w4a16_and_argmax():
    N, K, M, group = 16384, 1024, 4, 32
    wq, wsz = WL.w4a16_packed(N, K, group, 41)
    wq_d, wsz_d = dev(wq), dev(wsz)
    a = [dev(WL.activations_f16(M, K, 42 + v)) for v in (0, 1)]
    out = [torch.empty((M, N), dtype=torch.float32, device="cuda") for _ in (0, 1)]
    idx = [torch.empty(M, dtype=torch.int32, device="cuda") for _ in (0, 1)]
    val = [torch.empty(M, dtype=torch.float32, device="cuda") for _ in (0, 1)]

    def run(v):
        api.w4a16_gemm(a[v], wq_d, wsz_d, K, N, group, out=out[v], f32=True)
        api.argmax_rows(out[v], idx[v], val[v])
    _replays("w4a16 + argmax", run, lambda v: [out[v], idx[v], val[v]])


def test_graph_zero_tickets_then_split_gemv():
    """r4d_gemm_trellis_nt_m64_zero_tickets captured with the split launch that follows it (the engine's recovery
    sequence): the clear is a kernel node, so every replay starts from zeroed tickets although the buffer is
    poisoned before each one; every replay's output equals the eager launch on a fresh buffer."""
    K, N, M, skg = 6144, 5120, 4, 4
    words, _, svh = WL.trellis_linear(K, N, KB, 61)
    w_d, svh_d = dev(words), dev(svh)
    a = dev(WL.activations_f16(M, K, 62).view(np.uint16))
    want = _bits(api.trellis_gemm_m64(a, w_d, svh_d, K, N, KB, skg=skg, out_scale=OUT_SCALE))
    tk = api.TicketBuffer(N).t
    nbytes = api.lib().r4d_gemm_trellis_nt_m64_tickets_bytes(N)
    ws = torch.empty(api.lib().r4d_gemm_trellis_nt_m64_ws_bytes(M, N, skg) // 4, dtype=torch.float32, device="cuda")
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    banner("graph", "zero_tickets + split GEMV")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())

    def run():
        api.lib().r4d_gemm_trellis_nt_m64_zero_tickets(tk.data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream)
        api.trellis_gemm_m64(a, w_d, svh_d, K, N, KB, skg=skg, out=out, ws=ws, tickets=tk, out_scale=OUT_SCALE)
    with torch.cuda.stream(s):
        run()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            run()
    torch.cuda.synchronize()
    for r in range(3):
        tk.copy_(torch.randint(1, 1 << 20, tk.shape, dtype=torch.int32, device="cuda"))
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out), want), r
        assert int(tk.abs().sum()) == 0, r


def test_zero_tickets_byte_tail():
    """The clear covers exactly `bytes` bytes, a tail of 1-3 bytes past the last whole word included."""
    banner("zero_tickets tail")
    buf = torch.full((64,), 0x5A, dtype=torch.uint8, device="cuda")
    for nb in (1, 4, 7, 13, 60):
        buf.fill_(0x5A)
        api.lib().r4d_gemm_trellis_nt_m64_zero_tickets(buf.data_ptr(), nb, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        h = buf.cpu().numpy()
        assert not h[:nb].any() and (h[nb:] == 0x5A).all(), nb
