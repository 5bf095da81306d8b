"""GPU parity of the fused LM-head entry r4d_gemm_w4a16_nt_m64_f32_argmax through the C ABI: its logits are
bit-identical to r4d_gemm_w4a16_nt_m64_f32's on the same inputs, and its (index, value) per row bit-identical to the
oracle's argmax order (larger value first, then lower index, NaN never wins) over those logits -- so to the two-call
GEMM + r4dx_argmax_rows_f32 path. Cases: both MFMA forms and both row-tile counts, spare waves (N not a multiple of
the 256 columns of a workgroup), the full config-3 vocab, planted ties across workgroups, NaN and all-zero rows, and
back-to-back calls on one stream (the slots and the ticket clear themselves) with a smaller second call, HIP-graph
replays with eager calls between them, and two streams at once."""
import ctypes as C

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


def _bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def _check(a_d, wq_d, wsz_d, K, N, group):
    """Fused call vs the f32 GEMM entry and the oracle's argmax over its logits."""
    M = a_d.shape[0]
    ref = api.w4a16_gemm(a_d, wq_d, wsz_d, K, N, group, f32=True)
    c, idx, val = api.w4a16_gemm_argmax(a_d, wq_d, wsz_d, K, N, group)
    torch.cuda.synchronize()
    logits = ref.cpu().numpy()
    assert np.array_equal(_bits(c.cpu().numpy()), _bits(logits))
    idx, val = idx.cpu().numpy(), val.cpu().numpy()
    for m in range(M):
        v = C.c_float()
        i = O.lib().r4o_argmax_f32(ptr(np.ascontiguousarray(logits[m])), N, C.byref(v))
        assert int(idx[m]) == i, (m, int(idx[m]), i)
        assert _bits(val[m]) == _bits(v.value), (m, val[m], v.value)
    return logits, idx


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("M,N,K", [(1, 16, 448), (3, 1040, 512), (8, 4096, 5120), (9, 80, 704), (33, 528, 1024),
                                   (64, 512, 5120)])
def test_fused_argmax_shapes(group, M, N, K):
    banner("w4a16 argmax", group, M, N, K)
    wq, wsz = WL.w4a16_packed(N, K, group, 21 + M)
    a = WL.activations_f16(M, K, 22).view(np.uint16)
    _check(dev(a), dev(wq), dev(wsz), K, N, group)


@pytest.mark.parametrize("group", [32, 64])
def test_fused_argmax_config3(group):
    """The full vocab (N = 248 320, 970 workgroups over the 64 slots) at M = 1 and 8, then M = 8 again and
    M = 1 again: each call's slots start clear."""
    N, K = 248320, 5120
    wq, wsz = WL.w4a16_packed(N, K, group, 31)
    a = WL.activations_f16(8, K, 32).view(np.uint16)
    wq_d, wsz_d, a_d = dev(wq), dev(wsz), dev(a)
    for M in (1, 8, 8, 1):
        banner("w4a16 argmax config3", group, M)
        _check(a_d[:M], wq_d, wsz_d, K, N, group)


def test_fused_argmax_ties_nan_zero():
    """A tie planted across workgroups (the winning column's 16-column tile copied to a later tile: the
    lower index wins), a row whose activations hold a NaN (every logit NaN: index 0, value -inf), and an
    all-zero row (every logit +0: index 0)."""
    group, N, K = 64, 8192, 1024
    wq, wsz = WL.w4a16_packed(N, K, group, 41)
    a = WL.activations_f16(3, K, 42).view(np.uint16).copy()
    a[1, 17] = 0x7E00   # f16 NaN
    a[2, :] = 0
    a_d = dev(a)
    logits, idx = _check(a_d, dev(wq), dev(wsz), K, N, group)
    assert int(idx[1]) == 0 and int(idx[2]) == 0
    # copy the tile of row 0's winner to the last tile: the same logits there, the earlier column still wins
    win = int(idx[0])
    t_src, t_dst = win // 16, N // 16 - 1
    if t_src == t_dst:
        t_dst = 0
    wq_t = wq.reshape(N // 16, -1).copy()
    wsz_t = wsz.reshape(N // 16, -1).copy()
    wq_t[t_dst], wsz_t[t_dst] = wq_t[t_src], wsz_t[t_src]
    banner("w4a16 argmax tie", win, t_dst)
    logits2, idx2 = _check(a_d, dev(wq_t.reshape(-1)), dev(wsz_t.reshape(-1)), K, N, group)
    twin = t_dst * 16 + win % 16
    assert _bits(logits2[0, twin]) == _bits(logits2[0, win])
    assert int(idx2[0]) == min(win, twin)


def test_fused_argmax_graph_replays_and_two_streams():
    """Captured in a HIP graph and replayed three times with eager launches between the replays (the slots and the
    ticket must be clear at every replay), each replay against the eager result; then two streams running the entry
    at once on different inputs (each stream has its own slots and ticket)."""
    group, N, K = 64, 16384, 2048
    wq, wsz = WL.w4a16_packed(N, K, group, 51)
    a = WL.activations_f16(8, K, 52).view(np.uint16)
    b = WL.activations_f16(8, K, 53).view(np.uint16)
    wq_d, wsz_d, a_d, b_d = dev(wq), dev(wsz), dev(a), dev(b)
    banner("w4a16 argmax graph")
    c_ref, i_ref, v_ref = api.w4a16_gemm_argmax(a_d, wq_d, wsz_d, K, N, group)
    torch.cuda.synchronize()
    i_ref, v_ref = i_ref.cpu().numpy(), v_ref.cpu().numpy()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    out = torch.empty((8, N), dtype=torch.float32, device="cuda")
    idx = torch.empty(8, dtype=torch.int32, device="cuda")
    val = torch.empty(8, dtype=torch.float32, device="cuda")
    with torch.cuda.stream(s):
        api.w4a16_gemm_argmax(a_d, wq_d, wsz_d, K, N, group, out=out, out_idx=idx, out_val=val)   # scratch of s
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            api.w4a16_gemm_argmax(a_d, wq_d, wsz_d, K, N, group, out=out, out_idx=idx, out_val=val)
    torch.cuda.synchronize()
    for r in range(3):
        idx.fill_(-1)
        val.fill_(0.0)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(idx.cpu().numpy(), i_ref), r
        assert np.array_equal(_bits(val.cpu().numpy()), _bits(v_ref)), r
        # eager work between the replays, on the same stream's scratch and on the default stream's
        with torch.cuda.stream(s):
            api.w4a16_gemm_argmax(b_d[:3], wq_d, wsz_d, K, N, group)
        api.w4a16_gemm_argmax(b_d[:5], wq_d, wsz_d, K, N, group)
        torch.cuda.synchronize()
    banner("w4a16 argmax two streams")
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for st in (s1, s2):
        with torch.cuda.stream(st):
            api.w4a16_gemm_argmax(a_d[:1], wq_d, wsz_d, K, N, group)
    torch.cuda.synchronize()
    for _ in range(3):
        with torch.cuda.stream(s1):
            ca, ia, va = api.w4a16_gemm_argmax(a_d, wq_d, wsz_d, K, N, group)
        with torch.cuda.stream(s2):
            cb, ib, vb = api.w4a16_gemm_argmax(b_d, wq_d, wsz_d, K, N, group)
        torch.cuda.synchronize()
        for c, i, v in ((ca, ia, va), (cb, ib, vb)):
            logits = c.cpu().numpy()
            for m in range(8):
                vv = C.c_float()
                assert int(i[m]) == O.lib().r4o_argmax_f32(ptr(np.ascontiguousarray(logits[m])), N, C.byref(vv))
                assert _bits(v[m].item()) == _bits(vv.value)
