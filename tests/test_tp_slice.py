"""The tensor-parallel share of a trellis linear (container.rank_slice, docs/trellis-kernel.md:187-203), on the CPU:
a rank's words decode (oracle) to exactly its rows / k-range of the full Q, its svh / suh are the right cuts, the
shares of all ranks tile the linear, and ranges that are not 128-aligned are refused. The ranks' kernels on the GPU
are tests/test_tp_share_gpu.py's."""
import numpy as np
import pytest

import oracle_lib as O
from r4dx_amd import container as CT
from r4dx_amd import workloads as WL


def _lin(K, N, KB, parts=(), seed=0, nsuh=1):
    words, _, svh = WL.trellis_linear(K, N, KB, seed)
    suh = [WL.signs(K, seed + 10 + i) for i in range(nsuh)]
    return CT.TrellisLinear("t", words, suh, svh, K, N, KB, list(parts), 0)


@pytest.mark.parametrize("tp", [2, 4])
def test_column_slice_rows(tp):
    K, N, KB = 256, 1024, 4
    lin = _lin(K, N, KB)
    q = O.decode_pair_grid(lin.words, K, N, KB)
    cols = []
    for r in range(tp):
        s = CT.rank_slice(lin, r, tp, "col")
        assert (s.K, s.N, s.parts) == (K, N // tp, [])
        qs = O.decode_pair_grid(s.words, s.K, s.N, KB)
        c = slice(r * N // tp, (r + 1) * N // tp)
        assert np.array_equal(qs, q[:, c]) and np.array_equal(s.svh, lin.svh[c])
        assert np.array_equal(s.suh[0], lin.suh[0])
        cols.append(qs)
    assert np.array_equal(np.concatenate(cols, axis=1), q)


def test_column_slice_two_parts_and_segments():
    """gate | up: a rank takes its run of each part, its parts the runs' widths; a one-input fused linear's own
    segments (qkv) cut it the same way with one part."""
    K, N, KB = 128, 1024, 5
    lin = _lin(K, N, KB, parts=(512, 512), nsuh=2)
    q = O.decode_pair_grid(lin.words, K, N, KB)
    for r in range(2):
        s = CT.rank_slice(lin, r, 2, "col")
        assert s.parts == [256, 256] and len(s.suh) == 2
        want = np.concatenate([q[:, 256 * r:256 * r + 256], q[:, 512 + 256 * r:512 + 256 * r + 256]], axis=1)
        assert np.array_equal(O.decode_pair_grid(s.words, K, 512, KB), want)
    one = _lin(K, 1280, KB, seed=3)
    q1 = O.decode_pair_grid(one.words, K, 1280, KB)
    s = CT.rank_slice(one, 1, 2, "col", segments=[256, 256, 768])
    assert s.N == 640 and s.parts == []
    want = np.concatenate([q1[:, 128:256], q1[:, 384:512], q1[:, 896:1280]], axis=1)
    assert np.array_equal(O.decode_pair_grid(s.words, K, 640, KB), want)
    with pytest.raises(ValueError):  # segments that cut across a part boundary
        CT.rank_slice(lin, 0, 2, "col", segments=[256, 768])


@pytest.mark.parametrize("tp", [2, 3])
def test_row_slice_k_range(tp):
    K, N, KB = 256 * tp, 256, 4
    lin = _lin(K, N, KB, seed=5)
    q = O.decode_pair_grid(lin.words, K, N, KB)
    kc = K // tp
    parts = []
    for r in range(tp):
        s = CT.rank_slice(lin, r, tp, "row")
        assert (s.K, s.N) == (kc, N) and np.array_equal(s.svh, lin.svh)
        assert np.array_equal(s.suh[0], lin.suh[0][r * kc:(r + 1) * kc])
        qs = O.decode_pair_grid(s.words, kc, N, KB)
        assert np.array_equal(qs, q[r * kc:(r + 1) * kc])
        parts.append(qs)
    assert np.array_equal(np.concatenate(parts), q)


def test_row_parallel_outputs_add_up():
    """The ranks' linears (input transform of their k-range, the output transform of their partial) add up to the
    full linear in fp64: the transform is blockwise in K and linear after the sum."""
    K, N, KB, M = 512, 256, 4, 3
    lin = _lin(K, N, KB, seed=7)
    x = WL.activations_f16(M, K, 8).view(np.uint16)
    full = O.linear_from_a(O.transform_input(x, False, lin.suh[0]), O.decode_pair_grid(lin.words, K, N, KB), lin.svh)
    tot = np.zeros_like(full)
    for r in range(2):
        s = CT.rank_slice(lin, r, 2, "row")
        xa = np.ascontiguousarray(x[:, r * 256:(r + 1) * 256])
        tot += O.linear_from_a(O.transform_input(xa, False, s.suh[0]), O.decode_pair_grid(s.words, 256, N, KB), s.svh)
    # the per-rank f16 rounding of the transformed input is the same rounding of the same values
    assert np.allclose(tot, full, rtol=1e-12, atol=1e-12 * np.abs(full).max())


def test_refusals():
    lin = _lin(256, 384, 4)
    with pytest.raises(ValueError):
        CT.rank_slice(lin, 0, 2, "col")      # 192 rows per rank
    with pytest.raises(ValueError):
        CT.rank_slice(lin, 0, 4, "row")      # 64 k per rank
    with pytest.raises(ValueError):
        CT.rank_slice(lin, 2, 2, "row")
    with pytest.raises(ValueError):
        CT.rank_slice(lin, 0, 2, "diag")


def test_tp2_shapes_are_128_aligned():
    """Every projection of the model splits at TP = 2 (docs/trellis-kernel.md:197-203)."""
    for name, K, N in WL.LAYER_SHAPES:
        key = "mlp.gate_up" if name in ("mlp.gate", "mlp.up") else name
        kind, segs = WL.TP_KINDS[key]
        if kind == "row":
            assert (K // 2) % 128 == 0
        else:
            assert all((s // 2) % 128 == 0 for s in (segs or [N]))
