"""One tensor-parallel rank's share of the model's trellis linears at TP = 2, on the one GPU (the rank's kernels at
their real shard shapes; no collective is part of this build):
  * every projection's rank share (container.rank_slice) through the input transform and the GEMV / M = 256 GEMM,
    against the fp64 oracle of that share (bf16 bar: 2^-8 relative, 1e-3 rms floor);
  * column-parallel: the ranks' outputs are the full linear's columns bit for bit at the same SKG (the kernels'
    columns do not depend on N), one part and gate | up;
  * row-parallel: the ranks' fp32 partial sums add up to the full linear's sums (1e-3 relative, 1e-4 rms floor),
    the sum an all-reduce would form before (raw) or after (bf16) the output transform."""
import numpy as np
import pytest

import oracle_lib as O
from r4dx_amd import container as CT
from r4dx_amd import workloads as WL

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no GPU", allow_module_level=True)

from r4dx_amd import api  # noqa: E402
from gpu_util import banner, close_rel, host_u16  # noqa: E402

SHAPES = {name: (K, N) for name, K, N in WL.LAYER_SHAPES}


def _full(name, KB, seed):
    if name == "mlp.gate_up":
        K, N0 = SHAPES["mlp.gate"]
        words, _, svh = WL.trellis_linear(K, 2 * N0, KB, seed)
        return CT.TrellisLinear(name, words, [WL.signs(K, seed + 5), WL.signs(K, seed + 6)], svh, K, 2 * N0, KB,
                                [N0, N0], 0)
    K, N = SHAPES[name]
    words, suh, svh = WL.trellis_linear(K, N, KB, seed)
    return CT.TrellisLinear(name, words, [suh], svh, K, N, KB, [], 0)


def _x(M, K, seed):
    x = O.f32_to_bf16_bits(np.random.default_rng(seed).normal(0, 1, (M, K)).astype(np.float32))
    return x, torch.from_numpy(x.view(np.int16)).to("cuda").view(torch.bfloat16)


def _run(lin, dt, xd, skg, raw=False):
    """The linear at an explicit SKG: transform, then the M <= 64 or the M = 256 GEMM."""
    a = api.trellis_input(xd, dt["suh"], lin.prescale_log2)
    a1 = a[1] if len(a) > 1 else None
    ns = lin.parts[0] if lin.parts else None
    osc = float(np.float32(np.ldexp(1.0, -lin.prescale_log2) / np.sqrt(128.0)))
    fn = api.trellis_gemm_m64 if xd.shape[0] <= 64 else api.trellis_gemm_m256
    return fn(a[0], dt["words"], None if raw else dt["svh"], lin.K, lin.N, lin.KB, skg=skg, a1=a1, n_split=ns,
              out_scale=osc, raw=raw)


@pytest.mark.parametrize("name", list(WL.TP_KINDS))
def test_rank_share_vs_oracle(name):
    KB = 4 if len(name) % 2 else 5
    kind, segs = WL.TP_KINDS[name]
    lin = _full(name, KB, 40 + len(name))
    share = CT.rank_slice(lin, 1, 2, kind, segs)
    dt = api.trellis_linear_to_device(share, "cuda")
    q = O.decode_pair_grid(share.words, share.K, share.N, KB)
    for M in (1, 8):
        banner("tp2 share", name, kind, share.K, share.N, KB, M)
        x, xd = _x(M, share.K, M)
        y = api.trellis_linear(xd, share, dt)
        torch.cuda.synchronize()
        a = [O.transform_input(x, True, s, share.prescale_log2) for s in share.suh]
        ref = O.linear_from_a(a[0], q, share.svh, share.prescale_log2, a1=a[1] if len(a) > 1 else None,
                              n_split=share.parts[0] if share.parts else None)
        assert close_rel(O.bf16_bits_to_f32(host_u16(y)), ref, 2.0**-8, 1e-3) <= 1.0


@pytest.mark.parametrize("name,M", [("attn.k", 1), ("attn.k", 256), ("mlp.gate_up", 1), ("mlp.gate_up", 256),
                                    ("gdn.qkv", 4)])
def test_column_parallel_ranks_are_the_full_columns(name, M):
    banner("tp2 column identity", name, M)
    KB = 4
    kind, segs = WL.TP_KINDS[name]
    lin = _full(name, KB, 60)
    skg = api.trellis_gemv_skg(lin.K, lin.N, KB) if M <= 64 else api.trellis_m256_skg(lin.K, lin.N, KB)
    _, xd = _x(M, lin.K, 61)
    full = host_u16(_run(lin, api.trellis_linear_to_device(lin, "cuda"), xd, skg))
    cuts = []
    n0 = 0
    for seg in (segs or [lin.N]):
        cuts.append((n0, seg))
        n0 += seg
    for r in range(2):
        share = CT.rank_slice(lin, r, 2, kind, segs)
        got = host_u16(_run(share, api.trellis_linear_to_device(share, "cuda"), xd, skg))
        torch.cuda.synchronize()
        want = np.concatenate([full[:, a + r * c // 2:a + (r + 1) * c // 2] for a, c in cuts], axis=1)
        assert np.array_equal(got, want), r


@pytest.mark.parametrize("name,M", [("mlp.down", 1), ("attn.o", 16), ("gdn.out", 256)])
def test_row_parallel_partials_add_up(name, M):
    banner("tp2 row partials", name, M)
    KB = 5
    lin = _full(name, KB, 70)
    x, xd = _x(M, lin.K, 71)
    pick = api.trellis_gemv_skg if M <= 64 else api.trellis_m256_skg
    full = _run(lin, api.trellis_linear_to_device(lin, "cuda"), xd, pick(lin.K, lin.N, KB), raw=True)
    tot = torch.zeros_like(full, dtype=torch.float64)
    for r in range(2):
        share = CT.rank_slice(lin, r, 2, "row")
        xr = xd[:, r * share.K:(r + 1) * share.K].contiguous()
        tot += _run(share, api.trellis_linear_to_device(share, "cuda"), xr, pick(share.K, share.N, KB),
                    raw=True).double()
    torch.cuda.synchronize()
    assert close_rel(tot.cpu().numpy(), full.double().cpu().numpy(), 1e-3, 1e-4) <= 1.0
