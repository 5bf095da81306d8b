"""The trellis container loader (r4dx_amd/container.py): the metadata gate of src/model/trellis_meta.h:70-209 --
every field this runtime does not implement, a malformed linear and an unverified container refused -- the
tensor layout of docs/trellis-kernel.md:105-117 (sizes and the rate cross-checked), and (GPU) a loaded
linear's output against the fp64 oracle."""
import copy
import json

import numpy as np
import pytest

from r4dx_amd import container as CT
from r4dx_amd import workloads as WL

GOOD = {
    "quant": {"trellis": {
        "format": "r4dx-trellis", "version": 1, "codebook": "mul1",
        "codebook_consts": {"mult": "0x83dcd12d", "k_inv_f16": "0x1eee", "k_bias_f16": "0xc931"},
        "state_bits": 16, "tail_biting": True, "position_order": "exl3-tensor-core",
        "bitstream": "ring-u32-msb-first", "tile_grid": "n32-pairs-k-major",
        "hadamard": {"block": 128, "order": "sylvester-natural", "scale": "1/sqrt(128)",
                     "input": "x*suh then H", "output": "H then *svh"},
        "prescale_log2": 0,
        "linears": {"l0.gdn.in_proj_qkv": {"bits": 4},
                    "l0.mlp.gate_up": {"bits": 5, "parts": [256, 256], "prescale_log2": 3}},
    }},
    "r4dx_convert_run": {"trellis": {"verify": {"result": "pass (bit-exact)", "failed": 0, "checked": 3}}},
}


def _edit(path, value):
    m = copy.deepcopy(GOOD)
    node = m
    for k in path[:-1]:
        node = node[k]
    if value is KeyError:
        del node[path[-1]]
    else:
        node[path[-1]] = value
    return m


def test_metadata_accepts_the_contract():
    spec = CT.parse_trellis_metadata(GOOD, "x.r4dx")
    assert spec.prescale_log2 == 0 and spec.hf_tensors() == 3
    assert spec.linears["l0.gdn.in_proj_qkv"].bits == 4 and spec.linears["l0.gdn.in_proj_qkv"].parts == []
    gu = spec.linears["l0.mlp.gate_up"]
    assert gu.bits == 5 and gu.parts == [256, 256] and gu.prescale_log2 == 3
    assert CT.parse_trellis_metadata({}, "x") is None
    assert CT.parse_trellis_metadata({"quant": {"w4a16": {}}}, "x") is None


T = ("quant", "trellis")


@pytest.mark.parametrize("path,value", [
    (T + ("format",), "exl3"), (T + ("version",), 2), (T + ("codebook",), "3inst"),
    (T + ("codebook_consts", "mult"), "0x83dcd12e"), (T + ("codebook_consts",), KeyError),
    (T + ("state_bits",), 15), (T + ("tail_biting",), False), (T + ("position_order",), "row-major"),
    (T + ("bitstream",), "ring-u32-lsb-first"), (T + ("tile_grid",), "n16"), (T + ("hadamard", "block"), 64),
    (T + ("hadamard", "input"), "H then x*suh"), (T + ("prescale_log2",), 17), (T + ("prescale_log2",), KeyError),
    (T + ("linears",), {}), (T + ("linears", "l0.gdn.in_proj_qkv", "bits"), 6),
    (T + ("linears", "l0.gdn.in_proj_qkv", "rate"), 4), (T + ("linears", "l0.mlp.gate_up", "parts"), [256, 200]),
    (T + ("linears", "l0.mlp.gate_up", "parts"), [512]), (T + ("linears", "l0.mlp.gate_up", "prescale_log2"), -17),
    (("r4dx_convert_run",), KeyError), (("r4dx_convert_run", "trellis", "verify", "result"), "FAILED"),
    (("r4dx_convert_run", "trellis", "verify", "result"), "pending"),
    (("r4dx_convert_run", "trellis", "verify", "failed"), 1), (("r4dx_convert_run", "trellis", "verify", "checked"), 2),
])
def test_metadata_refusals(path, value):
    with pytest.raises(ValueError, match="refusing to load"):
        CT.parse_trellis_metadata(_edit(path, value), "x.r4dx")


def _write_case(tmp_path, KB=4, K=256, N=512, bits_meta=None):
    words, suh, svh = WL.trellis_linear(K, N, KB, 3)
    words2, suh2, svh2 = WL.trellis_linear(K, N, 5, 4)
    suh2b = WL.signs(K, 9)
    meta = copy.deepcopy(GOOD)
    meta["quant"]["trellis"]["linears"]["l0.gdn.in_proj_qkv"]["bits"] = bits_meta or KB
    tensors = {}
    tensors.update(CT.trellis_tensors("l0.gdn.in_proj_qkv", words, [suh], svh))
    tensors.update(CT.trellis_tensors("l0.mlp.gate_up", words2, [suh2, suh2b], svh2))
    p = str(tmp_path / "t.r4dx")
    CT.write_container(p, meta, tensors)
    return p, (words, suh, svh), (words2, suh2, suh2b, svh2)


def test_container_round_trip(tmp_path):
    p, (words, suh, svh), (words2, suh2, suh2b, svh2) = _write_case(tmp_path)
    header, off = CT.read_header(p)
    assert header["__metadata__"] == json.loads(json.dumps(GOOD)) or "quant" in header["__metadata__"]
    a = CT.load_trellis_linear(p, "l0.gdn.in_proj_qkv")
    assert (a.K, a.N, a.KB, a.parts) == (256, 512, 4, []) and np.array_equal(a.words, words)
    assert np.array_equal(a.suh[0], suh.astype(np.float16).astype(np.float32))
    assert np.array_equal(a.svh, svh.astype(np.float16).astype(np.float32))
    b = CT.load_trellis_linear(p, "l0.mlp.gate_up")
    assert (b.K, b.N, b.KB, b.parts, b.prescale_log2) == (256, 512, 5, [256, 256], 3)
    assert np.array_equal(b.words, words2) and len(b.suh) == 2
    assert np.array_equal(b.suh[1], suh2b.astype(np.float32))
    with pytest.raises(KeyError):
        CT.load_trellis_linear(p, "l0.attn.o")


def test_container_rate_cross_check(tmp_path):
    """A linear whose word bytes do not match its metadata rate is refused."""
    p, _, _ = _write_case(tmp_path, KB=4, bits_meta=5)
    with pytest.raises(ValueError, match="word bytes"):
        CT.load_trellis_linear(p, "l0.gdn.in_proj_qkv")


@pytest.mark.gpu
def test_container_linear_on_gpu(tmp_path):
    """Loaded linears (one part at KB 4, a two-part gate_up at KB 5 with prescale 3) through transform + GEMV
    (M = 1, 8) and the M = 256 GEMM, against the fp64 oracle (within bf16 rounding)."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import oracle_lib as O
    from gpu_util import banner, close_rel, host_u16
    from r4dx_amd import api
    p, _, _ = _write_case(tmp_path)
    for base in ("l0.gdn.in_proj_qkv", "l0.mlp.gate_up"):
        lin = CT.load_trellis_linear(p, base)
        dt = api.trellis_linear_to_device(lin, "cuda")
        q = O.decode_pair_grid(lin.words, lin.K, lin.N, lin.KB)
        for M in (1, 8, 256):
            banner("container", base, M)
            x = O.f32_to_bf16_bits(np.random.default_rng(M).normal(0, 1, (M, lin.K)).astype(np.float32))
            xd = torch.from_numpy(x.view(np.int16)).to("cuda").view(torch.bfloat16)
            y = api.trellis_linear(xd, lin, dt)
            torch.cuda.synchronize()
            a = [O.transform_input(x, True, s, lin.prescale_log2) for s in lin.suh]
            ref = O.linear_from_a(a[0], q, lin.svh, lin.prescale_log2, a1=a[1] if len(a) > 1 else None,
                                  n_split=lin.parts[0] if lin.parts else None)
            got = O.bf16_bits_to_f32(host_u16(y))
            assert close_rel(got, ref, 2.0**-8, 1e-3) <= 1.0
