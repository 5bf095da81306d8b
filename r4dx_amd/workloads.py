"""Synthetic inputs of the benchmark workloads (numpy, seeded).  No network, no checkpoints: the
trellis words are uniform random uint32 (every 32-bit word is a valid ring), the Hadamard signs are
random +-1, and the channel scales are log-normal, exactly as the configs describe."""
import numpy as np

# Config 1 / 2: one 27B-class hybrid layer's projections, (name, K in, N out)
LAYER_SHAPES = [
    ("gdn.qkv", 5120, 10240),
    ("gdn.z", 5120, 6144),
    ("gdn.out", 6144, 5120),
    ("attn.q", 5120, 6144),
    ("attn.k", 5120, 1024),
    ("attn.v", 5120, 1024),
    ("attn.o", 6144, 5120),
    ("mlp.gate", 5120, 17408),
    ("mlp.up", 5120, 17408),
    ("mlp.down", 17408, 5120),
]


# Tensor-parallel kinds of those projections (docs/trellis-kernel.md:191-203): column-parallel linears split every
# output segment (gdn.qkv's q, k, v segments; mlp.gate | mlp.up's two parts), row-parallel ones split K. At TP = 2
# every rank range is 128-aligned; one GPU runs one rank's share.
TP_KINDS = {
    "gdn.qkv": ("col", [2048, 2048, 6144]),
    "gdn.z": ("col", None),
    "gdn.out": ("row", None),
    "attn.q": ("col", None),
    "attn.k": ("col", None),
    "attn.v": ("col", None),
    "attn.o": ("row", None),
    "mlp.gate_up": ("col", [17408, 17408]),
    "mlp.down": ("row", None),
}


# The engine's launch groups for those projections: (input group, linears); a linear with two names is a
# fused two-part linear (part 1 from the first part's N on, reading its own input transform).
LAYER_GROUPS = [
    ("gdn.in", [("gdn.qkv",), ("gdn.z",)]),
    ("gdn.out", [("gdn.out",)]),
    ("attn.in", [("attn.q",), ("attn.k",), ("attn.v",)]),
    ("attn.o", [("attn.o",)]),
    ("mlp.in", [("mlp.gate", "mlp.up")]),
    ("mlp.down", [("mlp.down",)]),
]


def trellis_words(K, N, KB, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, 2**32, size=K * N * KB // 32, dtype=np.uint64).astype(np.uint32)


def signs(n, seed):
    rng = np.random.default_rng(seed)
    return np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)


def svh_scales(N, seed):
    """+-1 * lognormal(ln 0.01, 0.3), rounded to fp16 then widened (the container stores fp16)."""
    rng = np.random.default_rng(seed)
    s = np.where(rng.random(N) < 0.5, -1.0, 1.0) * rng.lognormal(np.log(0.01), 0.3, N)
    return s.astype(np.float16).astype(np.float32)


def activations_f16(M, K, seed, outlier_frac=0.0, outlier_scale=20.0, bf16_exact=False):
    """f16 activations ~N(0,1) (a fraction of columns scaled as outlier channels). bf16_exact: each value rounded
    first to bf16 precision (nearest even), so the same numbers are exact in bf16 and in f16 (|x| < 2^16) -- an input
    that the bf16 and the f16 forms of the input transform read identically."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if outlier_frac > 0:
        cols = rng.choice(K, max(1, int(round(K * outlier_frac))), replace=False)
        x[:, cols] *= outlier_scale
    if bf16_exact:
        u = x.view(np.uint32).astype(np.uint64)
        x = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)
    return x.astype(np.float16)


def trellis_linear(K, N, KB, seed):
    """(words, suh, svh) of one trellis linear."""
    return trellis_words(K, N, KB, seed), signs(K, seed + 1), svh_scales(N, seed + 2)


def w4a16_packed(N, K, group, seed):
    """The LM-head workload's (w4a16) weights directly in the packed form: uniform random nibbles, per (row, group)
    an fp16 scale ~ lognormal around 0.02 and an int4 zero point uniform in 0..15.
    Returns (wq uint32 [N*K/8], wsz uint32 [N/16][K/group][16])."""
    rng = np.random.default_rng(seed)
    wq = rng.integers(0, 2**32, N * K // 8, dtype=np.uint64).astype(np.uint32)
    gpr = K // group
    sc = rng.lognormal(np.log(0.02), 0.3, (N // 16, gpr, 16)).astype(np.float16).view(np.uint16)
    zero = rng.integers(0, 16, (N // 16, gpr, 16))
    nz = (-(1024.0 + zero)).astype(np.float16).view(np.uint16)
    wsz = (sc.astype(np.uint32) | (nz.astype(np.uint32) << 16)).reshape(-1)
    return wq, wsz


def int8_case(K, N, seed, M=256):
    """The int8 prefill workload: activations f16 Student-t (nu = 4); weights int8 uniform in [-127, 127] with an
    fp32 scale per output column (log-normal around 0.01)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_t(4, (M, K)).astype(np.float16)
    w8 = rng.integers(-127, 128, (N, K)).astype(np.int8)
    sw = rng.lognormal(np.log(0.01), 0.3, N).astype(np.float32)
    return x, w8, sw
