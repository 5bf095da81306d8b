"""ctypes face of the CPU oracle (oracle/_build/libr4o.so) and, when built, of the reference's own
CPU references (oracle/_ref/libr4dref.so).  Test infrastructure: only tests/, the smoke check and
bench.py's cpu_baseline leg import this module."""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
LIB_PATH = os.path.join(ORACLE_DIR, "_build", "libr4o.so")
REF_PATH = os.path.join(ORACLE_DIR, "_ref", "libr4dref.so")

P = C.c_void_p
I64 = C.c_int64
I32 = C.c_int


def ptr(a):
    return a.ctypes.data_as(P) if a is not None else None


_lib = None
_ref = None

_SIGS = {
    "r4o_f16_to_f32": (C.c_float, [C.c_uint16]),
    "r4o_f32_to_f16": (C.c_uint16, [C.c_float]),
    "r4o_f32_to_bf16": (C.c_uint16, [C.c_float]),
    "r4o_codebook": (None, [P]),
    "r4o_trellis_state": (C.c_uint32, [P, I32, I32]),
    "r4o_tc_perm": (I32, [I32]),
    "r4o_pair_grid_index": (C.c_size_t, [I64, I32, I64, I64]),
    "r4o_to_pair_grid": (None, [P, I64, I64, I32, P]),
    "r4o_decode_pair_grid": (None, [P, I64, I64, I32, P, I32]),
    "r4o_fwht128_f32": (None, [P]),
    "r4o_fwht128_f64": (None, [P]),
    "r4o_transform_scale": (C.c_float, [I32]),
    "r4o_transform_input": (None, [P, I32, I64, I64, P, I32, P]),
    "r4o_silu_mul_bf16": (None, [P, I64, I64, I64, P]),
    "r4o_attn_gate_mul_bf16": (None, [P, P, I64, P]),
    "r4o_raw_sums_f64": (None, [P, P, I64, I64, I64, I64, P, P, I32]),
    "r4o_linear_from_a": (None, [P, P, I64, I64, I64, I64, P, P, I32, P, I32]),
    "r4o_epilogue_from_raw": (None, [P, I64, I64, P, C.c_float, P]),
    "r4o_i8_rs_half": (C.c_uint16, [C.c_float]),
    "r4o_i8_seff": (C.c_float, [C.c_float]),
    "r4o_i8_quant_w": (C.c_int8, [C.c_uint16, C.c_uint16]),
    "r4o_i8_quant_act": (C.c_int8, [C.c_float, C.c_float]),
    "r4o_i8_quant_act_blk": (None, [P, I32, I32, P, P]),
    "r4o_i8_quant_act_row": (None, [P, I32, I32, P, P]),
    "r4o_i8_quant_w_blk": (None, [P, I32, I32, P, P]),
    "r4o_i8_quant_w_col": (None, [P, I32, I32, P, P]),
    "r4o_i8_gemm_i32": (None, [P, P, I32, I32, I32, P, I32]),
    "r4o_i8_gemm_ref": (None, [P, P, P, P, I32, I32, I32, I32, P, I32]),
    "r4o_a8_offset": (C.c_size_t, [I32, I32, I32]),
    "r4o_pack_a8": (None, [P, I32, P]),
    "r4o_w8_offset": (C.c_size_t, [I32, I32, I32]),
    "r4o_pack_w8": (None, [P, I32, I32, P]),
    "r4o_w4_quantize": (None, [P, I32, I32, I32, P, P, P]),
    "r4o_w4_pack": (None, [P, I32, I32, P]),
    "r4o_w4_pack_scales": (None, [P, P, I32, I32, I32, P]),
    "r4o_w4_dequant": (None, [P, P, I32, I32, I32, P]),
    "r4o_w4_gemm_ref": (None, [P, P, P, I32, I32, I32, I32, P, I32]),
    "r4o_argmax_f32": (C.c_int32, [P, I64, P]),
    "r4o_wq_table": (None, [P, I64, I64, I32, P]),
    "r4o_wq_apply": (None, [P, I64, I64, I32, P, P]),
    "r4o_now_seconds": (C.c_double, []),
    "r4o_max_threads": (I32, []),
}

_REF_SIGS = {
    "ref_codebook": (None, [P]),
    "ref_trellis_state": (C.c_uint32, [P, I32, I32]),
    "ref_tc_perm": (I32, [I32]),
    "ref_to_pair_grid": (None, [P, I64, I64, I32, P]),
    "ref_decode_pair_grid": (None, [P, I64, I64, I32, P]),
    "ref_fwht_lds_f32": (None, [P]),
    "ref_transform_input_bf16": (None, [P, I64, I64, P, I32, P]),
    "ref_linear_from_a": (None, [P, P, I64, I64, I64, I64, P, P, I32, P]),
    "ref_epilogue_from_raw": (None, [P, I64, I64, P, C.c_float, P]),
    "ref_i8_quant_w_blk": (None, [P, I32, I32, P, P]),
    "ref_i8_quant_w_col": (None, [P, I32, I32, P, P]),
    "ref_i8_quant_act_blk": (None, [P, I32, P, P]),
    "ref_i8_quant_act_row": (None, [P, I32, P, P]),
    "ref_i8_gemm": (None, [P, P, P, P, I32, I32, I32, I32, P]),
    "ref_a8_offset": (C.c_size_t, [I32, I32, I32]),
    "ref_w8_offset": (C.c_size_t, [I32, I32, I32]),
    "ref_i8_quant_w": (C.c_int8, [C.c_uint16, C.c_uint16]),
    "ref_i8_rs_half": (C.c_uint16, [C.c_float]),
    "ref_w4_quantize_pack": (None, [P, I32, I32, I32, P, P]),
    "ref_argmax": (C.c_int32, [P, I64, P]),
    "ref_wq_table": (None, [P, I64, I64, I32, P]),
    "ref_wq_apply": (None, [P, I64, I64, I32, P, P]),
    "ref_f32_to_f16": (C.c_uint16, [C.c_float]),
    "ref_f32_to_bf16": (C.c_uint16, [C.c_float]),
}


def _bind(lib, sigs):
    for name, (res, args) in sigs.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


def build():
    """Compile the oracle (and oracle/_ref when the reference checkout is present)."""
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = _bind(C.CDLL(LIB_PATH), _SIGS)
    return _lib


def ref():
    """The reference's own CPU references, or None when oracle/_ref was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        _ref = _bind(C.CDLL(REF_PATH), _REF_SIGS)
    return _ref


# ---- numpy conveniences ---------------------------------------------------------------------------
def codebook():
    out = np.empty(65536, np.uint16)
    lib().r4o_codebook(ptr(out))
    return out


def decode_pair_grid(grid, K, N, KB, nthreads=0):
    q = np.empty((K, N), np.uint16)
    lib().r4o_decode_pair_grid(ptr(grid), K, N, KB, ptr(q), nthreads)
    return q


def transform_input(x_bits, x_is_bf16, suh, prescale=0):
    M, K = x_bits.shape
    a = np.empty((M, K), np.uint16)
    lib().r4o_transform_input(ptr(np.ascontiguousarray(x_bits)), int(x_is_bf16), M, K,
                              ptr(np.ascontiguousarray(suh, np.float32)), prescale, ptr(a))
    return a


def raw_sums(a0, q, a1=None, n_split=None, nthreads=0):
    M, K = a0.shape
    N = q.shape[1]
    s = np.empty((M, N), np.float64)
    lib().r4o_raw_sums_f64(ptr(a0), ptr(a1), N if n_split is None else n_split, M, K, N, ptr(q),
                           ptr(s), nthreads)
    return s


def linear_from_a(a0, q, svh, prescale=0, a1=None, n_split=None, nthreads=0):
    M, K = a0.shape
    N = q.shape[1]
    y = np.empty((M, N), np.float64)
    lib().r4o_linear_from_a(ptr(a0), ptr(a1), N if n_split is None else n_split, M, K, N, ptr(q),
                            ptr(np.ascontiguousarray(svh, np.float32)), prescale, ptr(y), nthreads)
    return y


def epilogue_from_raw(s, svh, out_scale):
    M, N = s.shape
    c = np.empty((M, N), np.uint16)
    lib().r4o_epilogue_from_raw(ptr(np.ascontiguousarray(s, np.float32)), M, N,
                                ptr(np.ascontiguousarray(svh, np.float32)), out_scale, ptr(c))
    return c


def wq_table(q, group):
    """src/model/fake_quant_w.h:118-128: scale table [K/group][N] of Q (f16 bits [K][N])."""
    K, N = q.shape
    t = np.empty((K // group, N), np.float32)
    lib().r4o_wq_table(ptr(np.ascontiguousarray(q, np.uint16)), K, N, group, ptr(t))
    return t


def wq_apply(q, group, t=None):
    """src/model/fake_quant_w.h:130-138 then f16: the rounded weight Q' (f16 bits [K][N])."""
    K, N = q.shape
    q = np.ascontiguousarray(q, np.uint16)
    t = wq_table(q, group) if t is None else np.ascontiguousarray(t, np.float32)
    out = np.empty((K, N), np.uint16)
    lib().r4o_wq_apply(ptr(q), K, N, group, ptr(t), ptr(out))
    return out


def f16_bits_to_f32(b):
    return np.asarray(b, np.uint16).view(np.float16).astype(np.float32)


def bf16_bits_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x):
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r
