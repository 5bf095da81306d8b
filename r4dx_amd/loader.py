"""Loads libr4d_mi355x.so and declares the ctypes signatures of include/r4d_mi355x.h."""
import ctypes as C
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libr4d_mi355x.so")
HEADER = os.path.join(os.path.dirname(PKG), "include", "r4d_mi355x.h")

I64, I32, F32, SZ, P = C.c_int64, C.c_int, C.c_float, C.c_size_t, C.c_void_p
CSTR = C.c_char_p
I64P = C.POINTER(C.c_int64)
I32P = C.POINTER(C.c_int)

SIGS = {
    "r4d_gemm_trellis_nt_m64": (None, [I64, I64, I32, I64, I64, I64, I64, I64] + [I32] * 11 + [F32, I64]),
    "r4d_gemm_trellis_nt_m64_raw": (None, [I64, I64, I32, I64, I64, I64, I64] + [I32] * 11 + [I64, I64]),
    "r4d_gemm_trellis_nt_m64_has_rate": (I32, [I32]),
    "r4d_gemm_trellis_nt_m64_max_m": (I32, []),
    "r4d_gemm_trellis_nt_m64_ws_bytes": (SZ, [I32, I32, I32]),
    "r4d_gemm_trellis_nt_m64_tickets_bytes": (SZ, [I32]),
    "r4d_gemm_trellis_nt_m64_zero_tickets": (None, [I64, SZ, I64]),
    "r4d_trellis_reconstruct_f16": (None, [I64, I64, I32, I32, I32, I64]),
    "r4d_gemm_trellis_nt_m64_check": (CSTR, [I32] * 9),
    "r4d_mi355x_trellis_gemv_skg": (I32, [I32, I32, I32]),
    "r4d_gemm_trellis_nt_m256": (None, [I64, I64, I32, I64, I64, I64, I64, I64] + [I32] * 8 + [F32, I64, I32]),
    "r4d_gemm_trellis_nt_m256_check": (CSTR, [I32] * 10),
    "r4d_gemm_trellis_nt_m256_ws_bytes": (SZ, [I32, I32, I32]),
    "r4d_gemm_trellis_nt_m256_raw": (None, [I64, I64, I32, I64, I64, I64, I64] + [I32] * 5 + [I64]),
    "r4d_mi355x_trellis_m256_skg": (I32, [I32, I32, I32]),
    "r4d_gemm_w4a16_nt_m64": (None, [I64, I64, I64, I64] + [I32] * 8 + [I64]),
    "r4d_gemm_w4a16_nt_m64_max_m": (I32, []),
    "r4d_gemm_w4a16_nt_m64_group": (I32, []),
    "r4d_gemm_w4a16_nt_m64_has_group": (I32, [I32]),
    "r4d_gemm_w4a16_nt_m64_g": (None, [I32, I64, I64, I64, I64] + [I32] * 8 + [I64]),
    "r4d_gemm_w4a16_nt_m64_check": (CSTR, [I32] * 4),
    "r4d_gemm_w4a16_nt_m64_f32": (None, [I32, I64, I64, I64, I64, I32, I32, I32, I64]),
    "r4dx_argmax_f32": (None, [I64, I64, I64, I64]),
    "r4dx_argmax_val_f32": (None, [I64, I64, I64, I64, I64]),
    "r4dx_argmax_bf16": (None, [I64, I64, I64, I64]),
    "r4dx_argmax_val_bf16": (None, [I64, I64, I64, I64, I64]),
    "r4dx_argmax_rows_f32": (None, [I64] * 8),
    "r4d_gemm_w4a16_nt_m64_f32_argmax": (None, [I32, I64, I64, I64, I64, I64, I64, I32, I32, I32, I64]),
    "r4d_trellis_i8_quant_act": (None, [I64, I64, I64, I32, I64, I32, I64]),
    "r4d_trellis_i8_quant_act_row": (None, [I64, I64, I64, I32, I64, I32, I64]),
    "r4d_i8_quant_act_plain": (None, [I64, I64, I64, I32, I32, I32, I64]),
    "r4d_gemm_i8_dense": (None, [I64] * 7 + [I32] * 5 + [I64]),
    "r4d_gemm_i8_dense_raw": (None, [I64] * 5 + [I32] * 4 + [I64]),
    "r4d_i8_pack_w": (None, [I64, I64, I32, I32, I64]),
    "r4d_gemm_i8_dense_check": (CSTR, [I32] * 4),
    "r4d_gemm_i8_dense_ws_bytes": (SZ, [I32] * 3),
    "r4d_mi355x_i8_skg": (I32, [I32, I32]),
    "r4d_mi355x_i8_dense_skg": (I32, [I32, I32, I32]),
    "r4d_trellis_i8_wscale_count": (SZ, [I32, I32]),
    "r4d_trellis_i8_wscale": (None, [I64, I64, I32, I32, I32, I64]),
    "r4d_trellis_i8_dump_w": (None, [I64, I64, I64, I64, I32, I32, I32, I64]),
    "r4d_gemm_trellis_nt_i8": (None, [I64, I64, I64, I64, I32] + [I64] * 6 + [I32] * 6 + [F32, I64]),
    "r4d_gemm_trellis_nt_i8_check": (CSTR, [I32] * 7),
    "r4d_gemm_trellis_nt_i8_ws_bytes": (SZ, [I32] * 3),
    "r4d_trellis_i8_wscale_col_count": (SZ, [I32, I32]),
    "r4d_trellis_i8_wscale_col": (None, [I64, I64, I32, I32, I32, I64]),
    "r4d_trellis_i8_dump_w_col": (None, [I64, I64, I64, I64, I32, I32, I32, I64]),
    "r4d_gemm_trellis_nt_i8c": (None, [I64, I64, I64, I64, I32] + [I64] * 6 + [I32] * 6 + [F32, I64]),
    "r4dx_trellis_gemv_xf": (None, [I64, I32, I64, I64, I32, I32] + [I64] * 5 + [I32] * 5 + [F32, I64]),
    "r4dx_trellis_gemv_xf_check": (CSTR, [I32] * 7),
    "r4dx_trellis_gemv_xf_parts_check": (CSTR, [I32, I32P] + [I32] * 6),
    "r4dx_trellis_gemv_xf_parts": (None, [I64, I32, I64P, I32P, I32, I32] + [I64] * 5 + [I32] * 5 + [F32, I64]),
    "r4dx_trellis_input_i8": (None, [I64, I64, I64, I32, I64P, I64P, I64P, I32, I64]),
    "r4dx_trellis_input_i8r": (None, [I64, I64, I64, I32, I64P, I64P, I64P, I32, I64]),
    "r4dx_trellis_input_bf16": (None, [I64, I64, I64, I32, I64P, I64P, I32, I64]),
    "r4dx_trellis_input_f16": (None, [I64, I64, I64, I32, I64P, I64P, I32, I64]),
    "r4dx_fwht128_f32": (None, [I64, I64, I32, I64]),
    "r4dx_gemm_trellis_nt_m64_parts_check": (CSTR, [I32, I32P, I32, I32, I32, I32, I32, I32]),
    "r4dx_gemm_trellis_nt_m64_parts": (None, [I64P, I32P, I32] + [I64] * 5 + [I32] * 5 + [F32, I64]),
    "r4dx_gemm_trellis_nt_m256_parts_check": (CSTR, [I32, I32P, I32, I32, I32, I32, I32]),
    "r4dx_gemm_trellis_nt_m256_parts": (None, [I64P, I32P, I32] + [I64] * 5 + [I32] * 5 + [F32, I64]),
    "r4d_trellis_wscale_count": (SZ, [I32, I32, I32]),
    "r4d_trellis_wscale_f32": (None, [I64, I64, I32, I32, I32, I32, I64]),
    "r4d_gemm_trellis_nt_m64_wq": (None, [I64, I64, I32, I64, I64, I64, I64, I64] + [I32] * 11 + [F32, I64, I32, I64]),
    "r4d_gemm_trellis_nt_m64_raw_wq": (None, [I64, I64, I32, I64, I64, I64, I64] + [I32] * 11 + [I64, I32, I64]),
    "r4d_gemm_trellis_nt_m256_wq": (None, [I64, I64, I32, I64, I64, I64, I64, I64] + [I32] * 8 + [F32, I64, I32, I64, I32]),
    "r4dx_silu_mul_trellis_bf16": (None, [I64] * 6 + [I32, I64]),
    "r4dx_attn_gate_mul_trellis_bf16": (None, [I64] * 6 + [I32, I64]),
    "r4dx_silu_mul_trellis_i8": (None, [I64] * 7 + [I32, I64]),
    "r4dx_attn_gate_mul_trellis_i8": (None, [I64] * 7 + [I32, I64]),
    "r4dx_silu_mul_trellis_i8r": (None, [I64] * 7 + [I32, I64]),
    "r4dx_attn_gate_mul_trellis_i8r": (None, [I64] * 7 + [I32, I64]),
    "r4dx_silu_mul_wide_bf16": (None, [I64] * 6),
    "r4dx_model_attn_gate_mul_bf16": (None, [I64] * 5),
    "r4dx_gemm_trellis_nt_m64_noalloc": (None, [I64, I64, I32, I64, I64, I64] + [I32] * 6 + [F32, I64]),
    "r4dx_gemm_trellis_nt_m64_noalloc_check": (CSTR, [I32] * 6),
    "r4dx_gemm_trellis_nt_m64_noalloc_max_ws_bytes": (SZ, []),
}

_lib = None


def header_symbols():
    """Every function name declared in include/r4d_mi355x.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(r4dx?_[a-z0-9_]+)\s*\(", text)))


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() "
                               "(python -m r4dx_amd.build); there is no fallback path")
        _lib = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGS.items():
            f = getattr(_lib, name)
            f.restype = res
            f.argtypes = args
    return _lib
