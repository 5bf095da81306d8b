"""Python mirrors of the C entry points, over torch device tensors.  Each call validates through the
library's own _check entry (or the same rules) first, so an illegal shape raises ValueError here
instead of an uncaught C++ exception crossing ctypes."""
import ctypes as C

import numpy as np
import torch

from .loader import lib


def _p(t):
    return 0 if t is None else t.data_ptr()


def _stream(stream=None):
    s = torch.cuda.current_stream() if stream is None else stream
    return s.cuda_stream


class TicketBuffer:
    """The per-linear tickets of the split GEMMs, r4d_gemm_trellis_nt_m64_tickets_bytes(N) (one 128-byte line per
    128-column group; zeroed once, every complete launch leaves them zero)."""

    def __init__(self, N, device="cuda"):
        nbytes = lib().r4d_gemm_trellis_nt_m64_tickets_bytes(N)
        self.t = torch.zeros(max(1, nbytes // 4), dtype=torch.int32, device=device)


def _wq_args(wq, K, KB):
    """(table pointer, gsh) of a _wq call, with the entries' own rules raised here as ValueError."""
    tab, gsh = wq
    if tab is None:
        raise ValueError("the _wq entry needs a scale table (trellis_wscale)")
    if gsh not in (1, 2, 3) or K % (16 << gsh):
        raise ValueError("gsh must be 1, 2 or 3 with 16 << gsh dividing K")
    if KB not in (4, 5):
        raise ValueError("KB must be 4 or 5")
    return _p(tab), gsh


def trellis_gemv_skg(K, N, KB):
    return lib().r4d_mi355x_trellis_gemv_skg(K, N, KB)


def trellis_gemm_m64(a0, w, svh, K, N, KB, skg=None, a1=None, n_split=None, out=None, ws=None,
                     tickets=None, out_scale=1.0, raw=False, stream=None, sk=0, clk=None, wq=None):
    """C = r4d_gemm_trellis_nt_m64 (bf16 [M][N]) or, raw=True, its _raw fp32 A @ Q. sk = 1: the one-wave-per-
    pair summation order that r4d_gemm_trellis_nt_m256 reproduces bit for bit. clk (raw only): an int64
    device tensor of 4 that receives workgroup (0, 0)'s shader clock and wall clock at entry and at the end
    of its own work. wq = (table, gsh): the _wq entry, every decoded weight fake-quantized to int8 under the
    table of trellis_wscale (not with clk)."""
    L = lib()
    M = a0.shape[0]
    skg = trellis_gemv_skg(K, N, KB) if skg is None else skg
    n_split = N if n_split is None else n_split
    if ws is None and skg > 1:
        ws = torch.empty(L.r4d_gemm_trellis_nt_m64_ws_bytes(M, N, skg) // 4, dtype=torch.float32,
                         device=a0.device)
    if tickets is None and skg > 1:
        tickets = TicketBuffer(N, a0.device).t
    msg = L.r4d_gemm_trellis_nt_m64_check(M, K, N, n_split, KB, skg, 0 if raw else 1,
                                          int(svh is not None), int(ws is not None and tickets is not None))
    if msg:
        raise ValueError(msg.decode())
    if wq is not None:
        if clk is not None:
            raise ValueError("the _wq entries take no clock probe")
        tab, gsh = _wq_args(wq, K, KB)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32 if raw else torch.bfloat16, device=a0.device)
    st = _stream(stream)
    if wq is not None:
        if raw:
            L.r4d_gemm_trellis_nt_m64_raw_wq(_p(a0), _p(a1), n_split, _p(w), _p(out), _p(ws), _p(tickets),
                                             M, K, N, KB, 0, sk, 0, 0, skg, 0, 0, tab, gsh, st)
        else:
            L.r4d_gemm_trellis_nt_m64_wq(_p(a0), _p(a1), n_split, _p(w), _p(svh), _p(out), _p(ws), _p(tickets),
                                         M, K, N, KB, 0, sk, 0, 0, skg, 0, 0, float(out_scale), tab, gsh, st)
    elif raw:
        L.r4d_gemm_trellis_nt_m64_raw(_p(a0), _p(a1), n_split, _p(w), _p(out), _p(ws), _p(tickets),
                                      M, K, N, KB, 0, sk, 0, 0, skg, 0, 0, _p(clk), st)
    else:
        L.r4d_gemm_trellis_nt_m64(_p(a0), _p(a1), n_split, _p(w), _p(svh), _p(out), _p(ws), _p(tickets),
                                  M, K, N, KB, 0, sk, 0, 0, skg, 0, 0, float(out_scale), st)
    return out


def trellis_gemm_m64_parts(a_parts, n0, w, svh, K, N, KB, skg=None, out=None, ws=None, tickets=None,
                           out_scale=1.0, stream=None):
    """r4dx_gemm_trellis_nt_m64_parts: one linear whose columns [n0[p], n0[p + 1]) read a_parts[p] (bf16 [M][N])."""
    L = lib()
    M = a_parts[0].shape[0]
    parts = len(a_parts)
    skg = trellis_gemv_skg(K, N, KB) if skg is None else skg
    if ws is None and skg > 1:
        ws = torch.empty(L.r4d_gemm_trellis_nt_m64_ws_bytes(M, N, skg) // 4, dtype=torch.float32, device=w.device)
    if tickets is None and skg > 1:
        tickets = TicketBuffer(N, w.device).t
    n0a = (C.c_int * parts)(*n0)
    msg = L.r4dx_gemm_trellis_nt_m64_parts_check(parts, n0a, M, K, N, KB, skg, int(ws is not None and tickets is not None))
    if msg:
        raise ValueError(msg.decode())
    if any(a.shape != (M, K) for a in a_parts) or svh is None:
        raise ValueError("every part input is [M][K]; svh is required")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=w.device)
    pa = (C.c_int64 * parts)(*[a.data_ptr() for a in a_parts])
    L.r4dx_gemm_trellis_nt_m64_parts(pa, n0a, parts, _p(w), _p(svh), _p(out), _p(ws), _p(tickets), M, K, N, KB, skg,
                                     float(out_scale), _stream(stream))
    return out


def trellis_gemm_m256_parts(a_parts, n0, w, svh, K, N, KB, skg=None, out=None, ws=None, tickets=None,
                            out_scale=1.0, stream=None):
    """r4dx_gemm_trellis_nt_m256_parts: the M = 128 / 256 GEMM of one linear whose columns [n0[p], n0[p + 1]) read
    a_parts[p] (bf16 [M][N])."""
    L = lib()
    M = a_parts[0].shape[0]
    parts = len(a_parts)
    skg = trellis_m256_skg(K, N, KB) if skg is None else skg
    n0a = (C.c_int * parts)(*n0)
    msg = L.r4dx_gemm_trellis_nt_m256_parts_check(parts, n0a, M, K, N, KB, skg)
    if msg:
        raise ValueError(msg.decode())
    if any(a.shape != (M, K) for a in a_parts) or svh is None:
        raise ValueError("every part input is [M][K]; svh is required")
    if ws is None:
        ws = torch.empty(L.r4d_gemm_trellis_nt_m256_ws_bytes(M, N, skg) // 4, dtype=torch.float32, device=w.device)
    if tickets is None:
        tickets = TicketBuffer(N, w.device).t
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=w.device)
    pa = (C.c_int64 * parts)(*[a.data_ptr() for a in a_parts])
    L.r4dx_gemm_trellis_nt_m256_parts(pa, n0a, parts, _p(w), _p(svh), _p(out), _p(ws), _p(tickets), M, K, N, KB, skg,
                                      float(out_scale), _stream(stream))
    return out


def trellis_m256_skg(K, N, KB):
    return lib().r4d_mi355x_trellis_m256_skg(K, N, KB)


def trellis_gemm_m256(a0, w, svh, K, N, KB, skg=None, a1=None, n_split=None, out=None, ws=None,
                      tickets=None, out_scale=1.0, raw=False, stream=None, wq=None, sk=0):
    """C = r4d_gemm_trellis_nt_m256 (bf16 [M][N], M = 128 or 256) or, raw=True, fp32 A @ Q. wq = (table, gsh):
    r4d_gemm_trellis_nt_m256_wq (bf16 only). sk: the M = 64 row's SK to reproduce (0 / 1 / 2: the one-wave order;
    4 / 8 / 16: the 4-wave order, bf16 entries only -- the raw entry has no SK)."""
    L = lib()
    M = a0.shape[0]
    skg = trellis_m256_skg(K, N, KB) if skg is None else skg
    n_split = N if n_split is None else n_split
    if raw and sk not in (0, 1, 2):
        raise ValueError("r4d_gemm_trellis_nt_m256_raw computes the one-wave order only (sk 0, 1 or 2)")
    msg = L.r4d_gemm_trellis_nt_m256_check(M, K, N, n_split, KB, sk, 0, skg, 0, 0)
    if msg:
        raise ValueError(msg.decode())
    if wq is not None:
        if raw:
            raise ValueError("r4d_gemm_trellis_nt_m256_wq has no raw form")
        _wq_args(wq, K, KB)
    # ws and tickets as the reference requires them (r4d.h:406-407): the split slices and the balanced form's
    # hand-over of cut units use them
    if ws is None:
        ws = torch.empty(L.r4d_gemm_trellis_nt_m256_ws_bytes(M, N, skg) // 4, dtype=torch.float32,
                         device=a0.device)
    if tickets is None:
        tickets = TicketBuffer(N, a0.device).t
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32 if raw else torch.bfloat16, device=a0.device)
    st = _stream(stream)
    if wq is not None:
        if raw:
            raise ValueError("r4d_gemm_trellis_nt_m256_wq has no raw form")
        tab, gsh = _wq_args(wq, K, KB)
        L.r4d_gemm_trellis_nt_m256_wq(_p(a0), _p(a1), n_split, _p(w), _p(svh), _p(out), _p(ws), _p(tickets),
                                      M, K, N, KB, sk, 0, skg, 0, float(out_scale), st, 0, tab, gsh)
    elif raw:
        L.r4d_gemm_trellis_nt_m256_raw(_p(a0), _p(a1), n_split, _p(w), _p(out), _p(ws), _p(tickets),
                                       M, K, N, KB, skg, st)
    else:
        L.r4d_gemm_trellis_nt_m256(_p(a0), _p(a1), n_split, _p(w), _p(svh), _p(out), _p(ws), _p(tickets),
                                   M, K, N, KB, sk, 0, skg, 0, float(out_scale), st, 0)
    return out


def trellis_wscale(w, K, N, KB, gsh, out=None, stream=None):
    """The fake-quant scale table [K / 16 >> gsh][N] of r4d_trellis_wscale_f32 (fp32 max|Q| / 127 per column
    and group of 2^gsh k-tiles, 1 for an all-zero group)."""
    L = lib()
    n = L.r4d_trellis_wscale_count(K, N, gsh)
    if n == 0 or KB not in (4, 5) or N % 32 or K % (16 << gsh) or (K // 16) % 4:
        raise ValueError("trellis_wscale: KB 4 or 5, N a multiple of 32, gsh 1..3, 16 << gsh and 64 dividing K")
    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=w.device)
    L.r4d_trellis_wscale_f32(_p(w), _p(out), K, N, KB, gsh, _stream(stream))
    return out


def trellis_reconstruct(w, K, N, KB, stream=None):
    q = torch.empty((K, N), dtype=torch.int16, device=w.device)
    lib().r4d_trellis_reconstruct_f16(_p(w), _p(q), K, N, KB, _stream(stream))
    return q


def trellis_input(x, suh_list, prescale=0, bf16=True, outs=None, stream=None):
    M, K = x.shape
    n = len(suh_list)
    if not 1 <= n <= 3 or K % 128:
        raise ValueError("nout must be 1..3 and K a multiple of 128")
    if outs is None:
        outs = [torch.empty((M, K), dtype=torch.float16, device=x.device) for _ in range(n)]
    suh = (C.c_int64 * n)(*[s.data_ptr() for s in suh_list])
    out = (C.c_int64 * n)(*[o.data_ptr() for o in outs])
    f = lib().r4dx_trellis_input_bf16 if bf16 else lib().r4dx_trellis_input_f16
    f(_p(x), M, K, n, suh, out, prescale, _stream(stream))
    return outs


def fwht128(x, stream=None):
    lib().r4dx_fwht128_f32(_p(x), x.numel() // 128, 0, _stream(stream))
    return x


def w4a16_gemm(a, wq, wsz, K, N, group=64, out=None, f32=False, stream=None):
    """C = r4d_gemm_w4a16_nt_m64_g (bf16) or, f32=True, r4d_gemm_w4a16_nt_m64_f32 (fp32 logits)."""
    L = lib()
    M = a.shape[0]
    msg = L.r4d_gemm_w4a16_nt_m64_check(group, M, K, N)
    if msg:
        raise ValueError(msg.decode())
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32 if f32 else torch.bfloat16, device=a.device)
    st = _stream(stream)
    if f32:
        L.r4d_gemm_w4a16_nt_m64_f32(group, _p(a), _p(wq), _p(wsz), _p(out), M, K, N, st)
    else:
        L.r4d_gemm_w4a16_nt_m64_g(group, _p(a), _p(wq), _p(wsz), _p(out), M, K, N, 0, 0, 0, 0, 0, st)
    return out


_argmax_streams = set()   # (device, stream) pairs whose argmax scratch the library has allocated


def _argmax_scratch_ready(device, st):
    key = (device, st)
    if key not in _argmax_streams and torch.cuda.is_current_stream_capturing():
        # the library allocates a stream's argmax scratch at its first call, which graph capture forbids
        raise ValueError("argmax: the stream's first argmax is under graph capture; run one on it before capturing")
    _argmax_streams.add(key)


def w4a16_gemm_argmax(a, wq, wsz, K, N, group=64, out=None, out_idx=None, out_val=None, stream=None):
    """fp32 logits [M][N] and their per-row argmax (int32 [M], fp32 [M]) in one launch
    (r4d_gemm_w4a16_nt_m64_f32_argmax)."""
    L = lib()
    M = a.shape[0]
    msg = L.r4d_gemm_w4a16_nt_m64_check(group, M, K, N)
    if msg:
        raise ValueError(msg.decode())
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=a.device)
    if out_idx is None:
        out_idx = torch.empty(M, dtype=torch.int32, device=a.device)
    if out_val is None:
        out_val = torch.empty(M, dtype=torch.float32, device=a.device)
    st = _stream(stream)
    _argmax_scratch_ready(a.device.index, st)
    L.r4d_gemm_w4a16_nt_m64_f32_argmax(group, _p(a), _p(wq), _p(wsz), _p(out), _p(out_idx), _p(out_val), M, K, N, st)
    return out, out_idx, out_val


def argmax_rows(logits, out_idx=None, out_val=None, stream=None):
    """Per-row argmax of a [rows][vocab] fp32 or bf16 tensor: (int32 [rows], fp32 [rows])."""
    L = lib()
    rows, vocab = logits.shape
    if out_idx is None:
        out_idx = torch.empty(rows, dtype=torch.int32, device=logits.device)
    if out_val is None:
        out_val = torch.empty(rows, dtype=torch.float32, device=logits.device)
    if not 1 <= rows <= 64 or vocab < 1:
        raise ValueError("argmax: rows must be 1..64 and vocab >= 1")
    st = _stream(stream)
    _argmax_scratch_ready(logits.device.index, st)
    if logits.dtype == torch.float32:
        L.r4dx_argmax_rows_f32(_p(logits), logits.stride(0), _p(out_idx), _p(out_val), 1, rows, vocab, st)
    elif logits.dtype == torch.bfloat16 and rows == 1:
        L.r4dx_argmax_val_bf16(_p(logits), _p(out_idx), _p(out_val), vocab, st)
    else:
        raise ValueError("fp32 rows or a single bf16 row")
    return out_idx, out_val


def i8_quant(x, blk=False, ref_layout=True, stream=None):
    """Activation quantizer: x f16 [M][K] -> (a8 int8, sa fp32). ref_layout: the A8 fragment layout (M = 256,
    r4d_trellis_i8_quant_act / _row, what the GEMMs read); else plain [M][K] (r4d_i8_quant_act_plain)."""
    L = lib()
    M, K = x.shape
    a8 = torch.empty(M * K, dtype=torch.int8, device=x.device)
    sa = torch.empty((K // 128) * M if blk else M, dtype=torch.float32, device=x.device)
    st = _stream(stream)
    if ref_layout:
        f = L.r4d_trellis_i8_quant_act if blk else L.r4d_trellis_i8_quant_act_row
        f(_p(x), _p(a8), _p(sa), 1, 0, K, st)
    else:
        L.r4d_i8_quant_act_plain(_p(x), _p(a8), _p(sa), M, K, int(blk), st)
    return a8, sa


def i8_pack_w(wp, out=None, stream=None):
    """Plain int8 [N][K] -> the W8 block layout (r4d_i8_pack_w)."""
    N, K = wp.shape
    out = torch.empty(N * K, dtype=torch.int8, device=wp.device) if out is None else out
    lib().r4d_i8_pack_w(_p(wp), _p(out), N, K, _stream(stream))
    return out


def i8_dense_skg(K, N, scale_mode=0):
    """The dense GEMM's launch form (r4d_mi355x_i8_dense_skg): 0 = stream-K, else the K split."""
    return lib().r4d_mi355x_i8_dense_skg(K, N, scale_mode)


class I8Workspace:
    """ws + the self-resetting tickets of a split int8 launch (one per linear; never two launches in flight)."""

    def __init__(self, N, skg, device):
        nb = lib().r4d_gemm_i8_dense_ws_bytes(256, N, skg)
        self.ws = torch.empty(max(1, nb // 4), dtype=torch.int32, device=device)
        self.tickets = torch.zeros(max(1, N // 128), dtype=torch.int32, device=device)


def i8_dense_gemm(a8, sa, w8, sw, K, N, scale_mode=0, skg=None, raw=False, out=None, work=None, stream=None):
    """C f16 [256][N] = r4d_gemm_i8_dense (a8 A8 layout, w8 W8 block layout), or raw=True the exact int32
    sums (r4d_gemm_i8_dense_raw)."""
    L = lib()
    M = 256
    skg = i8_dense_skg(K, N, scale_mode) if skg is None else skg
    msg = L.r4d_gemm_i8_dense_check(M, K, N, skg)
    if msg:
        raise ValueError(msg.decode())
    if work is None:
        work = I8Workspace(N, skg, a8.device)
    if out is None:
        out = torch.empty((M, N), dtype=torch.int32 if raw else torch.float16, device=a8.device)
    st = _stream(stream)
    if raw:
        L.r4d_gemm_i8_dense_raw(_p(a8), _p(w8), _p(out), _p(work.ws), _p(work.tickets), M, K, N, skg, st)
    else:
        L.r4d_gemm_i8_dense(_p(a8), _p(sa), _p(w8), _p(sw), _p(out), _p(work.ws), _p(work.tickets), M, K, N, skg,
                            scale_mode, st)
    return out


def trellis_i8_table(w, K, N, KB, coarse=False, stream=None):
    """The weight scale table: SW [K/128][N] (r4d_trellis_i8_wscale) or SWC [N] (coarse, _wscale_col)."""
    L = lib()
    n = L.r4d_trellis_i8_wscale_col_count(K, N) if coarse else L.r4d_trellis_i8_wscale_count(K, N)
    sw = torch.empty(n, dtype=torch.float32, device=w.device)
    (L.r4d_trellis_i8_wscale_col if coarse else L.r4d_trellis_i8_wscale)(_p(w), _p(sw), K, N, KB, _stream(stream))
    return sw


def trellis_i8_dump(w, sw, K, N, KB, coarse=False, plain=True, stream=None):
    """The int8 weights the GEMM quantizes on the fly: (w8 block layout, plain [N][K] or None)."""
    L = lib()
    w8 = torch.empty(N * K, dtype=torch.int8, device=w.device)
    wp = torch.empty((N, K), dtype=torch.int8, device=w.device) if plain else None
    f = L.r4d_trellis_i8_dump_w_col if coarse else L.r4d_trellis_i8_dump_w
    f(_p(w), _p(sw), _p(w8), _p(wp) if plain else 0, K, N, KB, _stream(stream))
    return w8, wp


def trellis_gemm_i8(a8, sa, w, sw, svh, K, N, KB, coarse=False, a8_1=None, sa_1=None, n_split=None, skw=2, skg=1,
                    out=None, ws=None, out_scale=1.0, stream=None):
    """C bf16 [256][N] = r4d_gemm_trellis_nt_i8 (per-128 scales) or _i8c (coarse)."""
    L = lib()
    M = 256
    n_split = N if n_split is None else n_split
    msg = L.r4d_gemm_trellis_nt_i8_check(M, K, N, n_split, KB, skw, skg)
    if msg:
        raise ValueError(msg.decode())
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a8.device)
    if ws is None and skg > 1:
        ws = torch.empty(L.r4d_gemm_trellis_nt_i8_ws_bytes(M, N, skg) // 4, dtype=torch.float32, device=a8.device)
    f = L.r4d_gemm_trellis_nt_i8c if coarse else L.r4d_gemm_trellis_nt_i8
    f(_p(a8), _p(sa), _p(a8_1) if a8_1 is not None else 0, _p(sa_1) if sa_1 is not None else 0, n_split, _p(w), _p(sw),
      _p(svh), _p(out), _p(ws) if ws is not None else 0, 0, M, K, N, KB, skw, skg, out_scale, _stream(stream))
    return out


def trellis_gemv_xf(x, suh, w, svh, K, N, KB, skg=None, suh1=None, n_split=None, prescale=0, bf16=False, out=None,
                    ws=None, tickets=None, out_scale=1.0, stream=None):
    """The input transform fused into the GEMV (r4dx_trellis_gemv_xf): x f16/bf16 bits [M][K] -> C bf16 [M][N]."""
    L = lib()
    M = x.shape[0]
    if skg is None:   # the planner's split, lowered to whole 128-blocks per slice
        skg = trellis_gemv_skg(K, N, KB)
        while (K // 128) % skg:
            skg -= 1
    n_split = N if n_split is None else n_split
    have_ws = skg > 1 or (ws is not None and tickets is not None)
    msg = L.r4dx_trellis_gemv_xf_check(M, K, N, n_split, KB, skg, int(have_ws))
    if msg:
        raise ValueError(msg.decode())
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    if have_ws and ws is None:
        ws = torch.empty(max(1, skg * M * N), dtype=torch.float32, device=x.device)
    if have_ws and tickets is None:
        tickets = TicketBuffer(N, x.device).t
    L.r4dx_trellis_gemv_xf(_p(x), int(bf16), _p(suh), _p(suh1), n_split, prescale, _p(w), _p(svh), _p(out),
                           _p(ws) if have_ws else 0, _p(tickets) if have_ws else 0, M, K, N, KB, skg, out_scale,
                           _stream(stream))
    return out


def trellis_gemv_xf_parts(x, suh_parts, n0, w, svh, K, N, KB, skg=None, prescale=0, bf16=False, out=None, ws=None,
                          tickets=None, out_scale=1.0, stream=None):
    """r4dx_trellis_gemv_xf_parts: the input transform fused into the parts launch -- columns [n0[p], n0[p + 1]) use
    suh_parts[p]; x f16/bf16 bits [M][K] -> C bf16 [M][N]."""
    L = lib()
    M = x.shape[0]
    parts = len(suh_parts)
    if skg is None:   # the planner's split, lowered to whole 128-blocks per slice
        skg = trellis_gemv_skg(K, N, KB)
        while (K // 128) % skg:
            skg -= 1
    have_ws = skg > 1 or (ws is not None and tickets is not None)
    n0a = (C.c_int * parts)(*n0)
    msg = L.r4dx_trellis_gemv_xf_parts_check(parts, n0a, M, K, N, KB, skg, int(have_ws))
    if msg:
        raise ValueError(msg.decode())
    if x.shape != (M, K) or svh is None or not -24 <= prescale <= 24:
        raise ValueError("x is [M][K], svh is required, |prescale| <= 24")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    if have_ws and ws is None:
        ws = torch.empty(max(1, skg * M * N), dtype=torch.float32, device=x.device)
    if have_ws and tickets is None:
        tickets = TicketBuffer(N, x.device).t
    sa = (C.c_int64 * parts)(*[s.data_ptr() for s in suh_parts])
    L.r4dx_trellis_gemv_xf_parts(_p(x), int(bf16), sa, n0a, parts, prescale, _p(w), _p(svh), _p(out),
                                 _p(ws) if have_ws else 0, _p(tickets) if have_ws else 0, M, K, N, KB, skg,
                                 float(out_scale), _stream(stream))
    return out


def trellis_input_i8(x, suh_list, prescale=0, row_scale=False, outs=None, stream=None):
    """The input transform fused with the activation quantizer (r4dx_trellis_input_i8 / _i8r): x bf16 bits
    [256][K] -> per output (a8 A8 layout, sa [K/128][256] or [256]); outs: preallocated (a8, sa) pairs."""
    M, K = x.shape
    n = len(suh_list)
    if outs is None:
        outs = [(torch.empty(M * K, dtype=torch.int8, device=x.device),
                 torch.empty(M if row_scale else (K // 128) * M, dtype=torch.float32, device=x.device))
                for _ in range(n)]
    a8 = [o[0] for o in outs]
    sa = [o[1] for o in outs]
    arr = lambda ts: (C.c_int64 * n)(*[t.data_ptr() for t in ts])
    f = lib().r4dx_trellis_input_i8r if row_scale else lib().r4dx_trellis_input_i8
    f(_p(x), M, K, n, arr(suh_list), arr(a8), arr(sa), prescale, _stream(stream))
    return list(zip(a8, sa))


def silu_mul(gate_up, intermediate, out=None, stream=None):
    """r4dx_silu_mul_wide_bf16: bf16 [rows][intermediate] = bf16(g * sigmoid(g) * u) from gate_up bf16 rows
    [gate | up] (row stride gate_up.stride(0))."""
    rows = gate_up.shape[0]
    if out is None:
        out = torch.empty((rows, intermediate), dtype=gate_up.dtype, device=gate_up.device)
    lib().r4dx_silu_mul_wide_bf16(_p(gate_up), _p(out), rows, intermediate, gate_up.stride(0), _stream(stream))
    return out


def attn_gate_mul(attn_out, gate, out=None, stream=None):
    """r4dx_model_attn_gate_mul_bf16: bf16(attn_out * sigmoid(gate)) elementwise."""
    if out is None:
        out = torch.empty_like(attn_out)
    lib().r4dx_model_attn_gate_mul_bf16(_p(attn_out), _p(gate), _p(out), attn_out.numel(), _stream(stream))
    return out


def _producer_check(K, rows, prescale):
    if K <= 0 or K % 128 or not 0 <= rows <= 65535 or abs(prescale) > 24:
        raise ValueError("K must be a positive multiple of 128, rows 0..65535, |prescale| <= 24")


def silu_mul_trellis(gate_up, intermediate, suh, prescale=0, quant=None, out=None, stream=None):
    """The MLP producer fused into mlp.down's input transform: quant None -> f16 A [rows][intermediate]
    (r4dx_silu_mul_trellis_bf16); 'blk' / 'row' -> (a8, sa) for the int8 GEMM (r4dx_silu_mul_trellis_i8 / _i8r,
    rows == 256)."""
    rows, stride = gate_up.shape[0], gate_up.stride(0)
    _producer_check(intermediate, rows, prescale)
    if stride < 2 * intermediate:
        raise ValueError("gate_up's row stride must be >= 2 * intermediate")
    st = _stream(stream)
    if quant is None:
        if out is None:
            out = torch.empty((rows, intermediate), dtype=torch.float16, device=gate_up.device)
        lib().r4dx_silu_mul_trellis_bf16(_p(gate_up), rows, intermediate, stride, _p(suh), _p(out), prescale, st)
        return out
    if rows != 256:
        raise ValueError("the int8 forms take exactly 256 rows")
    a8, sa = out if out is not None else (
        torch.empty(256 * intermediate, dtype=torch.int8, device=gate_up.device),
        torch.empty(256 if quant == "row" else (intermediate // 128) * 256, dtype=torch.float32, device=gate_up.device))
    f = lib().r4dx_silu_mul_trellis_i8r if quant == "row" else lib().r4dx_silu_mul_trellis_i8
    f(_p(gate_up), rows, intermediate, stride, _p(suh), _p(a8), _p(sa), prescale, st)
    return a8, sa


def attn_gate_mul_trellis(attn_out, gate, suh, prescale=0, quant=None, out=None, stream=None):
    """The attention output gate fused into attn.o's input transform: quant None -> f16 A [rows][K]
    (r4dx_attn_gate_mul_trellis_bf16); 'blk' / 'row' -> (a8, sa) (r4dx_attn_gate_mul_trellis_i8 / _i8r)."""
    rows, K = attn_out.shape
    _producer_check(K, rows, prescale)
    st = _stream(stream)
    if quant is None:
        if out is None:
            out = torch.empty((rows, K), dtype=torch.float16, device=attn_out.device)
        lib().r4dx_attn_gate_mul_trellis_bf16(_p(attn_out), _p(gate), rows, K, _p(suh), _p(out), prescale, st)
        return out
    if rows != 256:
        raise ValueError("the int8 forms take exactly 256 rows")
    a8, sa = out if out is not None else (
        torch.empty(256 * K, dtype=torch.int8, device=attn_out.device),
        torch.empty(256 if quant == "row" else (K // 128) * 256, dtype=torch.float32, device=attn_out.device))
    f = lib().r4dx_attn_gate_mul_trellis_i8r if quant == "row" else lib().r4dx_attn_gate_mul_trellis_i8
    f(_p(attn_out), _p(gate), rows, K, _p(suh), _p(a8), _p(sa), prescale, st)
    return a8, sa


def trellis_linear_to_device(lin, device):
    """A container.TrellisLinear's arrays as device tensors: words int32, suh fp32 per part, svh fp32."""
    return {"words": torch.from_numpy(lin.words.view(np.int32)).to(device),
            "suh": [torch.from_numpy(s).to(device) for s in lin.suh],
            "svh": torch.from_numpy(lin.svh).to(device)}


def trellis_linear(x, lin, dev_t, out_scale=None, stream=None):
    """y bf16 [M][N] = the trellis linear `lin` (container.TrellisLinear, its device tensors dev_t) of x bf16
    [M][K]: the input transform (one output per part, the linear's prescale), then r4d_gemm_trellis_nt_m64
    (M <= 64) or r4d_gemm_trellis_nt_m256 (M = 128 or 256), a two-part linear split at its first part. The
    default out_scale is the engine's float(2^-prescale / sqrt(128)) (src/model/linear.cpp:1074)."""
    M, K = x.shape
    if out_scale is None:
        out_scale = float(np.float32(np.ldexp(1.0, -lin.prescale_log2) / np.sqrt(128.0)))
    if K != lin.K:
        raise ValueError(f"x has K = {K}, the linear {lin.base} K = {lin.K}")
    a = trellis_input(x, dev_t["suh"], lin.prescale_log2, stream=stream)
    a1 = a[1] if len(a) > 1 else None
    n_split = lin.parts[0] if lin.parts else None
    if M <= 64:
        return trellis_gemm_m64(a[0], dev_t["words"], dev_t["svh"], lin.K, lin.N, lin.KB, a1=a1, n_split=n_split,
                                out_scale=out_scale, stream=stream)
    return trellis_gemm_m256(a[0], dev_t["words"], dev_t["svh"], lin.K, lin.N, lin.KB, a1=a1, n_split=n_split,
                             out_scale=out_scale, stream=stream)
