"""The MI355X tuning plan of a trellis linear: which kernel runs an M-row chunk and with which split knobs.

Replaces the reference's RDNA4 tables (src/model/gemm_tuning_table_trellis*.inc) and the rules around them
(`TrellisTuningFor`, `PlanTrellisM256`, `PlanTrellisI8`, src/model/linear.cpp:680-767), keeping their
contract:

* every M <= 16 gets the same (SK, SKG), so a verify row's bits equal the decode row's (the row-identity rule,
  src/model/linear.cpp:33-53);
* the M = 64 band's row is (SK = 2, SKG of the M = 256 plan): SK 1 and 2 both name the one-wave-per-pair order
  r4d_gemm_trellis_nt_m256 reproduces bit for bit, so an M = 256 chunk and four M = 64 chunks of the same rows
  agree, and SK = 2 lets the engine's PlanTrellisM256 (src/model/linear.cpp:705-722, skw <= SK, skw from
  {2, 4, 8}) find its K-slice grouping;
* every SKG is a power of two up to 8, the only values the engine's tuning rows may hold (TrellisRowFits,
  src/model/linear.cpp:243-255);
* a plan is refused, with the reason, when the shape breaks the loader's rules (KB 4 or 5 for the prefill
  kernels, 1 or 2 parts, whole 128-blocks, a part boundary inside N) or the kernel's own `_check` refuses it --
  so a plan never names a launch that would throw.
"""
from dataclasses import dataclass

from .loader import lib

DECODE_M = 16          # rows that share the decode tuning
CHUNK_M = 64           # the M = 64 band
PREFILL_M = 256        # the prefill GEMMs' rows


@dataclass
class Plan:
    ok: bool
    why: str = ""
    kernel: str = ""   # "m64" (r4d_gemm_trellis_nt_m64), "m256", "i8" / "i8c"
    SK: int = 0        # m64: 1 or 2 = one wave per tile pair over its slice, 4 = four waves in k order
    SKG: int = 1       # K slices across the grid
    skw: int = 0       # int8: the caller's skw argument (checked, not a kernel knob here)


def _shape_why(N, K, kb, parts, part_n0, rates=(3, 4, 5)):
    if kb not in rates:
        return f"KB is not one of {rates}"
    if parts not in (1, 2):
        return "trellis parts is not 1 or 2"
    if N <= 0 or K <= 0 or N > 0x7FFFFFFF or K > 0x7FFFFFFF:
        return "shape out of range"
    if N % 128 or K % 128:
        return "N and K must be whole 128-blocks"
    if parts == 2 and (part_n0 <= 0 or part_n0 >= N or part_n0 % 128):
        return "part boundary is not a whole 128-block inside N"
    return ""


def m256_skg(N, K, kb):
    return int(lib().r4d_mi355x_trellis_m256_skg(K, N, kb))


def linear_tuning(N, K, kb, M, parts=1, part_n0=None):
    """The (SK, SKG) of r4d_gemm_trellis_nt_m64 for an M-row chunk (M <= 64)."""
    why = _shape_why(N, K, kb, parts, part_n0 or 0)
    if why:
        return Plan(False, why)
    if not 1 <= M <= CHUNK_M:
        return Plan(False, "M must be 1..64 for r4d_gemm_trellis_nt_m64")
    if M <= DECODE_M:
        SK, SKG = 4, int(lib().r4d_mi355x_trellis_gemv_skg(K, N, kb))
    else:
        SK, SKG = 2, m256_skg(N, K, kb)
    n_split = part_n0 if parts == 2 else N
    msg = lib().r4d_gemm_trellis_nt_m64_check(M, K, N, n_split, kb, SKG, 1, 1, 1)
    if msg:
        return Plan(False, msg.decode())
    return Plan(True, "", "m64", SK, SKG)


def plan_trellis_m256(N, K, kb, parts=1, part_n0=None, M=PREFILL_M):
    """PlanTrellisM256 (linear.cpp:680-722): the M = 64 band's (SK = 2, SKG), skw = 2 (the first of the engine's
    preference order {2, 4, 8, 2} not above SK)."""
    why = _shape_why(N, K, kb, parts, part_n0 or 0, rates=(4, 5))
    if why:
        return Plan(False, why)
    skg = m256_skg(N, K, kb)
    n_split = part_n0 if parts == 2 else N
    msg = lib().r4d_gemm_trellis_nt_m256_check(M, K, N, n_split, kb, 2, 1, skg, 4, 2)
    if msg:
        return Plan(False, msg.decode())
    return Plan(True, "", "m256", 2, skg, 2)


def plan_trellis_i8(N, K, kb, parts=1, part_n0=None, coarse=False):
    """PlanTrellisI8 (linear.cpp:724-766): this build's skg per shape (no table row needed) and the first skw
    (2, 4, 8: the caller's argument, checked but not a kernel knob here) the kernel's own rules accept."""
    why = _shape_why(N, K, kb, parts, part_n0 or 0, rates=(4, 5))
    if why:
        return Plan(False, why)
    n_split = part_n0 if parts == 2 else N
    first = ""
    # the library's skg first, then smaller splits: (K / 128) must hold skw * skg, and a rank K such as 8704
    # (68 blocks = 4 * 17) takes skg 4 alone but no skw >= 2 beside it
    skg = int(lib().r4d_mi355x_i8_skg(K, N))
    while skg >= 1:
        for skw in (2, 4, 8):
            msg = lib().r4d_gemm_trellis_nt_i8_check(PREFILL_M, K, N, n_split, kb, skw, skg)
            if not msg:
                return Plan(True, "", "i8c" if coarse else "i8", 0, skg, skw)
            first = first or msg.decode()
        skg //= 2
    return Plan(False, first)
