"""The trellis int8 kernel's per-128 weight scale: rs = f16(min(1 / s_eff, 60000)) is formed with the hardware
reciprocal (about 1 ulp) instead of an IEEE divide. The claim the kernel rests on: for every table entry the format
produces -- s_eff = fp32(1 / rs) of an f16 rs in [2^-14, 60000] -- any fp32 within 3 ulps of 1 / s_eff converts back
to the same rs. Checked exhaustively (every normal f16 up to 60000)."""
import numpy as np


def test_reciprocal_of_seff_returns_rs_within_three_ulps():
    h = np.arange(0x0400, 0x7C00, dtype=np.uint16).view(np.float16)
    h = h[h.astype(np.float32) <= 60000]
    seff = np.float32(1.0) / h.astype(np.float32)
    exact = np.float32(1.0) / seff
    for d in range(-3, 4):
        r = (exact.view(np.int32) + np.int32(d)).view(np.float32)
        back = np.minimum(r, np.float32(60000)).astype(np.float16)
        assert np.array_equal(back.view(np.uint16), h.view(np.uint16)), d
