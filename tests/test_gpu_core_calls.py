"""Host-pointer core calls (sp_vht2_forward_f32, sp_band_quantize, sp_band_dequantize,
sp_band_dequantize_partial) against the oracle, bit for bit."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import oracle_py as O  # noqa: E402
import sp_hip as S  # noqa: E402


def test_core_vht2_and_band_codec():
    print("core host-pointer calls", flush=True)
    L = S.lib()
    rng = np.random.default_rng(21)
    for hd in (64, 128, 256):
        x = rng.standard_normal(hd).astype(np.float32)
        y = x.copy()
        L.sp_vht2_forward_f32(C.c_void_p(y.ctypes.data), hd)
        np.testing.assert_array_equal(y.view(np.uint32), O.vht2(x[None])[0].view(np.uint32))
        bits = [5, 5, 4, 3]
        obc, sbc = O.band_config(hd, bits), S.band_config(hd, bits)
        rec = np.zeros(obc.total_bytes, np.uint8)
        L.sp_band_quantize(C.c_void_p(y.ctypes.data), C.c_void_p(rec.ctypes.data), C.byref(sbc))
        want = O.band_quantize(y, obc)
        np.testing.assert_array_equal(rec, want)
        for mb in (-1, 0, 2, 4):
            out = np.full(hd, np.nan, np.float32)
            if mb < 0:
                L.sp_band_dequantize(C.c_void_p(rec.ctypes.data), C.c_void_p(out.ctypes.data), C.byref(sbc))
            else:
                L.sp_band_dequantize_partial(C.c_void_p(rec.ctypes.data), C.c_void_p(out.ctypes.data), C.byref(sbc), mb)
            ref = O.band_dequantize(rec, obc, mb)
            np.testing.assert_array_equal(out, ref, err_msg=f"hd {hd} max_bands {mb}")
