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


def test_core_calls_refuse_what_they_cannot_run():
    """A length with a prime factor above 11, or a band layout the codec rejects,
    leaves the caller's buffer as it was (and sets sp_hip_last_error)."""
    L = S.lib()
    x = np.arange(13, dtype=np.float32)
    y = x.copy()
    L.sp_vht2_forward_f32(C.c_void_p(y.ctypes.data), 13)
    np.testing.assert_array_equal(y, x)
    assert "13" in S.last_error()
    bad = S.band_config(128, [5, 5, 4, 3])
    bad.band_bits[1] = 0  # a zero-bit band
    coeff = np.ones(128, np.float32)
    rec = np.full(bad.total_bytes + 8, 0xAB, np.uint8)
    L.sp_band_quantize(C.c_void_p(coeff.ctypes.data), C.c_void_p(rec.ctypes.data), C.byref(bad))
    assert (rec == 0xAB).all()
    out = np.full(128, 3.0, np.float32)
    L.sp_band_dequantize_partial(C.c_void_p(rec.ctypes.data), C.c_void_p(out.ctypes.data), C.byref(bad), 2)
    assert (out == 3.0).all()
    assert "band" in S.last_error()
