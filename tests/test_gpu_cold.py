"""Warm tier (sp_hip_cold_*: the pinned host mirror of a layer's records): positions
written back land at their ring slots for every head, a restore puts them back
byte for byte, and once the ring has wrapped it keeps only the newest positions."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import sp_hip as S  # noqa: E402
from gpu_util import d2h, dev, p  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def ring(cl):
    n = cl.capacity
    return np.frombuffer(C.string_at(cl.h_pinned, n), np.uint8).reshape(cl.n_heads, cl.cap_pos, cl.packed_stride)


def test_cold_writeback_restore_and_ring():
    say("cold tier")
    L, H, hd, ms, layer = 2, 4, 128, 100, 1
    stream = torch.cuda.current_stream().cuda_stream
    cc = S.ShipCache(S.config(hd, L, H), ms, stream=stream)
    Lb = S.lib()
    x = np.random.default_rng(3).standard_normal((L * H * ms, hd)).astype(np.float16)
    xt = dev(x.view(np.uint16))
    S.check(Lb.sp_hip_write_all(cc.ref, 0, ms, p(xt), p(xt), S.DTYPE_F16))
    kB = cc.c.k_bands.total_bytes
    slab = C.c_void_p(cc.c.d_k_cache + layer * H * ms * kB)
    recs = d2h(cc.c.d_k_cache, L * H * ms * kB).reshape(L, H, ms, kB)[layer].copy()
    sptr = C.c_void_p(stream)
    # a mirror with room for every position: write back in two steps, clear the slab, restore
    cl = S.SpHipColdLayer()
    S.check(Lb.sp_hip_cold_layer_init(C.byref(cl), 0, kB, H, ms))
    assert cl.cap_pos == ms
    S.check(Lb.sp_hip_cold_writeback(C.byref(cl), slab, 0, 60, sptr))
    S.check(Lb.sp_hip_cold_writeback(C.byref(cl), slab, 60, 20, sptr))
    torch.cuda.synchronize()
    assert (cl.oldest_pos, cl.newest_pos, cl.ring_mode) == (0, 79, 0)
    np.testing.assert_array_equal(ring(cl)[:, :80], recs[:, :80])
    S.check(Lb.sp_hip_memset(slab, 0, H * ms * kB, sptr))
    S.check(Lb.sp_hip_cold_restore(C.byref(cl), slab, 80, sptr))
    torch.cuda.synchronize()
    back = d2h(cc.c.d_k_cache, L * H * ms * kB).reshape(L, H, ms, kB)[layer]
    np.testing.assert_array_equal(back[:, :80], recs[:, :80])
    assert not back[:, 80:].any()
    assert Lb.sp_hip_cold_restore(C.byref(cl), slab, 81, sptr) == -1  # position 80 was never written back
    Lb.sp_hip_cold_layer_free(C.byref(cl))
    # a 32-position ring: positions past it wrap, the oldest leave, restores from 0 are refused
    S.check(Lb.sp_hip_write_all(cc.ref, 0, ms, p(xt), p(xt), S.DTYPE_F16))
    cl = S.SpHipColdLayer()
    S.check(Lb.sp_hip_cold_layer_init(C.byref(cl), 32 * H * kB + 5, kB, H, ms))
    assert cl.cap_pos == 32
    S.check(Lb.sp_hip_cold_writeback(C.byref(cl), slab, 0, 20, sptr))
    S.check(Lb.sp_hip_cold_writeback(C.byref(cl), slab, 20, 30, sptr))  # wraps at 32
    S.check(Lb.sp_hip_cold_writeback(C.byref(cl), slab, 5, 2, sptr))    # older than the ring: dropped
    torch.cuda.synchronize()
    assert (cl.oldest_pos, cl.newest_pos, cl.ring_mode) == (18, 49, 1)
    r = ring(cl)
    for pos in range(18, 50):
        np.testing.assert_array_equal(r[:, pos % 32], recs[:, pos], err_msg=f"position {pos}")
    assert Lb.sp_hip_cold_restore(C.byref(cl), slab, 10, sptr) == -1
    Lb.sp_hip_cold_layer_free(C.byref(cl))
    cc.free()
