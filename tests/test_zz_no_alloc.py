"""sp_hip_attn_decode_bands_noalloc (decode attention with its workspace in a
fixed per-GPU device array, no allocation) against sp_hip_attn_decode_bands
(the cache's workspace): two calls in a row, the second smaller, through both
attention kernels, bit-identical scores and outputs; a call that needs more
workspace than the array holds is refused and leaves its outputs alone."""
import ctypes as C
import math
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import sp_hip as S  # noqa: E402
import workloads as W  # noqa: E402
from gpu_util import dev, empty_f32, host, p, stream  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


H, HD, MAX_SEQ, N_WRITTEN = 8, 128, 131072, 32768


@pytest.fixture(scope="module")
def cache():
    cc = S.ShipCache(S.config(HD, 1, H), MAX_SEQ, stream=torch.cuda.current_stream().cuda_stream)
    k16, v16 = W.cfg2_kv(n_heads=H, n_pos=N_WRITTEN, hd=HD, seed=77)
    L = S.lib()
    for h in range(H):
        kt, vt = dev(k16[h].view(np.uint16)), dev(v16[h].view(np.uint16))
        S.check(L.sp_hip_write_k_batch_f16(cc.ref, 0, h, 0, N_WRITTEN, p(kt)))
        S.check(L.sp_hip_write_v_batch_f16(cc.ref, 0, h, 0, N_WRITTEN, p(vt)))
    torch.cuda.synchronize()
    yield cc
    cc.free()


def _call(fn, cc, n_kv, qt, n_q, max_bands):
    sc, out = empty_f32(n_q * n_kv), empty_f32(n_q * HD)
    S.check(fn(cc.ref, 0, n_kv, p(qt), n_q, C.c_float(1.0 / math.sqrt(HD)), p(sc), p(out), max_bands, stream()))
    return host(sc), host(out)


@pytest.mark.parametrize("path", ["mfma", "general"])
def test_noalloc_matches_workspace_entry_point(cache, path, monkeypatch):
    if path == "general":
        monkeypatch.setenv("SP_HIP_NO_MFMA_ATTN", "1")
    L = S.lib()
    # a 32K call over every KV head, then a smaller call (fewer positions, fewer
    # query heads, two K bands) that reuses the array the first one filled
    for n_kv, n_q, mb in ((N_WRITTEN, 32, -1), (3001, 16, 2)):
        say(f"noalloc path={path} n_kv={n_kv} n_q={n_q} max_bands={mb}")
        q = W.cfg2_q(n_q=n_q, hd=HD, pos=n_kv, seed=n_kv)
        qt = dev(q)
        s_na, o_na = _call(L.sp_hip_attn_decode_bands_noalloc, cache, n_kv, qt, n_q, mb)
        s_ws, o_ws = _call(L.sp_hip_attn_decode_bands, cache, n_kv, qt, n_q, mb)
        assert np.isfinite(s_na).all() and np.isfinite(o_na).all()
        assert np.abs(o_na).max() > 0
        np.testing.assert_array_equal(s_na, s_ws)
        np.testing.assert_array_equal(o_na, o_ws)


def test_noalloc_refuses_oversized_calls(cache):
    L = S.lib()
    cap = L.sp_hip_attn_noalloc_max_floats()
    assert cap == (16 << 20) // 4
    # 64*128 + 64*ceil(n_kv/256)*130 floats + the 256 arrival counters (one per 64-word
    # line, plus one line of alignment slack): over 16 MiB from 502 splits on
    n_q = 64
    counters = 256 * 64 + 64
    n_kv = 502 * 256
    assert n_q * HD + n_q * ((n_kv + 255) // 256) * (HD + 2) + counters > cap
    qt = dev(np.ones((n_q, HD), np.float32))
    sc = torch.full((n_q * n_kv,), 7.0, dtype=torch.float32, device="cuda")
    out = torch.full((n_q * HD,), 7.0, dtype=torch.float32, device="cuda")
    rc = L.sp_hip_attn_decode_bands_noalloc(cache.ref, 0, n_kv, p(qt), n_q, C.c_float(1.0), p(sc), p(out), -1,
                                            stream())
    assert rc == -1
    assert b"scratch" in S.lib().sp_hip_last_error()
    assert bool((sc == 7.0).all()) and bool((out == 7.0).all())
    # one split fewer fits, and gives what the workspace entry point gives
    n_kv = 501 * 256
    assert n_q * HD + n_q * ((n_kv + 255) // 256) * (HD + 2) + counters <= cap
    rc = L.sp_hip_attn_decode_bands_noalloc(cache.ref, 0, n_kv, p(qt), n_q, C.c_float(1.0), None, p(out), -1,
                                            stream())
    assert rc == 0
    ref = empty_f32(n_q * HD)
    S.check(L.sp_hip_attn_decode_bands(cache.ref, 0, n_kv, p(qt), n_q, C.c_float(1.0), None, p(ref), -1, stream()))
    got = host(out)
    assert np.isfinite(got).all() and np.abs(got).max() > 0
    np.testing.assert_array_equal(got, host(ref))


def test_noalloc_under_graph_capture(cache):
    """The allocation-free call captured in a HIP graph (torch.cuda.graph): an
    eager call first (it looks up the scratch address), then one captured call,
    replayed three times with the query buffer refilled between replays, each
    replay equal to sp_hip_attn_decode_bands on the same query (eager work and
    synchronisations between the replays)."""
    L = S.lib()
    n_kv, n_q = 4096, 32
    scale = C.c_float(1.0 / math.sqrt(HD))
    qs = [W.cfg2_q(n_q=n_q, hd=HD, pos=n_kv, seed=s) for s in (5, 6)]
    qt = dev(qs[0])
    sc, out = empty_f32(n_q * n_kv), empty_f32(n_q * HD)
    S.check(L.sp_hip_attn_decode_bands_noalloc(cache.ref, 0, n_kv, p(qt), n_q, scale, p(sc), p(out), -1, stream()))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    say("noalloc graph capture")
    with torch.cuda.graph(g, stream=side):
        rc = L.sp_hip_attn_decode_bands_noalloc(cache.ref, 0, n_kv, p(qt), n_q, scale, p(sc), p(out), -1,
                                                C.c_void_p(side.cuda_stream))
    assert rc == 0, S.lib().sp_hip_last_error()
    for i in (1, 0, 1):
        qt.copy_(torch.from_numpy(qs[i]).cuda())
        sc.fill_(7.0)
        out.fill_(7.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        s_ref, o_ref = _call(L.sp_hip_attn_decode_bands, cache, n_kv, qt, n_q, -1)
        np.testing.assert_array_equal(host(sc), s_ref)
        np.testing.assert_array_equal(host(out), o_ref)
