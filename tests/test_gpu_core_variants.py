"""The core's sqfree and hierarchical caches on host vectors (sp_sqfree_cache_t,
sp_hier_cache_t) and the sqfree bridge (sp_llama_sqfree_*), on the GPU.

tests/cpp/sqfree_patch_replay is plain C linked against libshannon_prime_hip.so
alone; it replays the b8861 hook's sqfree sequence (init with K 5,4,4,4,5, V
mirroring K, then per token/layer/head a write at position 0 and a read back)
and the sqfree bridge's. Every reconstruction equals the oracle's sqfree round
trip bit for bit."""
import ctypes as C
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import oracle_py as O  # noqa: E402
import sp_hip as S  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
REPLAY = os.path.join(HERE, "cpp", "sqfree_patch_replay")


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def fp16_values(shape, seed):
    """Gaussian values with Student-t (nu = 4) outlier channels, rounded to fp16 and
    held as fp32 (what the hook gathers from an fp16 cache)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32)
    ch = rng.choice(shape[-1], 6, replace=False)
    x[..., ch] *= rng.standard_t(4, x[..., ch].shape).astype(np.float32) * 3
    return x.astype(np.float16).astype(np.float32)


def sqfree_roundtrip(x32, hd, sk, bits, rb, spinor):
    pad = O.sqfree_pad_dim(hd)
    km, bc = O.Knight(pad, sk), O.band_config(sk, bits)
    x16 = x32.reshape(-1, hd).astype(np.float16).view(np.uint16)
    rec = O.sqfree_compress_f16(x16, hd, km, bc, rb, spinor)
    return O.sqfree_decompress_f32(rec, hd, km, bc, rb, spinor).reshape(x32.shape), rec


def test_b8861_sqfree_sequence_replay(tmp_path, monkeypatch):
    if not os.path.exists(REPLAY):
        pytest.fail("tests/cpp/sqfree_patch_replay is not built (make -C tests/cpp)")
    hd, L, H, T = 128, 2, 4, 5
    x = fp16_values((2, L, T, H, hd), seed=8861)
    x.tofile(tmp_path / "x.bin")
    env = {k: v for k, v in os.environ.items() if not k.startswith("SHANNON_PRIME_")}
    env.update(SHANNON_PRIME_SQFREE="1", SHANNON_PRIME_SPINOR="1", SHANNON_PRIME_RESIDUAL_BITS="3")
    say("replay b8861 sqfree sequence")
    r = subprocess.run([REPLAY, str(tmp_path), str(hd), str(L), str(H), str(T)], capture_output=True, text=True,
                       timeout=120, env=env)
    sys.stdout.write(r.stdout + r.stderr)
    assert r.returncode == 0, r.stderr
    pad, sk, nres, bk, corr = r.stdout.split()
    assert (int(pad), int(sk), int(nres), int(bk)) == (154, 77, 77, 98)  # shannon_prime_sqfree.cu:683-686
    want, _ = sqfree_roundtrip(x, hd, 77, [5, 4, 4, 4, 5], 3, True)
    hook = np.fromfile(tmp_path / "hook.bin", np.float32).reshape(x.shape)
    bridge = np.fromfile(tmp_path / "bridge.bin", np.float32).reshape(x.shape)
    np.testing.assert_array_equal(hook.view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(bridge.view(np.uint32), want.view(np.uint32))
    assert float(corr) > 0.95
    assert abs(float(corr) - O.correlation(x[0, 0, 0, 0], want[0, 0, 0, 0])) < 1e-6


def test_core_sqfree_cache_and_calibration():
    hd, L, H, T = 128, 2, 2, 40
    cfg = S.config(hd, L, H, k_bits=(5, 4, 4, 4, 5), v_bits=(5, 4, 4, 4, 5))
    c = S.SpSqfreeCache()
    Lb = S.lib()
    S.check(Lb.sp_sqfree_cache_init(C.byref(c), C.byref(cfg), T, 3, 0), "sqfree_cache_init")
    assert (c.pad_dim, c.mask.sk_k, c.mask.n_res, c.bytes_per_pos_k) == (154, 77, 77, 88)
    km = O.Knight(154, 77)
    assert np.ctypeslib.as_array(c.mask.skeleton_idx, (77,)).tolist() == km.skeleton_idx.tolist()
    assert np.ctypeslib.as_array(c.mask.csr_offsets, (78,)).tolist() == km.csr_offsets.tolist()
    x = fp16_values((2, L, H, T, hd), seed=5)
    out = np.zeros_like(x)
    for side, (wr, rd) in enumerate(((Lb.sp_sqfree_write_k, Lb.sp_sqfree_read_k),
                                     (Lb.sp_sqfree_write_v, Lb.sp_sqfree_read_v))):
        for layer in range(L):
            for h in range(H):
                for t in range(T):
                    wr(C.byref(c), layer, h, t, x[side, layer, h, t].ctypes.data_as(C.c_void_p))
        for layer in range(L):
            for h in range(H):
                for t in range(T):
                    rd(C.byref(c), layer, h, t, out[side, layer, h, t].ctypes.data_as(C.c_void_p))
    want, _ = sqfree_roundtrip(x, hd, 77, [5, 4, 4, 4, 5], 3, False)
    np.testing.assert_array_equal(out.view(np.uint32), want.view(np.uint32))
    # out-of-range calls are ignored (the output is left alone)
    sentinel = np.full(hd, 7.0, np.float32)
    Lb.sp_sqfree_read_k(C.byref(c), L, 0, 0, sentinel.ctypes.data_as(C.c_void_p))
    Lb.sp_sqfree_read_k(C.byref(c), 0, 0, T, sentinel.ctypes.data_as(C.c_void_p))
    assert (sentinel == 7.0).all()
    # Knight recalibration: a skewed variance profile moves the skeleton; the host
    # mask follows the device tables, and the cache still round-trips consistently
    assert Lb.sp_sqfree_calibrate_end(C.byref(c)) == -1
    S.check(Lb.sp_sqfree_calibrate_begin(C.byref(c)))
    rng = np.random.default_rng(9)
    skew = (rng.standard_normal((300, hd)) * np.linspace(3.0, 0.1, hd)).astype(np.float32)
    for v in skew:
        Lb.sp_sqfree_calibrate_feed(C.byref(c), v.ctypes.data_as(C.c_void_p))
    S.check(Lb.sp_sqfree_calibrate_end(C.byref(c)))
    skel = np.ctypeslib.as_array(c.mask.skeleton_idx, (77,)).copy()
    res = np.ctypeslib.as_array(c.mask.residual_idx, (77,)).copy()
    assert skel.tolist() != km.skeleton_idx.tolist()
    assert sorted(skel.tolist() + res.tolist()) == list(range(154))
    a = np.zeros(hd, np.float32)
    Lb.sp_sqfree_write_k(C.byref(c), 1, 1, 3, x[0, 1, 1, 3].ctypes.data_as(C.c_void_p))
    Lb.sp_sqfree_read_k(C.byref(c), 1, 1, 3, a.ctypes.data_as(C.c_void_p))
    assert O.correlation(a, x[0, 1, 1, 3]) > 0.9
    Lb.sp_sqfree_cache_free(C.byref(c))
    assert not c.dev


def test_core_hier_cache_calibrate_save_load(tmp_path):
    hd, L, H, T = 256, 1, 2, 24
    cfg = S.config(hd, L, H)
    hc = S.SpHierCache()
    Lb = S.lib()
    assert Lb.sp_hier_cache_init(C.byref(hc), C.byref(cfg), T, 2, 0, None, 2) == -1  # only level 0
    S.check(Lb.sp_hier_cache_init(C.byref(hc), C.byref(cfg), T, 0, 0, None, 2), "hier_cache_init")
    pad = O.sqfree_pad_dim(hd)
    si, ti = O.hier_geometry(pad)
    p0 = hc.predictors[0]
    assert (hc.pad_dim, hc.n_slots, p0.n_skeleton, p0.n_target, p0.target_res_bits) == (pad, 2, 30, 300, 2)
    assert np.ctypeslib.as_array(p0.skeleton_idx, (30,)).tolist() == si.tolist()
    assert not np.ctypeslib.as_array(hc.predictors[1].W, (300 * 30,)).any()  # zero until calibrated
    rng = np.random.default_rng(12)
    M = rng.standard_normal((hd, 10)).astype(np.float32)
    feed = (rng.standard_normal((400, 10)).astype(np.float32) @ M.T).astype(np.float16).astype(np.float32)
    S.check(Lb.sp_hier_cache_calibrate_begin(C.byref(hc)))
    for s in range(2):
        for v in feed[s * 200:(s + 1) * 200]:
            Lb.sp_hier_cache_calibrate_feed(C.byref(hc), s, v.ctypes.data_as(C.c_void_p))
    S.check(Lb.sp_hier_cache_calibrate_end(C.byref(hc)))
    Ws = [np.ctypeslib.as_array(hc.predictors[s].W, (300 * 30,)).copy().reshape(300, 30) for s in range(2)]
    assert all(np.abs(w.view(np.float16).astype(np.float32)).max() > 0 for w in Ws)
    x = fp16_values((2, H, T, hd), seed=13)
    out = np.zeros_like(x)
    for side, (wr, rd) in enumerate(((Lb.sp_hier_cache_write_k, Lb.sp_hier_cache_read_k),
                                     (Lb.sp_hier_cache_write_v, Lb.sp_hier_cache_read_v))):
        for h in range(H):
            for t in range(T):
                wr(C.byref(hc), 0, h, t, x[side, h, t].ctypes.data_as(C.c_void_p))
                rd(C.byref(hc), 0, h, t, out[side, h, t].ctypes.data_as(C.c_void_p))
    bc = O.band_config(30, [5, 5])
    for side in range(2):
        for h in range(H):
            x16 = x[side, h].astype(np.float16).view(np.uint16)
            rec = O.hier_compress_f16(x16, hd, pad, si, ti, bc, Ws[h], 2)
            want = O.hier_decompress_f32(rec, hd, pad, si, ti, bc, Ws[h], 2)
            np.testing.assert_array_equal(out[side, h].view(np.uint32), want.view(np.uint32))
    prefix = str(tmp_path / "hier")
    S.check(Lb.sp_hier_cache_save(C.byref(hc), prefix.encode(), T, C.c_uint64(77)))
    hc2 = S.SpHierCache()
    S.check(Lb.sp_hier_cache_init(C.byref(hc2), C.byref(cfg), T, 0, 0, None, 2))
    assert Lb.sp_hier_cache_load(C.byref(hc2), prefix.encode(), C.c_uint64(77)) == T
    for s in range(2):
        np.testing.assert_array_equal(np.ctypeslib.as_array(hc2.predictors[s].W, (9000,)).reshape(300, 30), Ws[s])
    back = np.zeros(hd, np.float32)
    Lb.sp_hier_cache_read_v(C.byref(hc2), 0, 1, 7, back.ctypes.data_as(C.c_void_p))
    np.testing.assert_array_equal(back.view(np.uint32), out[1, 1, 7].view(np.uint32))
    Lb.sp_hier_cache_free(C.byref(hc2))
    Lb.sp_hier_cache_free(C.byref(hc))
