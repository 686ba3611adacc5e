"""Calibration passes on the GPU (the reference's calibrate_begin / feed / end,
kv_cache.cpp:515-751): the variance-ranked K coefficient order of the ship and
shadow caches, the sqfree Knight-mask recalibration, and the hierarchical predictor
fit. The reference's calibrate_end
algorithms live in its absent core, so the rules here are this build's (stated in
the headers); each test recomputes them in numpy (float64) from the oracle's
bit-exact transforms of the same vectors."""
import ctypes as C
import math
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import oracle_py as O  # noqa: E402
import sp_hip as S  # noqa: E402
import workloads as W  # noqa: E402
from gpu_util import d2h, dev, empty_f32, host, p, stream  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def variance_order(coef):
    """Coefficients by descending variance sum2/n - (sum/n)^2 (float64), ties by index."""
    c = coef.astype(np.float64)
    n = c.shape[0]
    m = c.sum(axis=0) / n
    var = (c * c).sum(axis=0) / n - m * m
    return np.argsort(-var, kind="stable").astype(np.int32)


def calib_vectors(n, hd, seed):
    """fp16 vectors whose channels have very different scales, so the coefficient
    variances are well separated."""
    rng = np.random.default_rng(seed)
    scale = np.exp(rng.uniform(-2.0, 2.0, hd)).astype(np.float32)
    return (rng.standard_normal((n, hd)).astype(np.float32) * scale).astype(np.float16)


def test_ship_calibrate_var_order_and_apply():
    """Three feeds (fp16 rows, fp16 rows with a row stride, fp32 rows) of K vectors;
    the ranking equals numpy's over the oracle VHT2 of the same vectors. Applied,
    it becomes the K order: records, reconstructions and fused attention then match
    the oracle run with that order."""
    hd, H, n_ctx = 128, 2, 300
    x = calib_vectors(3000, hd, seed=60)
    cfg = S.config(hd, 1, H)
    cc = S.ShipCache(cfg, n_ctx, stream=torch.cuda.current_stream().cuda_stream)
    L = S.lib()
    S.check(L.sp_hip_calibrate_begin(cc.ref))
    a = dev(x[:1000].view(np.uint16))
    padded = np.zeros((1200, hd + 8), np.float16)
    padded[:, :hd] = x[1000:2200]
    b = dev(padded.view(np.uint16))
    c = dev(x[2200:].astype(np.float32))
    S.check(L.sp_hip_calibrate_feed(cc.ref, p(a), hd, 1000, S.DTYPE_F16))
    S.check(L.sp_hip_calibrate_feed(cc.ref, p(b), hd + 8, 1200, S.DTYPE_F16))
    S.check(L.sp_hip_calibrate_feed(cc.ref, p(c), hd, 800, S.DTYPE_F32))
    order = np.zeros(hd, np.int32)
    S.check(L.sp_hip_calibrate_end(cc.ref, C.c_void_p(order.ctypes.data), 1))
    want = variance_order(O.vht2(x.astype(np.float32)))
    np.testing.assert_array_equal(order, want)
    assert sorted(order.tolist()) == list(range(hd))
    # the applied order drives writes, reads and attention
    k16, v16 = W.cfg2_kv(n_heads=H, n_pos=n_ctx, hd=hd, seed=61)
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    for h in range(H):
        kt, vt = dev(k16[h].view(np.uint16)), dev(v16[h].view(np.uint16))
        L.sp_hip_write_k_batch_f16(cc.ref, 0, h, 0, n_ctx, p(kt))
        L.sp_hip_write_v_batch_f16(cc.ref, 0, h, 0, n_ctx, p(vt))
    torch.cuda.synchronize()
    kB = kbc.total_bytes
    kc = d2h(cc.c.d_k_cache, H * n_ctx * kB).reshape(H, n_ctx, kB)
    kref = np.stack([O.ship_compress_f16(k16[h].view(np.uint16), kbc, order) for h in range(H)])
    np.testing.assert_array_equal(kc, kref)
    out = empty_f32(n_ctx * H * hd)
    S.check(L.sp_hip_read_layer(cc.ref, 0, 0, n_ctx, p(out), None, H * hd, S.DTYPE_F32, -1))
    got = host(out).reshape(n_ctx, H, hd)
    for h in range(H):
        np.testing.assert_array_equal(got[:, h], O.ship_decompress_f32(kref[h], kbc, order))
    vref = np.stack([O.ship_compress_f16(v16[h].view(np.uint16), vbc) for h in range(H)])
    n_q = 2 * H
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_ctx, seed=62)
    scale = 1.0 / math.sqrt(hd)
    s_ref, o_ref = O.attn_decode(q, kref, vref, H, n_ctx, kbc, vbc, order, scale)
    sc, ob = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
    S.check(L.sp_hip_attn_decode(cc.ref, 0, n_ctx, p(dev(q)), n_q, C.c_float(scale), p(sc), p(ob), stream()))
    for g, r in ((host(sc).reshape(n_q, n_ctx), s_ref), (host(ob).reshape(n_q, hd), o_ref)):
        assert np.max(np.abs(g - r)) <= 1e-3 * np.max(np.abs(r))
    # end without data is an error
    S.check(L.sp_hip_calibrate_begin(cc.ref))
    assert L.sp_hip_calibrate_end(cc.ref, None, 0) == -1
    cc.free()


def test_shadow_calibrate_host_vectors():
    """The core API the engine calls (sp_shadow_calibrate_begin / feed / end with
    host fp32 vectors): var_order and use_var_reorder are set, and later K writes
    and reads use var_order as the coefficient order."""
    hd, n_pos = 128, 40
    cfg = S.config(hd, 1, 1)
    sc = S.SpShadowCache()
    L = S.lib()
    S.check(L.sp_shadow_cache_init(C.byref(sc), C.byref(cfg)))
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    kbuf = np.zeros(n_pos * kbc.total_bytes, np.uint8)
    vbuf = np.zeros(n_pos * vbc.total_bytes, np.uint8)
    kp = (C.POINTER(C.c_uint8) * 1)(kbuf.ctypes.data_as(C.POINTER(C.c_uint8)))
    vp = (C.POINTER(C.c_uint8) * 1)(vbuf.ctypes.data_as(C.POINTER(C.c_uint8)))
    sc.k_cache = C.cast(kp, C.POINTER(C.POINTER(C.c_uint8)))
    sc.v_cache = C.cast(vp, C.POINTER(C.POINTER(C.c_uint8)))
    x = calib_vectors(200, hd, seed=63).astype(np.float32)
    S.check(L.sp_shadow_calibrate_begin(C.byref(sc)))
    assert sc.calibrating == 1
    for i in range(x.shape[0]):
        L.sp_shadow_calibrate_feed(C.byref(sc), C.c_void_p(x[i].ctypes.data))
    assert sc.calib_n == x.shape[0]
    S.check(L.sp_shadow_calibrate_end(C.byref(sc)))
    assert sc.use_var_reorder == 1 and sc.calibrating == 0
    order = np.ctypeslib.as_array(sc.var_order, (hd,)).copy()
    np.testing.assert_array_equal(order, variance_order(O.vht2(x)))
    sums = np.ctypeslib.as_array(sc.calib_sum, (hd,))
    np.testing.assert_allclose(sums, O.vht2(x).astype(np.float64).sum(axis=0), rtol=1e-12, atol=1e-9)
    kv = np.random.default_rng(64).standard_normal((n_pos, hd)).astype(np.float32)
    L.sp_shadow_write_k_batch(C.byref(sc), 0, 0, 0, n_pos, C.c_void_p(kv.ctypes.data))
    np.testing.assert_array_equal(kbuf.reshape(n_pos, -1), O.ship_compress_f32(kv, kbc, order))
    back = np.zeros((n_pos, hd), np.float32)
    L.sp_shadow_read_k_batch(C.byref(sc), 0, 0, 0, n_pos, C.c_void_p(back.ctypes.data))
    np.testing.assert_array_equal(back, O.ship_decompress_f32(kbuf.reshape(n_pos, -1), kbc, order))
    L.sp_shadow_cache_free(C.byref(sc))


def lowrank_vectors(n, hd, rank, seed):
    """fp16 vectors near a rank-`rank` subspace, so targets are predictable from the
    skeleton."""
    rng = np.random.default_rng(seed)
    M = rng.standard_normal((hd, rank)).astype(np.float32)
    z = rng.standard_normal((n, rank)).astype(np.float32)
    return (z @ M.T + 0.05 * rng.standard_normal((n, hd)).astype(np.float32)).astype(np.float16)


def test_hier_calibrate_fit():
    """Two feeds into slot 2 (fp16, then fp32 with a row stride), none into the
    other slots: slot 2's W equals numpy's ridge least-squares fit on the oracle's
    padded transforms (fp16 within one unit in the last place); the other slots keep
    their W; and the fitted predictor shrinks the residual energy against W = 0."""
    hd, pad_expect, n_slots = 256, 330, 4
    pad = O.sqfree_pad_dim(hd)
    assert pad == pad_expect
    skel, tgt = O.hier_geometry(pad)
    ns, nt = len(skel), len(tgt)
    cfg = S.config(hd, 2, 2)
    hc = S.HierCache(cfg, pad, skel, tgt, S.band_config(ns, [5, 5]), 2, 64, n_slots,
                     stream=torch.cuda.current_stream().cuda_stream)
    W0 = W.hier_W(n_slots, nt, ns, seed=65)
    hc.upload_W(W0)
    L = S.lib()
    x = lowrank_vectors(2500, hd, 12, seed=66)
    S.check(L.sp_hip_hier_calibrate_begin(hc.ref))
    a = dev(x[:1500].view(np.uint16))
    padded = np.zeros((1000, hd + 4), np.float32)
    padded[:, :hd] = x[1500:].astype(np.float32)
    b = dev(padded)
    S.check(L.sp_hip_hier_calibrate_feed(hc.ref, 2, p(a), hd, 1500, S.DTYPE_F16))
    S.check(L.sp_hip_hier_calibrate_feed(hc.ref, 2, p(b), hd + 4, 1000, S.DTYPE_F32))
    ridge = 1e-6
    S.check(L.sp_hip_hier_calibrate_end(hc.ref, C.c_double(ridge)))
    Wg = d2h(hc.c.d_W, n_slots * nt * ns * 2).view(np.uint16).reshape(n_slots, nt, ns)
    for s in (0, 1, 3):
        np.testing.assert_array_equal(Wg[s], W0[s])
    c = O.pad_transform(x.astype(np.float32), hd, pad).astype(np.float64)
    S_, T_ = c[:, skel], c[:, tgt]
    Gss, Gts = S_.T @ S_, T_.T @ S_
    lam = ridge * np.trace(Gss) / ns
    Wref = np.linalg.solve(Gss + lam * np.eye(ns), Gts.T).T
    wr = Wref.astype(np.float32).astype(np.float16).view(np.uint16).astype(np.int32)
    diff = np.abs(Wg[2].astype(np.int32) - wr)
    assert diff.max() <= 1, diff.max()
    assert (diff == 0).mean() > 0.999
    fit = Wg[2].view(np.float16).astype(np.float64)
    res_fit = ((T_ - S_ @ fit.T) ** 2).sum()
    res_zero = (T_ ** 2).sum()
    assert res_fit < 0.2 * res_zero, (res_fit, res_zero)
    assert L.sp_hip_hier_calibrate_end(hc.ref, C.c_double(ridge)) == -1  # needs a new begin

    # sticky EMA: refit slots 0 and 2 on the same vectors, keep a quarter of the old W
    keep = 0.25
    S.check(L.sp_hip_hier_calibrate_begin(hc.ref))
    for s in (0, 2):
        S.check(L.sp_hip_hier_calibrate_feed(hc.ref, s, p(a), hd, 1500, S.DTYPE_F16))
        S.check(L.sp_hip_hier_calibrate_feed(hc.ref, s, p(b), hd + 4, 1000, S.DTYPE_F32))
    assert L.sp_hip_hier_calibrate_end_ema(hc.ref, C.c_double(ridge), C.c_float(1.5)) == -1
    S.check(L.sp_hip_hier_calibrate_end_ema(hc.ref, C.c_double(ridge), C.c_float(keep)))
    We = d2h(hc.c.d_W, n_slots * nt * ns * 2).view(np.uint16).reshape(n_slots, nt, ns)
    for s in (1, 3):
        np.testing.assert_array_equal(We[s], W0[s])
    for s, old in ((0, W0[0]), (2, Wg[2])):
        blend = keep * old.view(np.float16).astype(np.float64) + (1 - keep) * Wref
        want = blend.astype(np.float32).astype(np.float16).view(np.uint16).astype(np.int32)
        diff = np.abs(We[s].astype(np.int32) - want)
        assert diff.max() <= 1, (s, diff.max())
        assert (diff == 0).mean() > 0.999
    hc.free()


def mobius_mu(n):
    mu, d = 1, 2
    while d * d <= n:
        if n % d == 0:
            n //= d
            if n % d == 0:
                return 0
            mu = -mu
        d += 1
    return -mu if n > 1 else mu


def knight_tables(ranking, sk):
    """The Knight rule over a ranking: skeleton = its first sk entries, residuals =
    the rest; residual c (n = c+1) takes the proper divisors d of n whose
    coefficient d-1 is in the skeleton and mu(n/d) != 0, with sign mu(n/d)."""
    skel, res = list(ranking[:sk]), list(ranking[sk:])
    slot_of = {c: s for s, c in enumerate(skel)}
    off, slot, mu = [0], [], []
    for c in res:
        n = c + 1
        for d in range(1, n):
            if n % d == 0 and mobius_mu(n // d) != 0 and (d - 1) in slot_of:
                slot.append(slot_of[d - 1])
                mu.append(mobius_mu(n // d))
        off.append(len(slot))
    return [np.array(a, np.int32) for a in (skel, res, off, slot, mu)]


class CustomKnight:
    """An oracle Knight mask over given tables."""

    def __init__(self, pad, skel, res, off, slot, mu):
        self.keep = [np.ascontiguousarray(skel, np.int32), np.ascontiguousarray(res, np.int32),
                     np.ascontiguousarray(off, np.int32), np.ascontiguousarray(slot, np.int32),
                     np.ascontiguousarray(mu, np.int8)]
        P = lambda a, t: a.ctypes.data_as(C.POINTER(t))
        k = self.keep
        self.m = O.KnightMask(pad, len(skel), len(res), len(slot), P(k[0], C.c_int), P(k[1], C.c_int),
                              P(k[2], C.c_int), P(k[3], C.c_int), P(k[4], C.c_int8))
        self.n_res = len(res)


def test_sqfree_knight_recalibration():
    """Two feeds of K vectors into an hd 128 sqfree cache (pad 154, sk 77); the
    ranking equals numpy's over the oracle's padded transforms; applied, the device
    Knight tables follow the rule over that ranking, and records and
    reconstructions equal the oracle run with those tables."""
    hd, sk, n = 128, 77, 120
    pad = O.sqfree_pad_dim(hd)
    bits = [5, 4, 4, 4, 5]
    cfg = S.config(hd, 1, 1, k_bits=bits, v_bits=bits)
    cc = S.SqfreeCache(cfg, n, rbits=3, spinor=True, sk_k=sk, stream=torch.cuda.current_stream().cuda_stream)
    L = S.lib()
    x = calib_vectors(1500, hd, seed=70)
    S.check(L.sp_hip_sqfree_calibrate_begin(cc.ref))
    a = dev(x[:900].view(np.uint16))
    b = dev(x[900:].astype(np.float32))
    S.check(L.sp_hip_sqfree_calibrate_feed(cc.ref, p(a), hd, 900, S.DTYPE_F16))
    S.check(L.sp_hip_sqfree_calibrate_feed(cc.ref, p(b), hd, 600, S.DTYPE_F32))
    ranking = np.zeros(pad, np.int32)
    S.check(L.sp_hip_sqfree_calibrate_end(cc.ref, C.c_void_p(ranking.ctypes.data), 1))
    np.testing.assert_array_equal(ranking, variance_order(O.pad_transform(x.astype(np.float32), hd, pad)))
    skel, res, off, slot, mu = knight_tables(ranking, sk)
    assert cc.c.n_terms == len(slot)
    got = [np.zeros(len(skel), np.int32), np.zeros(len(res), np.int32), np.zeros(len(off), np.int32),
           np.zeros(max(len(slot), 1), np.int32), np.zeros(max(len(slot), 1), np.int32)]
    S.check(L.sp_hip_sqfree_get_tables(cc.ref, *[C.c_void_p(g.ctypes.data) for g in got]))
    for g, w in zip(got, (skel, res, off, slot, mu)):
        np.testing.assert_array_equal(g[:len(w)], w)
    km = CustomKnight(pad, skel, res, off, slot, mu)
    skel_bc = O.band_config(sk, bits)
    k16 = W.cfg4_kv(n_heads=1, n_pos=n, hd=hd, seed=71)[0].reshape(n, hd)
    ref = O.sqfree_compress_f16(k16.view(np.uint16), hd, km, skel_bc, 3, True)
    rec = O.sqfree_decompress_f32(ref, hd, km, skel_bc, 3, True)
    kt = dev(k16.view(np.uint16))
    S.check(L.sp_hip_sqfree_write_batch(cc.ref, 0, 0, 0, 0, n, p(kt), S.DTYPE_F16))
    np.testing.assert_array_equal(d2h(cc.c.d_k_cache, n * ref.shape[1]).reshape(n, -1), ref)
    out = empty_f32(n * hd)
    S.check(L.sp_hip_sqfree_read_batch(cc.ref, 0, 0, 0, 0, n, p(out), S.DTYPE_F32))
    np.testing.assert_array_equal(host(out).reshape(n, hd).view(np.uint32), rec.view(np.uint32))
    cc.free()

