"""System 1/2 dual cache (DualKvCache's route table, routed writes and merged read)
on the GPU: every position of the merged read equals the oracle's reconstruction
from the cache that owns it, bit for bit, and each cache holds records only at the
positions routed to it."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import oracle_py as O  # noqa: E402
import sp_hip as S  # noqa: E402
import workloads as W  # noqa: E402
from gpu_util import d2h, dev, host, p  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def row(t, i, stride):
    """Device pointer to fp16 row i of a [n][stride] tensor."""
    import ctypes as C
    return C.c_void_p(t.data_ptr() + 2 * i * stride)


def _rows(x16, pad_row):
    """[H][n][hd] fp16 -> llama.cpp cache rows [n][H*hd + pad_row] (padding = 0)."""
    H, n, hd = x16.shape
    r = np.zeros((n, H * hd + pad_row), np.float16)
    for h in range(H):
        r[:, h * hd:(h + 1) * hd] = x16[h]
    return r


@pytest.mark.parametrize("kind,hd", [("sqfree", 128), ("hier", 128), ("hier", 256)])
def test_dual_routed_write_and_merged_read(kind, hd):
    """sqfree at hd 128 and hier at hd 256 (the default 30/300 geometry) read their
    listed positions through the one-vector-per-lane kernels, hier at hd 128 through
    the one-vector-per-wave kernel."""
    say(f"dual cache kind={kind} hd={hd}")
    L, H, ms, pad_row, layer = 2, 2, 200, 8, 1
    stream = torch.cuda.current_stream().cuda_stream
    ship = S.ShipCache(S.config(hd, L, H), ms, stream=stream)
    pad = O.sqfree_pad_dim(hd)
    if kind == "sqfree":
        bits = [5, 4, 4, 4, 5]
        sk = pad // 2
        sys2 = S.SqfreeCache(S.config(hd, L, H, k_bits=bits, v_bits=bits), ms, rbits=3, spinor=True, sk_k=sk,
                             stream=stream)
        km, sbc = O.Knight(pad, sk), O.band_config(sk, bits)

        def ref2(x16, slot):
            r = O.sqfree_compress_f16(x16.view(np.uint16), hd, km, sbc, 3, True)
            return r, O.sqfree_decompress_f32(r, hd, km, sbc, 3, True)
        kind_c = S.DUAL_SQFREE
    else:
        skel, tgt = O.hier_geometry(pad)
        sbc = O.band_config(len(skel), [5, 5])
        Wm = W.hier_W(L * H, len(tgt), len(skel), seed=77)
        sys2 = S.HierCache(S.config(hd, L, H), pad, skel, tgt, S.band_config(len(skel), [5, 5]), 2, ms, L * H,
                           stream=stream)
        sys2.upload_W(Wm)

        def ref2(x16, slot):
            r = O.hier_compress_f16(x16.view(np.uint16), hd, pad, skel, tgt, sbc, Wm[slot], 2)
            return r, O.hier_decompress_f32(r, hd, pad, skel, tgt, sbc, Wm[slot], 2)
        kind_c = S.DUAL_HIER
    dc = S.DualCache(ship, sys2, kind_c, 1.0)
    Lb = S.lib()
    assert Lb.sp_hip_dual_owner_of(dc.ref, -1) == 1 and Lb.sp_hip_dual_route_position(dc.ref, ms, 9.0) == 0
    rng = np.random.default_rng(5 if kind == "sqfree" else 6)
    n = 156
    ent = rng.uniform(0.0, 2.0, n).astype(np.float32)
    ent[:40] = 0.1  # a System 1 prefill prefix
    for t in range(150):
        assert Lb.sp_hip_dual_route_position(dc.ref, t, float(ent[t])) == int(ent[t] >= 1.0)
    k16, v16 = W.cfg4_kv(n_heads=H, n_pos=n, hd=hd, seed=60)
    stride = H * hd + pad_row
    kt, vt = dev(_rows(k16, pad_row)), dev(_rows(v16, pad_row))
    # prefill in two chunks, then decode steps that are routed one at a time
    S.check(Lb.sp_hip_dual_write_layer(dc.ref, layer, 0, 100, p(kt), p(vt), stride, S.DTYPE_F16))
    S.check(Lb.sp_hip_dual_write_layer(dc.ref, layer, 100, 50, row(kt, 100, stride), row(vt, 100, stride), stride,
                                       S.DTYPE_F16))
    ko = torch.full((n * stride,), float("nan"), dtype=torch.float32, device="cuda")
    vo = torch.full((n * stride,), float("nan"), dtype=torch.float32, device="cuda")
    S.check(Lb.sp_hip_dual_read_merged(dc.ref, layer, 150, p(ko), p(vo), stride, S.DTYPE_F32))
    for t in range(150, n):
        Lb.sp_hip_dual_route_position(dc.ref, t, float(ent[t]))
        S.check(Lb.sp_hip_dual_write_layer(dc.ref, layer, t, 1, row(kt, t, stride), row(vt, t, stride), stride,
                                           S.DTYPE_F16))
    ko2 = torch.full((n * stride,), float("nan"), dtype=torch.float32, device="cuda")
    vo2 = torch.full((n * stride,), float("nan"), dtype=torch.float32, device="cuda")
    S.check(Lb.sp_hip_dual_read_merged(dc.ref, layer, n, p(ko2), p(vo2), stride, S.DTYPE_F32))
    torch.cuda.synchronize()
    own2 = ent >= 1.0
    assert Lb.sp_hip_dual_sys2_count(dc.ref) == int(own2.sum())
    assert Lb.sp_hip_dual_sys1_count(dc.ref) == ms - int(own2.sum())
    assert [Lb.sp_hip_dual_owner_of(dc.ref, t) for t in range(n)] == [2 if o else 1 for o in own2]
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    order = O.mobius_order(hd)
    B1 = (kbc.total_bytes, vbc.total_bytes)
    B2 = (sys2.c.bytes_per_pos_k, sys2.c.bytes_per_pos_v)
    for side, (x16, outs, c1, c2) in enumerate(((k16, (ko, ko2), ship.c.d_k_cache, sys2.c.d_k_cache),
                                                 (v16, (vo, vo2), ship.c.d_v_cache, sys2.c.d_v_cache))):
        r1 = d2h(c1, L * H * ms * B1[side]).reshape(L, H, ms, B1[side])
        r2 = d2h(c2, L * H * ms * B2[side]).reshape(L, H, ms, B2[side])
        assert not r1[0].any() and not r2[0].any(), "other layer written"
        for h in range(H):
            x = x16[h]
            bc, od = (kbc, order) if side == 0 else (vbc, None)
            ship_rec = O.ship_compress_f16(x.view(np.uint16), bc, od)
            ship_out = O.ship_decompress_f32(ship_rec, bc, od)
            rec2, out2 = ref2(x, layer * H + h)
            np.testing.assert_array_equal(r1[layer, h, :n][~own2], ship_rec[~own2])
            assert not r1[layer, h, :n][own2].any(), "System 1 written at a System 2 position"
            np.testing.assert_array_equal(r2[layer, h, :n][own2], rec2[own2])
            assert not r2[layer, h, :n][~own2].any(), "System 2 written at a System 1 position"
            want = np.where(own2[:, None], out2, ship_out)
            for kv_len, out in ((150, outs[0]), (n, outs[1])):
                g = host(out).reshape(n, stride)
                np.testing.assert_array_equal(g[:kv_len, h * hd:(h + 1) * hd].view(np.uint32),
                                              want[:kv_len].view(np.uint32), err_msg=f"side {side} head {h}")
                assert np.isnan(g[:kv_len, H * hd:]).all() and np.isnan(g[kv_len:]).all()
    # bad arguments launch nothing
    assert Lb.sp_hip_dual_read_merged(dc.ref, L, 10, p(ko), p(vo), stride, S.DTYPE_F32) == -1
    assert Lb.sp_hip_dual_read_merged(dc.ref, 0, ms + 1, p(ko), p(vo), stride, S.DTYPE_F32) == -1
    assert Lb.sp_hip_dual_write_layer(dc.ref, 0, ms - 1, 2, p(kt), p(vt), stride, S.DTYPE_F16) == -1
    dc.free()
    sys2.free()
    ship.free()


def test_dual_rejects_mismatched_caches():
    stream = torch.cuda.current_stream().cuda_stream
    ship = S.ShipCache(S.config(128, 1, 2), 64, stream=stream)
    bits = [5, 4, 4, 4, 5]
    sq = S.SqfreeCache(S.config(128, 1, 2, k_bits=bits, v_bits=bits), 65, sk_k=77, stream=stream)
    c = S.SpHipDualCache()
    import ctypes as C
    assert S.lib().sp_hip_dual_init(C.byref(c), ship.ref, S.DUAL_SQFREE, sq.ref, C.c_float(1.0)) == -1
    assert S.lib().sp_hip_dual_init(C.byref(c), ship.ref, 7, sq.ref, C.c_float(1.0)) == -1
    sq.free()
    ship.free()
