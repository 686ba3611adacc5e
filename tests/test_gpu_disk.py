"""Disk formats v3 (ship caches: band-major) and v2 (sqfree and hier caches:
records whole, in cache order): the file layouts against numpy restatements,
bit-exact round trips, partial loads that equal partial reads, v2 files read by
every loader (a partial load of a v2 file reads every band), and the header and
hash guards."""
import ctypes as C
import os
import struct
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


def fnv(b):
    h = 0xcbf29ce484222325
    for c in b:
        h = ((h ^ c) * 0x100000001b3) & (2 ** 64 - 1)
    return h


def segments(bits, hd, B):
    """(offset, length) of each band's [scale][codes] in a record, then any tail."""
    out, off = [], 0
    n = len(bits)
    for b, nb in enumerate(bits):
        sz = hd // n if b < n - 1 else hd - (hd // n) * (n - 1)
        ln = 2 + (sz * nb + 7) // 8
        out.append((off, ln))
        off += ln
    if off < B:
        out.append((off, B - off))
    return out


def records(ptr, L, H, ms, B):
    return d2h(ptr, L * H * ms * B).reshape(L, H, ms, B)


def band_major(rec_l, segs, n_pos):
    """numpy restatement of the v3 body of one side: segment-major, then head, then position."""
    return np.concatenate([rec_l[:, :n_pos, o:o + ln].reshape(-1) for o, ln in segs])


def fill_ship(cc, L, H, hd, n, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((L, n, H * hd)).astype(np.float16)
    for layer in range(L):
        t = dev(x[layer].view(np.uint16))
        S.check(S.lib().sp_hip_write_layer(cc.ref, layer, 0, n, p(t), p(t), H * hd, S.DTYPE_F16))
    torch.cuda.synchronize()


def test_ship_save_load_partial(tmp_path, monkeypatch):
    say("disk ship save/load/partial")
    L, H, hd, ms, n = 2, 2, 128, 300, 200
    stream = torch.cuda.current_stream().cuda_stream
    cfg = S.config(hd, L, H)
    a = S.ShipCache(cfg, ms, stream=stream)
    fill_ship(a, L, H, hd, n, 1)
    Lb = S.lib()
    prefix = str(tmp_path / "ctx")
    h_a, h_b = fnv(b"/models/a.gguf"), fnv(b"/models/b.gguf")
    S.check(Lb.sp_hip_cache_save(a.ref, prefix.encode(), n, h_a))
    kB, vB = 76, 50
    ka, va = records(a.c.d_k_cache, L, H, ms, kB), records(a.c.d_v_cache, L, H, ms, vB)
    ksegs, vsegs = segments([5, 5, 4, 3], hd, kB), segments([3], hd, vB)
    for layer in range(L):
        raw = open(f"{prefix}.L{layer}.bin", "rb").read()
        hdr = struct.unpack("<4sIQ10iQ", raw[:64])
        assert hdr[:12] == (b"VHT2", 3, h_a, n, layer, H, hd, 0, kB, vB, 4, 1), hdr
        assert hdr[13] == fnv(raw[:56])
        body = np.frombuffer(raw[64:], np.uint8)
        kb = band_major(ka[layer], ksegs, n)
        np.testing.assert_array_equal(body[:kb.size], kb)
        np.testing.assert_array_equal(body[kb.size:], band_major(va[layer], vsegs, n))
    # full load into a fresh cache
    b = S.ShipCache(cfg, ms, stream=stream)
    assert Lb.sp_hip_cache_load(b.ref, prefix.encode(), h_a) == n
    np.testing.assert_array_equal(records(b.c.d_k_cache, L, H, ms, kB), ka)
    np.testing.assert_array_equal(records(b.c.d_v_cache, L, H, ms, vB), va)
    # partial loads: bands past max_bands are cleared, and reads equal partial reads of the original
    for mb in (0, 1, 2):
        c = S.ShipCache(cfg, ms, stream=stream)
        fill_ship(c, L, H, hd, n, 9)  # stale contents must be replaced
        assert Lb.sp_hip_cache_load_partial(c.ref, prefix.encode(), h_a, mb) == n
        kc, vc = records(c.c.d_k_cache, L, H, ms, kB), records(c.c.d_v_cache, L, H, ms, vB)
        for s, (o, ln) in enumerate(ksegs):
            want = ka[:, :, :n, o:o + ln] if s < mb else 0
            np.testing.assert_array_equal(kc[:, :, :n, o:o + ln], np.broadcast_to(want, kc[:, :, :n, o:o + ln].shape))
        np.testing.assert_array_equal(vc[:, :, :n], va[:, :, :n] if mb >= 1 else 0 * va[:, :, :n])
        got = torch.empty(L * H * n * hd, dtype=torch.float32, device="cuda")
        ref = torch.empty(L * H * n * hd, dtype=torch.float32, device="cuda")
        S.check(Lb.sp_hip_read_all(c.ref, 0, n, p(got), None, S.DTYPE_F32, -1))
        S.check(Lb.sp_hip_read_all(a.ref, 0, n, p(ref), None, S.DTYPE_F32, mb))
        # equal as values: a cleared band decodes as (0 - max) * 0 = -0.0 where a partial read has +0.0
        np.testing.assert_array_equal(host(got), host(ref))
        c.free()
    # guards: another model, SP_DISK_HASH_STRICT=0, a shape mismatch, a truncated file, a bad header
    assert Lb.sp_hip_cache_load(b.ref, prefix.encode(), h_b) == -1
    assert b"hash" in Lb.sp_hip_last_error()
    monkeypatch.setenv("SP_DISK_HASH_STRICT", "0")
    assert Lb.sp_hip_cache_load(b.ref, prefix.encode(), h_b) == n
    monkeypatch.delenv("SP_DISK_HASH_STRICT")
    other = S.ShipCache(S.config(hd, L, H + 1), ms, stream=stream)
    assert Lb.sp_hip_cache_load(other.ref, prefix.encode(), h_a) == -1
    other.free()
    short = str(tmp_path / "short")
    for layer in range(L):
        raw = open(f"{prefix}.L{layer}.bin", "rb").read()
        open(f"{short}.L{layer}.bin", "wb").write(raw[:-7] if layer == 1 else raw)
    assert Lb.sp_hip_cache_load(b.ref, short.encode(), h_a) == -1
    bad = str(tmp_path / "bad")
    for layer in range(L):
        raw = bytearray(open(f"{prefix}.L{layer}.bin", "rb").read())
        raw[20] ^= 1  # the layer field, without resealing the header check
        open(f"{bad}.L{layer}.bin", "wb").write(bytes(raw))
    assert Lb.sp_hip_cache_load(b.ref, bad.encode(), h_a) == -1
    assert Lb.sp_hip_cache_load(b.ref, str(tmp_path / "missing").encode(), h_a) == -1
    for c_ in (a, b):
        c_.free()


def test_sqfree_and_hier_save_load(tmp_path):
    say("disk sqfree + hier save/load")
    L, H, hd, ms, n = 2, 2, 128, 160, 150
    stream = torch.cuda.current_stream().cuda_stream
    bits = [5, 4, 4, 4, 5]
    k16, v16 = W.cfg4_kv(n_heads=H, n_pos=n, hd=hd, seed=70)
    rows_k = np.concatenate([k16[h] for h in range(H)], axis=1)  # [n][H*hd]
    rows_v = np.concatenate([v16[h] for h in range(H)], axis=1)
    kt, vt = dev(np.ascontiguousarray(rows_k).view(np.uint16)), dev(np.ascontiguousarray(rows_v).view(np.uint16))
    Lb = S.lib()
    h = fnv(b"model")
    # sqfree
    cfg = S.config(hd, L, H, k_bits=bits, v_bits=bits)
    a = S.SqfreeCache(cfg, ms, rbits=3, spinor=True, sk_k=77, stream=stream)
    for layer in range(L):
        S.check(Lb.sp_hip_sqfree_write_layer(a.ref, layer, 0, n, p(kt), p(vt), H * hd, S.DTYPE_F16))
    prefix = str(tmp_path / "sq")
    S.check(Lb.sp_hip_sqfree_cache_save(a.ref, prefix.encode(), n, h))
    B = a.c.bytes_per_pos_k
    # v2: one whole-record segment per side, the records in cache order
    for layer in range(L):
        raw = open(f"{prefix}.L{layer}.bin", "rb").read()
        hdr = struct.unpack("<4sIQ10iQ", raw[:64])
        assert hdr[:2] == (b"VHT2", 2) and hdr[7] == 1 and hdr[8] == B and hdr[10:12] == (1, 1), hdr
        assert hdr[13] == fnv(raw[:56])
        body = np.concatenate([records(a.c.d_k_cache, L, H, ms, B)[layer, :, :n].reshape(-1),
                               records(a.c.d_v_cache, L, H, ms, B)[layer, :, :n].reshape(-1)])
        np.testing.assert_array_equal(np.frombuffer(raw[64:], np.uint8), body)
    b = S.SqfreeCache(cfg, ms, rbits=3, spinor=True, sk_k=77, stream=stream)
    assert Lb.sp_hip_sqfree_cache_load(b.ref, prefix.encode(), h) == n
    for ptr_a, ptr_b in ((a.c.d_k_cache, b.c.d_k_cache), (a.c.d_v_cache, b.c.d_v_cache)):
        np.testing.assert_array_equal(records(ptr_b, L, H, ms, B), records(ptr_a, L, H, ms, B))
    a.free()
    b.free()
    # hier, with its W file
    pad = O.sqfree_pad_dim(hd)
    skel, tgt = O.hier_geometry(pad)
    Wm = W.hier_W(L * H, len(tgt), len(skel), seed=71)
    cfg = S.config(hd, L, H)
    a = S.HierCache(cfg, pad, skel, tgt, S.band_config(len(skel), [5, 5]), 2, ms, L * H, stream=stream)
    a.upload_W(Wm)
    for layer in range(L):
        S.check(Lb.sp_hip_hier_write_layer(a.ref, layer, 0, n, p(kt), p(vt), H * hd, S.DTYPE_F16))
    prefix = str(tmp_path / "hier")
    S.check(Lb.sp_hip_hier_cache_save(a.ref, prefix.encode(), n, h))
    assert os.path.getsize(f"{prefix}.hier_w.bin") == 64 + Wm.size * 2
    raw = open(f"{prefix}.L1.bin", "rb").read()
    hdr = struct.unpack("<4sIQ10iQ", raw[:64])
    B = a.c.bytes_per_pos_k
    assert hdr[:2] == (b"VHT2", 2) and hdr[7] == 2 and hdr[10:12] == (1, 1), hdr
    body = np.concatenate([records(a.c.d_k_cache, L, H, ms, B)[1, :, :n].reshape(-1),
                           records(a.c.d_v_cache, L, H, ms, B)[1, :, :n].reshape(-1)])
    np.testing.assert_array_equal(np.frombuffer(raw[64:], np.uint8), body)
    b = S.HierCache(cfg, pad, skel, tgt, S.band_config(len(skel), [5, 5]), 2, ms, L * H, stream=stream)
    assert Lb.sp_hip_hier_cache_load(b.ref, prefix.encode(), h) == n
    B = a.c.bytes_per_pos_k
    for ptr_a, ptr_b in ((a.c.d_k_cache, b.c.d_k_cache), (a.c.d_v_cache, b.c.d_v_cache)):
        np.testing.assert_array_equal(records(ptr_b, L, H, ms, B), records(ptr_a, L, H, ms, B))
    np.testing.assert_array_equal(d2h(b.c.d_W, Wm.size * 2).view(np.uint16).reshape(Wm.shape), Wm)
    a.free()
    b.free()


def write_v2(prefix, recs_k, recs_v, n, h, kind, order_check):
    """v2 layer files from records [L][H][n_pos][B]: the 64-byte header (version 2,
    one segment per side) and the records whole, in cache order."""
    L, H, _, kB = recs_k.shape
    vB = recs_v.shape[3]
    hd = 128
    for layer in range(L):
        hdr = struct.pack("<4sIQ10i", b"VHT2", 2, h, n, layer, H, hd, kind, kB, vB, 1, 1, order_check)
        hdr += struct.pack("<Q", fnv(hdr))
        body = recs_k[layer, :, :n].tobytes() + recs_v[layer, :, :n].tobytes()
        open(f"{prefix}.L{layer}.bin", "wb").write(hdr + body)


def test_v2_files_load_into_ship_caches(tmp_path):
    """A ship cache and the shadow cache load v2 files (records whole) as well as
    their own v3 files; a partial load of a v2 file reads every band."""
    say("disk v2 into ship caches")
    L, H, hd, ms, n = 2, 2, 128, 96, 80
    stream = torch.cuda.current_stream().cuda_stream
    cfg = S.config(hd, L, H)
    kB, vB = 76, 50
    a = S.ShipCache(cfg, ms, stream=stream)
    fill_ship(a, L, H, hd, n, 21)
    rk, rv = records(a.c.d_k_cache, L, H, ms, kB), records(a.c.d_v_cache, L, H, ms, vB)
    order = O.mobius_order(hd).astype(np.int32)
    order_check = fnv(order.tobytes()) & 0xffffffff
    order_check -= (1 << 32) if order_check >= (1 << 31) else 0  # the header's int32 slot
    prefix = str(tmp_path / "v2")
    h = fnv(b"model-v2")
    write_v2(prefix, rk, rv, n, h, 0, order_check)
    Lb = S.lib()
    for partial in (False, True):
        b = S.ShipCache(cfg, ms, stream=stream)
        got = (Lb.sp_hip_cache_load_partial(b.ref, prefix.encode(), h, 1) if partial
               else Lb.sp_hip_cache_load(b.ref, prefix.encode(), h))
        assert got == n, S.last_error()
        np.testing.assert_array_equal(records(b.c.d_k_cache, L, H, ms, kB)[:, :, :n], rk[:, :, :n])
        np.testing.assert_array_equal(records(b.c.d_v_cache, L, H, ms, vB)[:, :, :n], rv[:, :, :n])
        b.free()
    # the shadow cache (host record buffers) reads the same files
    sc = S.SpShadowCache()
    S.check(Lb.sp_shadow_cache_init(C.byref(sc), C.byref(cfg)))
    bufs = [np.zeros(n * kB, np.uint8) for _ in range(L * H)] + [np.zeros(n * vB, np.uint8) for _ in range(L * H)]
    kp = (C.POINTER(C.c_uint8) * (L * H))(*[x.ctypes.data_as(C.POINTER(C.c_uint8)) for x in bufs[:L * H]])
    vp = (C.POINTER(C.c_uint8) * (L * H))(*[x.ctypes.data_as(C.POINTER(C.c_uint8)) for x in bufs[L * H:]])
    sc.k_cache = C.cast(kp, C.POINTER(C.POINTER(C.c_uint8)))
    sc.v_cache = C.cast(vp, C.POINTER(C.POINTER(C.c_uint8)))
    S.check(Lb.sp_shadow_cache_set_slot_capacity(C.byref(sc), n))
    assert Lb.sp_shadow_cache_load_partial(C.byref(sc), prefix.encode(), h, 1) == n, S.last_error()
    for layer in range(L):
        for hh in range(H):
            np.testing.assert_array_equal(bufs[layer * H + hh].reshape(n, kB), rk[layer, hh, :n])
            np.testing.assert_array_equal(bufs[L * H + layer * H + hh].reshape(n, vB), rv[layer, hh, :n])
    Lb.sp_shadow_cache_free(C.byref(sc))
    # another version number is refused
    raw = bytearray(open(f"{prefix}.L0.bin", "rb").read())
    raw[4] = 4
    raw[56:64] = struct.pack("<Q", fnv(bytes(raw[:56])))
    open(f"{prefix}.L0.bin", "wb").write(bytes(raw))
    b = S.ShipCache(cfg, ms, stream=stream)
    assert Lb.sp_hip_cache_load(b.ref, prefix.encode(), h) == -1
    assert "version" in S.last_error()
    b.free()
    a.free()


def test_load_rejects_another_coefficient_order(tmp_path):
    """A file written under the default Mobius order does not load into a cache
    whose K order was recalibrated (its records would decode under the wrong order)."""
    L, H, hd, ms, n = 1, 2, 128, 64, 32
    stream = torch.cuda.current_stream().cuda_stream
    cfg = S.config(hd, L, H)
    a = S.ShipCache(cfg, ms, stream=stream)
    fill_ship(a, L, H, hd, n, 3)
    prefix = str(tmp_path / "o")
    Lb = S.lib()
    S.check(Lb.sp_hip_cache_save(a.ref, prefix.encode(), n, 5))
    b = S.ShipCache(cfg, ms, stream=stream)
    x = (np.random.default_rng(4).standard_normal((256, hd)) * np.linspace(0.1, 3, hd)).astype(np.float16)
    xt = dev(x.view(np.uint16))
    S.check(Lb.sp_hip_calibrate_begin(b.ref))
    S.check(Lb.sp_hip_calibrate_feed(b.ref, p(xt), hd, 256, S.DTYPE_F16))
    S.check(Lb.sp_hip_calibrate_end(b.ref, None, 1))
    assert Lb.sp_hip_cache_load(b.ref, prefix.encode(), 5) == -1
    assert b"order" in Lb.sp_hip_last_error()
    a.free()
    b.free()


def test_shadow_files_match_the_device_cache(tmp_path):
    """The shadow cache (host record buffers) writes the same bytes as the device
    cache for the same vectors, and each loads the other's files; a partial load
    clears the bands past the limit."""
    say("disk shadow")
    L, H, hd, n = 2, 2, 128, 48
    cfg = S.config(hd, L, H)
    Lb = S.lib()
    kB, vB = 76, 50
    x = np.random.default_rng(8).standard_normal((L, H, n, hd)).astype(np.float32)

    def shadow():
        sc = S.SpShadowCache()
        S.check(Lb.sp_shadow_cache_init(C.byref(sc), C.byref(cfg)))
        bufs = [np.zeros(n * kB, np.uint8) for _ in range(L * H)] + [np.zeros(n * vB, np.uint8) for _ in range(L * H)]
        kp = (C.POINTER(C.c_uint8) * (L * H))(*[b.ctypes.data_as(C.POINTER(C.c_uint8)) for b in bufs[:L * H]])
        vp = (C.POINTER(C.c_uint8) * (L * H))(*[b.ctypes.data_as(C.POINTER(C.c_uint8)) for b in bufs[L * H:]])
        sc.k_cache = C.cast(kp, C.POINTER(C.POINTER(C.c_uint8)))
        sc.v_cache = C.cast(vp, C.POINTER(C.POINTER(C.c_uint8)))
        S.check(Lb.sp_shadow_cache_set_slot_capacity(C.byref(sc), n))
        return sc, bufs, (kp, vp)

    sa, ba, keep_a = shadow()
    for layer in range(L):
        for h in range(H):
            Lb.sp_shadow_write_k_batch(C.byref(sa), layer, h, 0, n, C.c_void_p(x[layer, h].ctypes.data))
            Lb.sp_shadow_write_v_batch(C.byref(sa), layer, h, 0, n, C.c_void_p(x[layer, h].ctypes.data))
    ps, pd = str(tmp_path / "shadow"), str(tmp_path / "dev")
    S.check(Lb.sp_shadow_cache_save(C.byref(sa), ps.encode(), n, 11))
    stream = torch.cuda.current_stream().cuda_stream
    cc = S.ShipCache(cfg, n, stream=stream)
    # the device cache takes the same fp32 vectors ([slot][pos][hd])
    S.check(Lb.sp_hip_write_all(cc.ref, 0, n, p(dev(x.reshape(-1, hd))), p(dev(x.reshape(-1, hd))), S.DTYPE_F32))
    S.check(Lb.sp_hip_cache_save(cc.ref, pd.encode(), n, 11))
    for layer in range(L):
        assert open(f"{ps}.L{layer}.bin", "rb").read() == open(f"{pd}.L{layer}.bin", "rb").read()
    # shadow loads the device files, device loads the shadow files
    sb, bb, keep_b = shadow()
    assert Lb.sp_shadow_cache_load(C.byref(sb), pd.encode(), 11) == n
    for a_, b_ in zip(ba, bb):
        np.testing.assert_array_equal(a_, b_)
    cd = S.ShipCache(cfg, n, stream=stream)
    assert Lb.sp_hip_cache_load(cd.ref, ps.encode(), 11) == n
    np.testing.assert_array_equal(d2h(cd.c.d_k_cache, L * H * n * kB), np.concatenate(ba[:L * H]))
    # partial: K bands 0..1 kept, 2..3 cleared; the single V band kept
    sp_, bp, keep_p = shadow()
    assert Lb.sp_shadow_cache_load_partial(C.byref(sp_), ps.encode(), 11, 2) == n
    for s in range(L * H):
        k_full, k_part = ba[s].reshape(n, kB), bp[s].reshape(n, kB)
        np.testing.assert_array_equal(k_part[:, :44], k_full[:, :44])
        assert not k_part[:, 44:].any()
        np.testing.assert_array_equal(bp[L * H + s], ba[L * H + s])
    assert Lb.sp_shadow_cache_load(C.byref(sb), ps.encode(), 12) == -1
    # files longer than the slot buffers are refused before any record changes,
    # and so is a layer set whose last file is bad
    small, bs, keep_s = shadow()
    S.check(Lb.sp_shadow_cache_set_slot_capacity(C.byref(small), n - 1))
    assert Lb.sp_shadow_cache_load(C.byref(small), ps.encode(), 11) == -1
    assert "room" in S.last_error()
    assert Lb.sp_shadow_cache_save(C.byref(small), str(tmp_path / "x").encode(), n, 11) == -1
    assert not any(b_.any() for b_ in bs)
    bad = str(tmp_path / "bad")
    for layer in range(L):
        data = open(f"{ps}.L{layer}.bin", "rb").read()
        open(f"{bad}.L{layer}.bin", "wb").write(data if layer + 1 < L else data[:-5])
    fresh, bf, keep_f = shadow()
    assert Lb.sp_shadow_cache_load(C.byref(fresh), bad.encode(), 11) == -1
    assert "truncated" in S.last_error()
    assert not any(b_.any() for b_ in bf)
    cbad = S.ShipCache(cfg, n, stream=stream)
    assert Lb.sp_hip_cache_load(cbad.ref, bad.encode(), 11) == -1
    assert not d2h(cbad.c.d_k_cache, L * H * n * kB).any()
    cbad.free()
    cshort = S.ShipCache(cfg, n - 1, stream=stream)
    assert Lb.sp_hip_cache_load(cshort.ref, ps.encode(), 11) == -1
    cshort.free()
    for sc_ in (sa, sb, sp_, small, fresh):
        Lb.sp_shadow_cache_free(C.byref(sc_))
    cc.free()
    cd.free()
