"""Ship codec on the GPU vs the CPU oracle: packed codes bit-exact, reconstructions
bit-exact (same fp32 operation order), across kernel families, dtypes, band
geometries, normalisation conventions, partial reads and edge cases."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import oracle_py as O  # noqa: E402
import sp_hip as S  # noqa: E402
import workloads as W  # noqa: E402
from gpu_util import d2h, decode, dev, empty_f16, empty_f32, empty_u8, encode, host, order_dev, p, stream  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


CASES = [
    # hd, bits, mobius, norm, ternary   (fast path when hd pow2 and bands on multiples of 8)
    (128, [5, 5, 4, 3], True, S.NORM_FINAL, 0),
    (128, [3], False, S.NORM_FINAL, 0),
    (128, [5, 5, 4, 3], True, S.NORM_STAGE, 0),
    (64, [5, 5, 4, 3], True, S.NORM_FINAL, 0),
    (256, [5, 5, 4, 3], True, S.NORM_FINAL, 0),
    (256, [3], False, S.NORM_FINAL, 0),
    (128, [5, 5, 4, 3], True, S.NORM_FINAL, 1 << 3),
    (64, [5, 4, 4], True, S.NORM_FINAL, 0),        # bands 21/21/22 -> generic kernels
    (96, [5, 4, 4], True, S.NORM_FINAL, 0),        # Vilenkin 2^5*3
    (96, [5], False, S.NORM_FINAL, 0),
    (128, [5] * 10, True, S.NORM_FINAL, 0),        # last band absorbs remainder
    (128, [8, 8, 8, 8], True, S.NORM_FINAL, 0),
    (128, [2, 1], True, S.NORM_FINAL, 0),          # draft "aggressive" preset
]


@pytest.mark.parametrize("hd,bits,mob,norm,tmask", CASES)
def test_encode_decode_bit_exact(hd, bits, mob, norm, tmask):
    say(f"case hd={hd} bits={bits} mob={mob} norm={norm} tmask={tmask}")
    n = 1000
    k16, _ = W.cfg1_kv(n_heads=1, n_pos=n, hd=hd, seed=hd + len(bits))
    x16 = k16.reshape(n, hd).view(np.uint16)
    obc = O.band_config(hd, bits, tmask)
    sbc = S.band_config(hd, bits, tmask)
    order = O.mobius_order(hd) if mob else None
    ref = O.ship_compress_f16(x16, obc, order, norm)
    ot = order_dev(hd) if mob else None
    xt = dev(x16)
    for generic in (False, True):
        got = host(encode(sbc, ot, xt, S.DTYPE_F16, n, hd, norm, generic)).reshape(n, -1)
        np.testing.assert_array_equal(got, ref, err_msg=f"codes generic={generic}")
    # fp32 entry point gives the same codes
    got32 = host(encode(sbc, ot, dev(k16.reshape(n, hd).astype(np.float32)), S.DTYPE_F32, n, hd, norm)).reshape(n, -1)
    np.testing.assert_array_equal(got32, ref)
    # decode: fp32 bit-exact, fp16 bit-exact
    rec = dev(ref.reshape(-1))
    r32 = O.ship_decompress_f32(ref, obc, order, norm)
    r16 = O.ship_decompress_f16(ref, obc, order, norm)
    for generic in (False, True):
        g32 = host(decode(sbc, ot, rec, S.DTYPE_F32, n, hd, norm, -1, generic)).reshape(n, hd)
        np.testing.assert_array_equal(g32.view(np.uint32), r32.view(np.uint32), err_msg=f"f32 generic={generic}")
        g16 = host(decode(sbc, ot, rec, S.DTYPE_F16, n, hd, norm, -1, generic), np.uint16).reshape(n, hd)
        np.testing.assert_array_equal(g16, r16, err_msg=f"f16 generic={generic}")


@pytest.mark.parametrize("hd", [128, 256])
@pytest.mark.parametrize("max_bands", [0, 1, 2, 3, 4, 7, -1])
def test_partial_reads(max_bands, hd):
    bits, n = [5, 5, 4, 3], 300
    k16, _ = W.cfg1_kv(n_heads=1, n_pos=n, hd=hd, seed=9)
    x16 = k16.reshape(n, hd).view(np.uint16)
    obc, sbc = O.band_config(hd, bits), S.band_config(hd, bits)
    order = O.mobius_order(hd)
    ref = O.ship_compress_f16(x16, obc, order)
    want = O.ship_decompress_f32(ref, obc, order, O.NORM_FINAL, max_bands)
    for generic in (False, True):
        got = host(decode(sbc, order_dev(hd), dev(ref.reshape(-1)), S.DTYPE_F32, n, hd, S.NORM_FINAL,
                          max_bands, generic)).reshape(n, hd)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_edge_inputs():
    """zeros, fp16 extremes, huge fp32 values (scale overflow -> zeroed band), subnormals."""
    hd, bits = 128, [5, 5, 4, 3]
    rng = np.random.default_rng(4)
    rows = [np.zeros(hd, np.float32), np.full(hd, 65504.0, np.float32), np.full(hd, -65504.0, np.float32),
            (rng.standard_normal(hd) * 1e-6).astype(np.float32), (rng.standard_normal(hd) * 6e-8).astype(np.float32)]
    big = rng.standard_normal(hd).astype(np.float32)
    big[3] = 1e30
    rows.append(big)
    one = np.zeros(hd, np.float32)
    one[17] = 1.0
    rows.append(one)
    x = np.stack(rows * 10).astype(np.float32)
    n = x.shape[0]
    obc, sbc = O.band_config(hd, bits), S.band_config(hd, bits)
    order = O.mobius_order(hd)
    ref = O.ship_compress_f32(x, obc, order)
    for generic in (False, True):
        got = host(encode(sbc, order_dev(hd), dev(x), S.DTYPE_F32, n, hd, S.NORM_FINAL, generic)).reshape(n, -1)
        np.testing.assert_array_equal(got, ref)
        rec = O.ship_decompress_f32(ref, obc, order)
        g = host(decode(sbc, order_dev(hd), dev(ref.reshape(-1)), S.DTYPE_F32, n, hd, S.NORM_FINAL, -1, generic))
        np.testing.assert_array_equal(g.reshape(n, hd).view(np.uint32), rec.view(np.uint32))


def test_empty_and_single():
    hd, bc = 128, S.band_config(128, [3])
    x = dev(np.zeros((1, hd), np.float32))
    out = empty_u8(64)
    S.check(S.lib().sp_hip_ship_encode(C.byref(bc), None, 0, p(x), S.DTYPE_F32, 0, hd, p(out), 0, 1, 0, stream()))
    torch.cuda.synchronize()
    assert int(out.sum()) == 0
    got = host(encode(bc, None, x, S.DTYPE_F32, 1, hd))
    np.testing.assert_array_equal(got[:50], O.ship_compress_f32(np.zeros((1, hd), np.float32), O.band_config(128, [3]))[0])


def test_codes_at_rounding_ties():
    """Quantizer inputs that sit exactly on a half-integer round half to even
    (__float2int_rn, shannon_prime_cuda.cu:186). Such inputs are rare (a few rows in
    65536 of Llama-like K/V), so the test writes a whole 8-head, 8192-position layer
    through the cache, checks with the oracle that it holds tied rows for both K and
    V, and compares every code."""
    H, hd, n = 8, 128, 8192
    k16, v16 = W.cfg1_kv(n_heads=H, n_pos=n, hd=hd, seed=3)
    order = O.mobius_order(hd)
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    kt_rows = W.tie_rows(k16.reshape(-1, hd).view(np.uint16), kbc, order, O.NORM_FINAL, O.vht2)
    vt_rows = W.tie_rows(v16.reshape(-1, hd).view(np.uint16), vbc, None, O.NORM_FINAL, O.vht2)
    say(f"tie rows: K {kt_rows.tolist()} V {vt_rows.tolist()}")
    assert len(kt_rows) and len(vt_rows)
    cc = S.ShipCache(S.config(hd, 1, H), n, stream=torch.cuda.current_stream().cuda_stream)
    kt = dev(np.ascontiguousarray(k16.transpose(1, 0, 2)).view(np.uint16))  # llama rows [pos][head][hd]
    vt = dev(np.ascontiguousarray(v16.transpose(1, 0, 2)).view(np.uint16))
    S.check(S.lib().sp_hip_write_layer(cc.ref, 0, 0, n, p(kt), p(vt), H * hd, S.DTYPE_F16))
    torch.cuda.synchronize()
    kc = d2h(cc.c.d_k_cache, H * n * kbc.total_bytes).reshape(H * n, -1)
    vc = d2h(cc.c.d_v_cache, H * n * vbc.total_bytes).reshape(H * n, -1)
    kref = O.ship_compress_f16(k16.reshape(-1, hd).view(np.uint16), kbc, order)
    vref = O.ship_compress_f16(v16.reshape(-1, hd).view(np.uint16), vbc)
    np.testing.assert_array_equal(kc[kt_rows], kref[kt_rows])
    np.testing.assert_array_equal(vc[vt_rows], vref[vt_rows])
    np.testing.assert_array_equal(kc, kref)
    np.testing.assert_array_equal(vc, vref)
    cc.free()


def _v3_records(codes, scales):
    """Records of the one-band 3-bit layout at hd 128: the fp16 scale, then the 128
    codes packed 3 bits each from bit 0 (the reference's band packing)."""
    n = codes.shape[0]
    bits = ((codes[:, :, None] >> np.arange(3)) & 1).astype(np.uint8).reshape(n, 384)
    rec = np.zeros((n, 50), np.uint8)
    rec[:, 0:2] = scales.astype(np.uint16).view(np.uint8).reshape(n, 2)
    rec[:, 2:] = np.packbits(bits, axis=1, bitorder="little")
    return rec


def _same_bits_or_both_nan(got, ref, ftype):
    gf, rf = got.view(ftype), ref.view(ftype)
    both_nan = np.isnan(gf) & np.isnan(rf)
    return np.all((got == ref) | both_nan)


@pytest.mark.parametrize("n", [64 * 9 + 17, 64])
def test_v_decode_crafted_records(n):
    """The one-band 3-bit V layout at hd 128 over records the encoder never
    writes: every code 0..7 (7 decodes to +4), scales across the fp16 range
    (subnormal, normal, large enough that outputs overflow fp16), and tiles
    holding a +0, -0, infinite or NaN scale; a partial last tile. fp16 and fp32
    outputs against the oracle, bit for bit (NaN outputs compared as NaN: the
    oracle runs on x86, whose default NaN has the sign bit set)."""
    say(f"v3 crafted-record decode n={n}")
    hd = 128
    rng = np.random.default_rng(n)
    codes = rng.integers(0, 8, (n, hd))
    scales = rng.integers(0x0400, 0x7bff, n).astype(np.uint16)  # normal fp16
    scales[rng.random(n) < 0.05] = rng.integers(1, 0x3ff, 1)[0]  # some subnormal
    scales[3] = 0x7bff  # 65504: outputs overflow fp16
    if n > 64:
        scales[64 + 5] = 0x0000   # tile 1: +0
        scales[128 + 63] = 0x8000  # tile 2: -0
        scales[256] = 0x7c00      # tile 4: +inf
        scales[320 + 9] = 0xfe00  # tile 5: NaN
        codes[448:512] = 3        # tile 7: all-zero coefficients with a zero scale
        scales[448:512] = 0x0000
    rec = _v3_records(codes, scales)
    obc, sbc = O.band_config(hd, [3]), S.band_config(hd, [3])
    rt = dev(rec.reshape(-1))
    r16 = O.ship_decompress_f16(rec, obc)
    r32 = O.ship_decompress_f32(rec, obc)
    g16 = host(decode(sbc, None, rt, S.DTYPE_F16, n, hd), np.uint16).reshape(n, hd)
    g32 = host(decode(sbc, None, rt, S.DTYPE_F32, n, hd)).reshape(n, hd)
    assert _same_bits_or_both_nan(g16, r16, np.float16), np.argwhere(g16 != r16)[:8]
    assert _same_bits_or_both_nan(g32.view(np.uint32), r32.view(np.uint32), np.float32), \
        np.argwhere(g32.view(np.uint32) != r32.view(np.uint32))[:8]
    # tiles without a non-finite scale match bit for bit, NaN aside
    good = np.ones(n, bool)
    if n > 64:
        good[256:384] = False
    assert np.array_equal(g16[good], r16[good])


@pytest.mark.parametrize("n_pos", [65536, 40001])
def test_multi_tile_blocks_bit_exact(n_pos):
    """Layer-wide calls large enough that every persistent block walks more than one
    64-vector tile (the grid is 16 single-wave blocks per CU, 4096 on MI355X):
    8 heads x 65536 positions are 8192 tiles, two per block, with the next tile's
    inputs prefetched across the tile boundary; 40001 positions give 626 tiles per
    head (the last one a single vector), so blocks walk one or two tiles and some
    tiles straddle nothing but a one-vector tail. K and V encode through write_all,
    both decodes through read_all (fp16), every code and every reconstructed value
    against the oracle."""
    H, hd = 8, 128
    say(f"multi-tile codec H={H} n_pos={n_pos}")
    k16, v16 = W.cfg2_kv(n_heads=H, n_pos=n_pos, hd=hd, seed=n_pos)
    cc = S.ShipCache(S.config(hd, 1, H), n_pos, stream=torch.cuda.current_stream().cuda_stream)
    L = S.lib()
    kt = dev(k16.reshape(H * n_pos, hd).view(np.uint16))
    vt = dev(v16.reshape(H * n_pos, hd).view(np.uint16))
    S.check(L.sp_hip_write_all(cc.ref, 0, n_pos, p(kt), p(vt), S.DTYPE_F16), "write_all")
    del kt, vt
    order = O.mobius_order(hd)
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    kref = O.ship_compress_f16(k16.reshape(-1, hd).view(np.uint16), kbc, order)
    vref = O.ship_compress_f16(v16.reshape(-1, hd).view(np.uint16), vbc)
    kc = d2h(cc.c.d_k_cache, kref.size).reshape(kref.shape)
    vc = d2h(cc.c.d_v_cache, vref.size).reshape(vref.shape)
    np.testing.assert_array_equal(kc, kref, err_msg="K codes")
    np.testing.assert_array_equal(vc, vref, err_msg="V codes")
    ko, vo = empty_f16(H * n_pos * hd), empty_f16(H * n_pos * hd)
    S.check(L.sp_hip_read_all(cc.ref, 0, n_pos, p(ko), p(vo), S.DTYPE_F16, -1), "read_all")
    np.testing.assert_array_equal(host(ko, np.uint16).reshape(-1, hd), O.ship_decompress_f16(kref, kbc, order),
                                  err_msg="K reconstruction")
    np.testing.assert_array_equal(host(vo, np.uint16).reshape(-1, hd), O.ship_decompress_f16(vref, vbc),
                                  err_msg="V reconstruction")
    cc.free()


@pytest.mark.parametrize("strided", [False, True])
def test_cache_hd96_vilenkin(strided):
    """hd 96 (Vilenkin 2^5*3) with the bridge defaults K 5/4/4 + Mobius and V 5 through
    the cache: contiguous [slot][pos][hd] rows (write_all/read_all) or llama cache rows
    with a head stride (write_layer/read_layer); codes and fp16/fp32 reconstructions
    bit-exact, including a partial last tile."""
    L_, H, hd, max_seq, n = 2, 4, 96, 200, 131
    say(f"cache hd96 strided={strided}")
    cfg = S.config(hd, L_, H, k_bits=(5, 4, 4), v_bits=(5,))
    cc = S.ShipCache(cfg, max_seq, stream=torch.cuda.current_stream().cuda_stream)
    order = O.mobius_order(hd)
    kbc, vbc = O.band_config(hd, [5, 4, 4]), O.band_config(hd, [5])
    assert (kbc.total_bytes, vbc.total_bytes) == (58, 62)
    k16, v16 = W.cfg3_kv(n_heads=L_ * H, n_pos=n, hd=hd, seed=96)  # [slot][pos][hd]
    if strided:
        for layer in range(L_):
            kt = dev(np.ascontiguousarray(k16[layer * H:(layer + 1) * H].transpose(1, 0, 2)).view(np.uint16))
            vt = dev(np.ascontiguousarray(v16[layer * H:(layer + 1) * H].transpose(1, 0, 2)).view(np.uint16))
            S.check(S.lib().sp_hip_write_layer(cc.ref, layer, 0, n, p(kt), p(vt), H * hd, S.DTYPE_F16))
    else:
        kt, vt = dev(k16.view(np.uint16)), dev(v16.view(np.uint16))  # both alive through the launch
        S.check(S.lib().sp_hip_write_all(cc.ref, 0, n, p(kt), p(vt), S.DTYPE_F16))
    torch.cuda.synchronize()
    kc = d2h(cc.c.d_k_cache, L_ * H * max_seq * 58).reshape(L_ * H, max_seq, 58)
    vc = d2h(cc.c.d_v_cache, L_ * H * max_seq * 62).reshape(L_ * H, max_seq, 62)
    for slot in range(L_ * H):
        kref = O.ship_compress_f16(k16[slot].view(np.uint16), kbc, order)
        vref = O.ship_compress_f16(v16[slot].view(np.uint16), vbc)
        np.testing.assert_array_equal(kc[slot, :n], kref, err_msg=f"K codes slot {slot}")
        np.testing.assert_array_equal(vc[slot, :n], vref, err_msg=f"V codes slot {slot}")
    for dtype in (S.DTYPE_F16, S.DTYPE_F32):
        mk = empty_f16 if dtype == S.DTYPE_F16 else empty_f32
        hdt = np.uint16 if dtype == S.DTYPE_F16 else np.uint32
        if strided:
            for layer in range(L_):
                kl, vl = mk(n * H * hd), mk(n * H * hd)
                S.check(S.lib().sp_hip_read_layer(cc.ref, layer, 0, n, p(kl), p(vl), H * hd, dtype, -1))
                ka = host(kl, hdt).reshape(n, H, hd).transpose(1, 0, 2)
                va = host(vl, hdt).reshape(n, H, hd).transpose(1, 0, 2)
                if layer == 0:
                    kall, vall = [ka], [va]
                else:
                    kall.append(ka)
                    vall.append(va)
            kg, vg = np.concatenate(kall), np.concatenate(vall)
        else:
            ko, vo = mk(L_ * H * n * hd), mk(L_ * H * n * hd)
            S.check(S.lib().sp_hip_read_all(cc.ref, 0, n, p(ko), p(vo), dtype, -1))
            kg, vg = host(ko, hdt).reshape(L_ * H, n, hd), host(vo, hdt).reshape(L_ * H, n, hd)
        for slot in range(L_ * H):
            if dtype == S.DTYPE_F16:
                kr = O.ship_decompress_f16(kc[slot, :n], kbc, order)
                vr = O.ship_decompress_f16(vc[slot, :n], vbc)
            else:
                kr = O.ship_decompress_f32(kc[slot, :n], kbc, order).view(np.uint32)
                vr = O.ship_decompress_f32(vc[slot, :n], vbc).view(np.uint32)
            np.testing.assert_array_equal(kg[slot], kr, err_msg=f"K recon slot {slot} dtype {dtype}")
            np.testing.assert_array_equal(vg[slot], vr, err_msg=f"V recon slot {slot} dtype {dtype}")
    cc.free()


def test_cache_slots_layer_and_all_layouts():
    """sp_hip_write_layer / read_layer (llama cache rows) and write_all / read_all agree with
    the oracle for every slot, including odd start positions (unaligned V records)."""
    L, H, hd, max_seq = 3, 4, 128, 96
    cfg = S.config(hd, L, H)
    cc = S.ShipCache(cfg, max_seq, stream=torch.cuda.current_stream().cuda_stream)
    order = O.mobius_order(hd)
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    rng = np.random.default_rng(12)
    start, n_tok = 13, 41
    k = rng.standard_normal((L, n_tok, H, hd)).astype(np.float16)
    v = rng.standard_normal((L, n_tok, H, hd)).astype(np.float16)
    for layer in range(L):
        kt, vt = dev(k[layer].view(np.uint16)), dev(v[layer].view(np.uint16))
        S.check(S.lib().sp_hip_write_layer(cc.ref, layer, start, n_tok, p(kt), p(vt), H * hd, S.DTYPE_F16))
    torch.cuda.synchronize()
    kB, vB = kbc.total_bytes, vbc.total_bytes
    kc = d2h(cc.c.d_k_cache, L * H * max_seq * kB).reshape(L, H, max_seq, kB)
    vc = d2h(cc.c.d_v_cache, L * H * max_seq * vB).reshape(L, H, max_seq, vB)
    for layer in range(L):
        for h in range(H):
            kref = O.ship_compress_f16(k[layer, :, h].view(np.uint16), kbc, order)
            vref = O.ship_compress_f16(v[layer, :, h].view(np.uint16), vbc)
            np.testing.assert_array_equal(kc[layer, h, start:start + n_tok], kref)
            np.testing.assert_array_equal(vc[layer, h, start:start + n_tok], vref)
            assert not kc[layer, h, :start].any() and not kc[layer, h, start + n_tok:].any()
            assert not vc[layer, h, :start].any() and not vc[layer, h, start + n_tok:].any()
    # read_layer back (fp32 rows)
    for layer in range(L):
        ko, vo = empty_f32(n_tok * H * hd), empty_f32(n_tok * H * hd)
        S.check(S.lib().sp_hip_read_layer(cc.ref, layer, start, n_tok, p(ko), p(vo), H * hd, S.DTYPE_F32, -1))
        ko = host(ko).reshape(n_tok, H, hd)
        vo = host(vo).reshape(n_tok, H, hd)
        for h in range(H):
            np.testing.assert_array_equal(ko[:, h], O.ship_decompress_f32(kc[layer, h, start:start + n_tok], kbc, order))
            np.testing.assert_array_equal(vo[:, h], O.ship_decompress_f32(vc[layer, h, start:start + n_tok], vbc))
    # read_all over every slot (fp16)
    ka, va = empty_f16(L * H * n_tok * hd), empty_f16(L * H * n_tok * hd)
    S.check(S.lib().sp_hip_read_all(cc.ref, start, n_tok, p(ka), p(va), S.DTYPE_F16, -1))
    ka = host(ka, np.uint16).reshape(L, H, n_tok, hd)
    for layer in range(L):
        for h in range(H):
            np.testing.assert_array_equal(ka[layer, h], O.ship_decompress_f16(kc[layer, h, start:start + n_tok], kbc, order))
    # out-of-range requests are rejected without launching
    kt = dev(k[0].view(np.uint16))
    assert S.lib().sp_hip_write_layer(cc.ref, L, 0, 1, p(kt), p(kt), H * hd, S.DTYPE_F16) == -1
    assert S.lib().sp_hip_write_layer(cc.ref, 0, max_seq - 1, 2, p(kt), p(kt), H * hd, S.DTYPE_F16) == -1
    assert S.lib().sp_hip_write_layer(cc.ref, 0, 0, 2, p(kt), p(kt), H * hd - 1, S.DTYPE_F16) == -1
    cc.free()


@pytest.mark.parametrize("kernel", ["narrow", "lane"])
@pytest.mark.parametrize("dtype,k_pad,max_bands", [("f16", 0, -1), ("f16", 4, 2), ("f32", 0, 3), ("f32", 3, -1)])
def test_roundtrip_cells(dtype, k_pad, max_bands, kernel, monkeypatch):
    """sp_hip_roundtrip_cells (the device post-decode hook): K as llama.cpp cache rows
    (row stride H*hd + k_pad: 16-byte pieces, or element by element when the rows
    are not 16-byte aligned), V in the transposed v_trans layout, 77 scattered cells
    plus one past max_seq. Records at the listed cells equal the oracle's records of
    the original vectors; the tensor at those cells holds the oracle's reconstruction
    (bands >= max_bands zero); every other cell and the row padding are untouched.
    Both kernels: head_dim/8 lanes per vector with K and V in one launch, and one
    vector per lane, one launch per side."""
    monkeypatch.setenv("SP_HIP_RT_KERNEL", kernel)
    say(f"roundtrip cells kernel={kernel} dtype={dtype} k_pad={k_pad} max_bands={max_bands}")
    L, H, hd, max_seq, kv_size, layer = 2, 4, 128, 300, 320, 1
    cfg = S.config(hd, L, H)
    cc = S.ShipCache(cfg, max_seq, stream=torch.cuda.current_stream().cuda_stream)
    order = O.mobius_order(hd)
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    rng = np.random.default_rng(50 + k_pad)
    kcs = H * hd + k_pad
    npdt = np.float16 if dtype == "f16" else np.float32
    k = rng.standard_normal((kv_size, kcs)).astype(npdt)
    v = rng.standard_normal((H * hd, kv_size)).astype(npdt)  # v_trans: [h*hd + d][cell]
    cells = np.concatenate([rng.choice(max_seq, 77, replace=False), [max_seq + 5]]).astype(np.int32)
    rng.shuffle(cells)
    kt, vt, ct = dev(k), dev(v), dev(cells)
    dt = S.DTYPE_F16 if dtype == "f16" else S.DTYPE_F32
    S.check(S.lib().sp_hip_roundtrip_cells(cc.ref, layer, p(ct), len(cells), p(kt), kcs, p(vt), 1, kv_size, dt,
                                           max_bands, None))
    kg, vg = host(kt), host(vt)
    kB, vB = kbc.total_bytes, vbc.total_bytes
    kc = d2h(cc.c.d_k_cache, L * H * max_seq * kB).reshape(L, H, max_seq, kB)
    vc = d2h(cc.c.d_v_cache, L * H * max_seq * vB).reshape(L, H, max_seq, vB)
    live = np.sort(cells[cells < max_seq])
    dead = np.setdiff1d(np.arange(kv_size), live)
    np.testing.assert_array_equal(kg[dead], k[dead])
    np.testing.assert_array_equal(vg[:, dead], v[:, dead])
    np.testing.assert_array_equal(kg[:, H * hd:], k[:, H * hd:])
    assert not kc[0].any() and not vc[0].any(), "other layer written"
    mask = np.zeros(max_seq, bool)
    mask[live] = True
    for h in range(H):
        xk, xv = k[live, h * hd:(h + 1) * hd], v[h * hd:(h + 1) * hd, live].T
        if dtype == "f16":
            kref = O.ship_compress_f16(xk.view(np.uint16), kbc, order)
            vref = O.ship_compress_f16(np.ascontiguousarray(xv).view(np.uint16), vbc)
            krec = O.ship_decompress_f16(kref, kbc, order, max_bands=max_bands).view(np.float16)
            vrec = O.ship_decompress_f16(vref, vbc, max_bands=max_bands).view(np.float16)
        else:
            kref = O.ship_compress_f32(xk, kbc, order)
            vref = O.ship_compress_f32(np.ascontiguousarray(xv), vbc)
            krec = O.ship_decompress_f32(kref, kbc, order, max_bands=max_bands)
            vrec = O.ship_decompress_f32(vref, vbc, max_bands=max_bands)
        np.testing.assert_array_equal(kc[layer, h, live], kref)
        np.testing.assert_array_equal(vc[layer, h, live], vref)
        assert not kc[layer, h, ~mask].any() and not vc[layer, h, ~mask].any()
        np.testing.assert_array_equal(kg[live, h * hd:(h + 1) * hd].view(np.uint8), krec.view(np.uint8))
        np.testing.assert_array_equal(vg[h * hd:(h + 1) * hd, live].T.copy().view(np.uint8), vrec.view(np.uint8))
    # layouts the entry point rejects
    assert S.lib().sp_hip_roundtrip_cells(cc.ref, layer, p(ct), len(cells), p(kt), H * hd - 1, None, 0, 0, dt, -1,
                                          None) == -1
    assert S.lib().sp_hip_roundtrip_cells(cc.ref, layer, p(ct), len(cells), None, 0, p(vt), 2, 2, dt, -1, None) == -1
    cc.free()



@pytest.mark.parametrize("hd,n_cells,calibrated,v_trans", [(64, 1, False, True), (128, 1, True, True),
                                                         (256, 5, False, False), (128, 300, True, False)])
def test_roundtrip_cells_any_order_and_width(hd, n_cells, calibrated, v_trans):
    """The narrow round trip at head_dim 64 / 128 / 256, a single decode cell, and a
    calibrated (variance-ranked) K order, which the one-vector-per-lane kernel does
    not take: records and reconstructions equal the oracle's with that order."""
    say(f"roundtrip narrow hd={hd} n_cells={n_cells} calibrated={calibrated} v_trans={v_trans}")
    L, H, max_seq, layer = 1, 4, 400, 0
    cfg = S.config(hd, L, H)
    cc = S.ShipCache(cfg, max_seq, stream=torch.cuda.current_stream().cuda_stream)
    Lb = S.lib()
    rng = np.random.default_rng(hd + n_cells)
    order = O.mobius_order(hd)
    if calibrated:
        calib = (rng.standard_normal((512, hd)) * np.linspace(0.1, 3.0, hd)).astype(np.float16)
        ct0 = dev(calib.view(np.uint16))
        S.check(Lb.sp_hip_calibrate_begin(cc.ref))
        S.check(Lb.sp_hip_calibrate_feed(cc.ref, p(ct0), hd, 512, S.DTYPE_F16))
        got = np.zeros(hd, np.int32)
        S.check(Lb.sp_hip_calibrate_end(cc.ref, got.ctypes.data_as(C.c_void_p), 1))
        order = got
        assert not np.array_equal(order, O.mobius_order(hd))
    kbc = O.band_config(hd, list(cfg.k_band_bits[:cfg.k_n_bands]))
    vbc = O.band_config(hd, list(cfg.v_band_bits[:cfg.v_n_bands]))
    row = H * hd
    k = rng.standard_normal((max_seq, row)).astype(np.float16)
    v = rng.standard_normal((row, max_seq) if v_trans else (max_seq, row)).astype(np.float16)
    cells = rng.choice(max_seq, n_cells, replace=False).astype(np.int32)
    kt, vt, ct = dev(k.view(np.uint16)), dev(v.view(np.uint16)), dev(cells)
    vcs, ves = (1, max_seq) if v_trans else (row, 1)
    S.check(Lb.sp_hip_roundtrip_cells(cc.ref, layer, p(ct), n_cells, p(kt), row, p(vt), vcs, ves, S.DTYPE_F16, -1,
                                      None))
    kg, vg = host(kt).view(np.float16).reshape(k.shape), host(vt).view(np.float16).reshape(v.shape)
    kB, vB = kbc.total_bytes, vbc.total_bytes
    kc = d2h(cc.c.d_k_cache, H * max_seq * kB).reshape(H, max_seq, kB)
    vc = d2h(cc.c.d_v_cache, H * max_seq * vB).reshape(H, max_seq, vB)
    for h in range(H):
        xk = np.ascontiguousarray(k[cells, h * hd:(h + 1) * hd])
        xv = np.ascontiguousarray(v[h * hd:(h + 1) * hd, cells].T if v_trans else v[cells, h * hd:(h + 1) * hd])
        kref = O.ship_compress_f16(xk.view(np.uint16), kbc, order)
        vref = O.ship_compress_f16(xv.view(np.uint16), vbc)
        np.testing.assert_array_equal(kc[h, cells], kref)
        np.testing.assert_array_equal(vc[h, cells], vref)
        krec = O.ship_decompress_f16(kref, kbc, order).view(np.float16)
        vrec = O.ship_decompress_f16(vref, vbc).view(np.float16)
        np.testing.assert_array_equal(kg[cells, h * hd:(h + 1) * hd].view(np.uint16), krec.view(np.uint16))
        vgot = vg[h * hd:(h + 1) * hd, cells].T if v_trans else vg[cells, h * hd:(h + 1) * hd]
        np.testing.assert_array_equal(np.ascontiguousarray(vgot).view(np.uint16), vrec.view(np.uint16))
    cc.free()
