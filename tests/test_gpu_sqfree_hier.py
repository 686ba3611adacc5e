"""Sqfree+spinor and hierarchical Vilenkin codecs on the GPU vs the CPU oracle:
records bit-exact, reconstructions bit-exact."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import oracle_py as O  # noqa: E402
import sp_hip as S  # noqa: E402
import workloads as W  # noqa: E402
from gpu_util import d2h, dev, empty_f32, host, p  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("hd,bits,rbits,spinor,sk_frac", [
    (128, [5, 4, 4, 4, 5], 3, True, 0.0),    # reference CUDA geometry: sk_k = pad/2 = 77
    (128, [5, 4, 4, 4, 5], 3, True, 0.75),   # cfg 4: SK_FRAC 0.75 -> sk_k = 115
    (128, [3, 3, 3, 3, 3], 3, True, 0.0),    # SPINOR 3/3/3/3/3 (shannon_prime_llama_sqfree.c:27)
    (128, [5, 4, 4, 4, 5], 2, False, 0.0),
    (64, [5, 4, 4, 4, 5], 4, True, 0.0),
    (256, [5, 4, 4, 4, 5], 3, True, 0.0),
])
def test_sqfree_bit_exact(hd, bits, rbits, spinor, sk_frac):
    say(f"sqfree hd={hd} bits={bits} rbits={rbits} spinor={spinor} sk_frac={sk_frac}")
    n = 300
    k16, _ = W.cfg4_kv(n_heads=1, n_pos=n, hd=hd, seed=hd + rbits)
    x16 = k16.reshape(n, hd).view(np.uint16)
    pad = O.sqfree_pad_dim(hd)
    sk = int(pad * sk_frac) if sk_frac else pad // 2
    km = O.Knight(pad, sk)
    skel_bc = O.band_config(sk, bits)
    ref = O.sqfree_compress_f16(x16, hd, km, skel_bc, rbits, spinor)
    rec = O.sqfree_decompress_f32(ref, hd, km, skel_bc, rbits, spinor)
    cfg = S.config(hd, 1, 1, k_bits=bits, v_bits=bits)
    cc = S.SqfreeCache(cfg, n, rbits=rbits, spinor=spinor, sk_k=sk,
                       stream=torch.cuda.current_stream().cuda_stream)
    assert (cc.c.pad_dim, cc.c.sk_k, cc.c.n_res) == (pad, sk, pad - sk)
    # device Knight tables equal the oracle's
    sk_idx = np.zeros(sk, np.int32)
    res_idx = np.zeros(max(pad - sk, 1), np.int32)
    off = np.zeros(pad - sk + 1, np.int32)
    slot = np.zeros(max(cc.c.n_terms, 1), np.int32)
    mu = np.zeros(max(cc.c.n_terms, 1), np.int32)
    S.check(S.lib().sp_hip_sqfree_get_tables(cc.ref, C.c_void_p(sk_idx.ctypes.data),
                                             C.c_void_p(res_idx.ctypes.data), C.c_void_p(off.ctypes.data),
                                             C.c_void_p(slot.ctypes.data), C.c_void_p(mu.ctypes.data)))
    np.testing.assert_array_equal(sk_idx, km.skeleton_idx)
    np.testing.assert_array_equal(off, km.csr_offsets)
    assert cc.c.n_terms == km.n_terms
    np.testing.assert_array_equal(slot[:km.n_terms], km.csr_skel_slot)
    np.testing.assert_array_equal(mu[:km.n_terms], km.csr_mu_sign.astype(np.int32))
    assert cc.c.bytes_per_pos_k == ref.shape[1]
    xt = dev(x16)
    S.check(S.lib().sp_hip_sqfree_write_batch(cc.ref, 0, 0, 0, 0, n, p(xt), S.DTYPE_F16))
    got = d2h(cc.c.d_k_cache, n * ref.shape[1]).reshape(n, -1)
    np.testing.assert_array_equal(got, ref)
    out = empty_f32(n * hd)
    S.check(S.lib().sp_hip_sqfree_read_batch(cc.ref, 0, 0, 0, 0, n, p(out), S.DTYPE_F32))
    g = host(out).reshape(n, hd)
    np.testing.assert_array_equal(g.view(np.uint32), rec.view(np.uint32))
    # fp16 reads: the fp32 reconstruction rounded to nearest even
    out16 = torch.empty(n * hd, dtype=torch.float16, device="cuda")
    S.check(S.lib().sp_hip_sqfree_read_batch(cc.ref, 0, 0, 0, 0, n, p(out16), S.DTYPE_F16))
    np.testing.assert_array_equal(host(out16).reshape(n, hd).view(np.uint16), rec.astype(np.float16).view(np.uint16))
    corr = np.mean([O.correlation(a, b) for a, b in zip(k16.reshape(n, hd).astype(np.float32), g)])
    assert corr > 0.9, corr
    cc.free()


def test_sqfree_record_size_cfg4():
    """98 B at pad 154, sk_k 77, 5/4/4/4/5, rb 3, spinor (shannon_prime_sqfree.cu:683-686)."""
    cfg = S.config(128, 1, 1, k_bits=[5, 4, 4, 4, 5], v_bits=[5, 4, 4, 4, 5])
    cc = S.SqfreeCache(cfg, 4, rbits=3, spinor=True)
    assert cc.c.bytes_per_pos_k == 98
    cc.free()


@pytest.mark.parametrize("hd,rbits,skel_bits", [(256, 2, [5, 5]), (128, 2, [5, 5]), (128, 3, [5, 4, 4])])
def test_hier_bit_exact(hd, rbits, skel_bits):
    say(f"hier hd={hd} rbits={rbits} skel_bits={skel_bits}")
    n, n_slots = 200, 2
    pad = O.sqfree_pad_dim(hd)
    skel_idx, tgt_idx = O.hier_geometry(pad)
    skel_bc = O.band_config(len(skel_idx), skel_bits)
    Wm = W.hier_W(n_slots, len(tgt_idx), len(skel_idx), seed=hd)
    k16, _ = W.cfg5_kv(n_heads=n_slots, n_pos=n, hd=hd, seed=hd + 1)
    cfg = S.config(hd, 1, n_slots)
    hc = S.HierCache(cfg, pad, skel_idx, tgt_idx, S.band_config(len(skel_idx), skel_bits), rbits, n,
                     n_slots, stream=torch.cuda.current_stream().cuda_stream)
    hc.upload_W(Wm)
    B = O.hier_bytes(skel_bc, len(tgt_idx), rbits)
    assert hc.c.bytes_per_pos_k == B
    for slot in range(n_slots):
        x16 = k16[slot].view(np.uint16)
        ref = O.hier_compress_f16(x16, hd, pad, skel_idx, tgt_idx, skel_bc, Wm[slot], rbits)
        rec = O.hier_decompress_f32(ref, hd, pad, skel_idx, tgt_idx, skel_bc, Wm[slot], rbits)
        xt = dev(x16)
        S.check(S.lib().sp_hip_hier_write_batch(hc.ref, 1, 0, slot, 0, n, p(xt), S.DTYPE_F16))
        allv = d2h(hc.c.d_v_cache, n_slots * n * B).reshape(n_slots, n, B)
        np.testing.assert_array_equal(allv[slot], ref)
        out = empty_f32(n * hd)
        S.check(S.lib().sp_hip_hier_read_batch(hc.ref, 1, 0, slot, 0, n, p(out), S.DTYPE_F32))
        np.testing.assert_array_equal(host(out).reshape(n, hd).view(np.uint32), rec.view(np.uint32))
    hc.free()


@pytest.mark.parametrize("dtype", ["f16", "f32", "f32_tiny"])
def test_hier_default_geometry_lanes(dtype):
    """configs[4] geometry (hd 256 -> pad 330, 30 skeleton at 5/5, 300 targets at
    2 bits): the one-vector-per-lane kernels. 229 positions from position 4 (a
    partial last tile whose 103-byte records end 3 bytes into a dword), two slots,
    fp16 and fp32 inputs and outputs; f32_tiny scales the inputs to ~1e-37 so the
    predictor products are fp32 subnormals."""
    say(f"hier lanes dtype={dtype}")
    hd, rbits, n, start, n_slots = 256, 2, 229, 4, 2
    max_seq = start + n + 3
    pad = O.sqfree_pad_dim(hd)
    skel_idx, tgt_idx = O.hier_geometry(pad)
    skel_bc = O.band_config(len(skel_idx), [5, 5])
    B = O.hier_bytes(skel_bc, len(tgt_idx), rbits)
    assert (pad, B, (max_seq * B) % 4, (start * B) % 4, (n * B) % 4) == (330, 103, 0, 0, 3)
    Wm = W.hier_W(n_slots, len(tgt_idx), len(skel_idx), seed=21)
    k16, _ = W.cfg5_kv(n_heads=n_slots, n_pos=n, hd=hd, seed=22)
    cfg = S.config(hd, 1, n_slots)
    hc = S.HierCache(cfg, pad, skel_idx, tgt_idx, S.band_config(len(skel_idx), [5, 5]), rbits, max_seq,
                     n_slots, stream=torch.cuda.current_stream().cuda_stream)
    hc.upload_W(Wm)
    for slot in range(n_slots):
        if dtype == "f16":
            x16 = k16[slot].view(np.uint16)
            ref = O.hier_compress_f16(x16, hd, pad, skel_idx, tgt_idx, skel_bc, Wm[slot], rbits)
            xt = dev(x16)
            S.check(S.lib().sp_hip_hier_write_batch(hc.ref, 0, 0, slot, start, n, p(xt), S.DTYPE_F16))
        else:
            x32 = k16[slot].astype(np.float32) * np.float32(1.0 + 2.0 ** -12)
            if dtype == "f32_tiny":
                x32 = x32 * np.float32(1e-37)
            ref = O.hier_compress_f32(x32, hd, pad, skel_idx, tgt_idx, skel_bc, Wm[slot], rbits)
            xt = dev(x32)
            S.check(S.lib().sp_hip_hier_write_batch(hc.ref, 0, 0, slot, start, n, p(xt), S.DTYPE_F32))
        rec = O.hier_decompress_f32(ref, hd, pad, skel_idx, tgt_idx, skel_bc, Wm[slot], rbits)
        allk = d2h(hc.c.d_k_cache, n_slots * max_seq * B).reshape(n_slots, max_seq, B)
        np.testing.assert_array_equal(allk[slot, start:start + n], ref)
        assert not allk[slot, start + n:].any() and not allk[slot, :start].any(), "writes outside the batch"
        out = empty_f32(n * hd)
        S.check(S.lib().sp_hip_hier_read_batch(hc.ref, 0, 0, slot, start, n, p(out), S.DTYPE_F32))
        np.testing.assert_array_equal(host(out).reshape(n, hd).view(np.uint32), rec.view(np.uint32))
        out16 = torch.empty(n * hd, dtype=torch.float16, device="cuda")
        S.check(S.lib().sp_hip_hier_read_batch(hc.ref, 0, 0, slot, start, n, p(out16), S.DTYPE_F16))
        np.testing.assert_array_equal(host(out16).reshape(n, hd).view(np.uint16),
                                      rec.astype(np.float16).view(np.uint16))
    hc.free()


def _rows(x16, row_pad):
    """[H][n][hd] fp16 -> llama.cpp cache rows [n][H*hd + row_pad] (padding = 0x7e00 NaN sentinel)."""
    H, n, hd = x16.shape
    rows = np.full((n, H * hd + row_pad), 0x7e00, np.uint16)
    for h in range(H):
        rows[:, h * hd:(h + 1) * hd] = x16[h].view(np.uint16)
    return rows


@pytest.mark.parametrize("sk_frac", [0.75, 0.0])
def test_sqfree_layer_wide(sk_frac):
    """sp_hip_sqfree_write_layer / read_layer: every head of layer 1 in one launch
    from llama.cpp cache rows (row stride H*hd + 8), 150 tokens from position 3;
    records and fp32 reconstructions bit-exact against the oracle per head, row
    padding untouched."""
    say(f"sqfree layer-wide sk_frac={sk_frac}")
    hd, H, n, start, pad_row = 128, 4, 150, 3, 8
    k16, v16 = W.cfg4_kv(n_heads=H, n_pos=n, hd=hd, seed=31)
    pad = O.sqfree_pad_dim(hd)
    sk = int(pad * sk_frac) if sk_frac else pad // 2
    km = O.Knight(pad, sk)
    bits = [5, 4, 4, 4, 5]
    skel_bc = O.band_config(sk, bits)
    cfg = S.config(hd, 2, H, k_bits=bits, v_bits=bits)
    cc = S.SqfreeCache(cfg, start + n + 5, rbits=3, spinor=True, sk_k=sk,
                       stream=torch.cuda.current_stream().cuda_stream)
    B = cc.c.bytes_per_pos_k
    stride = H * hd + pad_row
    kt, vt = dev(_rows(k16, pad_row)), dev(_rows(v16, pad_row))
    S.check(S.lib().sp_hip_sqfree_write_layer(cc.ref, 1, start, n, p(kt), p(vt), stride, S.DTYPE_F16))
    ko = torch.full((n * stride,), float("nan"), dtype=torch.float32, device="cuda")
    vo = torch.full((n * stride,), float("nan"), dtype=torch.float32, device="cuda")
    S.check(S.lib().sp_hip_sqfree_read_layer(cc.ref, 1, start, n, p(ko), p(vo), stride, S.DTYPE_F32))
    ms = cc.c.max_seq_len
    for name, x16, cache, out in (("K", k16, cc.c.d_k_cache, ko), ("V", v16, cc.c.d_v_cache, vo)):
        allr = d2h(cache, 2 * H * ms * B).reshape(2 * H, ms, B)
        g = host(out).reshape(n, stride)
        assert np.isnan(g[:, H * hd:]).all(), "row padding written"
        for h in range(H):
            ref = O.sqfree_compress_f16(x16[h].view(np.uint16), hd, km, skel_bc, 3, True)
            rec = O.sqfree_decompress_f32(ref, hd, km, skel_bc, 3, True)
            np.testing.assert_array_equal(allr[H + h, start:start + n], ref, err_msg=f"{name} head {h}")
            assert not allr[h].any(), "layer 0 written"
            np.testing.assert_array_equal(g[:, h * hd:(h + 1) * hd].view(np.uint32), rec.view(np.uint32))
    cc.free()


def test_hier_layer_wide():
    """sp_hip_hier_write_layer / read_layer at the configs[4] geometry: both heads of
    layer 1 (slots 2, 3, each with its own W) in one launch from cache rows, 200
    tokens from position 4; bit-exact against the oracle per head."""
    say("hier layer-wide")
    hd, H, n, start, pad_row, rbits = 256, 2, 200, 4, 16, 2
    k16, v16 = W.cfg5_kv(n_heads=H, n_pos=n, hd=hd, seed=41)
    pad = O.sqfree_pad_dim(hd)
    skel_idx, tgt_idx = O.hier_geometry(pad)
    skel_bc = O.band_config(len(skel_idx), [5, 5])
    Wm = W.hier_W(2 * H, len(tgt_idx), len(skel_idx), seed=42)
    cfg = S.config(hd, 2, H)
    ms = start + n + 4
    hc = S.HierCache(cfg, pad, skel_idx, tgt_idx, S.band_config(len(skel_idx), [5, 5]), rbits, ms, 2 * H,
                     stream=torch.cuda.current_stream().cuda_stream)
    hc.upload_W(Wm)
    B = hc.c.bytes_per_pos_k
    stride = H * hd + pad_row
    kt, vt = dev(_rows(k16, pad_row)), dev(_rows(v16, pad_row))
    S.check(S.lib().sp_hip_hier_write_layer(hc.ref, 1, start, n, p(kt), p(vt), stride, S.DTYPE_F16))
    ko = torch.full((n * stride,), float("nan"), dtype=torch.float32, device="cuda")
    vo = torch.full((n * stride,), float("nan"), dtype=torch.float32, device="cuda")
    S.check(S.lib().sp_hip_hier_read_layer(hc.ref, 1, start, n, p(ko), p(vo), stride, S.DTYPE_F32))
    for name, x16, cache, out in (("K", k16, hc.c.d_k_cache, ko), ("V", v16, hc.c.d_v_cache, vo)):
        allr = d2h(cache, 2 * H * ms * B).reshape(2 * H, ms, B)
        g = host(out).reshape(n, stride)
        assert np.isnan(g[:, H * hd:]).all(), "row padding written"
        for h in range(H):
            slot = H + h
            ref = O.hier_compress_f16(x16[h].view(np.uint16), hd, pad, skel_idx, tgt_idx, skel_bc, Wm[slot], rbits)
            rec = O.hier_decompress_f32(ref, hd, pad, skel_idx, tgt_idx, skel_bc, Wm[slot], rbits)
            np.testing.assert_array_equal(allr[slot, start:start + n], ref, err_msg=f"{name} head {h}")
            np.testing.assert_array_equal(g[:, h * hd:(h + 1) * hd].view(np.uint32), rec.view(np.uint32))
    hc.free()


def test_hier_record_size_cfg5():
    pad = O.sqfree_pad_dim(256)
    skel_idx, tgt_idx = O.hier_geometry(pad)
    assert (pad, len(skel_idx), len(tgt_idx)) == (330, 30, 300)
    assert O.hier_bytes(O.band_config(30, [5, 5]), 300, 2) == 103


# The benched calls run every block of the persistent (decode) or resident (encode)
# grid over many 64-vector tiles, with the next tile's rows or records prefetched
# across tiles. SP_HIP_MAX_BLOCKS caps the grid so that inputs small enough for the
# CPU oracle take the same multi-tile path: 3 blocks over 4 heads x 900 tokens
# (60 tiles per side) is 20 tiles per block, the last tile of each head partial.
@pytest.mark.parametrize("sk_frac,v_bits", [(0.75, [5, 4, 4, 4, 5]), (0.75, [3]), (0.0, [5, 4, 4, 4, 5])])
def test_sqfree_multi_tile_blocks(sk_frac, v_bits, monkeypatch):
    """configs[3]'s codec (pad 154, skeleton 115 or 77, 3-bit residual, spinor;
    K 5/4/4/4/5, V 5/4/4/4/5 as the reference hook mirrors K, or V one 3-bit band
    as configs[3] asks) through the layer-wide write/read with every block walking
    ~20 tiles: records and fp32 reconstructions bit-exact against the oracle."""
    monkeypatch.setenv("SP_HIP_MAX_BLOCKS", "3")
    say(f"sqfree multi-tile sk_frac={sk_frac} v_bits={v_bits}")
    hd, H, n, start = 128, 4, 900, 5
    k16, v16 = W.cfg4_kv(n_heads=H, n_pos=n, hd=hd, seed=57)
    pad = O.sqfree_pad_dim(hd)
    sk = int(pad * sk_frac) if sk_frac else pad // 2
    km = O.Knight(pad, sk)
    k_bits = [5, 4, 4, 4, 5]
    kbc, vbc = O.band_config(sk, k_bits), O.band_config(sk, v_bits)
    cfg = S.config(hd, 1, H, k_bits=k_bits, v_bits=v_bits)
    cc = S.SqfreeCache(cfg, start + n + 2, rbits=3, spinor=True, sk_k=sk,
                       stream=torch.cuda.current_stream().cuda_stream)
    Bk, Bv = cc.c.bytes_per_pos_k, cc.c.bytes_per_pos_v
    if sk == 115:
        assert (Bk, Bv) == (100, 100 if len(v_bits) == 5 else 70)
    stride = H * hd
    kt, vt = dev(_rows(k16, 0)), dev(_rows(v16, 0))
    S.check(S.lib().sp_hip_sqfree_write_layer(cc.ref, 0, start, n, p(kt), p(vt), stride, S.DTYPE_F16))
    ko, vo = empty_f32(n * stride), empty_f32(n * stride)
    S.check(S.lib().sp_hip_sqfree_read_layer(cc.ref, 0, start, n, p(ko), p(vo), stride, S.DTYPE_F32))
    ms = cc.c.max_seq_len
    for name, x16, cache, B, bc, out in (("K", k16, cc.c.d_k_cache, Bk, kbc, ko), ("V", v16, cc.c.d_v_cache, Bv, vbc, vo)):
        allr = d2h(cache, H * ms * B).reshape(H, ms, B)
        g = host(out).reshape(n, stride)
        for h in range(H):
            ref = O.sqfree_compress_f16(x16[h].view(np.uint16), hd, km, bc, 3, True)
            rec = O.sqfree_decompress_f32(ref, hd, km, bc, 3, True)
            np.testing.assert_array_equal(allr[h, start:start + n], ref, err_msg=f"{name} head {h}")
            assert not allr[h, :start].any() and not allr[h, start + n:].any(), "writes outside the tokens"
            np.testing.assert_array_equal(g[:, h * hd:(h + 1) * hd].view(np.uint32), rec.view(np.uint32),
                                          err_msg=f"{name} head {h}")
    cc.free()


@pytest.mark.parametrize("sides", ["k_only", "k_and_v"])
def test_hier_multi_tile_blocks(sides, monkeypatch):
    """configs[4]'s hier codec (pad 330, 30 skeleton at 5/5, 300 targets at 2 bits)
    with the grid capped at 3 blocks: the one-sided encode (2 heads x 1000 tokens,
    32 tiles) and the two-sided K+V launch of a prefill chunk (64 tiles), then the
    decode, each block walking 10-22 tiles with the cross-tile prefetch; records and
    reconstructions bit-exact against the oracle."""
    monkeypatch.setenv("SP_HIP_MAX_BLOCKS", "3")
    say(f"hier multi-tile {sides}")
    hd, H, n, start, rbits = 256, 2, 1000, 3, 2
    k16, v16 = W.cfg5_kv(n_heads=H, n_pos=n, hd=hd, seed=61)
    pad = O.sqfree_pad_dim(hd)
    skel_idx, tgt_idx = O.hier_geometry(pad)
    skel_bc = O.band_config(len(skel_idx), [5, 5])
    Wm = W.hier_W(H, len(tgt_idx), len(skel_idx), seed=62)
    ms = start + n + 1
    hc = S.HierCache(S.config(hd, 1, H), pad, skel_idx, tgt_idx, S.band_config(len(skel_idx), [5, 5]), rbits, ms, H,
                     stream=torch.cuda.current_stream().cuda_stream)
    hc.upload_W(Wm)
    B = hc.c.bytes_per_pos_k
    stride = H * hd
    kt, vt = dev(_rows(k16, 0)), dev(_rows(v16, 0))
    S.check(S.lib().sp_hip_hier_write_layer(hc.ref, 0, start, n, p(kt), p(vt) if sides == "k_and_v" else None,
                                            stride, S.DTYPE_F16))
    ko, vo = empty_f32(n * stride), empty_f32(n * stride)
    S.check(S.lib().sp_hip_hier_read_layer(hc.ref, 0, start, n, p(ko), p(vo) if sides == "k_and_v" else None,
                                           stride, S.DTYPE_F32))
    checks = [("K", k16, hc.c.d_k_cache, ko)]
    if sides == "k_and_v":
        checks.append(("V", v16, hc.c.d_v_cache, vo))
    for name, x16, cache, out in checks:
        allr = d2h(cache, H * ms * B).reshape(H, ms, B)
        g = host(out).reshape(n, stride)
        for h in range(H):
            ref = O.hier_compress_f16(x16[h].view(np.uint16), hd, pad, skel_idx, tgt_idx, skel_bc, Wm[h], rbits)
            rec = O.hier_decompress_f32(ref, hd, pad, skel_idx, tgt_idx, skel_bc, Wm[h], rbits)
            np.testing.assert_array_equal(allr[h, start:start + n], ref, err_msg=f"{name} head {h}")
            np.testing.assert_array_equal(g[:, h * hd:(h + 1) * hd].view(np.uint32), rec.view(np.uint32),
                                          err_msg=f"{name} head {h}")
    if sides == "k_only":
        assert not d2h(hc.c.d_v_cache, H * ms * B).any(), "V written by a K-only call"
    hc.free()
