"""Pins the CPU oracle's ship codec against closed forms, invariants, brute force and
the reference's own logged figures (CPU only)."""
import math

import numpy as np
import pytest

import oracle_py as O
import workloads as W


def hadamard(n):
    H = np.array([[1.0]])
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H


# ---------------------------------------------------------------- VHT2 p=2

@pytest.mark.parametrize("n", [2, 4, 8, 16, 32, 64, 128, 256, 512])
@pytest.mark.parametrize("norm", [O.NORM_FINAL, O.NORM_STAGE])
def test_vht2_matches_sylvester_closed_form(n, norm):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((4, n)).astype(np.float32)
    y = np.stack([O.vht2(r, norm) for r in x])
    ref = x.astype(np.float64) @ hadamard(n).T / math.sqrt(n)
    np.testing.assert_allclose(y, ref, rtol=0, atol=2e-6 * math.sqrt(n) * np.abs(x).max())


def test_vht2_closed_form_catches_transposed_stage_order():
    # natural-order Sylvester: row 1 of H_n alternates +-; a bit-reversed
    # (sequency) ordering would put it elsewhere
    e1 = np.zeros(8, np.float32)
    e1[1] = 1.0
    y = O.vht2(e1)
    np.testing.assert_allclose(y * math.sqrt(8), [1, -1, 1, -1, 1, -1, 1, -1], atol=1e-6)


@pytest.mark.parametrize("n", [64, 128, 256])
def test_vht2_self_inverse_and_parseval(n):
    rng = np.random.default_rng(7)
    x = rng.standard_normal(n).astype(np.float32)
    y = O.vht2(x)
    assert abs(np.dot(y, y) - np.dot(x, x)) < 1e-4 * np.dot(x, x)
    np.testing.assert_allclose(O.vht2(y), x, atol=1e-5)


def test_vht2_final_norm_constant():
    # NEON path multiplies by 1.0f/sqrtf(n) computed in float
    assert np.float32(O.lib().spo_inv_sqrt_n(128)) == np.float32(1.0) / np.sqrt(np.float32(128))


# ---------------------------------------------------------------- Vilenkin

def cas_matrix(p):
    k = np.arange(p)
    a = 2 * np.pi * np.outer(k, k) / p
    return (np.cos(a) + np.sin(a)) / math.sqrt(p)


def vilenkin_dense(n):
    """Kronecker product of normalised cas blocks; first (smallest) prime acts on
    the fastest-varying index."""
    f = []
    d = n
    for p in (2, 3, 5, 7, 11):
        while d % p == 0:
            f.append(p)
            d //= p
    assert d == 1
    M = np.array([[1.0]])
    for p in f:
        M = np.kron(cas_matrix(p), M)
    return M


@pytest.mark.parametrize("n", [6, 12, 30, 66, 96, 105, 154, 330])
def test_vilenkin_matches_kronecker_closed_form(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    y = O.vht2(x)
    ref = vilenkin_dense(n) @ x.astype(np.float64)
    np.testing.assert_allclose(y, ref, atol=2e-5 * np.abs(x).max() * math.sqrt(n))
    np.testing.assert_allclose(O.vht2(y), x, atol=5e-5)


# ---------------------------------------------------------------- band geometry

@pytest.mark.parametrize("hd,bits,expect", [
    (128, [5, 5, 4, 3], 76),
    (128, [3], 50),
    (64, [5, 5, 4, 3], 42),     # shannon_prime_llama.h:337-338
    (96, [5, 4, 4], 58),
    (96, [5], 62),
    (77, [5, 4, 4, 4, 5], 55),  # sqfree skeleton at pad 154
])
def test_record_sizes(hd, bits, expect):
    assert O.band_config(hd, bits).total_bytes == expect


@pytest.mark.parametrize("hd,kbits,vbits,ratio", [
    (64, [5, 5, 4, 3], [3], 3.8),   # ppl_logs/dolphin1b-q8-vht2-5543-32chunks.log
    (64, [5, 4, 4], [5], 3.0),      # ppl_logs/vht2_32_postdec_v5.log
    (64, [8, 8, 8, 8], [8], 1.9),   # ppl_logs/dolphin1b-q8-vht2-8888-8chunks.log
    (128, [5, 5, 4, 3], [3], 4.1),  # android_build/test_adreno_phone.log
])
def test_logged_compression_ratios(hd, kbits, vbits, ratio):
    k = O.band_config(hd, kbits).total_bytes
    v = O.band_config(hd, vbits).total_bytes
    assert round(4 * hd / (k + v), 1) == ratio


def test_last_band_absorbs_remainder():
    bc = O.band_config(128, [5] * 10)
    assert bc.band_size == 12
    assert [bc.band_sz[b] for b in range(10)] == [12] * 9 + [20]


def test_ternary_band_is_two_bits():
    bc = O.band_config(128, [5, 5, 4, 3], ternary_mask=1 << 3)
    assert bc.band_bits[3] == 2
    assert bc.total_bytes == 22 + 22 + 18 + 2 + 8


# ---------------------------------------------------------------- fp16

def test_f16_conversion_matches_numpy_rne():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.9, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
                  1.5 * 2.0 ** -25, 2.0 ** -14, 6.1e-5, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11,
                  np.inf, -np.inf], np.float32)])
    got = np.array([O.f32_to_f16_bits(float(v)) for v in vals], dtype=np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, ref)
    back = np.array([O.lib().spo_f16_to_f32(int(h)) for h in ref], np.float32)
    np.testing.assert_array_equal(back, ref.view(np.float16).astype(np.float32))


# ---------------------------------------------------------------- quantizer

def unpack_band_codes(packed, bc):
    """Independent bit-string unpacking of a record: returns [(scale_f16_bits, codes)]."""
    out = []
    for b in range(bc.n_bands):
        off = bc.band_byte_off[b]
        sz, bits = bc.band_sz[b], bc.band_bits[b]
        h = int(packed[off]) | (int(packed[off + 1]) << 8)
        nbytes = (sz * bits + 7) // 8
        bitstr = "".join(format(int(x), "08b")[::-1] for x in packed[off + 2: off + 2 + nbytes])
        codes = [int(bitstr[i * bits:(i + 1) * bits][::-1], 2) for i in range(sz)]
        out.append((h, codes))
    return out


def test_quantizer_brute_force_nearest_code():
    rng = np.random.default_rng(11)
    bc = O.band_config(128, [5, 5, 4, 3])
    for _ in range(50):
        x = (rng.standard_normal(128) * rng.uniform(0.01, 20)).astype(np.float32)
        packed = O.band_quantize(x, bc)
        for b, (h, codes) in enumerate(unpack_band_codes(packed, bc)):
            off, sz, bits = bc.band_off[b], bc.band_sz[b], bc.band_bits[b]
            m = (1 << (bits - 1)) - 1
            xb = x[off:off + sz].astype(np.float64)
            amax = np.abs(xb).max()
            scale = np.float32(np.float32(amax) / np.float32(m))
            assert h == np.float16(scale).view(np.uint16)
            s16 = float(np.float16(scale))
            inv = np.float32(1.0) / np.float32(s16)
            for xi, u in zip(xb, codes):
                q = u - m
                # nearest integer to x*inv (ties to even), clamped
                t = float(np.float32(np.float32(xi) * inv))
                cands = range(-m, m + 1)
                best = min(cands, key=lambda c: (abs(c - t), c % 2))
                assert q == best


def test_quantizer_ties_round_half_even():
    """x*inv exactly on a half-integer: __float2int_rn (shannon_prime_cuda.cu:186)
    rounds half to even. A power-of-two scale makes inv exact, so the products are
    the chosen half-integers themselves."""
    for bits in (5, 4, 3, 2):
        m = (1 << (bits - 1)) - 1
        bc = O.band_config(8, [bits])
        s = np.float32(0.25)
        halves = [k + 0.5 for k in range(-m, m)]
        for i in range(0, len(halves), 7):
            chunk = halves[i:i + 7]
            x = np.array([m] + chunk + [0.0] * (7 - len(chunk)), np.float64) * float(s)
            (h, codes), = unpack_band_codes(O.band_quantize(x.astype(np.float32), bc), bc)
            assert h == np.float16(s).view(np.uint16)
            for t, u in zip(chunk, codes[1:]):
                assert u - m == int(np.rint(t)), (bits, t, u - m)
                assert (u - m) % 2 == 0


def test_quantizer_special_cases():
    bc = O.band_config(128, [5, 5, 4, 3])
    z = np.zeros(128, np.float32)
    packed = O.band_quantize(z, bc)
    for b, (h, codes) in enumerate(unpack_band_codes(packed, bc)):
        m = (1 << (bc.band_bits[b] - 1)) - 1
        assert h == 0 and all(c == m for c in codes)
    # element at amax maps to exactly +-max_val
    x = np.linspace(-1, 1, 128).astype(np.float32)
    x[5] = 7.0
    x[40] = -3.0
    codes = unpack_band_codes(O.band_quantize(x, bc), bc)
    assert codes[0][1][5] == 30 and codes[1][1][40 - 32] == 0
    # fp16 scale overflow -> dequantized band is all zero (non-finite guard)
    y = np.ones(128, np.float32)
    y[0] = 1e7
    rec = O.band_dequantize(O.band_quantize(y, bc), bc)
    assert np.all(rec[:32] == 0) and np.all(np.abs(rec[32:]) > 0)


def test_packing_known_answer():
    # one band of 8 values at 3 bits: codes 0..6 -> LSB-first stream
    bc = O.band_config(8, [3])
    x = np.array([-3, -2, -1, 0, 1, 2, 3, 3], np.float32)
    p = O.band_quantize(x, bc)
    assert p.tolist() == [0x00, 0x3c] + [0x88, 0xc6, 0xda]


def test_partial_dequant_semantics():
    bc = O.band_config(128, [5, 5, 4, 3])
    x = np.random.default_rng(3).standard_normal(128).astype(np.float32)
    p = O.band_quantize(x, bc)
    full = O.band_dequantize(p, bc)
    np.testing.assert_array_equal(O.band_dequantize(p, bc, max_bands=-1), full)
    np.testing.assert_array_equal(O.band_dequantize(p, bc, max_bands=4), full)
    assert np.all(O.band_dequantize(p, bc, max_bands=0) == 0)
    two = O.band_dequantize(p, bc, max_bands=2)
    np.testing.assert_array_equal(two[:64], full[:64])
    assert np.all(two[64:] == 0)


# ---------------------------------------------------------------- Mobius

def test_mobius_order_is_squarefree_first_permutation():
    o = O.mobius_order(128)
    assert sorted(o.tolist()) == list(range(128))
    sf = [i for i in range(128) if all((i + 1) % (p * p) for p in range(2, 12))]
    assert o[:len(sf)].tolist() == sf


# ---------------------------------------------------------------- fidelity (test_adreno log)

def test_ship_fidelity_thresholds_cfg1():
    k16, v16 = W.cfg1_kv(n_heads=2, n_pos=256)
    order = O.mobius_order(128)
    kbc, vbc = O.band_config(128, [5, 5, 4, 3]), O.band_config(128, [3])
    k = k16.reshape(-1, 128)
    v = v16.reshape(-1, 128)
    kr = O.ship_decompress_f32(O.ship_compress_f16(k.view(np.uint16), kbc, order), kbc, order)
    vr = O.ship_decompress_f32(O.ship_compress_f16(v.view(np.uint16), vbc), vbc)
    kc = np.mean([O.correlation(a, b) for a, b in zip(k.astype(np.float32), kr)])
    vc = np.mean([O.correlation(a, b) for a, b in zip(v.astype(np.float32), vr)])
    # android_build/test_adreno_phone.log: K > 0.985, V > 0.95 at hd=128
    assert kc > 0.985 and vc > 0.95, (kc, vc)


def test_f16_and_f32_entry_points_agree():
    k16, _ = W.cfg1_kv(n_heads=1, n_pos=64)
    k = k16.reshape(-1, 128)
    bc = O.band_config(128, [5, 5, 4, 3])
    o = O.mobius_order(128)
    np.testing.assert_array_equal(O.ship_compress_f16(k.view(np.uint16), bc, o),
                                  O.ship_compress_f32(k.astype(np.float32), bc, o))


def test_tree256_sum_exact_on_integers():
    rng = np.random.default_rng(5)
    for n in (1, 77, 128, 256, 300, 777):
        v = rng.integers(-1000, 1000, n).astype(np.float32)
        assert O.tree256_sum(v) == float(v.sum(dtype=np.int64))
        assert O.tree256_sum(v, take_abs=True) == float(np.abs(v).sum(dtype=np.int64))


def test_attention_oracle_matches_dense_softmax():
    k16, v16 = W.cfg2_kv(n_heads=2, n_pos=64)
    q = W.cfg2_q(n_q=4, pos=64)
    kbc, vbc = O.band_config(128, [5, 5, 4, 3]), O.band_config(128, [3])
    order = O.mobius_order(128)
    kp = np.stack([O.ship_compress_f16(k16[h].view(np.uint16), kbc, order) for h in range(2)])
    vp = np.stack([O.ship_compress_f16(v16[h].view(np.uint16), vbc) for h in range(2)])
    scale = 1 / math.sqrt(128)
    s, out = O.attn_decode(q, kp, vp, 2, 64, kbc, vbc, order, scale)
    kr = np.stack([O.ship_decompress_f32(kp[h], kbc, order) for h in range(2)]).astype(np.float64)
    vr = np.stack([O.ship_decompress_f32(vp[h], vbc) for h in range(2)]).astype(np.float64)
    for h in range(4):
        ref_s = kr[h // 2] @ q[h].astype(np.float64) * scale
        np.testing.assert_allclose(s[h], ref_s, rtol=1e-5, atol=1e-5)
        p = np.exp(ref_s - ref_s.max())
        p /= p.sum()
        np.testing.assert_allclose(out[h], p @ vr[h // 2], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("mb", [0, 1, 2, 3])
def test_band_limited_attention_oracle_matches_dense_softmax(mb):
    """Band-limited attention equals a dense softmax over the partial
    reconstructions (K and V bands >= mb read as 0); every band is the full one."""
    k16, v16 = W.cfg2_kv(n_heads=2, n_pos=48, seed=mb + 7)
    q = W.cfg2_q(n_q=4, pos=48, seed=mb + 8)
    kbc, vbc = O.band_config(128, [5, 5, 4, 3]), O.band_config(128, [3])
    order = O.mobius_order(128)
    kp = np.stack([O.ship_compress_f16(k16[h].view(np.uint16), kbc, order) for h in range(2)])
    vp = np.stack([O.ship_compress_f16(v16[h].view(np.uint16), vbc) for h in range(2)])
    scale = 1 / math.sqrt(128)
    s, out = O.attn_decode(q, kp, vp, 2, 48, kbc, vbc, order, scale, max_bands=mb)
    kr = np.stack([O.ship_decompress_f32(kp[h], kbc, order, max_bands=mb) for h in range(2)]).astype(np.float64)
    vr = np.stack([O.ship_decompress_f32(vp[h], vbc, max_bands=mb) for h in range(2)]).astype(np.float64)
    if mb == 0:
        assert not kr.any() and not vr.any()
    for h in range(4):
        ref_s = kr[h // 2] @ q[h].astype(np.float64) * scale
        np.testing.assert_allclose(s[h], ref_s, rtol=1e-5, atol=1e-5)
        p = np.exp(ref_s - ref_s.max())
        p /= p.sum()
        np.testing.assert_allclose(out[h], p @ vr[h // 2], rtol=1e-5, atol=1e-6)
    s4, o4 = O.attn_decode(q, kp, vp, 2, 48, kbc, vbc, order, scale, max_bands=4)
    s_all, o_all = O.attn_decode(q, kp, vp, 2, 48, kbc, vbc, order, scale)
    np.testing.assert_array_equal(s4, s_all)
    np.testing.assert_array_equal(o4, o_all)


def test_attention_oracle_takes_position_slices():
    """A sequence's range of a longer cache (a non-contiguous [H][start:start+n] slice)
    gives the same scores and output as the same records copied contiguously."""
    k16, v16 = W.cfg2_kv(n_heads=2, n_pos=200, seed=21)
    q = W.cfg2_q(n_q=4, pos=90, seed=22)
    kbc, vbc = O.band_config(128, [5, 5, 4, 3]), O.band_config(128, [3])
    order = O.mobius_order(128)
    kp = np.stack([O.ship_compress_f16(k16[h].view(np.uint16), kbc, order) for h in range(2)])
    vp = np.stack([O.ship_compress_f16(v16[h].view(np.uint16), vbc) for h in range(2)])
    scale = 1 / math.sqrt(128)
    for _ in range(3):  # allocations between calls would reuse a freed copy's memory
        s, out = O.attn_decode(q, kp[:, 70:160], vp[:, 70:160], 2, 90, kbc, vbc, order, scale)
        junk = [np.full(kp[:, 70:160].size, 255, np.uint8) for _ in range(4)]
        s2, o2 = O.attn_decode(q, kp[:, 70:160].copy(), vp[:, 70:160].copy(), 2, 90, kbc, vbc, order, scale)
        np.testing.assert_array_equal(s, s2)
        np.testing.assert_array_equal(out, o2)
        del junk
