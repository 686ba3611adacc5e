"""Pins of the oracle's sqfree+spinor and hierarchical functions (CPU).

Each stage of oracle/sp_oracle.c is compared with an independent numpy
restatement written from the reference's CUDA text (tests/np_restate.py), on
inputs chosen so that the plausible misreadings give different answers:
round-half-up truncation vs rint in the residual quantizers
(shannon_prime_sqfree.cu:526, shannon_prime_hier.cu:166), sat = mag*bits vs
mag (:520-522), the 1e-12 floor, the strict spinor comparison (:231), the
serial W.skel sum (shannon_prime_hier.cu:84-89), the 256-slot reduction order
of the pad mean and the residual magnitude, and the Knight CSR (mu(n/d) by
brute force). Whole records are then compared byte for byte."""
import math

import numpy as np
import pytest

import np_restate as R
import oracle_py as O

F32 = np.float32


# ---- Mobius function and the Knight CSR ----------------------------------------

def test_mobius_mu_known_values_and_mertens():
    known = [1, -1, -1, 0, -1, 1, -1, 0, 0, 1, -1, 0, -1, 1, 1, 0, -1, 0, -1, 0, 1, 1, -1, 0, 0, 1, 0, 0, -1, -1]
    assert [O.lib().spo_mobius_mu(n) for n in range(1, 31)] == known
    assert [R.mobius_mu(n) for n in range(1, 31)] == known
    # Mertens function M(n) = sum_{k<=n} mu(k): M(10) = -1, M(100) = 1, M(1000) = 2
    for n, m in ((10, -1), (100, 1), (1000, 2)):
        assert sum(O.lib().spo_mobius_mu(k) for k in range(1, n + 1)) == m


@pytest.mark.parametrize("pad,sk", [(66, 33), (105, 52), (154, 77), (154, 115), (330, 165), (330, 30)])
def test_knight_csr_equals_brute_force(pad, sk):
    km = O.Knight(pad, sk)
    skel, res, offs, slots, signs = R.knight_tables(pad, sk)
    assert km.skeleton_idx.tolist() == list(skel)
    assert km.residual_idx.tolist() == list(res)
    assert km.csr_offsets.tolist() == list(offs)
    assert km.csr_skel_slot.tolist() == list(slots)
    assert km.csr_mu_sign.tolist() == list(signs)


def test_mobius_predict_csr_sum():
    km = O.Knight(154, 77)
    rng = np.random.default_rng(5)
    skel = rng.standard_normal(77).astype(F32) * 10
    _, _, offs, slots, signs = R.knight_tables(154, 77)
    np.testing.assert_array_equal(O.mobius_predict(skel, km).view(np.uint32),
                                  R.mobius_predict(skel, offs, slots, signs).view(np.uint32))


# ---- pad mean ------------------------------------------------------------------------

def test_pad_mean_reduction_order():
    """The mean is summed in the 256-slot order: slot t = x[t] (hd <= 256),
    then slot[t] += slot[t + s] for s = 128 .. 1. With 1e8 at 0, -1e8 at 64 and
    1 at 1 the tree cancels the big pair first (sum 1); a left-to-right sum
    loses the 1 (sum 0)."""
    hd = 128
    x = np.zeros(hd, F32)
    x[0], x[64], x[1] = 1e8, -1e8, 1.0
    seq = F32(0)
    for v in x:
        seq = seq + v
    assert seq == 0.0 and R.tree256_sum(x) == 1.0
    want = F32(1.0) / F32(hd)
    assert O.tree256_sum(x) == 1.0
    np.testing.assert_array_equal(O.sqfree_pad(x, hd, 154)[hd:], np.full(154 - hd, want, F32))
    rng = np.random.default_rng(6)
    for hd, pad in ((64, 66), (96, 105), (128, 154), (256, 330)):
        x = rng.standard_normal(hd).astype(F32) * 5
        np.testing.assert_array_equal(O.sqfree_pad(x, hd, pad).view(np.uint32),
                                      R.sqfree_pad(x, hd, pad).view(np.uint32))
        assert abs(float(O.sqfree_pad(x, hd, pad)[-1]) - float(np.mean(x.astype(np.float64)))) < 1e-6


# ---- sqfree residual quantizer ----------------------------------------------------------

@pytest.mark.parametrize("bits,dev,want", [
    (1, [0.0, 1.0, 0.0, 1.0], [1, 1, 1, 1]),   # mag 0.5, step 1: dev 0 -> qf 0.5 -> (int)1.0 = 1 (rint: 0)
    (2, [0.5, 1.0, 0.5, 1.0], [2, 3, 2, 3]),   # mag 0.75, step 1: dev 1 -> qf 2.5 -> (int)3.0 = 3 (rint: 2)
])
def test_sqfree_quantizer_rounds_half_up(bits, dev, want):
    mag, lv = O.sqfree_residual_quantize(dev, bits)
    rmag, rlv = R.sqfree_residual_quantize(dev, bits)
    assert lv.tolist() == want == rlv
    assert mag == rmag
    # the misreading rint(qf) gives a different answer on these inputs
    assert R.sqfree_residual_quantize(dev, bits, round_half_up=False)[1] != want


def test_sqfree_quantizer_saturation_and_floor():
    rng = np.random.default_rng(7)
    for bits in (2, 3, 4):
        for _ in range(20):
            dev = (rng.standard_t(4, 77) * rng.uniform(0.01, 3)).astype(F32)
            mag, lv = O.sqfree_residual_quantize(dev, bits)
            rmag, rlv = R.sqfree_residual_quantize(dev, bits)
            assert mag == rmag and lv.tolist() == rlv
        # sat = mag*bits, not mag: random residuals tell them apart
        assert R.sqfree_residual_quantize(dev, bits, sat_times_bits=False)[1] != rlv
    # all-zero residual: mag is the 1e-12 floor, every level the centre rounded up
    mag, lv = O.sqfree_residual_quantize(np.zeros(40, F32), 3)
    assert mag == F32(1e-12) and set(lv.tolist()) == {4}
    # below the floor the encoder's sat is 1e-12 itself (not mag*bits): +-5e-13
    # quantizes to levels 5 / 2 (with sat = 3e-12 they would be 4 / 3)
    dev = np.array([5e-13, -5e-13] * 8, F32)
    mag, lv = O.sqfree_residual_quantize(dev, 3)
    assert mag == F32(1e-12) and lv.tolist() == [5, 2] * 8 == R.sqfree_residual_quantize(dev, 3)[1]


def test_sqfree_dequantizer():
    for bits in (1, 2, 3, 4):
        for mag in (F32(1e-12), F32(0.37), F32(2.5), F32(1234.5)):
            lv = np.arange(1 << bits, dtype=np.uint8)
            np.testing.assert_array_equal(O.sqfree_residual_dequantize(lv, bits, mag).view(np.uint32),
                                          R.sqfree_residual_dequantize(lv, bits, mag).view(np.uint32))
    # closed form at bits 3: step = 2*3*mag/7, levels 0..7 -> (l - 3.5)*step
    got = O.sqfree_residual_dequantize(np.arange(8, dtype=np.uint8), 3, F32(7.0))
    np.testing.assert_array_equal(got, (np.arange(8) - 3.5) * 6.0)


# ---- spinor -----------------------------------------------------------------------------

def test_spinor_strict_comparison():
    """bit = |a + p| < |a - p|: a tie (p = 0, or a = 0) keeps a - p and bit 0."""
    a = np.array([1, 1, -1, 0, 2, 0, 3, -0.25], F32)
    p = np.array([0, 1, 1, 1, -2, 0, 0.5, 0.25], F32)
    dev, sheet = O.spinor_extract(a, p)
    rdev, rsheet, bits = R.spinor_extract(a, p)
    assert bits.tolist() == [False, False, True, False, True, False, False, True]
    assert sheet.tolist() == [0b10010100] == list(rsheet)
    np.testing.assert_array_equal(dev, rdev)
    np.testing.assert_array_equal(dev, np.array([1, 0, 0, -1, 0, 0, 2.5, 0], F32))


def test_level_packing_lsb_first():
    lv = np.array([5, 2, 7, 1, 0, 6, 3], np.uint8)
    got = O.pack_levels(lv, 3)
    assert got.tolist() == list(R.pack_levels(lv, 3))
    # 5 | 2<<3 | 7<<6 | 1<<9 | 0<<12 | 6<<15 | 3<<18 = 0xf03d5
    assert got.tolist() == [0xd5, 0x03, 0x0f]


# ---- hier quantizer and predictor -------------------------------------------------------------

def test_hier_quantizer_rounds_half_even():
    dev = [1.0, 2.0, 1.0, 2.0]  # m 1.5, step 1, centre 1.5: qf 2.5 -> 2 (half even), 3.5 -> 4 -> 3
    mag, lv = O.hier_residual_quantize(dev, 2)
    assert lv.tolist() == [2, 3, 2, 3] == R.hier_residual_quantize(dev, 2)[1]
    assert mag == F32(1.5)
    assert R.hier_residual_quantize(dev, 2, half_even=False)[1] != [2, 3, 2, 3]
    rng = np.random.default_rng(8)
    for bits in (1, 2, 3):
        for _ in range(20):
            dev = (rng.standard_normal(300) * rng.uniform(0.01, 3)).astype(F32)
            mag, lv = O.hier_residual_quantize(dev, bits)
            rmag, rlv = R.hier_residual_quantize(dev, bits)
            assert mag == rmag and lv.tolist() == rlv
        # step = 2m/(L-1) with no bits factor: from 2 bits on the sqfree step
        # (2*m*bits/(L-1)) gives other levels
        if bits >= 2:
            assert R.sqfree_residual_quantize(dev, bits)[1] != rlv
    mag, lv = O.hier_residual_quantize(np.zeros(30, F32), 2)
    assert mag == F32(1e-12) and set(lv.tolist()) == {2}
    for bits in (1, 2, 3):
        lv = np.arange(1 << bits, dtype=np.uint8)
        for m in (F32(1e-12), F32(0.8), F32(3.25)):
            np.testing.assert_array_equal(O.hier_residual_dequantize(lv, bits, m).view(np.uint32),
                                          R.hier_residual_dequantize(lv, bits, m).view(np.uint32))


def test_hier_predict_serial_order():
    """acc += w*s for s ascending from 0.0f: with skel (1, 1e8, -1e8) and unit
    weights the 1 is absorbed (0); the descending order keeps it (1)."""
    W = np.array([[1.0, 1.0, -1.0]], np.float16).view(np.uint16)
    skel = np.array([1.0, 1e8, 1e8], F32)
    got = O.hier_predict(W, skel)
    assert got.tolist() == [0.0] == R.hier_predict(W.view(np.float16), skel).tolist()
    rev = F32(0)
    for s in (2, 1, 0):
        rev = rev + F32(np.float16(W.view(np.float16)[0, s])) * skel[s]
    assert rev == 1.0
    rng = np.random.default_rng(9)
    W = (rng.standard_normal((300, 30)) * 0.3).astype(np.float16)
    skel = (rng.standard_normal(30) * 20).astype(F32)
    np.testing.assert_array_equal(O.hier_predict(W.view(np.uint16), skel).view(np.uint32),
                                  R.hier_predict(W, skel).view(np.uint32))


# ---- whole records ----------------------------------------------------------------------------

def _vectors(n, hd, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, hd)).astype(F32)
    ch = rng.choice(hd, 4, replace=False)
    x[:, ch] *= rng.standard_t(4, (n, 4)).astype(F32) * 4
    return x.astype(np.float16).astype(F32)


@pytest.mark.parametrize("hd,sk,kbits,rbits,spinor", [
    (128, 77, [5, 4, 4, 4, 5], 3, 1),
    (128, 115, [5, 4, 4, 4, 5], 3, 1),
    (128, 77, [5, 4, 4, 4, 5], 3, 0),
    (64, 33, [5, 5, 4, 3], 2, 1),
    (96, 52, [5, 4, 4], 4, 0),
])
def test_sqfree_records_equal_numpy(hd, sk, kbits, rbits, spinor):
    pad = O.sqfree_pad_dim(hd)
    assert pad == R.pad_dim(hd)
    km = O.Knight(pad, sk)
    bc = O.band_config(sk, kbits)
    x = _vectors(12, hd, hd + sk)
    recs = O.sqfree_compress_f16(x.astype(np.float16).view(np.uint16), hd, km, bc, rbits, spinor)
    recon = O.sqfree_decompress_f32(recs, hd, km, bc, rbits, spinor)
    for i in range(len(x)):
        want = R.sqfree_compress(x[i], hd, sk, kbits, rbits, spinor)
        assert bytes(recs[i]) == want, f"record {i}"
        np.testing.assert_array_equal(recon[i].view(np.uint32),
                                      R.sqfree_decompress(want, hd, sk, kbits, rbits, spinor).view(np.uint32))


@pytest.mark.parametrize("hd", [128, 256])
def test_hier_records_equal_numpy(hd):
    pad = O.sqfree_pad_dim(hd)
    si, ti = O.hier_geometry(pad)
    rsi, rti = R.hier_geometry(pad)
    assert si.tolist() == list(rsi) and ti.tolist() == list(rti)
    kbits, rbits = [5, 5], 2
    bc = O.band_config(len(si), kbits)
    rng = np.random.default_rng(hd)
    W = (rng.standard_normal((len(ti), len(si))) * 0.2).astype(np.float16)
    x = _vectors(10, hd, hd + 1)
    recs = O.hier_compress_f16(x.astype(np.float16).view(np.uint16), hd, pad, si, ti, bc, W.view(np.uint16), rbits)
    recon = O.hier_decompress_f32(recs, hd, pad, si, ti, bc, W.view(np.uint16), rbits)
    for i in range(len(x)):
        want = R.hier_compress(x[i], hd, W, kbits, rbits)
        assert bytes(recs[i]) == want, f"record {i}"
        np.testing.assert_array_equal(recon[i].view(np.uint32),
                                      R.hier_decompress(want, hd, W, kbits, rbits).view(np.uint32))
