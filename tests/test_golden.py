"""The CPU oracle against the committed golden fixtures (tests/golden/*.npz,
written by tests/golden/make_fixtures.py): seeded inputs for configs 0-4 at
reduced sizes and the outputs the oracle gave for them. Codes and
reconstructions must match bit for bit, attention exactly (the oracle's
attention is deterministic float64 arithmetic), so any change to the oracle's
arithmetic shows here before it reaches the GPU parity tests."""
import math
import os

import numpy as np
import pytest

import oracle_py as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name))


@pytest.mark.parametrize("name", ["cfg0_ship_hd128.npz", "cfg2_ship_hd96.npz"])
def test_ship_fixture(name):
    f = load(name)
    hd = int(f["hd"])
    kbc, vbc = O.band_config(hd, list(f["k_bits"])), O.band_config(hd, list(f["v_bits"]))
    order = O.mobius_order(hd)
    np.testing.assert_array_equal(order, f["order"])
    kc = O.ship_compress_f16(f["k_in"], kbc, order)
    vc = O.ship_compress_f16(f["v_in"], vbc)
    np.testing.assert_array_equal(kc, f["k_codes"])
    np.testing.assert_array_equal(vc, f["v_codes"])
    np.testing.assert_array_equal(O.ship_decompress_f16(kc, kbc, order), f["k_rec16"])
    np.testing.assert_array_equal(O.ship_decompress_f16(vc, vbc), f["v_rec16"])
    np.testing.assert_array_equal(O.ship_decompress_f32(kc, kbc, order).view(np.uint32), f["k_rec32"].view(np.uint32))
    np.testing.assert_array_equal(O.ship_decompress_f32(vc, vbc).view(np.uint32), f["v_rec32"].view(np.uint32))
    np.testing.assert_array_equal(O.ship_decompress_f32(kc, kbc, order, max_bands=2).view(np.uint32),
                                  f["k_rec32_2bands"].view(np.uint32))


def test_attention_fixture():
    f = load("cfg1_attention_hd128.npz")
    hd, H = int(f["hd"]), int(f["n_kvh"])
    n_ctx = f["k_codes"].shape[1]
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    s, o = O.attn_decode(f["q"], f["k_codes"], f["v_codes"], H, n_ctx, kbc, vbc, O.mobius_order(hd),
                         float(f["kq_scale"]))
    assert float(f["kq_scale"]) == np.float32(1.0 / math.sqrt(hd))
    np.testing.assert_array_equal(s, f["scores"])
    np.testing.assert_array_equal(o, f["out"])


def test_sqfree_fixture():
    f = load("cfg3_sqfree_hd128.npz")
    hd, pad, sk = int(f["hd"]), int(f["pad"]), int(f["sk_k"])
    assert pad == O.sqfree_pad_dim(hd) and (pad, sk) == (154, 115)
    km = O.Knight(pad, sk)
    bc = O.band_config(sk, list(f["bits"]))
    codes = O.sqfree_compress_f16(f["x_in"], hd, km, bc, int(f["rbits"]), bool(f["spinor"]))
    np.testing.assert_array_equal(codes, f["codes"])
    rec = O.sqfree_decompress_f32(codes, hd, km, bc, int(f["rbits"]), bool(f["spinor"]))
    np.testing.assert_array_equal(rec.view(np.uint32), f["rec32"].view(np.uint32))


def test_hier_fixture():
    f = load("cfg4_hier_hd256.npz")
    hd, pad, rb = int(f["hd"]), int(f["pad"]), int(f["rbits"])
    sk, tg = f["skel_idx"], f["tgt_idx"]
    osk, otg = O.hier_geometry(pad)
    np.testing.assert_array_equal(sk, osk)
    np.testing.assert_array_equal(tg, otg)
    bc = O.band_config(len(sk), list(f["skel_bits"]))
    Wm = f["W"]
    codes = O.hier_compress_f16(f["x_in"], hd, pad, sk, tg, bc, Wm[0], rb)
    np.testing.assert_array_equal(codes, f["codes"])
    rec = O.hier_decompress_f32(codes, hd, pad, sk, tg, bc, Wm[0], rb)
    np.testing.assert_array_equal(rec.view(np.uint32), f["rec32"].view(np.uint32))
    n_ctx = f["k_codes"].shape[1]
    s, o = O.hier_attn_decode(f["q"], f["k_codes"], f["v_codes"], 2, n_ctx, hd, pad, sk, tg, bc, Wm, rb,
                              float(f["kq_scale"]))
    np.testing.assert_array_equal(s, f["scores"])
    np.testing.assert_array_equal(o, f["out"])
