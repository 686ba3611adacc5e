"""Decode attention over sqfree(+spinor) records in the oracle
(spo_sqfree_attn_decode), pinned two ways on the CPU:

* against its definition: each KV head's K and V records decompressed by the
  (separately pinned) spo_sqfree_decompress, K with the K skeleton bands and V with
  the V bands, then float64 softmax attention with GQA grouping h -> h // (n_q / n_kvh);
* against the coefficient-domain algebra the device kernel uses, restated here in
  float64 numpy from the record layout and the brute-force Knight tables of
  tests/np_restate.py: the length-pad Vilenkin transform V (the Kronecker closed form)
  is symmetric and its own inverse, so with q~ = kq_scale * V(q zero-padded to pad),
  score_t = q~ . c~_t, where c~_t[skeleton] = the dequantized bands and
  c~_t[residual r] = (sheet_r ? -1 : 1) * (M skel_t)_r + (level_r - centre) * step_t
  (M the Knight CSR as a dense +-1 matrix, step = 2 * mag * rbits / (L - 1)), and
  sum_t p_t V~_t = V(sum_t p_t c~_t)[:hd]. A mean-padded q, a sheet sign applied to the
  deviation instead of the prediction, or step = 2 * mag / (L - 1) fails it.
"""
import numpy as np
import pytest

import np_restate as R
import oracle_py as O
import workloads as W
from test_oracle_ship import vilenkin_dense


def _np_attn(q, K, V, kq_scale):
    """float64 softmax attention; K, V [n_kvh][n_ctx][hd]."""
    n_q, n_kvh = q.shape[0], K.shape[0]
    grp = n_q // n_kvh
    s = np.stack([K[h // grp].astype(np.float64) @ q[h].astype(np.float64) for h in range(n_q)]) * kq_scale
    p = np.exp(s - s.max(axis=1, keepdims=True))
    out = np.stack([(p[h] @ V[h // grp].astype(np.float64)) / p[h].sum() for h in range(n_q)])
    return s, out


def _setup(hd, sk_frac, kbits, vbits, rbits, spinor, n_kvh, n_ctx, seed):
    pad = O.sqfree_pad_dim(hd)
    sk = int(pad * sk_frac) if sk_frac else pad // 2
    km = O.Knight(pad, sk)
    kbc, vbc = O.band_config(sk, kbits), O.band_config(sk, vbits)
    k16, v16 = W.cfg4_kv(n_heads=n_kvh, n_pos=n_ctx, hd=hd, seed=seed)
    kp = np.stack([O.sqfree_compress_f16(k16[h].view(np.uint16), hd, km, kbc, rbits, spinor) for h in range(n_kvh)])
    vp = np.stack([O.sqfree_compress_f16(v16[h].view(np.uint16), hd, km, vbc, rbits, spinor) for h in range(n_kvh)])
    return pad, sk, km, kbc, vbc, kp, vp


CASES = [
    # hd, skeleton fraction (0: pad/2), K bits, V bits, residual bits, spinor, n_kvh, n_q, n_ctx
    (128, 0.75, [5, 4, 4, 4, 5], [3], 3, True, 2, 16, 41),            # configs[3]: V one 3-bit band, GQA 8
    (128, 0.75, [5, 4, 4, 4, 5], [5, 4, 4, 4, 5], 3, True, 1, 3, 29),  # V mirrors K (the reference hook)
    (128, 0.0, [5, 4, 4, 4, 5], [5, 4, 4, 4, 5], 3, True, 2, 4, 17),   # skeleton 77 (reference CUDA)
    (64, 0.0, [5, 4, 4, 4, 5], [3, 3], 4, True, 2, 2, 23),             # pad 66, 4-bit residuals
    (128, 0.0, [5, 4, 4, 4, 5], [5, 4, 4, 4, 5], 2, False, 1, 2, 19),  # no spinor
]


@pytest.mark.parametrize("hd,sk_frac,kbits,vbits,rbits,spinor,n_kvh,n_q,n_ctx", CASES)
def test_sqfree_attn_oracle_matches_definition(hd, sk_frac, kbits, vbits, rbits, spinor, n_kvh, n_q, n_ctx):
    pad, sk, km, kbc, vbc, kp, vp = _setup(hd, sk_frac, kbits, vbits, rbits, spinor, n_kvh, n_ctx, seed=hd + rbits)
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_ctx, seed=5)
    scale = 1.0 / np.sqrt(hd)
    s, o = O.sqfree_attn_decode(q, kp, vp, n_kvh, n_ctx, hd, km, kbc, vbc, rbits, spinor, scale)
    K = np.stack([O.sqfree_decompress_f32(kp[h], hd, km, kbc, rbits, spinor) for h in range(n_kvh)])
    V = np.stack([O.sqfree_decompress_f32(vp[h], hd, km, vbc, rbits, spinor) for h in range(n_kvh)])
    s_ref, o_ref = _np_attn(q, K, V, scale)
    np.testing.assert_allclose(s, s_ref, rtol=1e-6, atol=1e-6 * np.abs(s_ref).max())
    np.testing.assert_allclose(o, o_ref, rtol=1e-6, atol=1e-6 * np.abs(o_ref).max())
    # scores-only and output-only calls give the same arrays
    s2, _ = O.sqfree_attn_decode(q, kp, vp, n_kvh, n_ctx, hd, km, kbc, vbc, rbits, spinor, scale, want_out=False)
    _, o2 = O.sqfree_attn_decode(q, kp, vp, n_kvh, n_ctx, hd, km, kbc, vbc, rbits, spinor, scale, want_scores=False)
    np.testing.assert_array_equal(s2, s)
    np.testing.assert_array_equal(o2, o)


def _coefficients(packed, bc, pad, sk, rbits, spinor):
    """c~ [n][pad] of sqfree records from the layout alone:
    [skeleton bands][mag f32 LE][n_res rbits-bit levels, LSB-first][sheet bits, LSB-first]."""
    skel_idx, res_idx, offs, slots, signs = R.knight_tables(pad, sk)
    nr = len(res_idx)
    M = np.zeros((nr, sk))
    for r in range(nr):
        for j in range(offs[r], offs[r + 1]):
            M[r, slots[j]] += signs[j]
    n = packed.shape[0]
    skB = bc.total_bytes
    skel = np.stack([O.band_dequantize(packed[i, :skB], bc) for i in range(n)]).astype(np.float64)
    mag = packed[:, skB:skB + 4].copy().view(np.float32)[:, 0].astype(np.float64)
    rbytes = (nr * rbits + 7) // 8
    bits = np.unpackbits(packed[:, skB + 4:skB + 4 + rbytes], axis=1, bitorder="little")[:, :nr * rbits]
    lv = (bits.reshape(n, nr, rbits) * (1 << np.arange(rbits))).sum(axis=2)
    sign = np.ones((n, nr))
    if spinor:
        sheet = np.unpackbits(packed[:, skB + 4 + rbytes:], axis=1, bitorder="little")[:, :nr]
        sign = 1.0 - 2.0 * sheet
    L = 1 << rbits
    step = 2.0 * mag * rbits / (L - 1)
    c = np.zeros((n, pad))
    c[:, list(skel_idx)] = skel
    c[:, list(res_idx)] = sign * (skel @ M.T) + (lv - (L - 1) / 2.0) * step[:, None]
    return c


@pytest.mark.parametrize("hd,sk_frac,kbits,vbits,rbits,spinor,n_kvh,n_q,n_ctx", CASES)
def test_sqfree_attn_coefficient_form(hd, sk_frac, kbits, vbits, rbits, spinor, n_kvh, n_q, n_ctx):
    pad, sk, km, kbc, vbc, kp, vp = _setup(hd, sk_frac, kbits, vbits, rbits, spinor, n_kvh, n_ctx,
                                           seed=3 * hd + rbits)
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_ctx, seed=6)
    scale = 1.0 / np.sqrt(hd)
    s, o = O.sqfree_attn_decode(q, kp, vp, n_kvh, n_ctx, hd, km, kbc, vbc, rbits, spinor, scale)
    Vmat = vilenkin_dense(pad)
    np.testing.assert_allclose(Vmat, Vmat.T, atol=1e-12)
    grp = n_q // n_kvh
    for h in range(n_q):
        kh = h // grp
        qp = np.zeros(pad)
        qp[:hd] = q[h]
        qt = scale * (Vmat @ qp)
        ck = _coefficients(kp[kh], kbc, pad, sk, rbits, spinor)
        score = ck @ qt
        np.testing.assert_allclose(s[h], score, rtol=1e-4, atol=1e-4 * np.abs(score).max())
        p = np.exp(score - score.max())
        cv = _coefficients(vp[kh], vbc, pad, sk, rbits, spinor)
        ref = (Vmat @ ((p @ cv) / p.sum()))[:hd]
        np.testing.assert_allclose(o[h], ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
