"""Decode attention over hier records in the oracle (spo_hier_attn_decode),
pinned two ways on the CPU:

* against its definition: each KV head's records decompressed by the (separately
  pinned) spo_hier_decompress with that head's predictor, then float64 softmax
  attention with GQA grouping h -> h // (n_q / n_kvh);
* against the spectral-domain algebra the device kernels use, restated here in
  float64 numpy from the record layout alone: the transform V of length pad is
  symmetric and its own inverse, so with q~ = kq_scale * V(q zero-padded to pad),
  score_t = u . skel_t + q~_tgt . dev_t where u = q~_skel + W^T q~_tgt, and
  sum_t p_t V~_t = V(c)[:hd] with c_skel = sum p skel, c_tgt = W c_skel + sum p dev.
  A zero-vs-mean pad of q, a transposed W or a wrong level centre fails it.
"""
import numpy as np
import pytest

import oracle_py as O
import workloads as W


def _np_attn(q, K, V, kq_scale):
    """float64 softmax attention; K, V [n_kvh][n_ctx][hd]."""
    n_q, n_kvh = q.shape[0], K.shape[0]
    grp = n_q // n_kvh
    s = np.stack([K[h // grp].astype(np.float64) @ q[h].astype(np.float64) for h in range(n_q)]) * kq_scale
    p = np.exp(s - s.max(axis=1, keepdims=True))
    out = np.stack([(p[h] @ V[h // grp].astype(np.float64)) / p[h].sum() for h in range(n_q)])
    return s, out


def _setup(hd, rbits, skel_bits, n_kvh, n_ctx, seed):
    pad = O.sqfree_pad_dim(hd)
    skel_idx, tgt_idx = O.hier_geometry(pad)
    skel_bc = O.band_config(len(skel_idx), skel_bits)
    Wm = W.hier_W(n_kvh, len(tgt_idx), len(skel_idx), seed=seed)
    k16, v16 = W.cfg5_kv(n_heads=n_kvh, n_pos=n_ctx, hd=hd, seed=seed + 1)
    kp = np.stack([O.hier_compress_f16(k16[h].view(np.uint16), hd, pad, skel_idx, tgt_idx, skel_bc, Wm[h], rbits)
                   for h in range(n_kvh)])
    vp = np.stack([O.hier_compress_f16(v16[h].view(np.uint16), hd, pad, skel_idx, tgt_idx, skel_bc, Wm[h], rbits)
                   for h in range(n_kvh)])
    return pad, skel_idx, tgt_idx, skel_bc, Wm, kp, vp


CASES = [(256, 2, [5, 5], 2, 4, 37), (64, 3, [5, 4], 2, 2, 19), (96, 2, [4], 1, 3, 11)]


@pytest.mark.parametrize("hd,rbits,skel_bits,n_kvh,n_q,n_ctx", CASES)
def test_hier_attn_oracle_matches_definition(hd, rbits, skel_bits, n_kvh, n_q, n_ctx):
    pad, sk, tg, bc, Wm, kp, vp = _setup(hd, rbits, skel_bits, n_kvh, n_ctx, seed=hd + rbits)
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_ctx, seed=5)
    scale = 1.0 / np.sqrt(hd)
    s, o = O.hier_attn_decode(q, kp, vp, n_kvh, n_ctx, hd, pad, sk, tg, bc, Wm, rbits, scale)
    K = np.stack([O.hier_decompress_f32(kp[h], hd, pad, sk, tg, bc, Wm[h], rbits) for h in range(n_kvh)])
    V = np.stack([O.hier_decompress_f32(vp[h], hd, pad, sk, tg, bc, Wm[h], rbits) for h in range(n_kvh)])
    s_ref, o_ref = _np_attn(q, K, V, scale)
    np.testing.assert_allclose(s, s_ref, rtol=1e-6, atol=1e-6 * np.abs(s_ref).max())
    np.testing.assert_allclose(o, o_ref, rtol=1e-6, atol=1e-6 * np.abs(o_ref).max())


def _records(packed, bc, n_target, rbits):
    """Skeleton values, mag and levels of hier records, read from the layout:
    [skeleton bands][mag f32 LE][n_target rbits-bit levels, LSB-first]."""
    n = packed.shape[0]
    skB = bc.total_bytes
    skel = np.stack([O.band_dequantize(packed[i, :skB], bc) for i in range(n)]).astype(np.float64)
    mag = packed[:, skB:skB + 4].copy().view(np.float32)[:, 0].astype(np.float64)
    bits = np.unpackbits(packed[:, skB + 4:], axis=1, bitorder="little")[:, :n_target * rbits]
    lv = (bits.reshape(n, n_target, rbits) * (1 << np.arange(rbits))).sum(axis=2)
    return skel, mag, lv


@pytest.mark.parametrize("hd,rbits,skel_bits,n_kvh,n_q,n_ctx", CASES)
def test_hier_attn_spectral_form(hd, rbits, skel_bits, n_kvh, n_q, n_ctx):
    pad, sk, tg, bc, Wm, kp, vp = _setup(hd, rbits, skel_bits, n_kvh, n_ctx, seed=3 * hd + rbits)
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_ctx, seed=6)
    scale = 1.0 / np.sqrt(hd)
    s, o = O.hier_attn_decode(q, kp, vp, n_kvh, n_ctx, hd, pad, sk, tg, bc, Wm, rbits, scale)
    L = 1 << rbits
    centre = (L - 1) / 2.0
    Vmat = np.stack([O.vilenkin(np.eye(pad, dtype=np.float32)[i]) for i in range(pad)]).astype(np.float64)
    grp = n_q // n_kvh
    for h in range(n_q):
        kh = h // grp
        Wf = Wm[kh].view(np.float16).astype(np.float64)  # [n_target][n_skel]
        qp = np.zeros(pad)
        qp[:hd] = q[h]
        qs = scale * (Vmat @ qp)
        u = qs[sk] + Wf.T @ qs[tg]
        skel, mag, lv = _records(kp[kh], bc, len(tg), rbits)
        step = 2.0 * mag / (L - 1)
        score = skel @ u + step * (lv @ qs[tg] - centre * qs[tg].sum())
        np.testing.assert_allclose(s[h], score, rtol=1e-4, atol=1e-4 * np.abs(score).max())
        p = np.exp(score - score.max())
        vskel, vmag, vlv = _records(vp[kh], bc, len(tg), rbits)
        vstep = 2.0 * vmag / (L - 1)
        c = np.zeros(pad)
        cs = p @ vskel
        c[sk] = cs
        c[tg] = Wf @ cs + (p * vstep) @ (vlv - centre)
        ref = (Vmat @ (c / p.sum()))[:hd]
        np.testing.assert_allclose(o[h], ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())
