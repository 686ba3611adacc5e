"""Writes the golden fixtures of tests/golden/ from the CPU oracle (oracle/sp_oracle.c).

The reference ships no golden vectors for this path (its core is an absent
submodule), so these fixtures are this build's own: seeded inputs and the
oracle's outputs for configs 0-4 of BASELINE.json at reduced sizes. They pin
the oracle against regressions (tests/test_golden.py) and give the GPU path a
fixed target (tests/test_gpu_golden.py). Each file is a numpy .npz with plain
arrays (no pickled objects).

Run from the repository root:  python3 tests/golden/make_fixtures.py
"""
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_py as O  # noqa: E402
import workloads as W  # noqa: E402


def ship(name, hd, kbits, vbits, kv, n_pos, seed):
    """Ship codec: fp16 K/V in, codes, fp16 and fp32 reconstructions, and the
    K reconstruction from its first two bands."""
    k16, v16 = kv(n_heads=2, n_pos=n_pos, hd=hd, seed=seed)
    k = k16.reshape(-1, hd).view(np.uint16)
    v = v16.reshape(-1, hd).view(np.uint16)
    kbc, vbc = O.band_config(hd, kbits), O.band_config(hd, vbits)
    order = O.mobius_order(hd)
    kc = O.ship_compress_f16(k, kbc, order)
    vc = O.ship_compress_f16(v, vbc)
    np.savez_compressed(os.path.join(HERE, name), hd=hd, k_bits=np.array(kbits), v_bits=np.array(vbits),
                        order=order, k_in=k, v_in=v, k_codes=kc, v_codes=vc,
                        k_rec16=O.ship_decompress_f16(kc, kbc, order), v_rec16=O.ship_decompress_f16(vc, vbc),
                        k_rec32=O.ship_decompress_f32(kc, kbc, order), v_rec32=O.ship_decompress_f32(vc, vbc),
                        k_rec32_2bands=O.ship_decompress_f32(kc, kbc, order, max_bands=2))


def attention(name, n_q, H, n_ctx, hd):
    """Fused decode attention over ship records: the records (from seeded RoPE'd
    K and V), the query, and the oracle's scores and softmax.V."""
    k16, v16 = W.cfg2_kv(n_heads=H, n_pos=n_ctx, hd=hd, seed=n_ctx + 11)
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_ctx, seed=n_ctx + 12)
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    order = O.mobius_order(hd)
    kp = np.stack([O.ship_compress_f16(k16[h].view(np.uint16), kbc, order) for h in range(H)])
    vp = np.stack([O.ship_compress_f16(v16[h].view(np.uint16), vbc) for h in range(H)])
    scale = 1.0 / math.sqrt(hd)
    s, o = O.attn_decode(q, kp, vp, H, n_ctx, kbc, vbc, order, scale)
    np.savez_compressed(os.path.join(HERE, name), hd=hd, n_kvh=H, kq_scale=np.float32(scale), q=q.astype(np.float32),
                        k_codes=kp, v_codes=vp, scores=s, out=o)


def sqfree(name, hd, bits, rbits, spinor, sk_frac, n_pos, seed):
    k16, _ = W.cfg4_kv(n_heads=1, n_pos=n_pos, hd=hd, seed=seed)
    x = k16.reshape(n_pos, hd).view(np.uint16)
    pad = O.sqfree_pad_dim(hd)
    sk = int(pad * sk_frac)
    km = O.Knight(pad, sk)
    bc = O.band_config(sk, bits)
    codes = O.sqfree_compress_f16(x, hd, km, bc, rbits, spinor)
    np.savez_compressed(os.path.join(HERE, name), hd=hd, pad=pad, sk_k=sk, bits=np.array(bits), rbits=rbits,
                        spinor=int(spinor), x_in=x, codes=codes,
                        rec32=O.sqfree_decompress_f32(codes, hd, km, bc, rbits, spinor))


def hier(name, hd, rbits, skel_bits, n_pos, n_q, n_ctx, seed):
    """Hier codec (one slot) and fused attention over hier records (2 KV heads)."""
    pad = O.sqfree_pad_dim(hd)
    sk, tg = O.hier_geometry(pad)
    bc = O.band_config(len(sk), skel_bits)
    Wm = W.hier_W(2, len(tg), len(sk), seed=seed)
    k16, v16 = W.cfg5_kv(n_heads=2, n_pos=max(n_pos, n_ctx), hd=hd, seed=seed + 1)
    x = k16[0, :n_pos].view(np.uint16)
    codes = O.hier_compress_f16(x, hd, pad, sk, tg, bc, Wm[0], rbits)
    kp = np.stack([O.hier_compress_f16(k16[h, :n_ctx].view(np.uint16), hd, pad, sk, tg, bc, Wm[h], rbits)
                   for h in range(2)])
    vp = np.stack([O.hier_compress_f16(v16[h, :n_ctx].view(np.uint16), hd, pad, sk, tg, bc, Wm[h], rbits)
                   for h in range(2)])
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_ctx, seed=seed + 2)
    scale = 1.0 / math.sqrt(hd)
    s, o = O.hier_attn_decode(q, kp, vp, 2, n_ctx, hd, pad, sk, tg, bc, Wm, rbits, scale)
    np.savez_compressed(os.path.join(HERE, name), hd=hd, pad=pad, skel_idx=np.asarray(sk, np.int32),
                        tgt_idx=np.asarray(tg, np.int32), skel_bits=np.array(skel_bits), rbits=rbits, W=Wm,
                        x_in=x, codes=codes, rec32=O.hier_decompress_f32(codes, hd, pad, sk, tg, bc, Wm[0], rbits),
                        q=q.astype(np.float32), kq_scale=np.float32(scale), k_codes=kp, v_codes=vp, scores=s, out=o)


def main():
    # ship round trip at hd 128 (K 5/5/4/3 + Mobius, V 3), outlier channels x12
    ship("cfg0_ship_hd128.npz", 128, [5, 5, 4, 3], [3], W.cfg1_kv, 32, 201)
    # fused decompress-KQ, softmax and .V at the Llama-3 head ratio (GQA 4)
    attention("cfg1_attention_hd128.npz", 8, 2, 300, 128)
    # hd 96 (Vilenkin 2^5*3) with the bridge's defaults, K 5/4/4 + Mobius, V 5
    ship("cfg2_ship_hd96.npz", 96, [5, 4, 4], [5], W.cfg3_kv, 32, 203)
    # sqfree + spinor, pad 154, skeleton 0.75 (115) at 5/4/4/4/5, 3-bit residual
    sqfree("cfg3_sqfree_hd128.npz", 128, [5, 4, 4, 4, 5], 3, True, 0.75, 64, 204)
    # hier, hd 256 -> pad 330, 30 skeleton at 5/5, 2-bit targets; attention GQA 2
    hier("cfg4_hier_hd256.npz", 256, 2, [5, 5], 32, 4, 160, 205)


if __name__ == "__main__":
    main()
