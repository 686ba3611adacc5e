"""Seeded synthetic inputs for the five BASELINE configurations (reduced or full size).

All values are produced on the CPU with numpy's PCG64 so the GPU tests and the
oracle see identical fp16 inputs. Distributions follow BASELINE.json configs:
  cfg1: N(0,1) plus 4 seeded outlier channels per head scaled x12
  cfg2: N(0,1) with rotary embedding applied over positions (theta 500000)
  cfg3: N(0,1) times a per-head log-normal channel scale (sigma 0.5)
  cfg4: Gaussian with heavy-tailed Student-t(nu=4) outlier channels
  cfg5: N(0,1)
"""
import numpy as np


def rope(x, pos, theta=500000.0):
    """x: [..., n_pos, hd] rotated pairwise (i, i+hd/2) by pos * theta^(-2i/hd)."""
    hd = x.shape[-1]
    half = hd // 2
    inv = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / hd)
    ang = np.asarray(pos, dtype=np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[..., :half].astype(np.float64), x[..., half:].astype(np.float64)
    return np.concatenate([a * c - b * s, a * s + b * c], axis=-1).astype(np.float32)


def cfg1_kv(n_heads=8, n_pos=4096, hd=128, seed=1):
    """[n_heads, n_pos, hd] fp16 K and V: N(0,1) + 4 outlier channels/head x12."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(2):
        x = rng.standard_normal((n_heads, n_pos, hd), dtype=np.float32)
        for h in range(n_heads):
            ch = rng.choice(hd, 4, replace=False)
            x[h, :, ch] *= 12.0
        out.append(x.astype(np.float16))
    return out[0], out[1]


def cfg2_kv(n_heads=8, n_pos=1024, hd=128, seed=2, theta=500000.0):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n_heads, n_pos, hd), dtype=np.float32)
    k = rope(k, np.arange(n_pos), theta)
    v = rng.standard_normal((n_heads, n_pos, hd), dtype=np.float32)
    return k.astype(np.float16), v.astype(np.float16)


def cfg2_q(n_q=32, hd=128, pos=1024, seed=3, theta=500000.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n_q, 1, hd), dtype=np.float32)
    return rope(q, np.array([pos]), theta)[:, 0, :]


def cfg3_kv(n_heads=32, n_pos=256, hd=96, seed=4):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(2):
        scale = np.exp(0.5 * rng.standard_normal((n_heads, 1, hd))).astype(np.float32)
        x = rng.standard_normal((n_heads, n_pos, hd), dtype=np.float32) * scale
        out.append(x.astype(np.float16))
    return out[0], out[1]


def cfg4_kv(n_heads=4, n_pos=256, hd=128, seed=5, n_outlier=4):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(2):
        x = rng.standard_normal((n_heads, n_pos, hd), dtype=np.float32)
        for h in range(n_heads):
            ch = rng.choice(hd, n_outlier, replace=False)
            x[h][:, ch] = rng.standard_t(4, size=(n_pos, n_outlier)).astype(np.float32) * 3.0
        out.append(x.astype(np.float16))
    return out[0], out[1]


def cfg5_kv(n_heads=8, n_pos=128, hd=256, seed=6):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n_heads, n_pos, hd), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((n_heads, n_pos, hd), dtype=np.float32).astype(np.float16)
    return k, v


def hier_W(n_slots, n_target, n_skel, seed=7, scale=0.05):
    """Seeded fp16 predictor matrices [n_slots, n_target, n_skel] (as uint16 bits)."""
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((n_slots, n_target, n_skel)) * scale).astype(np.float16)
    return W.view(np.uint16)


def tie_rows(x16, bc, order=None, norm=1, vht2=None):
    """Indices of the rows of x16 (fp16 bits [n, hd]) for which some quantizer input
    x*inv is exactly a half-integer, so that the codes depend on round-half-to-even
    (__float2int_rn at shannon_prime_cuda.cu:186). The spectral values come from the
    oracle's VHT2 (passed in as `vht2`); scale, fp16 scale, inverse and product follow
    the quantizer's fp32 steps (shannon_prime_cuda.cu:160-186) in numpy float32."""
    x = vht2(np.ascontiguousarray(x16, dtype=np.uint16).view(np.float16).astype(np.float32), norm)
    if order is not None:
        x = x[:, np.asarray(order)]
    hits = np.zeros(x.shape[0], bool)
    for b in range(bc.n_bands):
        off, sz, bits = bc.band_off[b], bc.band_sz[b], bc.band_bits[b]
        maxv = (1 << (bits - 1)) - 1
        if maxv == 0:
            continue
        band = x[:, off:off + sz]
        amax = np.abs(band).max(1)
        scale = np.where(amax > 0, amax / np.float32(maxv), np.float32(0)).astype(np.float32)
        ss = scale.astype(np.float16).astype(np.float32)
        with np.errstate(divide="ignore"):
            inv = np.where(ss > 0, np.float32(1) / ss, np.float32(0)).astype(np.float32)
        prod = (band * inv[:, None]).astype(np.float32)
        hits |= (prod - np.floor(prod) == np.float32(0.5)).any(1)
    return np.nonzero(hits)[0]
