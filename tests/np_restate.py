"""Independent numpy restatement of the sqfree+spinor and hierarchical codecs --
test infrastructure, written from the reference's CUDA text, not from the C
oracle (oracle/sp_oracle.c), so that a misreading shared by the oracle and the
HIP kernels shows up as a byte difference here.

Every float32 operation below is one numpy float32 operation on float32
operands (one IEEE rounding each), in the order the reference kernels write
it; integer steps use Python ints. Where the reference's own kernels are not
reproducible on a CPU (the Vilenkin stage constants come from the device's
fast __cosf/__sinf, shannon_prime_sqfree.cu:40-43; the pad mean sums only the
first warp's partials, :133-144) this follows the build's documented choices:
Hartley constants cos+sin evaluated in double and rounded once, and the true
mean in the reference's 256-slot reduction order.
"""
import functools
import math

import numpy as np

F32 = np.float32


# ---- reductions, pad -------------------------------------------------------

def tree256_sum(v, take_abs=False):
    """The 256-thread block reduction of kernel_mean_abs
    (shannon_prime_sqfree.cu:493-509) and kernel_residual_magnitude
    (shannon_prime_hier.cu:115-144): thread t adds v[t], v[t+256], ... to 0.0f,
    then smem[t] += smem[t + s] for s = 128, 64, ..., 1."""
    v = np.asarray(v, F32)
    if take_abs:
        v = np.abs(v)
    slot = np.zeros(256, F32)
    for i in range(0, len(v), 256):
        part = v[i:i + 256]
        slot[:len(part)] = slot[:len(part)] + part
    s = 128
    while s > 0:
        slot[:s] = slot[:s] + slot[s:2 * s]
        s //= 2
    return slot[0]


def squarefree(n):
    if n < 1:
        return False
    d = 2
    while d * d <= n:
        if n % (d * d) == 0:
            return False
        d += 1
    return True


def pad_dim(hd):
    """Smallest squarefree integer >= hd whose prime factors are all <= 11."""
    n = hd
    while True:
        m = n
        for p in (2, 3, 5, 7, 11):
            while m % p == 0:
                m //= p
        if m == 1 and squarefree(n):
            return n
        n += 1


def sqfree_pad(x, hd, pad):
    """kernel_sqfree_pad (shannon_prime_sqfree.cu:118-151): the hd values, then
    their mean in every padded slot (mean = sum / (float)hd)."""
    x = np.asarray(x, F32)
    mean = tree256_sum(x[:hd]) / F32(hd)
    out = np.empty(pad, F32)
    out[:hd] = x[:hd]
    out[hd:] = mean
    return out


# ---- Vilenkin ---------------------------------------------------------------

def factors(n):
    f = []
    for p in (2, 3, 5, 7, 11):
        while n % p == 0:
            f.append(p)
            n //= p
    assert n == 1
    return f


def cas_table(p):
    C = np.empty((p, p), F32)
    for k in range(p):
        for j in range(p):
            a = 2.0 * math.pi * ((k * j) % p) / p
            C[k, j] = F32(math.cos(a) + math.sin(a))
    return C


def vilenkin(x):
    """kernel_vilenkin_inplace (shannon_prime_sqfree.cu:45-112): for each prime
    factor p ascending at stride s (s *= p after the stage), every group
    {base + k*s} becomes result[k] = (sum_j C[k][j]*g[j], from 0.0f, j
    ascending) * (1/sqrt(p))."""
    x = np.asarray(x, F32).copy()
    n = len(x)
    stride = 1
    for p in factors(n):
        C = cas_table(p)
        isp = F32(1.0) / np.sqrt(F32(p))
        blk = stride * p
        g = x.reshape(n // blk, p, stride)
        out = np.empty_like(g)
        for k in range(p):
            acc = np.zeros((n // blk, stride), F32)
            for j in range(p):
                acc = acc + C[k, j] * g[:, j, :]
            out[:, k, :] = acc * isp
        x = out.reshape(n)
        stride *= p
    return x


# ---- band quantizer (the skeleton's record head) ---------------------------

def band_spans(n, nb):
    size = n // nb
    return [(b * size, (n - b * size) if b == nb - 1 else size) for b in range(nb)]


def band_quantize(x, bits):
    """kernel_band_quantize_simple (shannon_prime_cuda.cu:131-204) -> bytes."""
    x = np.asarray(x, F32)
    out = bytearray()
    for (off, sz), nbit in zip(band_spans(len(x), len(bits)), bits):
        band = x[off:off + sz]
        maxv = (1 << (nbit - 1)) - 1
        amax = F32(0.0)
        for a in np.abs(band):
            if a > amax:
                amax = a
        scale = amax / F32(maxv) if amax > 0 else F32(0.0)
        sh = np.float16(scale)
        out += sh.tobytes()
        stored = F32(sh)
        inv = F32(1.0) / stored if stored > 0 else F32(0.0)
        acc = 0
        for i, v in enumerate(band):
            q = int(np.rint(v * inv))
            q = max(-maxv, min(maxv, q))
            acc |= (q + maxv) << (i * nbit)
        out += acc.to_bytes((sz * nbit + 7) // 8, "little")
    return bytes(out)


def band_bytes(n, bits):
    return sum(2 + (sz * b + 7) // 8 for (_, sz), b in zip(band_spans(n, len(bits)), bits))


def band_dequantize(rec, n, bits):
    """kernel_band_dequantize_simple (shannon_prime_cuda.cu:210-270)."""
    out = np.zeros(n, F32)
    pos = 0
    for (off, sz), nbit in zip(band_spans(n, len(bits)), bits):
        maxv = (1 << (nbit - 1)) - 1
        scale = F32(np.frombuffer(rec[pos:pos + 2], np.float16)[0])
        if not np.isfinite(scale):
            scale = F32(0.0)
        pos += 2
        nbytes = (sz * nbit + 7) // 8
        acc = int.from_bytes(rec[pos:pos + nbytes], "little")
        for i in range(sz):
            u = (acc >> (i * nbit)) & ((1 << nbit) - 1)
            out[off + i] = F32(u - maxv) * scale
        pos += nbytes
    return out


# ---- level packing ------------------------------------------------------------

def pack_levels(levels, nbit):
    """kernel_pack_levels (shannon_prime_sqfree.cu:552-564): LSB-first."""
    acc = 0
    for i, v in enumerate(levels):
        acc |= int(v) << (i * nbit)
    return acc.to_bytes((len(levels) * nbit + 7) // 8, "little")


def unpack_levels(data, n, nbit):
    acc = int.from_bytes(data, "little")
    return [(acc >> (i * nbit)) & ((1 << nbit) - 1) for i in range(n)]


# ---- Mobius function, squarefree-first order, Knight CSR -----------------------

def mobius_mu(n):
    """mu(n) by trial division."""
    k, d = 0, 2
    while d * d <= n:
        if n % d == 0:
            n //= d
            if n % d == 0:
                return 0
            k += 1
        d += 1
    if n > 1:
        k += 1
    return -1 if k % 2 else 1


def squarefree_first(n):
    """Indices i with i+1 squarefree ascending, then the rest ascending."""
    return [i for i in range(n) if squarefree(i + 1)] + [i for i in range(n) if not squarefree(i + 1)]


@functools.lru_cache(maxsize=None)
def knight_tables(pad, sk):
    """Skeleton = the first sk entries of the squarefree-first order; residual =
    the rest in that order. Residual coefficient c (n = c+1) gets one CSR term
    per divisor d < n, ascending, with mu(n/d) != 0 and coefficient d-1 in the
    skeleton: (skeleton slot of d-1, mu(n/d))."""
    order = squarefree_first(pad)
    skel, res = order[:sk], order[sk:]
    slot = {c: s for s, c in enumerate(skel)}
    offsets, slots, signs = [0], [], []
    for c in res:
        n = c + 1
        for d in range(1, n):
            if n % d == 0 and mobius_mu(n // d) != 0 and (d - 1) in slot:
                slots.append(slot[d - 1])
                signs.append(mobius_mu(n // d))
        offsets.append(len(slots))
    return tuple(skel), tuple(res), tuple(offsets), tuple(slots), tuple(signs)


def mobius_predict(skel, offsets, slots, signs):
    """kernel_mobius_predict (shannon_prime_sqfree.cu:179-203): pred[r] = sum
    from 0.0f of (float)mu * skel[slot] over the CSR row, in order."""
    skel = np.asarray(skel, F32)
    pred = np.zeros(len(offsets) - 1, F32)
    for r in range(len(pred)):
        acc = F32(0.0)
        for j in range(offsets[r], offsets[r + 1]):
            acc = acc + F32(signs[j]) * skel[slots[j]]
        pred[r] = acc
    return pred


# ---- spinor, sqfree residual quantizer ---------------------------------------

def spinor_extract(a, p):
    """kernel_spinor_extract (shannon_prime_sqfree.cu:212-240): v+ = a - p,
    v- = a + p, bit = |v-| < |v+| (strict), dev = the chosen one."""
    a, p = np.asarray(a, F32), np.asarray(p, F32)
    vp, vm = a - p, a + p
    bit = np.abs(vm) < np.abs(vp)
    dev = np.where(bit, vm, vp).astype(F32)
    sheet = bytearray((len(a) + 7) // 8)
    for r in np.nonzero(bit)[0]:
        sheet[r // 8] |= 1 << (r % 8)
    return dev, bytes(sheet), bit


def sqfree_residual_quantize(dev, nbit, round_half_up=True, sat_times_bits=True):
    """kernel_mean_abs + kernel_quantize_residual (shannon_prime_sqfree.cu:493-532):
    mag = max(sum|dev| / n, 1e-12); sat = mag*bits (1e-12 at the floor);
    step = 2*sat/(L-1); level = (int)(dev*(1/step) + center + 0.5), clamped.
    The two switches give the plausible misreadings (rint; sat = mag) that the
    pins must tell apart from the reference's rule."""
    dev = np.asarray(dev, F32)
    mag = tree256_sum(dev, take_abs=True) / F32(len(dev))
    if mag < F32(1e-12):
        mag = F32(1e-12)
    L = 1 << nbit
    center = F32(0.5) * F32(L - 1)
    if sat_times_bits:
        sat = mag * F32(nbit) if mag > F32(1e-12) else F32(1e-12)
    else:
        sat = mag
    step = (F32(2.0) * sat) / F32(L - 1)
    inv = F32(1.0) / step
    lv = []
    for v in dev:
        qf = v * inv + center
        q = int(math.trunc(float(qf + F32(0.5)))) if round_half_up else int(np.rint(qf))
        lv.append(max(0, min(L - 1, q)))
    return mag, lv


def sqfree_residual_dequantize(levels, nbit, mag):
    """kernel_dequantize_residual (shannon_prime_sqfree.cu:535-548)."""
    L = 1 << nbit
    center = F32(0.5) * F32(L - 1)
    step = (F32(2.0) * (F32(mag) * F32(nbit))) / F32(L - 1)
    return np.array([(F32(v) - center) * step for v in levels], F32)


# ---- sqfree record ----------------------------------------------------------

def sqfree_compress(x, hd, sk, kbits, rbits, spinor):
    """sp_cuda_sqfree_write_one (shannon_prime_sqfree.cu:750-853): record
    [skeleton bands][f32 mag][residual levels][sheet bits] (:683-686); the
    prediction uses the unquantized skeleton."""
    pad = pad_dim(hd)
    skel_idx, res_idx, offs, slots, signs = knight_tables(pad, sk)
    c = vilenkin(sqfree_pad(x, hd, pad))
    skel = c[list(skel_idx)]
    rec = band_quantize(skel, kbits)
    pred = mobius_predict(skel, offs, slots, signs)
    act = c[list(res_idx)]
    if spinor:
        dev, sheet, _ = spinor_extract(act, pred)
    else:
        dev, sheet = (act - pred).astype(F32), b""
    mag, lv = sqfree_residual_quantize(dev, rbits)
    return rec + np.array([mag], F32).tobytes() + pack_levels(lv, rbits) + sheet


def sqfree_decompress(rec, hd, sk, kbits, rbits, spinor):
    """sp_cuda_sqfree_read_one (shannon_prime_sqfree.cu:857-950): the prediction
    uses the dequantized skeleton."""
    pad = pad_dim(hd)
    skel_idx, res_idx, offs, slots, signs = knight_tables(pad, sk)
    nb = band_bytes(sk, kbits)
    skel = band_dequantize(rec[:nb], sk, kbits)
    c = np.zeros(pad, F32)
    c[list(skel_idx)] = skel
    nr = len(res_idx)
    pred = mobius_predict(skel, offs, slots, signs)
    mag = np.frombuffer(rec[nb:nb + 4], F32)[0]
    rbytes = (nr * rbits + 7) // 8
    lv = unpack_levels(rec[nb + 4:nb + 4 + rbytes], nr, rbits)
    dv = sqfree_residual_dequantize(lv, rbits, mag)
    sheet = rec[nb + 4 + rbytes:]
    for r in range(nr):
        p = pred[r]
        if spinor and (sheet[r // 8] >> (r % 8)) & 1:
            p = -p
        c[res_idx[r]] = p + dv[r]
    return vilenkin(c)[:hd]


# ---- hierarchical --------------------------------------------------------------

@functools.lru_cache(maxsize=None)
def hier_geometry(pad):
    """Skeleton = the first ceil(0.09*pad) of the squarefree-first order, targets
    the rest (the build's documented geometry)."""
    n_skel = max(1, (pad * 9 + 99) // 100)
    order = squarefree_first(pad)
    return tuple(order[:n_skel]), tuple(order[n_skel:])


def hier_predict(W16, skel):
    """kernel_hier_predict (shannon_prime_hier.cu:74-92): per target row,
    acc = 0.0f; for s ascending: acc += (float)W[t][s] * skel[s] (product
    rounded, then the add)."""
    W = np.asarray(W16, np.float16).astype(F32)
    skel = np.asarray(skel, F32)
    acc = np.zeros(W.shape[0], F32)
    for s in range(W.shape[1]):
        acc = acc + W[:, s] * skel[s]
    return acc


def hier_residual_quantize(dev, nbit, half_even=True):
    """kernel_residual_magnitude + kernel_quantize_residual
    (shannon_prime_hier.cu:115-171): m = max(sum|dev|/n, 1e-12); step =
    2*m/(L-1); center = (L-1)/2; level = __float2int_rn(dev*(1/step) + center)
    (half to even), clamped. half_even=False gives the sqfree rounding rule."""
    dev = np.asarray(dev, F32)
    m = tree256_sum(dev, take_abs=True) / F32(len(dev))
    if m < F32(1e-12):
        m = F32(1e-12)
    L = 1 << nbit
    step = (F32(2.0) * m) / F32(L - 1)
    center = F32(L - 1) / F32(2.0)
    inv = F32(1.0) / step if step > 0 else F32(0.0)
    lv = []
    for v in dev:
        qf = v * inv + center
        q = int(np.rint(qf)) if half_even else int(math.trunc(float(qf + F32(0.5))))
        lv.append(max(0, min(L - 1, q)))
    return m, lv


def hier_residual_dequantize(levels, nbit, m):
    L = 1 << nbit
    step = (F32(2.0) * F32(m)) / F32(L - 1)
    center = F32(L - 1) / F32(2.0)
    return np.array([(F32(v) - center) * step for v in levels], F32)


def hier_compress(x, hd, W16, kbits, rbits):
    """sp_cuda_hier_write_one (shannon_prime_hier.cu:399-486): record
    [skeleton bands][f32 mag][residual levels] (:331-335); prediction from the
    unquantized skeleton."""
    pad = pad_dim(hd)
    skel_idx, tgt_idx = hier_geometry(pad)
    c = vilenkin(sqfree_pad(x, hd, pad))
    skel = c[list(skel_idx)]
    rec = band_quantize(skel, kbits)
    dev = (c[list(tgt_idx)] - hier_predict(W16, skel)).astype(F32)
    m, lv = hier_residual_quantize(dev, rbits)
    return rec + np.array([m], F32).tobytes() + pack_levels(lv, rbits)


def hier_decompress(rec, hd, W16, kbits, rbits):
    """sp_cuda_hier_read_one (shannon_prime_hier.cu:490-571)."""
    pad = pad_dim(hd)
    skel_idx, tgt_idx = hier_geometry(pad)
    ns = len(skel_idx)
    nb = band_bytes(ns, kbits)
    skel = band_dequantize(rec[:nb], ns, kbits)
    pred = hier_predict(W16, skel)
    m = np.frombuffer(rec[nb:nb + 4], F32)[0]
    lv = unpack_levels(rec[nb + 4:], len(tgt_idx), rbits)
    dv = hier_residual_dequantize(lv, rbits, m)
    c = np.zeros(pad, F32)
    c[list(skel_idx)] = skel
    c[list(tgt_idx)] = pred + dv
    return vilenkin(c)[:hd]
