"""ctypes binding of the CPU oracle (oracle/libsp_oracle.so) -- test infrastructure.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module; the product library never does.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "_build", "libsp_oracle.so")

MAX_BANDS = 16
NORM_FINAL = 0
NORM_STAGE = 1


class BandConfig(C.Structure):
    _fields_ = [
        ("head_dim", C.c_int),
        ("n_bands", C.c_int),
        ("band_bits", C.c_int * MAX_BANDS),
        ("band_size", C.c_int),
        ("total_bytes", C.c_int),
        ("ternary_mask", C.c_uint32),
        ("band_off", C.c_int * MAX_BANDS),
        ("band_sz", C.c_int * MAX_BANDS),
        ("band_byte_off", C.c_int * MAX_BANDS),
    ]


class KnightMask(C.Structure):
    _fields_ = [
        ("pad_dim", C.c_int),
        ("sk_k", C.c_int),
        ("n_res", C.c_int),
        ("n_terms", C.c_int),
        ("skeleton_idx", C.POINTER(C.c_int)),
        ("residual_idx", C.POINTER(C.c_int)),
        ("csr_offsets", C.POINTER(C.c_int)),
        ("csr_skel_slot", C.POINTER(C.c_int)),
        ("csr_mu_sign", C.POINTER(C.c_int8)),
    ]


def _ensure_built():
    if not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-C", ORACLE_DIR], check=True, capture_output=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        _ensure_built()
        _lib = C.CDLL(ORACLE_SO)
        _lib.spo_f32_to_f16.restype = C.c_uint16
        _lib.spo_f32_to_f16.argtypes = [C.c_float]
        _lib.spo_f16_to_f32.restype = C.c_float
        _lib.spo_f16_to_f32.argtypes = [C.c_uint16]
        _lib.spo_inv_sqrt_n.restype = C.c_float
        _lib.spo_tree256_sum.restype = C.c_float
        _lib.spo_correlation_f32.restype = C.c_float
        _lib.spo_sqfree_residual_quantize.restype = C.c_float
        _lib.spo_sqfree_residual_dequantize.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_float, C.c_void_p]
        _lib.spo_hier_residual_quantize.restype = C.c_float
        _lib.spo_hier_residual_dequantize.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_float, C.c_void_p]
        _lib.spo_attn_decode.argtypes = [C.c_void_p] * 3 + [C.c_int] * 4 + [C.c_void_p] * 3 + \
            [C.c_int, C.c_float, C.c_void_p, C.c_void_p]
        _lib.spo_attn_decode_bands.argtypes = [C.c_void_p] * 3 + [C.c_int] * 4 + [C.c_void_p] * 3 + \
            [C.c_int, C.c_float, C.c_void_p, C.c_void_p, C.c_int]
    return _lib


def ptr(a):
    return C.c_void_p(a.ctypes.data) if a is not None else None


def band_config(hd, bits, ternary_mask=0):
    bc = BandConfig()
    arr = (C.c_int * MAX_BANDS)(*bits)
    lib().spo_band_config_init_ext(C.byref(bc), hd, len(bits), arr, C.c_uint32(ternary_mask))
    return bc


def mobius_order(n):
    o = np.zeros(n, dtype=np.int32)
    lib().spo_mobius_order(n, ptr(o))
    return o


def vht2(x, norm=NORM_FINAL):
    """Forward VHT2 of one vector, or of every row of a 2-D array."""
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    n = x.shape[-1]
    rows = x.reshape(-1, n)
    for r in range(rows.shape[0]):
        lib().spo_vht2_forward(C.c_void_p(rows.ctypes.data + r * n * 4), n, norm)
    return x


def f32_to_f16_bits(v):
    return lib().spo_f32_to_f16(C.c_float(v))


def ship_compress_f16(x16, bc, order=None, norm=NORM_FINAL):
    """x16: uint16 [n, hd] (fp16 bits) -> uint8 [n, B]"""
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    n, hd = x16.shape
    out = np.zeros((n, bc.total_bytes), dtype=np.uint8)
    o = None if order is None else np.ascontiguousarray(order, dtype=np.int32)
    lib().spo_ship_compress_batch_f16(ptr(x16), ptr(out), n, hd, C.byref(bc), ptr(o), norm)
    return out


def ship_roundtrip_f16_omp(x16, bc, order=None, norm=NORM_FINAL, threads=1):
    """Compress + decompress every vector, split over `threads` OpenMP threads
    (the all-core CPU baseline); returns the reconstructed fp16 bits."""
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    n = x16.shape[0]
    packed = np.empty((n, bc.total_bytes), np.uint8)
    out = np.empty_like(x16)
    o = None if order is None else np.ascontiguousarray(order, dtype=np.int32)
    lib().spo_ship_roundtrip_batch_f16_omp(ptr(x16), ptr(packed), ptr(out), n, x16.shape[1], C.byref(bc), ptr(o),
                                           norm, int(threads))
    return out


def ship_compress_f32(x, bc, order=None, norm=NORM_FINAL):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, hd = x.shape
    out = np.zeros((n, bc.total_bytes), dtype=np.uint8)
    o = None if order is None else np.ascontiguousarray(order, dtype=np.int32)
    lib().spo_ship_compress_batch_f32(ptr(x), ptr(out), n, hd, C.byref(bc), ptr(o), norm)
    return out


def ship_decompress_f32(packed, bc, order=None, norm=NORM_FINAL, max_bands=-1):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    n = packed.shape[0]
    out = np.zeros((n, bc.head_dim), dtype=np.float32)
    o = None if order is None else np.ascontiguousarray(order, dtype=np.int32)
    lib().spo_ship_decompress_batch_f32(ptr(packed), ptr(out), n, bc.head_dim, C.byref(bc),
                                        ptr(o), norm, max_bands)
    return out


def ship_decompress_f16(packed, bc, order=None, norm=NORM_FINAL, max_bands=-1):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    n = packed.shape[0]
    out = np.zeros((n, bc.head_dim), dtype=np.uint16)
    o = None if order is None else np.ascontiguousarray(order, dtype=np.int32)
    lib().spo_ship_decompress_batch_f16(ptr(packed), ptr(out), n, bc.head_dim, C.byref(bc),
                                        ptr(o), norm, max_bands)
    return out


def band_quantize(x, bc):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(bc.total_bytes, dtype=np.uint8)
    lib().spo_band_quantize(ptr(x), ptr(out), C.byref(bc))
    return out


def band_dequantize(packed, bc, max_bands=-1):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.zeros(bc.head_dim, dtype=np.float32)
    lib().spo_band_dequantize_partial(ptr(packed), ptr(out), C.byref(bc), max_bands)
    return out


def sqfree_pad_dim(hd):
    return lib().spo_sqfree_pad_dim(hd)


class Knight:
    def __init__(self, pad, sk_k):
        self.m = KnightMask()
        rc = lib().spo_knight_mask_init(C.byref(self.m), pad, sk_k)
        assert rc == 0
        m = self.m
        self.pad, self.sk_k, self.n_res, self.n_terms = m.pad_dim, m.sk_k, m.n_res, m.n_terms
        self.skeleton_idx = np.ctypeslib.as_array(m.skeleton_idx, (m.sk_k,)).copy()
        self.residual_idx = np.ctypeslib.as_array(m.residual_idx, (max(m.n_res, 1),))[: m.n_res].copy()
        self.csr_offsets = np.ctypeslib.as_array(m.csr_offsets, (m.n_res + 1,)).copy()
        if m.n_terms:
            self.csr_skel_slot = np.ctypeslib.as_array(m.csr_skel_slot, (m.n_terms,)).copy()
            self.csr_mu_sign = np.ctypeslib.as_array(m.csr_mu_sign, (m.n_terms,)).copy()
        else:
            self.csr_skel_slot = np.zeros(0, np.int32)
            self.csr_mu_sign = np.zeros(0, np.int8)

    def __del__(self):
        try:
            lib().spo_knight_mask_free(C.byref(self.m))
        except Exception:
            pass


def sqfree_bytes(skel_bc, n_res, rbits, spinor):
    return lib().spo_sqfree_bytes(C.byref(skel_bc), n_res, rbits, int(spinor))


def sqfree_compress_f16(x16, hd, km, skel_bc, rbits, spinor):
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    n = x16.shape[0]
    B = sqfree_bytes(skel_bc, km.n_res, rbits, spinor)
    out = np.zeros((n, B), dtype=np.uint8)
    lib().spo_sqfree_compress_batch_f16(ptr(x16), ptr(out), n, hd, C.byref(km.m), C.byref(skel_bc),
                                        rbits, int(spinor))
    return out


def sqfree_decompress_f32(packed, hd, km, skel_bc, rbits, spinor):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    n = packed.shape[0]
    out = np.zeros((n, hd), dtype=np.float32)
    lib().spo_sqfree_decompress_batch_f32(ptr(packed), ptr(out), n, hd, C.byref(km.m),
                                          C.byref(skel_bc), rbits, int(spinor))
    return out


def hier_geometry(pad):
    ns = C.c_int(0)
    lib().spo_hier_default_geometry(pad, C.byref(ns))
    n_skel = ns.value
    skel = np.zeros(n_skel, np.int32)
    tgt = np.zeros(pad - n_skel, np.int32)
    lib().spo_hier_indices(pad, n_skel, ptr(skel), ptr(tgt))
    return skel, tgt


def hier_bytes(skel_bc, n_target, rbits):
    return lib().spo_hier_bytes(C.byref(skel_bc), n_target, rbits)


def hier_compress_f16(x16, hd, pad, skel_idx, tgt_idx, skel_bc, W, rbits):
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    n = x16.shape[0]
    B = hier_bytes(skel_bc, len(tgt_idx), rbits)
    out = np.zeros((n, B), dtype=np.uint8)
    W = np.ascontiguousarray(W, dtype=np.uint16)
    lib().spo_hier_compress_batch_f16(ptr(x16), ptr(out), n, hd, pad, len(skel_idx), ptr(skel_idx),
                                      len(tgt_idx), ptr(tgt_idx), C.byref(skel_bc), ptr(W), rbits)
    return out


def pad_transform(x32, hd, pad):
    """fp32 vectors [n][hd] -> padded (true-mean fill, tree-256 order) and
    transformed [n][pad] (the sqfree / hier coefficients before any quantizing)."""
    x32 = np.ascontiguousarray(x32, dtype=np.float32)
    out = np.zeros((x32.shape[0], pad), np.float32)
    for i in range(x32.shape[0]):
        lib().spo_sqfree_pad(ptr(x32[i]), ptr(out[i]), hd, pad)
        lib().spo_vht2_forward(ptr(out[i]), pad, NORM_FINAL)
    return out


def hier_compress_f32(x32, hd, pad, skel_idx, tgt_idx, skel_bc, W, rbits):
    """fp32 vectors [n][hd] -> records [n][B] (spo_hier_compress per vector)."""
    x32 = np.ascontiguousarray(x32, dtype=np.float32)
    n = x32.shape[0]
    B = hier_bytes(skel_bc, len(tgt_idx), rbits)
    out = np.zeros((n, B), dtype=np.uint8)
    W = np.ascontiguousarray(W, dtype=np.uint16)
    for i in range(n):
        lib().spo_hier_compress(ptr(x32[i]), ptr(out[i]), hd, pad, len(skel_idx), ptr(skel_idx), len(tgt_idx),
                                ptr(tgt_idx), C.byref(skel_bc), ptr(W), rbits)
    return out


def hier_decompress_f32(packed, hd, pad, skel_idx, tgt_idx, skel_bc, W, rbits):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    n = packed.shape[0]
    out = np.zeros((n, hd), dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.uint16)
    lib().spo_hier_decompress_batch_f32(ptr(packed), ptr(out), n, hd, pad, len(skel_idx),
                                        ptr(skel_idx), len(tgt_idx), ptr(tgt_idx), C.byref(skel_bc),
                                        ptr(W), rbits)
    return out


def attn_decode(q, kpack, vpack, n_kvh, n_ctx, kbc, vbc, order, kq_scale, norm=NORM_FINAL,
                want_scores=True, want_out=True, max_bands=-1):
    q = np.ascontiguousarray(q, dtype=np.float32)
    n_q, hd = q.shape
    scores = np.zeros((n_q, n_ctx), np.float32) if want_scores else None
    out = np.zeros((n_q, hd), np.float32) if want_out else None
    o = None if order is None else np.ascontiguousarray(order, dtype=np.int32)
    kc, vc = np.ascontiguousarray(kpack), np.ascontiguousarray(vpack)  # held across the call
    lib().spo_attn_decode_bands(ptr(q), ptr(kc), ptr(vc),
                                n_q, n_kvh, n_ctx, hd, C.byref(kbc), C.byref(vbc), ptr(o), norm,
                                C.c_float(kq_scale), ptr(scores), ptr(out), max_bands)
    return scores, out


def hier_attn_decode(q, kpack, vpack, n_kvh, n_ctx, hd, pad, skel_idx, tgt_idx, skel_bc, W, rbits, kq_scale,
                     want_scores=True, want_out=True):
    """spo_hier_attn_decode: kpack/vpack [n_kvh][n_ctx][B] uint8, W [n_kvh][n_target][n_skel] fp16 bits."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    n_q = q.shape[0]
    scores = np.zeros((n_q, n_ctx), np.float32) if want_scores else None
    out = np.zeros((n_q, hd), np.float32) if want_out else None
    s = np.ascontiguousarray(skel_idx, dtype=np.int32)
    t = np.ascontiguousarray(tgt_idx, dtype=np.int32)
    w = np.ascontiguousarray(W, dtype=np.uint16)
    kc, vc = np.ascontiguousarray(kpack), np.ascontiguousarray(vpack)  # held across the call
    lib().spo_hier_attn_decode(ptr(q), ptr(kc), ptr(vc),
                               n_q, n_kvh, n_ctx, hd, pad, len(s), ptr(s), len(t), ptr(t), C.byref(skel_bc),
                               ptr(w), rbits, C.c_float(kq_scale), ptr(scores), ptr(out))
    return scores, out


def sqfree_attn_decode(q, kpack, vpack, n_kvh, n_ctx, hd, km, kbc, vbc, rbits, spinor, kq_scale,
                       want_scores=True, want_out=True):
    """spo_sqfree_attn_decode: kpack/vpack [n_kvh][n_ctx][B] uint8 (K with kbc, V with vbc)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    n_q = q.shape[0]
    scores = np.zeros((n_q, n_ctx), np.float32) if want_scores else None
    out = np.zeros((n_q, hd), np.float32) if want_out else None
    kc, vc = np.ascontiguousarray(kpack), np.ascontiguousarray(vpack)  # held across the call
    lib().spo_sqfree_attn_decode(ptr(q), ptr(kc), ptr(vc),
                                 n_q, n_kvh, n_ctx, hd, C.byref(km.m), C.byref(kbc), C.byref(vbc), rbits,
                                 int(spinor), C.c_float(kq_scale), ptr(scores), ptr(out))
    return scores, out


def correlation(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    b = np.ascontiguousarray(b, dtype=np.float32).ravel()
    return lib().spo_correlation_f32(ptr(a), ptr(b), a.size)


def tree256_sum(v, take_abs=False):
    v = np.ascontiguousarray(v, dtype=np.float32)
    return lib().spo_tree256_sum(ptr(v), v.size, int(take_abs))


# ---- individual stages of the sqfree / hier codecs ----

def spinor_extract(a, p):
    a = np.ascontiguousarray(a, np.float32)
    p = np.ascontiguousarray(p, np.float32)
    dev = np.zeros_like(a)
    sheet = np.zeros((len(a) + 7) // 8, np.uint8)
    lib().spo_spinor_extract(ptr(a), ptr(p), len(a), ptr(dev), ptr(sheet))
    return dev, sheet


def sqfree_residual_quantize(dev, bits):
    dev = np.ascontiguousarray(dev, np.float32)
    lv = np.zeros(len(dev), np.uint8)
    mag = lib().spo_sqfree_residual_quantize(ptr(dev), len(dev), bits, ptr(lv))
    return np.float32(mag), lv


def sqfree_residual_dequantize(lv, bits, mag):
    lv = np.ascontiguousarray(lv, np.uint8)
    out = np.zeros(len(lv), np.float32)
    lib().spo_sqfree_residual_dequantize(ptr(lv), len(lv), bits, C.c_float(mag), ptr(out))
    return out


def hier_residual_quantize(dev, bits):
    dev = np.ascontiguousarray(dev, np.float32)
    lv = np.zeros(len(dev), np.uint8)
    mag = lib().spo_hier_residual_quantize(ptr(dev), len(dev), bits, ptr(lv))
    return np.float32(mag), lv


def hier_residual_dequantize(lv, bits, mag):
    lv = np.ascontiguousarray(lv, np.uint8)
    out = np.zeros(len(lv), np.float32)
    lib().spo_hier_residual_dequantize(ptr(lv), len(lv), bits, C.c_float(mag), ptr(out))
    return out


def hier_predict(W16, skel):
    W16 = np.ascontiguousarray(W16, np.uint16)
    skel = np.ascontiguousarray(skel, np.float32)
    out = np.zeros(W16.shape[0], np.float32)
    lib().spo_hier_predict(ptr(W16), ptr(skel), ptr(out), W16.shape[0], W16.shape[1])
    return out


def mobius_predict(skel, km):
    skel = np.ascontiguousarray(skel, np.float32)
    out = np.zeros(max(km.n_res, 1), np.float32)
    lib().spo_mobius_predict(ptr(skel), C.byref(km.m), ptr(out))
    return out[:km.n_res]


def pack_levels(lv, bits):
    lv = np.ascontiguousarray(lv, np.uint8)
    out = np.zeros((len(lv) * bits + 7) // 8, np.uint8)
    lib().spo_pack_levels(ptr(lv), len(lv), bits, ptr(out))
    return out


def sqfree_pad(x, hd, pad):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(pad, np.float32)
    lib().spo_sqfree_pad(ptr(x), ptr(out), hd, pad)
    return out


def vilenkin(x):
    """Forward Vilenkin / VHT2 of one vector (the oracle's dispatch)."""
    return vht2(x)
