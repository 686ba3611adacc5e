"""ctypes binding of libshannon_prime_hip.so (the MI355X codec library).

Loads the in-tree library built by ``make -C shannon-prime-llama_amd``. There is
no fallback: if the library is missing or no gfx950 device is visible, the
calls that need the GPU raise.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libshannon_prime_hip.so")
INCLUDE_DIR = os.path.join(os.path.dirname(HERE), "include")

SP_MAX_BANDS = 16
DTYPE_F32 = 0
DTYPE_F16 = 1
NORM_FINAL = 0
NORM_STAGE = 1


class SpConfig(C.Structure):
    _fields_ = [
        ("head_dim", C.c_int), ("n_layers", C.c_int), ("n_heads_kv", C.c_int),
        ("k_n_bands", C.c_int), ("k_band_bits", C.c_int * SP_MAX_BANDS),
        ("v_n_bands", C.c_int), ("v_band_bits", C.c_int * SP_MAX_BANDS),
        ("use_mobius_mask", C.c_int), ("k_ternary_mask", C.c_uint32),
        ("v_ternary_mask", C.c_uint32), ("use_fp8", C.c_int), ("vht2_norm", C.c_int),
    ]


class SpBandConfig(C.Structure):
    _fields_ = [
        ("head_dim", C.c_int), ("n_bands", C.c_int), ("band_bits", C.c_int * SP_MAX_BANDS),
        ("band_size", C.c_int), ("total_bytes", C.c_int), ("ternary_mask", C.c_uint32),
    ]


class SpMobiusMask(C.Structure):
    _fields_ = [("n", C.c_int), ("order", C.POINTER(C.c_int))]


class SpShadowCache(C.Structure):
    _fields_ = [
        ("config", SpConfig), ("k_bands", SpBandConfig), ("v_bands", SpBandConfig),
        ("mobius_mask", SpMobiusMask), ("k_cache", C.POINTER(C.POINTER(C.c_uint8))),
        ("v_cache", C.POINTER(C.POINTER(C.c_uint8))), ("calibrating", C.c_int),
        ("calib_sum", C.POINTER(C.c_double)), ("calib_sum2", C.POINTER(C.c_double)),
        ("calib_n", C.c_longlong), ("var_order", C.POINTER(C.c_int)), ("use_var_reorder", C.c_int),
        ("dev", C.c_void_p),
    ]


class SpHipCache(C.Structure):
    _fields_ = [
        ("config", SpConfig), ("k_bands", SpBandConfig), ("v_bands", SpBandConfig),
        ("d_k_cache", C.c_void_p), ("d_v_cache", C.c_void_p), ("max_seq_len", C.c_int),
        ("d_mobius_order", C.c_void_p), ("d_mobius_inv", C.c_void_p),
        ("stream", C.c_void_p), ("priv", C.c_void_p),
    ]


class SpHipSqfreeCache(C.Structure):
    _fields_ = [
        ("config", SpConfig), ("pad_dim", C.c_int), ("sk_k", C.c_int), ("n_res", C.c_int),
        ("n_terms", C.c_int), ("residual_bits", C.c_int), ("use_spinor", C.c_int),
        ("k_bands", SpBandConfig), ("v_bands", SpBandConfig),
        ("d_skeleton_idx", C.c_void_p), ("d_residual_idx", C.c_void_p),
        ("d_csr_offsets", C.c_void_p), ("d_csr_skel_slot", C.c_void_p),
        ("d_csr_mu_sign", C.c_void_p), ("d_k_cache", C.c_void_p), ("d_v_cache", C.c_void_p),
        ("bytes_per_pos_k", C.c_int), ("bytes_per_pos_v", C.c_int), ("max_seq_len", C.c_int),
        ("n_slots", C.c_int), ("stream", C.c_void_p), ("priv", C.c_void_p),
    ]


class SpHipHierCache(C.Structure):
    _fields_ = [
        ("config", SpConfig), ("pad_dim", C.c_int), ("n_skeleton", C.c_int),
        ("n_target", C.c_int), ("target_res_bits", C.c_int), ("n_slots", C.c_int),
        ("max_seq_len", C.c_int), ("d_W", C.c_void_p), ("d_skeleton_idx", C.c_void_p),
        ("d_target_idx", C.c_void_p), ("skel_bands", SpBandConfig), ("d_k_cache", C.c_void_p),
        ("d_v_cache", C.c_void_p), ("bytes_per_pos_k", C.c_int), ("bytes_per_pos_v", C.c_int),
        ("stream", C.c_void_p), ("priv", C.c_void_p),
    ]


class SpHipDualCache(C.Structure):
    _fields_ = [("sys1", C.c_void_p), ("sys2", C.c_void_p), ("sys2_kind", C.c_int),
                ("entropy_threshold", C.c_float), ("max_seq_len", C.c_int), ("priv", C.c_void_p)]


DUAL_SQFREE, DUAL_HIER = 1, 2


class SpHipColdLayer(C.Structure):
    _fields_ = [("h_pinned", C.c_void_p), ("capacity", C.c_int64), ("packed_stride", C.c_int),
                ("n_heads", C.c_int), ("max_seq_len", C.c_int), ("cap_pos", C.c_int64), ("write_head", C.c_int64),
                ("oldest_pos", C.c_int64), ("newest_pos", C.c_int64), ("ring_mode", C.c_int),
                ("initialized", C.c_int)]


class SpLlamaParams(C.Structure):
    _fields_ = [
        ("head_dim", C.c_int), ("n_layers", C.c_int), ("n_heads_kv", C.c_int),
        ("max_seq_len", C.c_int), ("backend", C.c_int), ("gpu_context", C.c_void_p),
        ("arch_name", C.c_char_p),
    ]


class SpLlamaMemory(C.Structure):
    _fields_ = [("compressed_bytes", C.c_size_t), ("baseline_bytes", C.c_size_t),
                ("compression_ratio", C.c_float), ("n_positions", C.c_int)]


class SpKnightMask(C.Structure):
    _fields_ = [("pad_dim", C.c_int), ("sk_k", C.c_int), ("n_res", C.c_int), ("n_terms", C.c_int),
                ("skeleton_idx", C.POINTER(C.c_int)), ("residual_idx", C.POINTER(C.c_int)),
                ("csr_offsets", C.POINTER(C.c_int)), ("csr_skel_slot", C.POINTER(C.c_int)),
                ("csr_mu_sign", C.POINTER(C.c_int8))]


class SpSqfreeCache(C.Structure):
    """The core's sqfree cache on host vectors (sp_sqfree_cache_t)."""
    _fields_ = [("config", SpConfig), ("pad_dim", C.c_int), ("mask", SpKnightMask),
                ("k_bands", SpBandConfig), ("v_bands", SpBandConfig), ("residual_bits", C.c_int),
                ("use_spinor", C.c_int), ("max_seq_len", C.c_int), ("bytes_per_pos_k", C.c_int),
                ("bytes_per_pos_v", C.c_int), ("dev", C.c_void_p)]


class SpHierPredictor(C.Structure):
    _fields_ = [("pad_dim", C.c_int), ("n_skeleton", C.c_int), ("n_target", C.c_int),
                ("skeleton_idx", C.POINTER(C.c_int)), ("target_idx", C.POINTER(C.c_int)),
                ("skel_bands", SpBandConfig), ("target_res_bits", C.c_int), ("W", C.POINTER(C.c_uint16))]


class SpHierCache(C.Structure):
    """The core's hierarchical cache on host vectors (sp_hier_cache_t)."""
    _fields_ = [("config", SpConfig), ("pad_dim", C.c_int), ("n_slots", C.c_int), ("max_seq_len", C.c_int),
                ("level", C.c_int), ("predictors", C.POINTER(SpHierPredictor)), ("bytes_per_pos", C.c_int),
                ("dev", C.c_void_p)]


class SpLlamaSqfreeConfig(C.Structure):
    _fields_ = [("sqfree_enabled", C.c_int), ("spinor_enabled", C.c_int), ("residual_bits", C.c_int),
                ("sk_frac", C.c_float), ("k_band_bits", C.c_int * SP_MAX_BANDS), ("n_k_bands", C.c_int)]


BACKEND_CPU, BACKEND_CUDA, BACKEND_VULKAN, BACKEND_ADRENO, BACKEND_HEXAGON, BACKEND_HIP = range(6)
ROLE_DEFAULT, ROLE_TARGET, ROLE_DRAFT = range(3)

_lib = None


def lib():
    """Load the library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built: run `make -C {HERE}`")
        L = C.CDLL(LIB_PATH)
        vp, i, f, ll = C.c_void_p, C.c_int, C.c_float, C.c_longlong
        L.sp_hip_last_error.restype = C.c_char_p
        L.sp_hip_attn_noalloc_max_floats.restype = C.c_size_t
        L.sp_llama_sqfree_init.restype = vp
        L.sp_llama_sqfree_init.argtypes = [i, i, i, i]
        L.sp_llama_sqfree_free.argtypes = [vp]
        L.sp_llama_sqfree_write_kv.argtypes = [vp, i, i, i, vp, vp]
        L.sp_llama_sqfree_read_k.argtypes = [vp, i, i, i, vp]
        L.sp_llama_sqfree_read_v.argtypes = [vp, i, i, i, vp]
        L.sp_llama_sqfree_validate_k.argtypes = [vp, vp, i]
        L.sp_llama_sqfree_validate_k.restype = f
        L.sp_llama_sqfree_get_cache.argtypes = [vp]
        L.sp_llama_sqfree_get_cache.restype = C.POINTER(SpSqfreeCache)
        L.sp_hip_event_create.restype = vp
        L.sp_hip_event_elapsed_ms.restype = f
        L.sp_hip_event_elapsed_ms.argtypes = [vp, vp]
        L.sp_hip_event_record.argtypes = [vp, vp]
        L.sp_hip_event_destroy.argtypes = [vp]
        L.sp_hip_stream_sync.argtypes = [vp]
        L.sp_hip_ship_encode.argtypes = [vp, vp, i, vp, i, ll, ll, vp, ll, i, i, vp]
        L.sp_hip_ship_decode.argtypes = [vp, vp, i, i, vp, ll, vp, i, ll, ll, i, i, vp]
        L.sp_hip_ship_encode_generic.argtypes = L.sp_hip_ship_encode.argtypes
        L.sp_hip_ship_decode_generic.argtypes = L.sp_hip_ship_decode.argtypes
        L.sp_hip_write_layer.argtypes = [vp, i, i, i, vp, vp, ll, i]
        L.sp_hip_read_layer.argtypes = [vp, i, i, i, vp, vp, ll, i, i]
        L.sp_hip_write_all.argtypes = [vp, i, i, vp, vp, i]
        L.sp_hip_roundtrip_cells.argtypes = [vp, i, vp, i, vp, ll, vp, ll, ll, i, i, vp]
        L.sp_hip_calibrate_begin.argtypes = [vp]
        L.sp_hip_calibrate_feed.argtypes = [vp, vp, ll, i, i]
        L.sp_hip_calibrate_end.argtypes = [vp, vp, i]
        L.sp_hip_sqfree_calibrate_begin.argtypes = [vp]
        L.sp_hip_sqfree_calibrate_feed.argtypes = [vp, vp, ll, i, i]
        L.sp_hip_sqfree_calibrate_end.argtypes = [vp, vp, i]
        L.sp_hip_hier_calibrate_begin.argtypes = [vp]
        L.sp_hip_hier_calibrate_feed.argtypes = [vp, i, vp, ll, i, i]
        L.sp_hip_hier_calibrate_end.argtypes = [vp, C.c_double]
        L.sp_hip_hier_calibrate_end_ema.argtypes = [vp, C.c_double, C.c_float]
        L.sp_shadow_calibrate_begin.argtypes = [vp]
        L.sp_shadow_calibrate_feed.argtypes = [vp, vp]
        L.sp_shadow_calibrate_end.argtypes = [vp]
        L.sp_shadow_write_k_batch.argtypes = [vp, i, i, i, i, vp]
        L.sp_shadow_read_k_batch.argtypes = [vp, i, i, i, i, vp]
        L.sp_hip_read_all.argtypes = [vp, i, i, vp, vp, i, i]
        L.sp_hip_attn_decode.argtypes = [vp, i, i, vp, i, f, vp, vp, vp]
        L.sp_hip_attn_decode_bands.argtypes = [vp, i, i, vp, i, f, vp, vp, i, vp]
        u64, cp = C.c_uint64, C.c_char_p
        L.sp_fnv1a64.argtypes = [vp, C.c_size_t]
        L.sp_fnv1a64.restype = u64
        for name in ("sp_hip_cache_save", "sp_hip_sqfree_cache_save", "sp_hip_hier_cache_save"):
            getattr(L, name).argtypes = [vp, cp, i, u64]
        for name in ("sp_hip_cache_load", "sp_hip_sqfree_cache_load", "sp_hip_hier_cache_load"):
            getattr(L, name).argtypes = [vp, cp, u64]
        L.sp_hip_cache_load_partial.argtypes = [vp, cp, u64, i]
        L.sp_shadow_cache_save.argtypes = [vp, cp, i, u64]
        L.sp_shadow_cache_load.argtypes = [vp, cp, u64]
        L.sp_shadow_cache_load_partial.argtypes = [vp, cp, u64, i]
        L.sp_hip_memset.argtypes = [vp, i, C.c_size_t, vp]
        L.sp_hip_dual_init.argtypes = [vp, vp, i, vp, f]
        L.sp_hip_dual_free.argtypes = [vp]
        L.sp_hip_dual_route_position.argtypes = [vp, i, f]
        L.sp_hip_dual_owner_of.argtypes = [vp, i]
        L.sp_hip_dual_sys1_count.argtypes = [vp]
        L.sp_hip_dual_sys2_count.argtypes = [vp]
        L.sp_hip_dual_write_layer.argtypes = [vp, i, i, i, vp, vp, ll, i]
        L.sp_hip_dual_read_merged.argtypes = [vp, i, i, vp, vp, ll, i]
        L.sp_hip_attn_decode_all_layers.argtypes = [vp, i, vp, i, f, vp, vp]
        L.sp_hip_attn_scores_all_layers.argtypes = [vp, i, vp, i, f, vp, i, vp]
        L.sp_hip_attn_decode_f16.argtypes = [vp, vp, i, i, i, i, i, vp, i, f, vp, vp, vp]
        L.sp_hip_sqfree_write_batch.argtypes = [vp, i, i, i, i, i, vp, i]
        L.sp_hip_sqfree_read_batch.argtypes = [vp, i, i, i, i, i, vp, i]
        L.sp_hip_hier_write_batch.argtypes = [vp, i, i, i, i, i, vp, i]
        L.sp_hip_hier_read_batch.argtypes = [vp, i, i, i, i, i, vp, i]
        L.sp_hip_sqfree_write_layer.argtypes = [vp, i, i, i, vp, vp, ll, i]
        L.sp_hip_sqfree_read_layer.argtypes = [vp, i, i, i, vp, vp, ll, i]
        L.sp_hip_hier_write_layer.argtypes = [vp, i, i, i, vp, vp, ll, i]
        L.sp_hip_hier_read_layer.argtypes = [vp, i, i, i, vp, vp, ll, i]
        L.sp_hip_hier_attn_decode.argtypes = [vp, i, i, vp, i, f, vp, vp, vp]
        L.sp_hip_sqfree_attn_decode.argtypes = [vp, i, i, vp, i, f, vp, vp, vp]
        for name in ("sp_hip_attn_decode_seqs", "sp_hip_sqfree_attn_decode_seqs", "sp_hip_hier_attn_decode_seqs"):
            getattr(L, name).argtypes = [vp, i, i, vp, vp, vp, i, f, vp, vp, vp]
        L.sp_hip_vht2_forward.argtypes = [vp, i, i, i, vp]
        L.sp_hip_band_quantize.argtypes = [vp, vp, vp, i, vp]
        L.sp_hip_band_dequantize.argtypes = [vp, vp, vp, i, vp]
        L.sp_hip_mobius_reorder.argtypes = [vp, vp, i, i, vp]
        L.sp_hip_mobius_unreorder.argtypes = [vp, vp, i, i, vp]
        L.sp_llama_init.restype = vp
        L.sp_llama_init_with_role.restype = vp
        L.sp_llama_init_config.restype = vp
        L.sp_llama_free.argtypes = [vp]
        for n in ("sp_llama_write_k", "sp_llama_write_v"):
            getattr(L, n).argtypes = [vp, i, i, i, vp]
        for n in ("sp_llama_read_k", "sp_llama_read_v"):
            getattr(L, n).argtypes = [vp, i, i, i, vp]
        for n in ("sp_llama_read_k_partial", "sp_llama_read_v_partial"):
            getattr(L, n).argtypes = [vp, i, i, i, vp, i]
        for n in ("sp_llama_write_k_batch", "sp_llama_write_v_batch", "sp_llama_read_k_batch",
                  "sp_llama_read_v_batch"):
            getattr(L, n).argtypes = [vp, i, i, i, i, vp]
        L.sp_llama_write_kv.argtypes = [vp, i, i, i, vp, vp]
        L.sp_llama_memory.restype = SpLlamaMemory
        L.sp_llama_memory.argtypes = [vp]
        L.sp_llama_validate_k.restype = f
        L.sp_llama_validate_k.argtypes = [vp, vp, i]
        L.sp_llama_clear_range.argtypes = [vp, i, i]
        L.sp_llama_get_backend.argtypes = [vp]
        for n in ("sp_llama_get_k_buf", "sp_llama_get_v_buf", "sp_llama_get_hexagon_k_buf"):
            getattr(L, n).restype = vp
            getattr(L, n).argtypes = [vp, i, i]
        L.sp_llama_get_hip_cache.restype = vp
        L.sp_llama_get_hip_cache.argtypes = [vp]
        L.sp_llama_get_k_total_bytes.argtypes = [vp]
        L.sp_llama_get_v_total_bytes.argtypes = [vp]
        L.sp_llama_get_freq_factors.restype = vp
        L.sp_llama_get_freq_factors.argtypes = [vp]
        L.sp_llama_get_n_freqs.argtypes = [vp]
        L.sp_correlation_f32.restype = f
        L.sp_compression_ratio.restype = f
        L.sp_f16_to_f32.restype = f
        L.sp_f32_to_f16.restype = C.c_uint16
        L.sp_f32_to_f16.argtypes = [f]
        _lib = L
    return _lib


def last_error():
    return lib().sp_hip_last_error().decode()


def check(rc, what="call"):
    if rc != 0:
        raise RuntimeError(f"{what} failed: {last_error()}")


def config(head_dim, n_layers=1, n_heads_kv=1, k_bits=(5, 5, 4, 3), v_bits=(3,), mobius=True,
           norm=NORM_FINAL, k_ternary=0, v_ternary=0):
    cfg = SpConfig()
    lib().sp_config_init(C.byref(cfg), head_dim, n_layers, n_heads_kv)
    cfg.k_n_bands = len(k_bits)
    for j, b in enumerate(k_bits):
        cfg.k_band_bits[j] = b
    cfg.v_n_bands = len(v_bits)
    for j, b in enumerate(v_bits):
        cfg.v_band_bits[j] = b
    cfg.use_mobius_mask = int(mobius)
    cfg.vht2_norm = norm
    cfg.k_ternary_mask = k_ternary
    cfg.v_ternary_mask = v_ternary
    return cfg


def band_config(hd, bits, ternary_mask=0):
    bc = SpBandConfig()
    arr = (C.c_int * SP_MAX_BANDS)(*bits)
    lib().sp_band_config_init_ext(C.byref(bc), hd, len(bits), arr, C.c_uint32(ternary_mask))
    return bc


class ShipCache:
    """sp_hip_cache_t owner (device-resident ship cache)."""

    def __init__(self, cfg, max_seq, stream=0):
        self.c = SpHipCache()
        check(lib().sp_hip_cache_init(C.byref(self.c), C.byref(cfg), max_seq, C.c_void_p(stream)),
              "sp_hip_cache_init")
        self.ref = C.byref(self.c)

    def free(self):
        if self.c.priv:
            lib().sp_hip_cache_free(self.ref)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class SqfreeCache:
    def __init__(self, cfg, max_seq, rbits=3, spinor=True, sk_k=0, stream=0):
        self.c = SpHipSqfreeCache()
        check(lib().sp_hip_sqfree_cache_init_ex(C.byref(self.c), C.byref(cfg), max_seq, rbits,
                                                int(spinor), sk_k, C.c_void_p(stream)),
              "sp_hip_sqfree_cache_init_ex")
        self.ref = C.byref(self.c)

    def free(self):
        if self.c.priv:
            lib().sp_hip_sqfree_cache_free(self.ref)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HierCache:
    def __init__(self, cfg, pad, skel_idx, target_idx, skel_bc, rbits, max_seq, n_slots, stream=0):
        import numpy as np
        self.c = SpHipHierCache()
        s = np.ascontiguousarray(skel_idx, dtype=np.int32)
        t = np.ascontiguousarray(target_idx, dtype=np.int32)
        check(lib().sp_hip_hier_cache_init(C.byref(self.c), C.byref(cfg), pad, len(s), len(t), rbits,
                                           s.ctypes.data_as(C.c_void_p), t.ctypes.data_as(C.c_void_p),
                                           C.byref(skel_bc), max_seq, n_slots, C.c_void_p(stream)),
              "sp_hip_hier_cache_init")
        self.ref = C.byref(self.c)

    def upload_W(self, W_u16):
        import numpy as np
        W = np.ascontiguousarray(W_u16, dtype=np.uint16)
        check(lib().sp_hip_hier_cache_upload_W(self.ref, W.ctypes.data_as(C.c_void_p)), "upload_W")

    def free(self):
        if self.c.priv:
            lib().sp_hip_hier_cache_free(self.ref)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DualCache:
    """sp_hip_dual_cache_t over a ship cache and a sqfree or hier cache (both stay
    owned by the caller)."""

    def __init__(self, sys1, sys2, kind, threshold):
        self.c = SpHipDualCache()
        self.sys1, self.sys2 = sys1, sys2  # keep the caches alive
        check(lib().sp_hip_dual_init(C.byref(self.c), sys1.ref, kind, sys2.ref, C.c_float(threshold)),
              "sp_hip_dual_init")
        self.ref = C.byref(self.c)

    def free(self):
        if self.c.priv:
            lib().sp_hip_dual_free(self.ref)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def header_symbols():
    """Every function name declared in include/*.h (for the export check)."""
    import re
    names = set()
    for fn in sorted(os.listdir(INCLUDE_DIR)):
        if not fn.endswith(".h"):
            continue
        txt = open(os.path.join(INCLUDE_DIR, fn)).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        txt = re.sub(r"//[^\n]*", "", txt)
        for m in re.finditer(r"\b(sp_\w+)\s*\(", txt):
            pre = txt[max(0, m.start() - 80):m.start()]
            if "#define" in pre.split("\n")[-1]:
                continue
            names.add(m.group(1))
    return sorted(names)
