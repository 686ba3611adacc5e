"""C-ABI library: loads, exports every declared symbol, host-side logic agrees with the
oracle (CPU only, no compute calls on a GPU)."""
import ctypes as C
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle_py as O
import sp_hip as S


def test_library_exports_every_declared_symbol():
    L = S.lib()
    names = S.header_symbols()
    assert len(names) > 80
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_headers_compile_as_c_and_cpp(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "shannon_prime.h"\n#include "sp_hip.h"\n#include "shannon_prime_llama.h"\n'
                   "int main(void){sp_config_t c; sp_config_init(&c,128,1,1); return c.k_n_bands==4?0:1;}\n")
    for comp, ext in (("gcc", "c"), ("g++", "cpp")):
        f = tmp_path / f"t.{ext}"
        f.write_text(src.read_text())
        r = subprocess.run([comp, "-fsyntax-only", "-Wall", "-Werror", "-I", S.INCLUDE_DIR, str(f)],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("hd,bits,tmask", [(128, [5, 5, 4, 3], 0), (128, [3], 0), (64, [5, 4, 4], 0),
                                           (96, [5, 4, 4], 0), (128, [5, 5, 4, 3], 8),
                                           (77, [5, 4, 4, 4, 5], 0), (128, [5] * 10, 0)])
def test_band_geometry_matches_oracle(hd, bits, tmask):
    a = S.band_config(hd, bits, tmask)
    b = O.band_config(hd, bits, tmask)
    assert (a.total_bytes, a.band_size, a.n_bands) == (b.total_bytes, b.band_size, b.n_bands)
    assert list(a.band_bits)[:len(bits)] == list(b.band_bits)[:len(bits)]
    for band in range(len(bits)):
        off, sz = C.c_int(), C.c_int()
        S.lib().sp_band_span(C.byref(a), band, C.byref(off), C.byref(sz))
        assert (off.value, sz.value) == (b.band_off[band], b.band_sz[band])


@pytest.mark.parametrize("n", [64, 96, 128, 154, 256, 330])
def test_mobius_table_matches_oracle(n):
    m = S.SpMobiusMask()
    assert S.lib().sp_mobius_mask_init(C.byref(m), n) == 0
    got = np.ctypeslib.as_array(m.order, (n,)).copy()
    S.lib().sp_mobius_mask_free(C.byref(m))
    np.testing.assert_array_equal(got, O.mobius_order(n))


def test_sqfree_pad_dims():
    for hd in (64, 96, 128, 256, 100, 200):
        assert S.lib().sp_sqfree_pad_dim(hd) == O.sqfree_pad_dim(hd)
    assert [S.lib().sp_sqfree_pad_dim(h) for h in (64, 128, 256, 96)] == [66, 154, 330, 105]


def test_hier_default_geometry_matches_oracle():
    for pad in (66, 154, 330, 105):
        n_skel = S.lib().sp_hier_default_geometry(pad, None, None)
        sk = np.zeros(n_skel, np.int32)
        tg = np.zeros(pad - n_skel, np.int32)
        assert S.lib().sp_hier_default_geometry(pad, C.c_void_p(sk.ctypes.data), C.c_void_p(tg.ctypes.data)) == n_skel
        osk, otg = O.hier_geometry(pad)
        np.testing.assert_array_equal(sk, osk)
        np.testing.assert_array_equal(tg, otg)
    assert S.lib().sp_hier_default_geometry(330, None, None) == 30  # cfg 5: 30 skeleton, 300 targets
    assert S.lib().sp_hier_default_geometry(0, None, None) == -1


def test_host_fp16_helpers_match_oracle():
    rng = np.random.default_rng(1)
    vals = rng.standard_normal(2000).astype(np.float32) * 10.0 ** rng.integers(-8, 6, 2000)
    for v in vals:
        assert S.lib().sp_f32_to_f16(float(v)) == O.f32_to_f16_bits(float(v))


def test_compression_ratio():
    cfg = S.config(128)
    assert abs(S.lib().sp_compression_ratio(C.byref(cfg)) - 512 / 126) < 1e-5


def test_bridge_disabled_returns_null(monkeypatch):
    monkeypatch.delenv("SHANNON_PRIME_ENABLED", raising=False)
    p = S.SpLlamaParams(128, 2, 2, 16, S.BACKEND_CPU, None, None)
    assert not S.lib().sp_llama_init(C.byref(p))
    monkeypatch.setenv("SHANNON_PRIME_ENABLED", "1")
    monkeypatch.setenv("SHANNON_PRIME_DRAFT_ENABLED", "0")
    assert not S.lib().sp_llama_init_with_role(C.byref(p), 2)


def test_bridge_null_safety():
    L = S.lib()
    L.sp_llama_free(None)
    assert L.sp_llama_get_backend(None) == -1
    assert not L.sp_llama_get_k_buf(None, 0, 0)
    assert L.sp_llama_get_n_freqs(None) == 0
    mem = L.sp_llama_memory(None)
    assert mem.compressed_bytes == 0


@pytest.mark.skipif(os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK),
                    reason="GPU visible: the no-GPU failure path does not apply")
def test_init_fails_loudly_without_gpu():
    cfg = S.config(128, 1, 1)
    c = S.SpHipCache()
    assert S.lib().sp_hip_cache_init(C.byref(c), C.byref(cfg), 16, None) == -1
    assert "gfx950" in S.last_error() or S.last_error()
    sc = S.SpShadowCache()
    assert S.lib().sp_shadow_cache_init(C.byref(sc), C.byref(cfg)) == -1


def test_fnv1a64_known_answers():
    """sp_fnv1a64 (the disk files' model hash and header check) against the published
    FNV-1a 64-bit test vectors (offset basis 0xcbf29ce484222325, prime 0x100000001b3)."""
    L = S.lib()
    for msg, want in ((b"", 0xcbf29ce484222325), (b"a", 0xaf63dc4c8601ec8c), (b"foobar", 0x85944171f73967e8)):
        assert L.sp_fnv1a64(msg, len(msg)) == want, msg


def test_cpp_kv_cache_header_compiles():
    """include/sp_kv_cache.hpp (the C++ KvCache mirror) is self-contained C++17."""
    inc = os.path.join(os.path.dirname(__file__), "..", "include")
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-fsyntax-only", "-x", "c++", "-I", inc,
                        "-"], input='#include "sp_kv_cache.hpp"\n', capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


class _Knight(C.Structure):
    _fields_ = [("pad_dim", C.c_int), ("sk_k", C.c_int), ("n_res", C.c_int), ("n_terms", C.c_int),
                ("skeleton_idx", C.POINTER(C.c_int)), ("residual_idx", C.POINTER(C.c_int)),
                ("csr_offsets", C.POINTER(C.c_int)), ("csr_skel_slot", C.POINTER(C.c_int)),
                ("csr_mu_sign", C.POINTER(C.c_int8))]


@pytest.mark.parametrize("pad,sk", [(154, 77), (154, 115), (330, 165), (66, 1)])
def test_knight_mask_matches_oracle(pad, sk):
    """sp_knight_mask_init (host tables, no GPU) equals the oracle's Knight tables."""
    L = S.lib()
    m = _Knight()
    assert L.sp_knight_mask_init(C.byref(m), pad, sk, None) == 0
    ref = O.Knight(pad, sk)
    assert (m.pad_dim, m.sk_k, m.n_res, m.n_terms) == (pad, sk, ref.n_res, ref.n_terms)
    np.testing.assert_array_equal(np.ctypeslib.as_array(m.skeleton_idx, (sk,)), ref.skeleton_idx)
    np.testing.assert_array_equal(np.ctypeslib.as_array(m.residual_idx, (m.n_res,)), ref.residual_idx)
    np.testing.assert_array_equal(np.ctypeslib.as_array(m.csr_offsets, (m.n_res + 1,)), ref.csr_offsets)
    if m.n_terms:
        np.testing.assert_array_equal(np.ctypeslib.as_array(m.csr_skel_slot, (m.n_terms,)), ref.csr_skel_slot)
        np.testing.assert_array_equal(np.ctypeslib.as_array(m.csr_mu_sign, (m.n_terms,)), ref.csr_mu_sign)
    L.sp_knight_mask_free(C.byref(m))
    assert L.sp_knight_mask_init(C.byref(m), pad, pad + 1, None) == -1


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus 2 exits with status 2 and says so, before any GPU work."""
    root = os.path.join(os.path.dirname(__file__), "..")
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=root)
    assert r.returncode == 2, (r.returncode, r.stderr[-500:])
    assert "one GPU" in r.stderr
