"""The shannon_prime_llama bridge (src/tools/shannon_prime_llama.h:97-341) on the GPU:
host fp32 vectors in and out through the CPU (shadow cache) and HIP backends, checked
against the oracle's compress -> decompress of the same vectors (bit-exact), plus
partial-band reads, clear_range and the memory report."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import oracle_py as O  # noqa: E402
import sp_hip as S  # noqa: E402
import workloads as W  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def fptr(a):
    return C.c_void_p(a.ctypes.data)


@pytest.fixture
def bridge_env(monkeypatch):
    def make(backend):
        monkeypatch.setenv("SHANNON_PRIME_ENABLED", "1")
        monkeypatch.setenv("SHANNON_PRIME_BACKEND", backend)
        for v in ("SHANNON_PRIME_K_BITS", "SHANNON_PRIME_V_BITS", "SHANNON_PRIME_MOBIUS",
                  "SHANNON_PRIME_TERNARY_BANDS", "SHANNON_PRIME_VHT2_NORM"):
            monkeypatch.delenv(v, raising=False)
    return make


@pytest.mark.parametrize("backend", ["hip", "cpu"])
def test_bridge_roundtrip_matches_oracle(backend, bridge_env):
    say(f"bridge backend={backend}")
    bridge_env(backend)
    hd, n_layers, H, max_seq, n = 128, 2, 2, 96, 40
    torch.cuda.synchronize()
    p = S.SpLlamaParams(hd, n_layers, H, max_seq, S.BACKEND_HIP if backend == "hip" else S.BACKEND_CPU, None, None)
    L = S.lib()
    ctx = L.sp_llama_init(C.byref(p))
    assert ctx, S.last_error()
    try:
        k16, v16 = W.cfg2_kv(n_heads=H, n_pos=n, hd=hd, seed=11)
        kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
        order = O.mobius_order(hd)
        for h in range(H):
            k = np.ascontiguousarray(k16[h].astype(np.float32))
            v = np.ascontiguousarray(v16[h].astype(np.float32))
            # batch write of the first n-1 positions, single-vector write of the last
            L.sp_llama_write_k_batch(ctx, 1, h, 0, n - 1, fptr(k))
            L.sp_llama_write_v_batch(ctx, 1, h, 0, n - 1, fptr(v))
            L.sp_llama_write_k(ctx, 1, h, n - 1, fptr(k[n - 1]))
            L.sp_llama_write_v(ctx, 1, h, n - 1, fptr(v[n - 1]))
            kref = O.ship_decompress_f32(O.ship_compress_f32(k, kbc, order), kbc, order)
            vref = O.ship_decompress_f32(O.ship_compress_f32(v, vbc), vbc)
            kout = np.empty_like(k)
            vout = np.empty_like(v)
            L.sp_llama_read_k_batch(ctx, 1, h, 0, n, fptr(kout))
            L.sp_llama_read_v_batch(ctx, 1, h, 0, n, fptr(vout))
            np.testing.assert_array_equal(kout.view(np.uint32), kref.view(np.uint32))
            np.testing.assert_array_equal(vout.view(np.uint32), vref.view(np.uint32))
            one = np.empty(hd, np.float32)
            L.sp_llama_read_k(ctx, 1, h, 7, fptr(one))
            np.testing.assert_array_equal(one.view(np.uint32), kref[7].view(np.uint32))
            for mb in (0, 2):
                L.sp_llama_read_k_partial(ctx, 1, h, 5, fptr(one), mb)
                part = O.ship_decompress_f32(O.ship_compress_f32(k[5:6], kbc, order), kbc, order, max_bands=mb)[0]
                np.testing.assert_array_equal(one.view(np.uint32), part.view(np.uint32))
        mem = L.sp_llama_memory(ctx)
        assert mem.compressed_bytes > 0 and mem.baseline_bytes > mem.compressed_bytes
        # clear_range zeroes the records: a cleared vector reads back as zeros
        L.sp_llama_clear_range(ctx, 0, 8)
        z = np.ones(hd, np.float32)
        L.sp_llama_read_k(ctx, 1, 0, 3, fptr(z))
        assert not z.any()
    finally:
        L.sp_llama_free(ctx)


def test_hip_backend_exposes_device_cache(bridge_env):
    bridge_env("hip")
    p = S.SpLlamaParams(128, 1, 2, 16, S.BACKEND_HIP, None, None)
    L = S.lib()
    ctx = L.sp_llama_init(C.byref(p))
    assert ctx, S.last_error()
    try:
        assert L.sp_llama_get_backend(ctx) == S.BACKEND_HIP
        assert L.sp_llama_get_hip_cache(ctx)
        assert L.sp_llama_get_k_buf(ctx, 0, 1)
        assert L.sp_llama_get_k_total_bytes(ctx) == 76 and L.sp_llama_get_v_total_bytes(ctx) == 50
    finally:
        L.sp_llama_free(ctx)
