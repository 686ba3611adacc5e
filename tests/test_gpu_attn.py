"""Fused decompress-attention decode vs the oracle (scores and softmax.V within 1e-3
relative in fp32), GQA grouping, split boundaries, and the fp16 baseline kernel."""
import ctypes as C
import functools
import math
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import oracle_py as O  # noqa: E402
import sp_hip as S  # noqa: E402
import workloads as W  # noqa: E402
from gpu_util import d2h, dev, empty_f32, host, p, stream  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel_close(got, ref, tol=1e-3, floor=1e-2):
    """Elementwise relative bound |got - ref| <= tol * max(|ref|, floor * max|ref|):
    every entry of at least 1% of the array's largest magnitude is within `tol`
    of itself; smaller entries (scores near zero, where a relative bound has no
    meaning) are held to tol * 1% of the largest."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    bound = tol * np.maximum(np.abs(ref), floor * np.abs(ref).max())
    err = np.abs(got - ref)
    if not (bound > 0).any():  # an all-zero reference: the result must be exactly zero
        np.testing.assert_array_equal(got, ref)
        return
    ratio = np.divide(err, bound, out=np.where(err > 0, np.inf, 0.0), where=bound > 0)
    worst = int(np.argmax(ratio))
    assert np.all(err <= bound), ("elementwise", worst, got.ravel()[worst], ref.ravel()[worst],
                                  float(ratio.max()))


ATTN_CASES = [
    (8, 2, 300, 128, True),      # GQA 4, a partial second split, odd max_seq (V tiles 2-byte aligned)
    (32, 8, 1024, 128, True),    # Llama-3-8B head layout
    (4, 4, 256, 128, False),     # MHA, exactly one split, no Mobius
    (16, 2, 4099, 128, True),    # GQA 8, 17 splits, a 3-position last tile
    (3, 3, 1, 128, True),        # a single position
    (16, 8, 777, 256, True),     # Gemma-3 head_dim (general kernel)
    (8, 8, 129, 64, True),       # general kernel
    (12, 4, 700, 128, True),     # GQA 3: one unused head column of the score matrix cores
    (20, 4, 333, 128, True),     # GQA 5: a second column set, three of its heads unused
]


def general_kernel_only(monkeypatch):
    """Route decode attention to the general kernel (sp_attn.hip's split kernel)."""
    monkeypatch.setenv("SP_HIP_NO_MFMA_ATTN", "1")
    monkeypatch.setenv("SP_HIP_NO_LANE_ATTN", "1")


@pytest.mark.parametrize("path", ["default", "general"])
@pytest.mark.parametrize("n_q,H,n_ctx,hd,mob", ATTN_CASES)
def test_fused_attention_matches_oracle(n_q, H, n_ctx, hd, mob, path, monkeypatch):
    """The default launch runs the matrix-core kernel at hd 128 (K 5/5/4/3, V 3-bit),
    the one-position-per-lane kernel at hd 64 and the general kernel at hd 256;
    path "general" forces the general kernel everywhere. All meet 1e-3."""
    if path == "general":
        general_kernel_only(monkeypatch)
    elif hd == 256:
        pytest.skip("the default launch at head_dim 256 is the general kernel (path general)")
    say(f"attn path={path} n_q={n_q} H={H} n_ctx={n_ctx} hd={hd} mob={mob}")
    k16, v16 = W.cfg2_kv(n_heads=H, n_pos=n_ctx, hd=hd, seed=n_ctx)
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_ctx, seed=n_ctx + 1)
    cfg = S.config(hd, 2, H, mobius=mob)
    cc = S.ShipCache(cfg, n_ctx + 5, stream=torch.cuda.current_stream().cuda_stream)
    layer = 1
    for h in range(H):
        kt, vt = dev(k16[h].view(np.uint16)), dev(v16[h].view(np.uint16))
        S.lib().sp_hip_write_k_batch_f16(cc.ref, layer, h, 0, n_ctx, p(kt))
        S.lib().sp_hip_write_v_batch_f16(cc.ref, layer, h, 0, n_ctx, p(vt))
    torch.cuda.synchronize()
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    order = O.mobius_order(hd) if mob else None
    kref = np.stack([O.ship_compress_f16(k16[h].view(np.uint16), kbc, order) for h in range(H)])
    vref = np.stack([O.ship_compress_f16(v16[h].view(np.uint16), vbc) for h in range(H)])
    scale = 1.0 / math.sqrt(hd)
    s_ref, o_ref = O.attn_decode(q, kref, vref, H, n_ctx, kbc, vbc, order, scale)
    qt = dev(q)
    sc, out = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
    S.check(S.lib().sp_hip_attn_decode(cc.ref, layer, n_ctx, p(qt), n_q, C.c_float(scale), p(sc), p(out),
                                       stream()))
    rel_close(host(sc).reshape(n_q, n_ctx), s_ref)
    rel_close(host(out).reshape(n_q, hd), o_ref)
    # scores-only mode (the reference op's output) and output-only mode agree
    sc2, out2 = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
    S.check(S.lib().sp_hip_attn_decode(cc.ref, layer, n_ctx, p(qt), n_q, C.c_float(scale), p(sc2), None, stream()))
    S.check(S.lib().sp_hip_attn_decode(cc.ref, layer, n_ctx, p(qt), n_q, C.c_float(scale), None, p(out2), stream()))
    np.testing.assert_array_equal(host(sc2), host(sc))
    np.testing.assert_array_equal(host(out2), host(out))
    cc.free()


@pytest.mark.parametrize("path", ["default", "general"])
@pytest.mark.parametrize("n_q,H,n_ctx,k_bits,v_bits,runs", [
    (32, 32, 300, (5, 4, 4), (5,), 0),      # configs[2] (Phi-3-mini, MHA) at the bridge's hd-96 bands
    (32, 32, 4096, (5, 4, 4), (5,), 0),     # configs[2]'s per-sequence shape: 64 tiles per head
    (16, 4, 3000, (5, 4, 4), (5,), 3),      # GQA 4, runs of 15-16 tiles, a ragged last tile
    (24, 8, 777, (5, 4, 4), (5,), 0),       # GQA 3
    (16, 4, 1037, (5, 5, 4, 3), (3,), 0),   # the shipping bands at hd 96, GQA 4 (general kernel only)
])
def test_hd96_attention_matches_oracle(n_q, H, n_ctx, k_bits, v_bits, runs, path, monkeypatch):
    """head_dim 96 (Vilenkin 2^5 * 3): the bridge's bands (K 5/4/4 + Mobius, V 5) run
    the one-position-per-lane kernel by default, other bands the general kernel;
    scores and output within 1e-3 of the oracle, several splits or runs and a ragged
    last tile."""
    hd = 96
    if path == "general":
        general_kernel_only(monkeypatch)
    if runs:
        monkeypatch.setenv("SP_HIP_ATTN_LANE_RUNS", str(runs))
    say(f"attn hd96 path={path} n_q={n_q} H={H} n_ctx={n_ctx} k={k_bits} v={v_bits}")
    k16, v16 = W.cfg3_kv(n_heads=H, n_pos=n_ctx, hd=hd, seed=n_ctx)
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_ctx, seed=n_ctx + 1)
    cfg = S.config(hd, 1, H, k_bits=k_bits, v_bits=v_bits)
    cc = S.ShipCache(cfg, n_ctx, stream=torch.cuda.current_stream().cuda_stream)
    for h in range(H):
        kt, vt = dev(k16[h].view(np.uint16)), dev(v16[h].view(np.uint16))
        S.lib().sp_hip_write_k_batch_f16(cc.ref, 0, h, 0, n_ctx, p(kt))
        S.lib().sp_hip_write_v_batch_f16(cc.ref, 0, h, 0, n_ctx, p(vt))
    torch.cuda.synchronize()
    kbc, vbc = O.band_config(hd, list(k_bits)), O.band_config(hd, list(v_bits))
    order = O.mobius_order(hd)
    kref = np.stack([O.ship_compress_f16(k16[h].view(np.uint16), kbc, order) for h in range(H)])
    vref = np.stack([O.ship_compress_f16(v16[h].view(np.uint16), vbc) for h in range(H)])
    scale = 1.0 / math.sqrt(hd)
    s_ref, o_ref = O.attn_decode(q, kref, vref, H, n_ctx, kbc, vbc, order, scale)
    qt = dev(q)
    sc, out = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
    S.check(S.lib().sp_hip_attn_decode(cc.ref, 0, n_ctx, p(qt), n_q, C.c_float(scale), p(sc), p(out), stream()))
    torch.cuda.synchronize()
    rel_close(host(sc).reshape(n_q, n_ctx), s_ref)
    rel_close(host(out).reshape(n_q, hd), o_ref)
    # band limits: K and V bands >= max_bands read as 0
    for mb in (2, 1):
        s_b, o_b = O.attn_decode(q, kref, vref, H, n_ctx, kbc, vbc, order, scale, max_bands=mb)
        sc, out = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
        S.check(S.lib().sp_hip_attn_decode_bands(cc.ref, 0, n_ctx, p(qt), n_q, C.c_float(scale), p(sc), p(out), mb,
                                                 stream()))
        rel_close(host(sc).reshape(n_q, n_ctx), s_b)
        rel_close(host(out).reshape(n_q, hd), o_b)
    cc.free()


@pytest.mark.parametrize("path", ["mfma", "general"])
@pytest.mark.parametrize("n_q,H,n_ctx", [(8, 2, 300), (32, 8, 1100)])
def test_band_limited_attention_matches_oracle(n_q, H, n_ctx, path, monkeypatch):
    """sp_hip_attn_decode_bands for every band limit 0..4 and -1 against the oracle
    over the partial reconstructions (1e-3); a limit of 4 or -1 equals the full call
    bit for bit."""
    if path == "general":
        general_kernel_only(monkeypatch)
    hd = 128
    k16, v16 = W.cfg2_kv(n_heads=H, n_pos=n_ctx, hd=hd, seed=n_ctx + 3)
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_ctx, seed=n_ctx + 4)
    cfg = S.config(hd, 1, H)
    cc = S.ShipCache(cfg, n_ctx, stream=torch.cuda.current_stream().cuda_stream)
    L = S.lib()
    for h in range(H):
        kt, vt = dev(k16[h].view(np.uint16)), dev(v16[h].view(np.uint16))
        L.sp_hip_write_k_batch_f16(cc.ref, 0, h, 0, n_ctx, p(kt))
        L.sp_hip_write_v_batch_f16(cc.ref, 0, h, 0, n_ctx, p(vt))
    torch.cuda.synchronize()
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    order = O.mobius_order(hd)
    kref = np.stack([O.ship_compress_f16(k16[h].view(np.uint16), kbc, order) for h in range(H)])
    vref = np.stack([O.ship_compress_f16(v16[h].view(np.uint16), vbc) for h in range(H)])
    scale = 1.0 / math.sqrt(hd)
    qt = dev(q)
    sc_full, out_full = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
    S.check(L.sp_hip_attn_decode(cc.ref, 0, n_ctx, p(qt), n_q, C.c_float(scale), p(sc_full), p(out_full), stream()))
    for mb in (0, 1, 2, 3, 4, -1):
        say(f"attn bands path={path} n_q={n_q} H={H} n_ctx={n_ctx} max_bands={mb}")
        sc, out = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
        S.check(L.sp_hip_attn_decode_bands(cc.ref, 0, n_ctx, p(qt), n_q, C.c_float(scale), p(sc), p(out), mb,
                                           stream()))
        if mb in (4, -1):
            np.testing.assert_array_equal(host(sc), host(sc_full))
            np.testing.assert_array_equal(host(out), host(out_full))
            continue
        s_ref, o_ref = O.attn_decode(q, kref, vref, H, n_ctx, kbc, vbc, order, scale, max_bands=mb)
        rel_close(host(sc).reshape(n_q, n_ctx), s_ref)
        rel_close(host(out).reshape(n_q, hd), o_ref)
    cc.free()


@pytest.mark.parametrize("hd,k_bits,v_bits,n_q,H,n_ctx", [
    (96, (5, 4, 4), (5,), 8, 2, 700),        # configs[2]'s bands: the lane kernel's three K bands
    (64, (5, 5, 4, 3), (3,), 12, 4, 333),    # hd 64 shipping bands, GQA 3
])
def test_lane_band_limited_attention_matches_oracle(hd, k_bits, v_bits, n_q, H, n_ctx):
    """The one-position-per-lane kernel's band limits (sp_hip_attn_decode_bands): K bands
    past the limit, and V when the limit is 0, read as 0, against the oracle over the
    partial reconstructions (1e-3); the full band count and -1 equal the full call."""
    k16, v16 = W.cfg3_kv(n_heads=H, n_pos=n_ctx, hd=hd, seed=n_ctx + 5)
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_ctx, seed=n_ctx + 6)
    cc = S.ShipCache(S.config(hd, 1, H, k_bits=k_bits, v_bits=v_bits), n_ctx + 1,
                     stream=torch.cuda.current_stream().cuda_stream)
    L = S.lib()
    for h in range(H):
        kt, vt = dev(k16[h].view(np.uint16)), dev(v16[h].view(np.uint16))
        S.check(L.sp_hip_write_k_batch_f16(cc.ref, 0, h, 0, n_ctx, p(kt)))
        S.check(L.sp_hip_write_v_batch_f16(cc.ref, 0, h, 0, n_ctx, p(vt)))
    kbc, vbc = O.band_config(hd, list(k_bits)), O.band_config(hd, list(v_bits))
    order = O.mobius_order(hd)
    kref = np.stack([O.ship_compress_f16(k16[h].view(np.uint16), kbc, order) for h in range(H)])
    vref = np.stack([O.ship_compress_f16(v16[h].view(np.uint16), vbc) for h in range(H)])
    scale = 1.0 / math.sqrt(hd)
    qt = dev(q)
    sc_full, out_full = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
    S.check(L.sp_hip_attn_decode(cc.ref, 0, n_ctx, p(qt), n_q, C.c_float(scale), p(sc_full), p(out_full), stream()))
    nb = len(k_bits)
    for mb in list(range(nb)) + [nb, -1]:
        say(f"lane attn bands hd={hd} n_q={n_q} H={H} n_ctx={n_ctx} max_bands={mb}")
        sc, out = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
        S.check(L.sp_hip_attn_decode_bands(cc.ref, 0, n_ctx, p(qt), n_q, C.c_float(scale), p(sc), p(out), mb,
                                           stream()))
        if mb in (nb, -1):
            np.testing.assert_array_equal(host(sc), host(sc_full))
            np.testing.assert_array_equal(host(out), host(out_full))
            continue
        s_ref, o_ref = O.attn_decode(q, kref, vref, H, n_ctx, kbc, vbc, order, scale, max_bands=mb)
        rel_close(host(sc).reshape(n_q, n_ctx), s_ref)
        rel_close(host(out).reshape(n_q, hd), o_ref)
    cc.free()


# The shapes the bench times. The matrix-core kernel (k_attn_wave) gives each wave
# one 64-position tile while the context fits one round of 16-wave blocks (one per
# CU): 8 KV heads at 32768 positions are 4096 tiles on 256 blocks, one tile per wave,
# and a layer is one launch whose last block per KV head merges the blocks'
# partials. 16600 (260 tiles per head, the last one partial) ends each head with a
# partial tile. 40000 (625 tiles per head, 5000 in all) is more than one round, so
# each wave walks two tiles with an online softmax across them (the multi-tile path).
# (4, 1, 40000) and (8, 1, 40000): one KV head, so its blocks all count on one
# counter and the last of them merges every block's partials.
LONG_CASES = [(32, 8, 32768), (32, 8, 16600), (32, 8, 40000), (4, 1, 40000), (8, 1, 40000)]


@functools.lru_cache(maxsize=1)
def _long_case(n_q, H, n_ctx, hd):
    """Inputs and oracle records of one long case (shared by both kernel paths)."""
    k16, v16 = W.cfg2_kv(n_heads=H, n_pos=n_ctx, hd=hd, seed=n_ctx + 11)
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_ctx, seed=n_ctx + 12)
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    kref = O.ship_compress_f16(k16.reshape(-1, hd).view(np.uint16), kbc, O.mobius_order(hd)).reshape(H, n_ctx, -1)
    vref = O.ship_compress_f16(v16.reshape(-1, hd).view(np.uint16), vbc).reshape(H, n_ctx, -1)
    return k16, v16, q, kref, vref


@pytest.mark.parametrize("path", ["mfma", "general"])
@pytest.mark.parametrize("n_q,H,n_ctx", LONG_CASES)
def test_long_context_attention_matches_oracle(n_q, H, n_ctx, path, monkeypatch):
    """configs[1]'s per-layer decode (GQA 4 at 32K) and the ragged and 3-split
    variants, all bands and two K bands, scores and output, against the oracle."""
    if path == "general":
        monkeypatch.setenv("SP_HIP_NO_MFMA_ATTN", "1")
    hd = 128
    say(f"long attn path={path} n_q={n_q} H={H} n_ctx={n_ctx}")
    k16, v16, q, kref, vref = _long_case(n_q, H, n_ctx, hd)
    cc = S.ShipCache(S.config(hd, 1, H), n_ctx, stream=torch.cuda.current_stream().cuda_stream)
    L = S.lib()
    kt = dev(k16.reshape(H * n_ctx, hd).view(np.uint16))
    vt = dev(v16.reshape(H * n_ctx, hd).view(np.uint16))
    S.check(L.sp_hip_write_all(cc.ref, 0, n_ctx, p(kt), p(vt), S.DTYPE_F16), "write_all")
    del kt, vt
    kbc, vbc = O.band_config(hd, [5, 5, 4, 3]), O.band_config(hd, [3])
    order = O.mobius_order(hd)
    np.testing.assert_array_equal(d2h(cc.c.d_k_cache, kref.size).reshape(kref.shape), kref)
    scale = 1.0 / math.sqrt(hd)
    qt = dev(q)
    for mb in (-1, 2):
        say(f"  max_bands={mb}")
        s_ref, o_ref = O.attn_decode(q, kref, vref, H, n_ctx, kbc, vbc, order, scale, max_bands=mb)
        sc, out = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
        S.check(L.sp_hip_attn_decode_bands(cc.ref, 0, n_ctx, p(qt), n_q, C.c_float(scale), p(sc), p(out), mb,
                                           stream()))
        rel_close(host(sc).reshape(n_q, n_ctx), s_ref)
        rel_close(host(out).reshape(n_q, hd), o_ref)
        sc2, out2 = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
        S.check(L.sp_hip_attn_decode_bands(cc.ref, 0, n_ctx, p(qt), n_q, C.c_float(scale), p(sc2), None, mb,
                                           stream()))
        S.check(L.sp_hip_attn_decode_bands(cc.ref, 0, n_ctx, p(qt), n_q, C.c_float(scale), None, p(out2), mb,
                                           stream()))
        np.testing.assert_array_equal(host(sc2), host(sc))
        np.testing.assert_array_equal(host(out2), host(out))
    cc.free()


def test_all_layer_loops_equal_per_layer_calls():
    """sp_hip_attn_decode_all_layers and sp_hip_attn_scores_all_layers (all bands and
    two K bands) return, bit for bit, what the per-layer calls return."""
    L, H, n_q, n_ctx, hd = 3, 2, 8, 700, 128
    say(f"all-layer loops L={L} H={H} n_q={n_q} n_ctx={n_ctx}")
    cc = S.ShipCache(S.config(hd, L, H), n_ctx, stream=torch.cuda.current_stream().cuda_stream)
    lib = S.lib()
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    k = torch.randn((L * H, n_ctx, hd), generator=g, device="cuda").half()
    v = torch.randn((L * H, n_ctx, hd), generator=g, device="cuda").half()
    S.check(lib.sp_hip_write_all(cc.ref, 0, n_ctx, C.c_void_p(k.data_ptr()), C.c_void_p(v.data_ptr()), S.DTYPE_F16),
            "write_all")
    q = torch.randn((L, n_q, hd), generator=g, device="cuda")
    scale = C.c_float(1.0 / math.sqrt(hd))
    qp = C.c_void_p(q.data_ptr())
    out_all = torch.empty((L, n_q, hd), device="cuda")
    S.check(lib.sp_hip_attn_decode_all_layers(cc.ref, n_ctx, qp, n_q, scale, C.c_void_p(out_all.data_ptr()), stream()))
    for mb in (-1, 2):
        sc_all = torch.empty((L, n_q, n_ctx), device="cuda")
        S.check(lib.sp_hip_attn_scores_all_layers(cc.ref, n_ctx, qp, n_q, scale, C.c_void_p(sc_all.data_ptr()), mb,
                                                  stream()))
        for layer in range(L):
            sc1, out1 = torch.empty((n_q, n_ctx), device="cuda"), torch.empty((n_q, hd), device="cuda")
            S.check(lib.sp_hip_attn_decode_bands(cc.ref, layer, n_ctx, C.c_void_p(q[layer].data_ptr()), n_q, scale,
                                                 C.c_void_p(sc1.data_ptr()), C.c_void_p(out1.data_ptr()), mb,
                                                 stream()))
            torch.cuda.synchronize()
            assert torch.equal(sc_all[layer], sc1), (mb, layer)
            if mb == -1:
                assert torch.equal(out_all[layer], out1), layer
    cc.free()


def test_attention_rejects_bad_shapes():
    cfg = S.config(128, 1, 2)
    cc = S.ShipCache(cfg, 64)
    q = empty_f32(8 * 128)
    o = empty_f32(8 * 128)
    L = S.lib()
    assert L.sp_hip_attn_decode(cc.ref, 0, 65, p(q), 8, C.c_float(1.0), None, p(o), stream()) == -1  # n_kv > max_seq
    assert L.sp_hip_attn_decode(cc.ref, 1, 10, p(q), 8, C.c_float(1.0), None, p(o), stream()) == -1  # layer
    assert L.sp_hip_attn_decode(cc.ref, 0, 10, p(q), 3, C.c_float(1.0), None, p(o), stream()) == -1  # n_q % H
    assert L.sp_hip_attn_decode(cc.ref, 0, 10, p(q), 0, C.c_float(1.0), None, p(o), stream()) == -1
    cc.free()


def test_fp16_baseline_attention_matches_dense():
    n_q, H, n_ctx, hd = 8, 2, 600, 128
    rng = np.random.default_rng(3)
    k = rng.standard_normal((1, H, n_ctx, hd)).astype(np.float16)
    v = rng.standard_normal((1, H, n_ctx, hd)).astype(np.float16)
    q = rng.standard_normal((n_q, hd)).astype(np.float32)
    scale = 1.0 / math.sqrt(hd)
    kt, vt, qt = dev(k.view(np.uint16)), dev(v.view(np.uint16)), dev(q)
    sc, out = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
    S.check(S.lib().sp_hip_attn_decode_f16(p(kt), p(vt), H, n_ctx, hd, 0, n_ctx, p(qt), n_q, C.c_float(scale),
                                           p(sc), p(out), stream()))
    kk = k[0].astype(np.float64)
    vv = v[0].astype(np.float64)
    s_ref = np.stack([kk[h // 4] @ q[h] for h in range(n_q)]) * scale
    pr = np.exp(s_ref - s_ref.max(1, keepdims=True))
    pr /= pr.sum(1, keepdims=True)
    o_ref = np.stack([pr[h] @ vv[h // 4] for h in range(n_q)])
    rel_close(host(sc).reshape(n_q, n_ctx), s_ref)
    rel_close(host(out).reshape(n_q, hd), o_ref)
