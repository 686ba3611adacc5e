"""Fused decode attention over hier records (sp_hip_hier_attn_decode) against the
oracle's spo_hier_attn_decode (records decompressed by the hier read path, then
float64 softmax attention): scores and softmax.V within 1e-3 relative in fp32."""
import ctypes as C
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
from test_gpu_attn import rel_close  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _hier_cache(hd, rbits, skel_bits, H, n_kv, seed, layers=2):
    """A 2-layer hier cache with layer 1's K and V written from seeded vectors;
    returns the cache, the geometry and the oracle's records of layer 1."""
    pad = O.sqfree_pad_dim(hd)
    sk, tg = O.hier_geometry(pad)
    bc = O.band_config(len(sk), skel_bits)
    Wm = W.hier_W(layers * H, len(tg), len(sk), seed=seed)
    k16, v16 = W.cfg5_kv(n_heads=H, n_pos=n_kv, hd=hd, seed=seed + 1)
    hc = S.HierCache(S.config(hd, layers, H), pad, sk, tg, S.band_config(len(sk), skel_bits), rbits, n_kv + 3,
                     layers * H, stream=torch.cuda.current_stream().cuda_stream)
    hc.upload_W(Wm)
    B = hc.c.bytes_per_pos_k
    kp, vp = [], []
    for h in range(H):
        slot = H + h
        for is_v, x in ((0, k16[h]), (1, v16[h])):
            xt = dev(x.view(np.uint16))
            S.check(S.lib().sp_hip_hier_write_batch(hc.ref, is_v, 1, h, 0, n_kv, p(xt), S.DTYPE_F16))
        kp.append(O.hier_compress_f16(k16[h].view(np.uint16), hd, pad, sk, tg, bc, Wm[slot], rbits))
        vp.append(O.hier_compress_f16(v16[h].view(np.uint16), hd, pad, sk, tg, bc, Wm[slot], rbits))
    torch.cuda.synchronize()
    kp, vp = np.stack(kp), np.stack(vp)
    ms = n_kv + 3
    allk = d2h(hc.c.d_k_cache, layers * H * ms * B).reshape(layers * H, ms, B)
    np.testing.assert_array_equal(allk[H:, :n_kv], kp)  # the cache holds the oracle's records
    return hc, (pad, sk, tg, bc, Wm[H:]), kp, vp


CASES = [
    # hd, rbits, skeleton bands, H, n_q, n_kv, runs cap (chunks of 256 positions for the
    # chunk kernel, tiles of 64 for the lane kernel)
    (256, 2, [5, 5], 2, 4, 300, 0),     # configs[4] geometry, GQA 2, a partial second chunk
    (256, 2, [5, 5], 2, 4, 1100, 2),    # two runs of 2-3 chunks each: online softmax across chunks
    (64, 3, [5, 4], 2, 2, 517, 1),      # pad 66, 3-bit levels straddling bytes, one run of 3 chunks
    (96, 2, [4], 2, 6, 257, 0),         # pad 105, GQA 3 (odd: a lone last head), 1-position last chunk
    (256, 2, [5, 5], 1, 1, 1, 0),       # a single position
    (256, 2, [5, 5], 8, 16, 2000, 3),   # configs[4] head layout (8 KV heads, GQA 2), 3 runs of 2-3 chunks
    (256, 2, [5, 5], 2, 8, 700, 2),     # GQA 4: two head pairs per window item
    (256, 2, [5, 5], 1, 8, 333, 0),     # GQA 8: window and skeleton items in two rounds per lane
    (256, 2, [5, 5], 2, 6, 260, 1),     # GQA 3: a pair with one real head
    # the bench's run sizing (no cap): three resident blocks per CU spread over the KV
    # heads, so about 96 runs per head, which the merge splits over its run groups
    (256, 2, [5, 5], 8, 16, 25000, 0),  # configs[4] head layout: 96 runs per head (98 chunks)
    (256, 2, [5, 5], 1, 2, 25000, 0),   # one KV head: 98 runs of one chunk, three run groups of
                                        # 32-33 runs each in the merge
    (256, 2, [5, 5], 1, 2, 40000, 0),   # 157 runs: each merge run group (3 x 48 loads a pass)
                                        # takes a second pass
    (256, 2, [5, 5], 1, 2, 75300, 49),  # 49 runs of 6-7 chunks (295 chunks): long online softmax
                                        # chains and the scores-only instance's K prefetch across
                                        # chunks
]


@pytest.mark.parametrize("path", ["default", "runtime", "lane", "window"])
@pytest.mark.parametrize("hd,rbits,skel_bits,H,n_q,n_kv,runs", CASES)
def test_hier_attention_matches_oracle(hd, rbits, skel_bits, H, n_q, n_kv, runs, path, monkeypatch):
    """The default launch runs the 256-position chunk kernel (2-bit levels at up to 4
    query heads per KV head: the V coefficient sums on the matrix cores), and past its
    LDS limit (more than 4 query heads per KV head at pad 330) the one-position-per-lane
    split kernel of the configs[4] geometry (hd 256, skeleton 5/5, 2-bit targets). At
    that geometry the chunk kernel runs its compile-time-geometry instance; path
    "runtime" keeps the instance that reads the geometry from the call
    (SP_HIP_HIER_ATTN_CT=0), path "lane" selects the lane kernel wherever it fits
    (SP_HIP_HIER_ATTN_LANE=1), path "window" keeps the chunk kernel's V sums on the VALU
    (SP_HIP_HIER_ATTN_VM=0)."""
    lane_geo = hd == 256 and rbits == 2 and list(skel_bits) == [5, 5]
    if path == "lane":
        if not lane_geo:
            pytest.skip("the lane kernel serves the configs[4] geometry only")
        monkeypatch.setenv("SP_HIP_HIER_ATTN_LANE", "1")
    if path == "runtime":
        if not lane_geo or n_q // H > 4:
            pytest.skip("the compile-time instances serve the configs[4] geometry at up to 4 query heads per KV head")
        monkeypatch.setenv("SP_HIP_HIER_ATTN_CT", "0")
    if path == "window":
        if rbits != 2 or n_q // H > 4:
            pytest.skip("the matrix-core V sums serve 2-bit levels at up to 4 query heads per KV head")
        monkeypatch.setenv("SP_HIP_HIER_ATTN_VM", "0")
    if runs:
        monkeypatch.setenv("SP_HIP_HIER_ATTN_RUNS", str(runs))
    say(f"hier attn path={path} hd={hd} rbits={rbits} bands={skel_bits} H={H} n_q={n_q} n_kv={n_kv} runs={runs}")
    hc, (pad, sk, tg, bc, Wl), kp, vp = _hier_cache(hd, rbits, skel_bits, H, n_kv, seed=hd + n_kv)
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_kv, seed=n_kv + 7)
    scale = 1.0 / math.sqrt(hd)
    s_ref, o_ref = O.hier_attn_decode(q, kp, vp, H, n_kv, hd, pad, sk, tg, bc, Wl, rbits, scale)
    qt = dev(q)
    sc, out = empty_f32(n_q * n_kv), empty_f32(n_q * hd)
    S.check(S.lib().sp_hip_hier_attn_decode(hc.ref, 1, n_kv, p(qt), n_q, C.c_float(scale), p(sc), p(out),
                                            stream()))
    torch.cuda.synchronize()
    rel_close(host(sc).reshape(n_q, n_kv), s_ref)
    rel_close(host(out).reshape(n_q, hd), o_ref)
    # scores-only and output-only calls give the same arrays
    sc2, out2 = empty_f32(n_q * n_kv), empty_f32(n_q * hd)
    S.check(S.lib().sp_hip_hier_attn_decode(hc.ref, 1, n_kv, p(qt), n_q, C.c_float(scale), p(sc2), None, stream()))
    S.check(S.lib().sp_hip_hier_attn_decode(hc.ref, 1, n_kv, p(qt), n_q, C.c_float(scale), None, p(out2), stream()))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(sc2), host(sc))
    np.testing.assert_array_equal(host(out2), host(out))
    hc.free()


def test_hier_attention_rejects_bad_calls():
    say("hier attn bad calls")
    hc, _, _, _ = _hier_cache(256, 2, [5, 5], 2, 40, seed=3)
    qt = dev(np.zeros((4, 256), np.float32))
    sc, out = empty_f32(4 * 40), empty_f32(4 * 256)
    L = S.lib()
    f = C.c_float(0.0625)
    assert L.sp_hip_hier_attn_decode(hc.ref, 1, 40, p(qt), 3, f, p(sc), p(out), stream()) == -1  # 3 % 2
    assert L.sp_hip_hier_attn_decode(hc.ref, 1, 44, p(qt), 4, f, p(sc), p(out), stream()) == -1  # past max_seq
    assert L.sp_hip_hier_attn_decode(hc.ref, 2, 40, p(qt), 4, f, p(sc), p(out), stream()) == -1  # no layer 2
    assert L.sp_hip_hier_attn_decode(hc.ref, 1, 40, p(qt), 4, f, None, None, stream()) == -1
    assert L.sp_hip_hier_attn_decode(hc.ref, 1, 40, p(qt), 18, f, p(sc), p(out), stream()) == -1  # G 9 > 8
    hc.free()
