"""Fused decode attention over sqfree+spinor records (sp_hip_sqfree_attn_decode)
against the oracle's spo_sqfree_attn_decode (records decompressed by the sqfree read
path, then float64 softmax attention): scores and softmax.V within 1e-3 relative in
fp32, elementwise."""
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


def _rows(x16):
    """[H][n][hd] fp16 -> llama.cpp cache rows [n][H*hd]."""
    H, n, hd = x16.shape
    return np.ascontiguousarray(x16.transpose(1, 0, 2).reshape(n, H * hd)).view(np.uint16)


def _sqfree_cache(sk, v_bits, H, n_kv, seed, layers=2):
    """A 2-layer sqfree cache (hd 128, pad 154, K 5/4/4/4/5, 3-bit residuals, spinor)
    with layer 1's K and V written from seeded configs[3]-distributed vectors; returns
    the cache and the oracle's records of layer 1 (checked equal to the cache's)."""
    hd, pad = 128, 154
    k_bits = [5, 4, 4, 4, 5]
    km = O.Knight(pad, sk)
    kbc, vbc = O.band_config(sk, k_bits), O.band_config(sk, v_bits)
    k16, v16 = W.cfg4_kv(n_heads=H, n_pos=n_kv, hd=hd, seed=seed)
    cc = S.SqfreeCache(S.config(hd, layers, H, k_bits=k_bits, v_bits=v_bits), n_kv + 3, rbits=3, spinor=True,
                       sk_k=sk, stream=torch.cuda.current_stream().cuda_stream)
    kt, vt = dev(_rows(k16)), dev(_rows(v16))
    S.check(S.lib().sp_hip_sqfree_write_layer(cc.ref, 1, 0, n_kv, p(kt), p(vt), H * hd, S.DTYPE_F16))
    kp = np.stack([O.sqfree_compress_f16(k16[h].view(np.uint16), hd, km, kbc, 3, True) for h in range(H)])
    vp = np.stack([O.sqfree_compress_f16(v16[h].view(np.uint16), hd, km, vbc, 3, True) for h in range(H)])
    ms = n_kv + 3
    Bk, Bv = cc.c.bytes_per_pos_k, cc.c.bytes_per_pos_v
    allk = d2h(cc.c.d_k_cache, layers * H * ms * Bk).reshape(layers * H, ms, Bk)
    allv = d2h(cc.c.d_v_cache, layers * H * ms * Bv).reshape(layers * H, ms, Bv)
    np.testing.assert_array_equal(allk[H:, :n_kv], kp)  # the cache holds the oracle's records
    np.testing.assert_array_equal(allv[H:, :n_kv], vp)
    return cc, km, kbc, vbc, kp, vp


CASES = [
    # skeleton, V bits, H, n_q, n_kv, runs cap
    (115, [3], 4, 32, 3000, 0),               # configs[3]: GQA 8, V one 3-bit band, 47 tiles per head, partial last
    (115, [3], 4, 32, 3000, 5),               # runs of 9-10 tiles: online softmax across a run's tiles
    (115, [5, 4, 4, 4, 5], 2, 8, 777, 0),     # V mirrors K (the reference hook), GQA 4
    (77, [5, 4, 4, 4, 5], 2, 4, 130, 1),      # skeleton 77 (reference CUDA), GQA 2, one run of 3 tiles
    (115, [3], 2, 6, 200, 0),                 # GQA 3 (an unused head column of the V sums' halves)
    (115, [3], 2, 10, 333, 2),                # GQA 5
    (77, [5, 4, 4, 4, 5], 3, 3, 64, 0),       # MHA, exactly one tile
    (115, [3], 1, 8, 1, 0),                   # a single position
    (115, [3], 1, 8, 20000, 0),               # 313 runs of one tile: each merge run group (6 x 48
                                              # loads a pass) takes a second pass
]


@pytest.mark.parametrize("groups", ["auto", "one"])
@pytest.mark.parametrize("sk,v_bits,H,n_q,n_kv,runs", CASES)
def test_sqfree_attention_matches_oracle(sk, v_bits, H, n_q, n_kv, runs, groups, monkeypatch):
    """groups "auto": the launcher splits each KV head's query heads over two blocks when
    twice the blocks still fit one resident round (these sizes always do, at an even
    GQA); "one" keeps one block per KV head and run (SP_HIP_SQFREE_ATTN_GROUPS=1)."""
    if runs:
        monkeypatch.setenv("SP_HIP_SQFREE_ATTN_RUNS", str(runs))
    if groups == "one":
        monkeypatch.setenv("SP_HIP_SQFREE_ATTN_GROUPS", "1")
    say(f"sqfree attn sk={sk} v_bits={v_bits} H={H} n_q={n_q} n_kv={n_kv} runs={runs} groups={groups}")
    cc, km, kbc, vbc, kp, vp = _sqfree_cache(sk, v_bits, H, n_kv, seed=sk + n_kv)
    hd = 128
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_kv, seed=n_kv + 3)
    scale = 1.0 / math.sqrt(hd)
    s_ref, o_ref = O.sqfree_attn_decode(q, kp, vp, H, n_kv, hd, km, kbc, vbc, 3, True, scale)
    qt = dev(q)
    L = S.lib()
    sc, out = empty_f32(n_q * n_kv), empty_f32(n_q * hd)
    S.check(L.sp_hip_sqfree_attn_decode(cc.ref, 1, n_kv, p(qt), n_q, C.c_float(scale), p(sc), p(out), stream()))
    rel_close(host(sc).reshape(n_q, n_kv), s_ref)
    rel_close(host(out).reshape(n_q, hd), o_ref)
    # scores-only and output-only calls give the same arrays
    sc2, out2 = empty_f32(n_q * n_kv), empty_f32(n_q * hd)
    S.check(L.sp_hip_sqfree_attn_decode(cc.ref, 1, n_kv, p(qt), n_q, C.c_float(scale), p(sc2), None, stream()))
    S.check(L.sp_hip_sqfree_attn_decode(cc.ref, 1, n_kv, p(qt), n_q, C.c_float(scale), None, p(out2), stream()))
    np.testing.assert_array_equal(host(sc2), host(sc))
    np.testing.assert_array_equal(host(out2), host(out))
    cc.free()


def test_sqfree_attention_bench_shape():
    """The shape the bench times for configs[3], one sequence's layer: 4 KV heads x
    16384 positions, 32 query heads (GQA 8), skeleton 115, V one 3-bit band, with
    the default run sizing (256 runs per KV head)."""
    say("sqfree attn bench shape")
    H, n_q, n_kv, hd = 4, 32, 16384, 128
    cc, km, kbc, vbc, kp, vp = _sqfree_cache(115, [3], H, n_kv, seed=91)
    q = W.cfg2_q(n_q=n_q, hd=hd, pos=n_kv, seed=92)
    scale = 1.0 / math.sqrt(hd)
    s_ref, o_ref = O.sqfree_attn_decode(q, kp, vp, H, n_kv, hd, km, kbc, vbc, 3, True, scale)
    qt = dev(q)
    sc, out = empty_f32(n_q * n_kv), empty_f32(n_q * hd)
    S.check(S.lib().sp_hip_sqfree_attn_decode(cc.ref, 1, n_kv, p(qt), n_q, C.c_float(scale), p(sc), p(out),
                                              stream()))
    rel_close(host(sc).reshape(n_q, n_kv), s_ref)
    rel_close(host(out).reshape(n_q, hd), o_ref)
    cc.free()


def test_sqfree_attention_rejects_bad_calls():
    say("sqfree attn bad calls")
    L = S.lib()
    cc, _, _, _, _, _ = _sqfree_cache(115, [3], 2, 40, seed=3)
    qt = dev(np.zeros((4, 128), np.float32))
    sc, out = empty_f32(4 * 40), empty_f32(4 * 128)
    f = C.c_float(0.0884)
    assert L.sp_hip_sqfree_attn_decode(cc.ref, 1, 40, p(qt), 3, f, p(sc), p(out), stream()) == -1  # 3 % 2
    assert L.sp_hip_sqfree_attn_decode(cc.ref, 1, 44, p(qt), 4, f, p(sc), p(out), stream()) == -1  # past max_seq
    assert L.sp_hip_sqfree_attn_decode(cc.ref, 2, 40, p(qt), 4, f, p(sc), p(out), stream()) == -1  # no layer 2
    assert L.sp_hip_sqfree_attn_decode(cc.ref, 1, 40, p(qt), 4, f, None, None, stream()) == -1
    assert L.sp_hip_sqfree_attn_decode(cc.ref, 1, 40, p(qt), 18, f, p(sc), p(out), stream()) == -1  # G 9 > 8
    cc.free()
    # a geometry without a fused kernel (hd 64 -> pad 66) is refused with the reason
    cc = S.SqfreeCache(S.config(64, 1, 1, k_bits=[5, 4, 4, 4, 5], v_bits=[5, 4, 4, 4, 5]), 8, rbits=3, spinor=True,
                       stream=torch.cuda.current_stream().cuda_stream)
    q64 = dev(np.zeros((1, 64), np.float32))
    assert L.sp_hip_sqfree_attn_decode(cc.ref, 0, 8, p(q64), 1, f, p(sc), None, stream()) == -1
    assert b"geometry" in L.sp_hip_last_error()
    cc.free()
