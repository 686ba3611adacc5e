"""Batched decode attention (several sequences of one layer in one call):
sp_hip_attn_decode_seqs, sp_hip_sqfree_attn_decode_seqs and
sp_hip_hier_attn_decode_seqs against the oracle run on each sequence's range of
records: scores and softmax.V within 1e-3 relative in fp32, elementwise."""
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
from gpu_util import dev, empty_f32, host, p, stream  # noqa: E402
from test_gpu_attn import rel_close  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _arr(v):
    a = np.ascontiguousarray(v, dtype=np.int32)
    return a, C.c_void_p(a.ctypes.data)


def _check(fn, cache_ref, layer, starts, lens, q, n_q, hd, scale, ref_fn):
    """Runs the batched entry point with scores and output, then scores-only and
    output-only, and checks every sequence against ref_fn(s0, n) -> (scores, out)."""
    n_seq = len(starts)
    sa, sp_ = _arr(starts)
    la, lp = _arr(lens)
    qt = dev(q.reshape(n_seq * n_q, hd))
    tot = n_q * int(np.sum(lens))
    sc, out = empty_f32(tot), empty_f32(n_seq * n_q * hd)
    S.check(fn(cache_ref, layer, n_seq, sp_, lp, p(qt), n_q, C.c_float(scale), p(sc), p(out), stream()))
    g_s, g_o = host(sc), host(out).reshape(n_seq, n_q, hd)
    off = 0
    for i, (s0, n) in enumerate(zip(starts, lens)):
        s_ref, o_ref = ref_fn(i, s0, n)
        rel_close(g_s[off:off + n_q * n].reshape(n_q, n), s_ref)
        rel_close(g_o[i], o_ref)
        off += n_q * n
    sc2, out2 = empty_f32(tot), empty_f32(n_seq * n_q * hd)
    S.check(fn(cache_ref, layer, n_seq, sp_, lp, p(qt), n_q, C.c_float(scale), p(sc2), None, stream()))
    S.check(fn(cache_ref, layer, n_seq, sp_, lp, p(qt), n_q, C.c_float(scale), None, p(out2), stream()))
    np.testing.assert_array_equal(host(sc2), g_s)
    np.testing.assert_array_equal(host(out2).reshape(n_seq, n_q, hd), g_o)


SHIP_CASES = [
    # hd, K bits, V bits, H, n_q, starts, lens, max_seq
    # the lane kernel, all five sequences in one launch (58- and 62-byte records at even
    # starts of an even max_seq: dword-aligned bases)
    (96, (5, 4, 4), (5,), 4, 8, [0, 4096, 5200, 5200, 9000], [4096, 1000, 1, 2500, 64], 9068),
    # an odd start (a base off dword alignment): one launch sequence per sequence
    (96, (5, 4, 4), (5,), 4, 8, [0, 3001, 700], [3001, 999, 2000], 4004),
    (128, (5, 5, 4, 3), (3,), 2, 8, [0, 3000, 100], [3000, 1500, 700], 4503),  # matrix-core kernel per sequence
    (64, (5, 5, 4, 3), (3,), 2, 4, [0, 600], [600, 333], 936),                  # the lane kernel at hd 64
]


@pytest.mark.parametrize("hd,k_bits,v_bits,H,n_q,starts,lens,ms", SHIP_CASES)
def test_ship_attention_seqs(hd, k_bits, v_bits, H, n_q, starts, lens, ms):
    say(f"attn seqs hd={hd} H={H} n_q={n_q} starts={starts} lens={lens} max_seq={ms}")
    assert ms >= max(s + n for s, n in zip(starts, lens))
    k16, v16 = W.cfg3_kv(n_heads=H, n_pos=ms, hd=hd, seed=hd + ms)
    cc = S.ShipCache(S.config(hd, 2, H, k_bits=k_bits, v_bits=v_bits), ms,
                     stream=torch.cuda.current_stream().cuda_stream)
    L = S.lib()
    for h in range(H):
        kt, vt = dev(k16[h].view(np.uint16)), dev(v16[h].view(np.uint16))
        S.check(L.sp_hip_write_k_batch_f16(cc.ref, 1, h, 0, ms, p(kt)))
        S.check(L.sp_hip_write_v_batch_f16(cc.ref, 1, h, 0, ms, p(vt)))
    kbc, vbc = O.band_config(hd, list(k_bits)), O.band_config(hd, list(v_bits))
    order = O.mobius_order(hd)
    kref = np.stack([O.ship_compress_f16(k16[h].view(np.uint16), kbc, order) for h in range(H)])
    vref = np.stack([O.ship_compress_f16(v16[h].view(np.uint16), vbc) for h in range(H)])
    q = np.stack([W.cfg2_q(n_q=n_q, hd=hd, pos=n, seed=17 + i) for i, n in enumerate(lens)])
    scale = 1.0 / math.sqrt(hd)

    def ref(i, s0, n):
        return O.attn_decode(q[i], kref[:, s0:s0 + n], vref[:, s0:s0 + n], H, n, kbc, vbc, order, scale)
    _check(L.sp_hip_attn_decode_seqs, cc.ref, 1, starts, lens, q, n_q, hd, scale, ref)
    cc.free()


def test_sqfree_attention_seqs():
    """configs[3]'s geometry (skeleton 115, V one 3-bit band, GQA 8), four sequences of
    unequal length in one launch each of prep, split and merge."""
    H, n_q, hd = 4, 32, 128
    starts, lens = [0, 2000, 2000, 5100], [2000, 3100, 1, 900]
    ms = 6003
    say(f"sqfree attn seqs lens={lens}")
    km = O.Knight(154, 115)
    kbc, vbc = O.band_config(115, [5, 4, 4, 4, 5]), O.band_config(115, [3])
    k16, v16 = W.cfg4_kv(n_heads=H, n_pos=ms, hd=hd, seed=5)
    cc = S.SqfreeCache(S.config(hd, 1, H, k_bits=[5, 4, 4, 4, 5], v_bits=[3]), ms, rbits=3, spinor=True, sk_k=115,
                       stream=torch.cuda.current_stream().cuda_stream)
    rows = lambda x: dev(np.ascontiguousarray(x.transpose(1, 0, 2).reshape(ms, H * hd)).view(np.uint16))
    kt, vt = rows(k16), rows(v16)
    S.check(S.lib().sp_hip_sqfree_write_layer(cc.ref, 0, 0, ms, p(kt), p(vt), H * hd, S.DTYPE_F16))
    kp = np.stack([O.sqfree_compress_f16(k16[h].view(np.uint16), hd, km, kbc, 3, True) for h in range(H)])
    vp = np.stack([O.sqfree_compress_f16(v16[h].view(np.uint16), hd, km, vbc, 3, True) for h in range(H)])
    q = np.stack([W.cfg2_q(n_q=n_q, hd=hd, pos=n, seed=31 + i) for i, n in enumerate(lens)])
    scale = 1.0 / math.sqrt(hd)

    def ref(i, s0, n):
        return O.sqfree_attn_decode(q[i], kp[:, s0:s0 + n], vp[:, s0:s0 + n], H, n, hd, km, kbc, vbc, 3, True, scale)
    _check(S.lib().sp_hip_sqfree_attn_decode_seqs, cc.ref, 0, starts, lens, q, n_q, hd, scale, ref)
    cc.free()


@pytest.mark.parametrize("n_q,starts,lens", [
    (4, [0, 1500, 2100], [1500, 600, 2400]),   # GQA 2: the chunk kernel, grid z = 3 sequences
    (16, [0, 700], [700, 1300]),               # GQA 8: the lane kernel
])
def test_hier_attention_seqs(n_q, starts, lens):
    """configs[4]'s geometry (hd 256, pad 330, skeleton 5/5, 2-bit targets), 2 KV heads."""
    H, hd, rbits = 2, 256, 2
    ms = max(s + n for s, n in zip(starts, lens)) + 2
    say(f"hier attn seqs n_q={n_q} lens={lens}")
    pad = O.sqfree_pad_dim(hd)
    sk, tg = O.hier_geometry(pad)
    bc = O.band_config(len(sk), [5, 5])
    Wm = W.hier_W(H, len(tg), len(sk), seed=9)
    k16, v16 = W.cfg5_kv(n_heads=H, n_pos=ms, hd=hd, seed=10)
    hc = S.HierCache(S.config(hd, 1, H), pad, sk, tg, S.band_config(len(sk), [5, 5]), rbits, ms, H,
                     stream=torch.cuda.current_stream().cuda_stream)
    hc.upload_W(Wm)
    L = S.lib()
    for h in range(H):
        for is_v, x in ((0, k16[h]), (1, v16[h])):
            xt = dev(x.view(np.uint16))
            S.check(L.sp_hip_hier_write_batch(hc.ref, is_v, 0, h, 0, ms, p(xt), S.DTYPE_F16))
    kp = np.stack([O.hier_compress_f16(k16[h].view(np.uint16), hd, pad, sk, tg, bc, Wm[h], rbits) for h in range(H)])
    vp = np.stack([O.hier_compress_f16(v16[h].view(np.uint16), hd, pad, sk, tg, bc, Wm[h], rbits) for h in range(H)])
    q = np.stack([W.cfg2_q(n_q=n_q, hd=hd, pos=n, seed=41 + i) for i, n in enumerate(lens)])
    scale = 1.0 / math.sqrt(hd)

    def ref(i, s0, n):
        return O.hier_attn_decode(q[i], kp[:, s0:s0 + n], vp[:, s0:s0 + n], H, n, hd, pad, sk, tg, bc, Wm, rbits,
                                  scale)
    _check(L.sp_hip_hier_attn_decode_seqs, hc.ref, 0, starts, lens, q, n_q, hd, scale, ref)
    hc.free()


def test_seqs_reject_bad_tables():
    say("attn seqs bad tables")
    hd, H = 96, 2
    cc = S.ShipCache(S.config(hd, 1, H, k_bits=(5, 4, 4), v_bits=(5,)), 100,
                     stream=torch.cuda.current_stream().cuda_stream)
    L = S.lib()
    qt = dev(np.zeros((65 * 2, hd), np.float32))
    out = empty_f32(65 * 2 * hd)
    f = C.c_float(0.1)
    for starts, lens in (([0], [101]), ([-1], [5]), ([10], [0]), ([0] * 65, [1] * 65)):
        sa, sp_ = _arr(starts)
        la, lp = _arr(lens)
        assert L.sp_hip_attn_decode_seqs(cc.ref, 0, len(starts), sp_, lp, p(qt), 2, f, None, p(out), stream()) == -1
    sa, sp_ = _arr([0])
    la, lp = _arr([10])
    assert L.sp_hip_attn_decode_seqs(cc.ref, 0, 0, sp_, lp, p(qt), 2, f, None, p(out), stream()) == -1
    assert L.sp_hip_attn_decode_seqs(cc.ref, 0, 1, None, lp, p(qt), 2, f, None, p(out), stream()) == -1
    cc.free()
