"""The HIP path through the C-ABI against the committed golden fixtures
(tests/golden/*.npz, from the CPU oracle; tests/test_golden.py pins the oracle
to the same files): ship codes and reconstructions (hd 128 and hd 96, fp16 and
fp32, a 2-band partial read), fused attention over ship records, sqfree+spinor
and hier codes and reconstructions, and fused attention over hier records.
Codes and reconstructions bit-exact; attention within 1e-3 elementwise."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import sp_hip as S  # noqa: E402
from gpu_util import d2h, decode, dev, empty_f32, encode, host, order_dev, p, stream  # noqa: E402
from test_gpu_attn import rel_close  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_hip = None


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def h2d(dptr, a):
    """Copy a numpy array's bytes to a raw device pointer owned by the library."""
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    a = np.ascontiguousarray(a)
    torch.cuda.synchronize()
    assert _hip.hipMemcpy(dptr, a.ctypes.data, a.nbytes, 1) == 0  # hipMemcpyHostToDevice


@pytest.mark.parametrize("name", ["cfg0_ship_hd128.npz", "cfg2_ship_hd96.npz"])
def test_ship_matches_fixture(name):
    say(f"golden {name}")
    f = load(name)
    hd = int(f["hd"])
    kbc, vbc = S.band_config(hd, list(f["k_bits"])), S.band_config(hd, list(f["v_bits"]))
    n = f["k_in"].shape[0]
    ot = order_dev(hd)
    kc = host(encode(kbc, ot, dev(f["k_in"]), S.DTYPE_F16, n, hd)).reshape(n, -1)
    vc = host(encode(vbc, None, dev(f["v_in"]), S.DTYPE_F16, n, hd)).reshape(n, -1)
    np.testing.assert_array_equal(kc, f["k_codes"])
    np.testing.assert_array_equal(vc, f["v_codes"])
    kt, vt = dev(f["k_codes"].reshape(-1)), dev(f["v_codes"].reshape(-1))
    np.testing.assert_array_equal(host(decode(kbc, ot, kt, S.DTYPE_F16, n, hd), np.uint16).reshape(n, hd), f["k_rec16"])
    np.testing.assert_array_equal(host(decode(vbc, None, vt, S.DTYPE_F16, n, hd), np.uint16).reshape(n, hd), f["v_rec16"])
    np.testing.assert_array_equal(host(decode(kbc, ot, kt, S.DTYPE_F32, n, hd)).reshape(n, hd).view(np.uint32),
                                  f["k_rec32"].view(np.uint32))
    np.testing.assert_array_equal(host(decode(vbc, None, vt, S.DTYPE_F32, n, hd)).reshape(n, hd).view(np.uint32),
                                  f["v_rec32"].view(np.uint32))
    np.testing.assert_array_equal(
        host(decode(kbc, ot, kt, S.DTYPE_F32, n, hd, max_bands=2)).reshape(n, hd).view(np.uint32),
        f["k_rec32_2bands"].view(np.uint32))


def test_attention_matches_fixture():
    say("golden attention")
    f = load("cfg1_attention_hd128.npz")
    hd, H = int(f["hd"]), int(f["n_kvh"])
    n_ctx = f["k_codes"].shape[1]
    q = f["q"]
    n_q = q.shape[0]
    cc = S.ShipCache(S.config(hd, 1, H), n_ctx, stream=torch.cuda.current_stream().cuda_stream)
    h2d(cc.c.d_k_cache, f["k_codes"])  # slots [head][max_seq = n_ctx][B] of layer 0
    h2d(cc.c.d_v_cache, f["v_codes"])
    sc, out = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
    S.check(S.lib().sp_hip_attn_decode(cc.ref, 0, n_ctx, p(dev(q)), n_q, C.c_float(float(f["kq_scale"])), p(sc),
                                       p(out), stream()))
    rel_close(host(sc).reshape(n_q, n_ctx), f["scores"])
    rel_close(host(out).reshape(n_q, hd), f["out"])
    cc.free()


def test_sqfree_matches_fixture():
    say("golden sqfree")
    f = load("cfg3_sqfree_hd128.npz")
    hd, sk, rb, sp = int(f["hd"]), int(f["sk_k"]), int(f["rbits"]), bool(f["spinor"])
    bits = [int(b) for b in f["bits"]]
    n = f["x_in"].shape[0]
    cc = S.SqfreeCache(S.config(hd, 1, 1, k_bits=bits, v_bits=bits), n, rbits=rb, spinor=sp, sk_k=sk,
                       stream=torch.cuda.current_stream().cuda_stream)
    S.check(S.lib().sp_hip_sqfree_write_batch(cc.ref, 0, 0, 0, 0, n, p(dev(f["x_in"])), S.DTYPE_F16))
    B = f["codes"].shape[1]
    assert cc.c.bytes_per_pos_k == B
    np.testing.assert_array_equal(d2h(cc.c.d_k_cache, n * B).reshape(n, B), f["codes"])
    out = empty_f32(n * hd)
    S.check(S.lib().sp_hip_sqfree_read_batch(cc.ref, 0, 0, 0, 0, n, p(out), S.DTYPE_F32))
    np.testing.assert_array_equal(host(out).reshape(n, hd).view(np.uint32), f["rec32"].view(np.uint32))
    cc.free()


def test_hier_matches_fixture():
    say("golden hier")
    f = load("cfg4_hier_hd256.npz")
    hd, pad, rb = int(f["hd"]), int(f["pad"]), int(f["rbits"])
    sk, tg = f["skel_idx"], f["tgt_idx"]
    n = f["x_in"].shape[0]
    n_ctx = f["k_codes"].shape[1]
    ms = max(n, n_ctx)
    hc = S.HierCache(S.config(hd, 1, 2), pad, sk, tg, S.band_config(len(sk), [int(b) for b in f["skel_bits"]]), rb,
                     ms, 2, stream=torch.cuda.current_stream().cuda_stream)
    hc.upload_W(f["W"])
    B = f["codes"].shape[1]
    assert hc.c.bytes_per_pos_k == B
    # codec: slot 0's K from the fixture's inputs
    S.check(S.lib().sp_hip_hier_write_batch(hc.ref, 0, 0, 0, 0, n, p(dev(f["x_in"])), S.DTYPE_F16))
    np.testing.assert_array_equal(d2h(hc.c.d_k_cache, n * B).reshape(n, B), f["codes"])
    out = empty_f32(n * hd)
    S.check(S.lib().sp_hip_hier_read_batch(hc.ref, 0, 0, 0, 0, n, p(out), S.DTYPE_F32))
    np.testing.assert_array_equal(host(out).reshape(n, hd).view(np.uint32), f["rec32"].view(np.uint32))
    # fused attention over the fixture's records (slots [head][max_seq][B])
    kr = np.zeros((2, ms, B), np.uint8)
    vr = np.zeros((2, ms, B), np.uint8)
    kr[:, :n_ctx], vr[:, :n_ctx] = f["k_codes"], f["v_codes"]
    h2d(hc.c.d_k_cache, kr)
    h2d(hc.c.d_v_cache, vr)
    q = f["q"]
    n_q = q.shape[0]
    sc, o = empty_f32(n_q * n_ctx), empty_f32(n_q * hd)
    S.check(S.lib().sp_hip_hier_attn_decode(hc.ref, 0, n_ctx, p(dev(q)), n_q, C.c_float(float(f["kq_scale"])), p(sc),
                                            p(o), stream()))
    rel_close(host(sc).reshape(n_q, n_ctx), f["scores"])
    rel_close(host(o).reshape(n_q, hd), f["out"])
    hc.free()
