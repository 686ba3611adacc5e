"""The C++ KvCache mirror (include/sp_kv_cache.hpp) on the GPU: tests/cpp/kv_cache_check
runs create_gpu / write_gpu / read_gpu / calibration / save_to_disk / load_from_disk
for the ship, sqfree and hier compositions; its reconstructions equal the oracle's
bit for bit (hier with the W the program fitted)."""
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import oracle_py as O  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "kv_cache_check")


def test_cpp_kv_cache_mirror(tmp_path):
    if not os.path.exists(BIN):
        pytest.fail("tests/cpp/kv_cache_check is not built (make -C tests/cpp)")
    print("cpp KvCache mirror", flush=True)
    r = subprocess.run([BIN, str(tmp_path)], capture_output=True, text=True, timeout=120)
    sys.stdout.write(r.stdout)
    assert r.returncode == 0, r.stderr
    L, H, hd, n = 2, 2, 128, 80
    x = np.fromfile(tmp_path / "x.bin", np.float32).reshape(L, n, H, hd)
    x16 = x.astype(np.float16)
    assert np.array_equal(x16.astype(np.float32), x)  # the inputs are fp16 values
    pad = O.sqfree_pad_dim(hd)
    kbc, order = O.band_config(hd, [5, 5, 4, 3]), O.mobius_order(hd)
    km, qbc = O.Knight(pad, pad // 2), O.band_config(pad // 2, [5, 4, 4, 4, 5])
    skel, tgt = O.hier_geometry(pad)
    hbc = O.band_config(len(skel), [5, 5])
    W = np.fromfile(tmp_path / "hier_W.bin", np.uint16).reshape(L * H, len(tgt), len(skel))
    for kind in ("ship", "sqfree", "hier"):
        for layer in range(L):
            y = np.fromfile(tmp_path / f"{kind}_y{layer}.bin", np.float32).reshape(n, H, hd)
            for h in range(H):
                u16 = np.ascontiguousarray(x16[layer, :, h]).view(np.uint16)
                if kind == "ship":
                    want = O.ship_decompress_f32(O.ship_compress_f16(u16, kbc, order), kbc, order)
                elif kind == "sqfree":
                    want = O.sqfree_decompress_f32(O.sqfree_compress_f16(u16, hd, km, qbc, 3, True), hd, km, qbc, 3, True)
                else:
                    w = W[layer * H + h]
                    want = O.hier_decompress_f32(O.hier_compress_f16(u16, hd, pad, skel, tgt, hbc, w, 2),
                                                 hd, pad, skel, tgt, hbc, w, 2)
                np.testing.assert_array_equal(y[:, h].view(np.uint32), want.view(np.uint32),
                                              err_msg=f"{kind} layer {layer} head {h}")
    assert np.abs(W.view(np.float16).astype(np.float32)).max() > 0  # the predictor was fitted
