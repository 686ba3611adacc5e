#!/usr/bin/env python3
"""Benchmark of the Shannon-Prime KV codec hot path on one MI355X.

Workload (Llama-3-8B-shaped): 32 layers x 8 KV heads x
32768 positions, head_dim 128, fp16 K (RoPE theta 500000) and V, seeded N(0,1),
already resident in HBM. One step = compress every K and V vector (K 5/5/4/3 +
Mobius, V flat 3-bit) and decompress every record back to fp16:
8,388,608 K + 8,388,608 V vectors.

Printed JSON line: metric/value (K+V vectors per second through compress +
decompress), HBM GB/s of algorithmic bytes, the dominant kernel's roofline
(HIP events on the launch stream), fused decompress-attention decode at 32K in
us/token (32 layers) beside uncompressed fp16 attention (torch batched GEMMs and
this library's fp16 kernel), the other configs' codec paths (hd 96 Vilenkin,
sqfree+spinor, hier) at their per-GPU shapes, and the CPU baseline (the oracle on
a bounded sample, one thread and all cores). With the CPU leg, a sample of the
full-size run is also checked against the oracle.
"""
import argparse
import ctypes as C
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "shannon-prime-llama_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0
LAYERS, KVH, HD, POS, NQ = 32, 8, 128, 32768, 32
K_BITS, V_BITS = (5, 5, 4, 3), (3,)
# kernels behind each codec step on gfx950 (one launch per step over all 256 slots)
KERNEL_NAMES = {"k_enc": "k_ship_encode_lane<Layout<128,5,5,4,3>, fp16, Mobius>",
                "v_enc": "k_ship_encode_lane<Layout<128,3>, fp16>",
                "k_dec": "k_ship_decode_lane<Layout<128,5,5,4,3>, fp16, Mobius>",
                "v_dec": "k_ship_decode_lane<Layout<128,3>, fp16>"}


# VALU instructions per 64-vector tile of each codec kernel, measured with rocprofv3
# (SQ_INSTS_VALU per wave over the tiles each wave walks; profiles/valu_codec_kernels.md).
# A wave64 VALU instruction issues over 4 cycles on a 16-lane SIMD, so at full issue a
# kernel needs tiles * VALU_PER_TILE * 4 / (SIMDs * engine clock): the VALU-issue bound,
# which the bit-exact codecs cannot move to the matrix cores.
VALU_PER_TILE = {"k_enc": 1693, "v_enc": 1608, "k_dec": 1559, "v_dec": 1799,  # configs[1], hd 128
                 "hd96_k_enc": 2089, "hd96_v_enc": 2087, "hd96_k_dec": 2225, "hd96_v_dec": 2224,
                 "sqfree_k_enc": 7256, "sqfree_v_enc": 7207, "sqfree_k_dec": 5802, "sqfree_v_dec": 5948,
                 "hier_enc": 32633, "hier_dec": 31228}
ENGINE_CLOCK_HZ = 2.4e9  # MI355X peak engine clock


def valu_bound_s(n_vec, per_tile, simds):
    """Seconds the VALU needs at full issue for n_vec vectors at per_tile instructions per 64."""
    return (n_vec / 64.0) * per_tile * 4.0 / (simds * ENGINE_CLOCK_HZ)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_bytes(hd, kB, vB):
    """Per-vector algorithmic HBM bytes: compress reads 2*hd fp16 and writes B;
    decompress reads B and writes 2*hd fp16."""
    return {"k_enc": 2 * hd + kB, "v_enc": 2 * hd + vB, "k_dec": kB + 2 * hd, "v_dec": vB + 2 * hd}


def make_inputs(torch, n_slots, pos, hd, seed=2, theta=500000.0):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    k = torch.empty((n_slots, pos, hd), dtype=torch.float16, device="cuda")
    v = torch.empty((n_slots, pos, hd), dtype=torch.float16, device="cuda")
    half = hd // 2
    inv = theta ** (-torch.arange(half, device="cuda", dtype=torch.float64) * 2.0 / hd)
    ang = torch.arange(pos, device="cuda", dtype=torch.float64)[:, None] * inv[None, :]
    cs, sn = torch.cos(ang).float(), torch.sin(ang).float()
    for s in range(0, n_slots, 16):
        e = min(n_slots, s + 16)
        x = torch.randn((e - s, pos, hd), generator=g, device="cuda", dtype=torch.float32)
        a, b = x[..., :half], x[..., half:]
        k[s:e] = torch.cat([a * cs - b * sn, a * sn + b * cs], dim=-1).half()
        v[s:e] = torch.randn((e - s, pos, hd), generator=g, device="cuda", dtype=torch.float32).half()
    return k, v


def cpu_threads():
    """Host threads for the all-core leg: the box's CPU share (OMP_NUM_THREADS there)."""
    n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(env))) if env and env.isdigit() else n


def cpu_baseline(target_s=8.0):
    """The oracle (scalar C restatement of the reference codec, -O2) round-tripping
    K and V vectors on this host: one thread (the reference's per-vector structure
    on the decode thread), then OpenMP over the host's cores. Bounded sample: the
    same seeded cfg2 vectors, repeated, about target_s seconds per leg."""
    import numpy as np
    import oracle_py as O
    import workloads as W
    kbc, vbc = O.band_config(HD, list(K_BITS)), O.band_config(HD, list(V_BITS))
    order = O.mobius_order(HD)
    k16, v16 = W.cfg2_kv(n_heads=8, n_pos=4096, hd=HD, seed=5)
    k = np.ascontiguousarray(k16.reshape(-1, HD).view(np.uint16))
    v = np.ascontiguousarray(v16.reshape(-1, HD).view(np.uint16))

    def leg(threads, n_rep):
        t0 = time.perf_counter()
        for _ in range(n_rep):
            O.ship_roundtrip_f16_omp(k, kbc, order, threads=threads)
            O.ship_roundtrip_f16_omp(v, vbc, None, threads=threads)
        return time.perf_counter() - t0

    out = {}
    for name, threads in (("single", 1), ("all", cpu_threads())):
        t1 = leg(threads, 1)
        reps = max(1, int(target_s / max(t1, 1e-6)))
        t = leg(threads, reps)
        out[name] = (threads, reps, t, 2 * k.shape[0] * reps / t)
    th, reps, t, vps = out["all"]
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), model)
    except OSError:
        pass
    return {"value": round(vps, 1), "unit": "KV vecs/s", "cores": th, "kind": "port",
            "single_thread_value": round(out["single"][3], 1), "cpu_model": model,
            "sample": f"{k.shape[0]} K + {v.shape[0]} V hd=128 fp16 vectors (cfg2 distribution) compress+"
                      f"decompress through the C oracle (-O2), repeated {reps}x on {th} OpenMP threads "
                      f"({t:.1f} s); single thread {out['single'][3]:.0f} vecs/s over {out['single'][2]:.1f} s; "
                      f"host nproc={os.cpu_count()}"}


def traffic_from_profile(kernel_key):
    """HBM bytes per launch of a codec kernel from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_ship_codec_cfg1.json")
    try:
        with open(path) as f:
            t = json.load(f)["per_launch_bytes"]
        return t.get(kernel_key)
    except (OSError, ValueError, KeyError):
        return None


def parity_sample(S, cc, k, v, kr, kB, vB, n_slots):
    """The checker, run with the CPU leg: three slots' records and K reconstructions
    from the full-size run against the oracle (codes and fp16 bits exact)."""
    import numpy as np
    import oracle_py as O
    kbc, vbc = O.band_config(HD, list(K_BITS)), O.band_config(HD, list(V_BITS))
    order = O.mobius_order(HD)
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    bad = 0
    for slot in (0, 131, n_slots - 1):
        p0, m = 1000, 256
        xk = k[slot, p0:p0 + m].cpu().numpy().view(np.uint16)
        rec = np.empty(m * kB, np.uint8)
        hip.hipMemcpy(rec.ctypes.data, cc.c.d_k_cache + (slot * POS + p0) * kB, rec.size, 2)
        bad += int((rec.reshape(m, kB) != O.ship_compress_f16(xk, kbc, order)).any())
        xv = v[slot, p0:p0 + m].cpu().numpy().view(np.uint16)
        recv = np.empty(m * vB, np.uint8)
        hip.hipMemcpy(recv.ctypes.data, cc.c.d_v_cache + (slot * POS + p0) * vB, recv.size, 2)
        bad += int((recv.reshape(m, vB) != O.ship_compress_f16(xv, vbc)).any())
        bad += int((kr[slot, p0:p0 + m].cpu().numpy().view(np.uint16) !=
                    O.ship_decompress_f16(rec.reshape(m, kB), kbc, order)).any())
    return bad


def seq_table(starts, lens):
    """int32 start and length arrays of a batched attention call, each as (array, pointer)."""
    import numpy as np
    out = []
    for v in (starts, lens):
        a = np.ascontiguousarray(v, dtype=np.int32)
        out.append((a, C.c_void_p(a.ctypes.data)))
    return out[0], out[1]


def bench_variants(torch, S, L, stream, reps=10):
    """Throughput of the other configs' codec paths at their per-GPU shapes (extra
    fields of the JSON line, not the headline): the configs[1] post-decode round
    trip over cache cells (one decode token, a 2048-cell prefill chunk; bytes count
    the fp16 vector read and written back plus the record), configs[2] ship codec at hd 96
    (Vilenkin 2^5*3, bridge default K 5/4/4, V 5), configs[3] sqfree+spinor
    (pad 154, skeleton 0.75, K/V 5/4/4/4/5, residual 3 bits), configs[4] hier (pad 330,
    30-coefficient skeleton at 5/5 bits, 2-bit residual). Rates count algorithmic
    bytes (2*hd fp16 in or out plus the record)."""
    sp = C.c_void_p(stream.cuda_stream)
    P = lambda t: C.c_void_p(t.data_ptr())
    g = torch.Generator(device="cuda")
    g.manual_seed(11)

    def timed(f):
        f()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            f()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps * 1e-3  # s

    simds = 4 * torch.cuda.get_device_properties(0).multi_processor_count

    def rate(n_vec, hd, B, t, valu_key=None):
        r = {"ms": round(t * 1e3, 4), "vecs_per_s": round(n_vec / t, 1),
             "gbs": round(n_vec * (2 * hd + B) / t / 1e9, 1)}
        if valu_key:
            vb = valu_bound_s(n_vec, VALU_PER_TILE[valu_key], simds)
            r.update({"valu_per_tile": VALU_PER_TILE[valu_key], "valu_bound_ms": round(vb * 1e3, 4),
                      "valu_frac": round(vb / t, 3)})
        return r

    out = {}
    # one layer of 32 heads x 65536 cells (16 sequences x 4096), hd 96
    H3, N3, hd3 = 32, 65536, 96
    cfg = S.config(hd3, 1, H3, k_bits=(5, 4, 4), v_bits=(5,))
    c3 = S.ShipCache(cfg, N3, stream.cuda_stream)
    x = (torch.randn((H3, N3, hd3), generator=g, device="cuda") *
         torch.exp(0.5 * torch.randn((H3, 1, hd3), generator=g, device="cuda"))).half()
    y = torch.empty_like(x)
    kB3, vB3 = c3.c.k_bands.total_bytes, c3.c.v_bands.total_bytes
    n3 = H3 * N3
    out["cfg3_hd96_ship"] = {
        "k_enc": rate(n3, hd3, kB3, timed(lambda: S.check(L.sp_hip_write_all(c3.ref, 0, N3, P(x), None, S.DTYPE_F16))),
                      "hd96_k_enc"),
        "v_enc": rate(n3, hd3, vB3, timed(lambda: S.check(L.sp_hip_write_all(c3.ref, 0, N3, None, P(x), S.DTYPE_F16))),
                      "hd96_v_enc"),
        "k_dec": rate(n3, hd3, kB3, timed(lambda: S.check(L.sp_hip_read_all(c3.ref, 0, N3, P(y), None, S.DTYPE_F16, -1))),
                      "hd96_k_dec"),
        "v_dec": rate(n3, hd3, vB3, timed(lambda: S.check(L.sp_hip_read_all(c3.ref, 0, N3, None, P(y), S.DTYPE_F16, -1))),
                      "hd96_v_dec"),
        "record_bytes": [kB3, vB3]}
    # configs[2] decode, batched: the 16 sequences as position ranges [4096 i, 4096 (i + 1)) of this
    # layer (K and V records from the writes above), one fused attention call for all of them
    NS3, NP3 = 16, 4096
    q3 = torch.randn((NS3, H3, hd3), generator=g, device="cuda")
    o3 = torch.empty((NS3, H3, hd3), device="cuda")
    sc3 = C.c_float(1.0 / math.sqrt(hd3))
    st3, ln3 = seq_table([NP3 * i for i in range(NS3)], [NP3] * NS3)
    t16b = timed(lambda: S.check(L.sp_hip_attn_decode_seqs(c3.ref, 0, NS3, st3[1], ln3[1], P(q3), H3, sc3, None,
                                                           P(o3), sp), "cfg2 attn seqs"))
    c3.free()
    # the same step as 16 single-sequence calls, one sequence per cache layer (distinct records, so
    # no call reads what an earlier one left in the caches)
    c3d = S.ShipCache(S.config(hd3, NS3, H3, k_bits=(5, 4, 4), v_bits=(5,)), NP3, stream.cuda_stream)
    xs = x.view(H3, NS3, NP3, hd3).transpose(0, 1).contiguous()  # [sequence][head][cell][d]
    S.check(L.sp_hip_write_all(c3d.ref, 0, NP3, P(xs), P(xs), S.DTYPE_F16), "cfg2 prefill")
    del xs

    def dec16():
        for sq in range(NS3):
            S.check(L.sp_hip_attn_decode(c3d.ref, sq, NP3, P(q3[sq]), H3, sc3, None, P(o3[sq]), sp), "cfg2 attn")
    t16 = timed(dec16)
    rec3 = NS3 * H3 * NP3 * (kB3 + vB3)
    out["cfg3_hd96_decode"] = {
        "step_layer_us": round(t16b * 1e6, 1), "us_per_token_32_layers": round(32 * t16b * 1e6, 1),
        "decode_tokens_per_s": round(NS3 / (32 * t16b), 1), "record_gbs": round(rec3 / t16b / 1e9, 1),
        "step_layer_us_16_calls": round(t16 * 1e6, 1),
        "record_floor_us": round(rec3 / (HBM_PEAK_GBS * 1e3), 1),
        "fp16_floor_us": round(NS3 * H3 * NP3 * 2 * hd3 * 2 / (HBM_PEAK_GBS * 1e3), 1),
        "layout": f"{NS3} sequences x {NP3} positions x {H3} heads (MHA), hd {hd3}, K 5/4/4 + V 5 records "
                  f"({kB3} + {vB3} B); per layer step: one batched fused attention call "
                  f"(sp_hip_attn_decode_seqs, one-position-per-lane kernel); step_layer_us_16_calls: "
                  f"{NS3} single-sequence calls"}
    c3d.free()
    del x, y
    # configs[1] post-decode hook on the device: sp_hip_roundtrip_cells over one layer's 8 heads,
    # K as cache rows and V transposed (v_trans), for a 1-token decode step and a 2048-cell prefill chunk
    H1, KV1, hd1 = 8, 32768, 128
    cfg = S.config(hd1, 1, H1)
    c1 = S.ShipCache(cfg, KV1, stream.cuda_stream)
    kt = torch.randn((KV1, H1 * hd1), generator=g, device="cuda").half()
    vt = torch.randn((H1 * hd1, KV1), generator=g, device="cuda").half()
    rt = {}
    for n_cells, c0 in ((1, 4097), (16, 5000), (256, 6000), (2048, 8192)):
        cells = torch.arange(c0, c0 + n_cells, dtype=torch.int32, device="cuda")

        def rt_call():
            S.check(L.sp_hip_roundtrip_cells(c1.ref, 0, P(cells), n_cells, P(kt), H1 * hd1, P(vt), 1, KV1,
                                             S.DTYPE_F16, -1, sp))
        nv = 2 * H1 * n_cells  # K and V vectors
        for kern in ("default", "narrow", "lane"):
            # the entry point reads SP_HIP_RT_KERNEL at each call
            if kern == "default":
                os.environ.pop("SP_HIP_RT_KERNEL", None)
            else:
                os.environ["SP_HIP_RT_KERNEL"] = kern
            t = timed(rt_call)
            key = f"cells_{n_cells}" + ("" if kern == "default" else f"_{kern}")
            rt[key] = {"us": round(t * 1e6, 2), "vecs_per_s": round(nv / t, 1),
                       "gbs": round(nv * (2 * 2 * hd1) / t / 1e9 + H1 * n_cells * (76 + 50) / t / 1e9, 1)}
        os.environ.pop("SP_HIP_RT_KERNEL", None)
    out["cfg1_roundtrip_cells"] = dict(rt, layout="K cache rows, V transposed (v_trans), one layer x 8 heads, fp16")
    # System 1/2 dual cache at the configs[1] layer shape (8 heads x 32768 positions, hd 128): System 1 the
    # ship cache above, System 2 a sqfree cache (pad 154, skeleton 77, 5/4/4/4/5, 3-bit residual, spinor)
    # owning a random 20% of the positions; one layer's merged K+V read into fp16 rows
    bits = [5, 4, 4, 4, 5]
    sq1 = S.SqfreeCache(S.config(hd1, 1, H1, k_bits=bits, v_bits=bits), KV1, rbits=3, spinor=True, sk_k=77,
                        stream=stream.cuda_stream)
    dc = S.DualCache(c1, sq1, S.DUAL_SQFREE, 1.0)
    own2 = torch.rand(KV1, generator=g, device="cuda").cpu().numpy() < 0.2
    for t in range(KV1):
        L.sp_hip_dual_route_position(dc.ref, t, 2.0 if own2[t] else 0.0)
    krow = torch.randn((KV1, H1 * hd1), generator=g, device="cuda").half()
    vrow = torch.randn((KV1, H1 * hd1), generator=g, device="cuda").half()
    S.check(L.sp_hip_dual_write_layer(dc.ref, 0, 0, KV1, P(krow), P(vrow), H1 * hd1, S.DTYPE_F16), "dual write")
    ko, vo = torch.empty_like(krow), torch.empty_like(vrow)
    t_m = timed(lambda: S.check(L.sp_hip_dual_read_merged(dc.ref, 0, KV1, P(ko), P(vo), H1 * hd1, S.DTYPE_F16),
                                "dual read"))
    t_1 = timed(lambda: S.check(L.sp_hip_read_layer(c1.ref, 0, 0, KV1, P(ko), P(vo), H1 * hd1, S.DTYPE_F16, -1),
                                "ship read"))
    n2 = int(own2.sum())
    out["cfg1_dual_merged_read"] = {
        "us": round(t_m * 1e6, 1), "ship_only_read_us": round(t_1 * 1e6, 1), "sys2_positions": n2,
        "vecs_per_s": round(2 * H1 * KV1 / t_m, 1),
        "layout": "one layer x 8 heads x 32768 positions, K+V, fp16 rows; System 2 = sqfree on 20% of positions"}
    dc.free()
    sq1.free()
    # the same with System 2 = hier at the configs[4] geometry (hd 256 -> pad 330, 30/300, 2-bit residual;
    # W random, one per slot) beside an hd 256 ship cache, 8 heads x 32768 positions
    import numpy as np
    hd4 = 256
    sk4, tg4 = np.zeros(30, np.int32), np.zeros(300, np.int32)
    assert L.sp_hier_default_geometry(330, C.c_void_p(sk4.ctypes.data), C.c_void_p(tg4.ctypes.data)) == 30
    c4 = S.ShipCache(S.config(hd4, 1, H1), KV1, stream.cuda_stream)
    hc4 = S.HierCache(S.config(hd4, 1, H1), 330, sk4, tg4, S.band_config(30, [5, 5]), 2, KV1, H1,
                      stream=stream.cuda_stream)
    hc4.upload_W((np.random.default_rng(9).standard_normal((H1, 300, 30)) * 0.05).astype(np.float16).view(np.uint16))
    dc4 = S.DualCache(c4, hc4, S.DUAL_HIER, 1.0)
    for t in range(KV1):
        L.sp_hip_dual_route_position(dc4.ref, t, 2.0 if own2[t] else 0.0)
    krow4 = torch.randn((KV1, H1 * hd4), generator=g, device="cuda").half()
    S.check(L.sp_hip_dual_write_layer(dc4.ref, 0, 0, KV1, P(krow4), P(krow4), H1 * hd4, S.DTYPE_F16), "dual4 write")
    ko4 = torch.empty_like(krow4)
    vo4 = torch.empty_like(krow4)
    t_m4 = timed(lambda: S.check(L.sp_hip_dual_read_merged(dc4.ref, 0, KV1, P(ko4), P(vo4), H1 * hd4, S.DTYPE_F16),
                                 "dual4 read"))
    t_14 = timed(lambda: S.check(L.sp_hip_read_layer(c4.ref, 0, 0, KV1, P(ko4), P(vo4), H1 * hd4, S.DTYPE_F16, -1),
                                 "ship4 read"))
    out["cfg4_dual_hier_merged_read"] = {
        "us": round(t_m4 * 1e6, 1), "ship_only_read_us": round(t_14 * 1e6, 1), "sys2_positions": n2,
        "layout": "one layer x 8 heads x 32768 positions, hd 256, K+V, fp16 rows; System 2 = hier (pad 330) on 20%"}
    dc4.free()
    hc4.free()
    c4.free()
    del krow4, ko4, vo4
    # disk format v3 at the configs[1] layer shape: 4 layers x 8 heads x 32768 positions (33 MB of records
    # per layer file), save, load, and a partial load of K band 0 (+ the one V band), files under /tmp
    import tempfile
    cd = S.ShipCache(S.config(hd1, 4, H1), KV1, stream.cuda_stream)
    xs = torch.randn((4 * H1 * KV1, hd1), generator=g, device="cuda").half()
    S.check(L.sp_hip_write_all(cd.ref, 0, KV1, P(xs), P(xs), S.DTYPE_F16), "disk fill")
    del xs
    torch.cuda.synchronize()
    with tempfile.TemporaryDirectory(dir="/tmp") as td:
        prefix = os.path.join(td, "ctx").encode()
        file_bytes = 4 * H1 * KV1 * (76 + 50)
        t0 = time.perf_counter()
        S.check(L.sp_hip_cache_save(cd.ref, prefix, KV1, 1), "save")
        t_save = time.perf_counter() - t0
        t0 = time.perf_counter()
        n_l = L.sp_hip_cache_load(cd.ref, prefix, 1)
        t_load = time.perf_counter() - t0
        t0 = time.perf_counter()
        n_p = L.sp_hip_cache_load_partial(cd.ref, prefix, 1, 1)
        t_part = time.perf_counter() - t0
    assert n_l == KV1 and n_p == KV1
    out["cfg1_disk_v3"] = {"save_ms": round(t_save * 1e3, 1), "load_ms": round(t_load * 1e3, 1),
                           "load_partial_1band_ms": round(t_part * 1e3, 1), "file_mb": round(file_bytes / 1e6, 1),
                           "partial_read_mb": round(4 * H1 * KV1 * (22 + 50) / 1e6, 1),
                           "layout": "4 layers x 8 heads x 32768 positions, K 76 B + V 50 B records, files in /tmp"}
    cd.free()
    c1.free()
    del kt, vt, krow, vrow, ko, vo
    # sqfree+spinor, 12 layers x 4 KV heads x 65536 cells (4 x 16384), hd 128 -> pad 154,
    # skeleton 0.75 * 154 = 115, K 5/4/4/4/5, V one 3-bit band (as configs[3] asks; the reference hook
    # mirrors K's bands into V instead), 3-bit residuals
    L4, H4, N4 = 12, 4, 65536
    bits4 = (5, 4, 4, 4, 5)
    cfg = S.config(128, L4, H4, k_bits=bits4, v_bits=(3,))
    pad4 = L.sp_sqfree_pad_dim(128)
    c4 = S.SqfreeCache(cfg, N4, rbits=3, spinor=True, sk_k=int(pad4 * 0.75), stream=stream.cuda_stream)
    # rows in llama.cpp's cache layout: [layer][cell][head * hd + d]; one launch per layer and side
    x = (torch.randn((L4, N4, H4 * 128), generator=g, device="cuda")).half()
    y = torch.empty_like(x)
    B4, B4v = c4.c.bytes_per_pos_k, c4.c.bytes_per_pos_v

    def sq_call(fn, is_v, buf):
        def f():
            for layer in range(L4):
                a, b = (None, P(buf[layer])) if is_v else (P(buf[layer]), None)
                S.check(fn(c4.ref, layer, 0, N4, a, b, H4 * 128, S.DTYPE_F16))
        return f

    nv4 = L4 * H4 * N4
    r_ke = rate(nv4, 128, B4, timed(sq_call(L.sp_hip_sqfree_write_layer, 0, x)), "sqfree_k_enc")
    r_ve = rate(nv4, 128, B4v, timed(sq_call(L.sp_hip_sqfree_write_layer, 1, x)), "sqfree_v_enc")
    r_kd = rate(nv4, 128, B4, timed(sq_call(L.sp_hip_sqfree_read_layer, 0, y)), "sqfree_k_dec")
    r_vd = rate(nv4, 128, B4v, timed(sq_call(L.sp_hip_sqfree_read_layer, 1, y)), "sqfree_v_dec")
    out["cfg4_sqfree_spinor"] = {"enc": r_ke, "dec": r_kd, "v_enc": r_ve, "v_dec": r_vd,
                                 "record_bytes": [B4, B4v], "pad_dim": pad4, "skeleton": c4.c.sk_k,
                                 "calls": f"{L4} layers x {H4} heads x {N4} positions, one call per layer and side "
                                          f"(enc/dec: K 5/4/4/4/5; v_enc/v_dec: V one 3-bit band)"}
    # configs[3] decode: fused attention over the sqfree records, batch 4: the four sequences are the
    # position ranges [16384 i, 16384 (i + 1)) of one cache layer (4 KV heads; K and V from distinct
    # rows), 32 query heads per sequence (GQA 8)
    NA4, NQ4, NB4 = 16384, 32, 4
    c4a = S.SqfreeCache(S.config(128, 1, H4, k_bits=bits4, v_bits=(3,)), NB4 * NA4, rbits=3, spinor=True,
                        sk_k=int(pad4 * 0.75), stream=stream.cuda_stream)
    S.check(L.sp_hip_sqfree_write_layer(c4a.ref, 0, 0, NB4 * NA4, P(x[0, :NB4 * NA4]), P(x[1, :NB4 * NA4]),
                                        H4 * 128, S.DTYPE_F16))
    q4 = torch.randn((NB4, NQ4, 128), generator=g, device="cuda")
    o4 = torch.empty((NB4, NQ4, 128), device="cuda")
    s4 = torch.empty((NQ4, NA4), device="cuda")
    sc4 = C.c_float(1.0 / math.sqrt(128))
    t_one = timed(lambda: S.check(L.sp_hip_sqfree_attn_decode(c4a.ref, 0, NA4, P(q4[0]), NQ4, sc4, None, P(o4[0]),
                                                              sp)))
    t_kq4 = timed(lambda: S.check(L.sp_hip_sqfree_attn_decode(c4a.ref, 0, NA4, P(q4[0]), NQ4, sc4, P(s4), None, sp)))
    st4, ln4 = seq_table([NA4 * i for i in range(NB4)], [NA4] * NB4)
    t_b4 = timed(lambda: S.check(L.sp_hip_sqfree_attn_decode_seqs(c4a.ref, 0, NB4, st4[1], ln4[1], P(q4), NQ4, sc4,
                                                                  None, P(o4), sp)))
    rec4 = H4 * NA4 * (B4 + B4v)
    out["cfg4_sqfree_fused_attn"] = {
        "layer_us": round(t_one * 1e6, 1), "kq_only_layer_us": round(t_kq4 * 1e6, 1),
        "batch4_step_layer_us": round(t_b4 * 1e6, 1), "us_per_step_48_layers": round(48 * t_b4 * 1e6, 1),
        "decode_tokens_per_s_48_layers": round(NB4 / (48 * t_b4), 1),
        "record_gbs": round(rec4 / t_one / 1e9, 1), "batch4_record_gbs": round(NB4 * rec4 / t_b4 / 1e9, 1),
        "record_floor_us": round(rec4 / (HBM_PEAK_GBS * 1e3), 2),
        "fp16_layer_floor_us": round(H4 * NA4 * 2 * 128 * 2 / (HBM_PEAK_GBS * 1e3), 2),
        "layout": f"{H4} KV heads x {NA4} positions, {NQ4} query heads (GQA 8), K {B4} B + V {B4v} B records "
                  f"(pad {pad4}, skeleton {c4a.c.sk_k}); layer_us: one sequence's call; batch4_step: one "
                  f"batched call (sp_hip_sqfree_attn_decode_seqs) over {NB4} sequences"}
    c4a.free()
    c4.free()
    del x, y
    # hier, hd 256 -> pad 330, 8 KV heads x (8 x 131072) cells of one layer in one launch per side
    H5, N5, hd5 = 8, 8 * 131072, 256
    pad5 = L.sp_sqfree_pad_dim(hd5)
    n_sk = L.sp_hier_default_geometry(pad5, None, None)
    import numpy as np
    sk = np.zeros(n_sk, np.int32)
    tg = np.zeros(pad5 - n_sk, np.int32)
    L.sp_hier_default_geometry(pad5, C.c_void_p(sk.ctypes.data), C.c_void_p(tg.ctypes.data))
    c5 = S.HierCache(S.config(hd5, 1, H5), pad5, sk, tg, S.band_config(n_sk, [5, 5]), 2, N5, H5,
                     stream=stream.cuda_stream)
    Wh = (np.random.default_rng(5).standard_normal((H5, pad5 - n_sk, n_sk)) * 0.05).astype(np.float16)
    c5.upload_W(Wh.view(np.uint16))
    x = torch.empty((N5, H5 * hd5), dtype=torch.float16, device="cuda")
    for r0 in range(0, N5, 1 << 18):  # bounded fp32 temporaries
        x[r0:r0 + (1 << 18)] = torch.randn((min(1 << 18, N5 - r0), H5 * hd5), generator=g, device="cuda").half()
    y = torch.empty_like(x)
    B5 = c5.c.bytes_per_pos_k

    def hi_write():
        S.check(L.sp_hip_hier_write_layer(c5.ref, 0, 0, N5, P(x), None, H5 * hd5, S.DTYPE_F16))

    def hi_read():
        S.check(L.sp_hip_hier_read_layer(c5.ref, 0, 0, N5, P(y), None, H5 * hd5, S.DTYPE_F16))

    out["cfg5_hier"] = {"enc": rate(H5 * N5, hd5, B5, timed(hi_write), "hier_enc"),
                        "dec": rate(H5 * N5, hd5, B5, timed(hi_read), "hier_dec"),
                        "record_bytes": B5, "pad_dim": pad5, "skeleton": n_sk,
                        "calls": f"1 layer x {H5} heads x {N5} positions, one call (K)"}
    # the reference caller's per-vector hook path through the bridge (host pointers): one
    # sp_llama_write_k / write_v / read_k / read_v per vector, each an H2D or D2H copy, a launch
    # and a stream sync (the Python call overhead, ~1 us, is included)
    saved = {k: os.environ.get(k) for k in ("SHANNON_PRIME_ENABLED", "SHANNON_PRIME_BACKEND")}
    os.environ["SHANNON_PRIME_ENABLED"] = "1"
    os.environ["SHANNON_PRIME_BACKEND"] = "hip"
    try:
        prm = S.SpLlamaParams(128, 2, 8, 4096, S.BACKEND_HIP, None, None)
        ctx = L.sp_llama_init(C.byref(prm))
        if ctx:
            vec = np.random.default_rng(3).standard_normal((64, 128)).astype(np.float32)
            outv = np.empty(128, np.float32)
            fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
            n_calls = 256
            times = {}
            for name, call in (("write_k", lambda i: L.sp_llama_write_k(ctx, 1, i % 8, i, fp(vec[i % 64]))),
                               ("write_v", lambda i: L.sp_llama_write_v(ctx, 1, i % 8, i, fp(vec[i % 64]))),
                               ("read_k", lambda i: L.sp_llama_read_k(ctx, 1, i % 8, i, fp(outv))),
                               ("read_v", lambda i: L.sp_llama_read_v(ctx, 1, i % 8, i, fp(outv)))):
                # the first calls load each kernel's code object (records at odd positions of a
                # 50 B V record are not 16 B aligned and take the row kernel) and allocate the
                # staging buffers: 64 untimed calls, then the median of individually timed ones
                for i in range(64):
                    call(i)
                per = []
                for i in range(n_calls):
                    t0 = time.perf_counter()
                    call(i)
                    per.append(time.perf_counter() - t0)
                times[name] = float(np.median(per)) * 1e6
            L.sp_llama_free(ctx)
            per_tok = 32 * 8 * (times["write_k"] + times["write_v"] + times["read_k"] + times["read_v"])
            out["cfg1_hook_per_vector"] = {
                "us_per_call_median": {k: round(v, 2) for k, v in times.items()},
                "us_per_token_32x8_write_and_read": round(per_tok, 1),
                "layout": "bridge backend hip, hd 128, one fp32 vector per call (host pointer), synchronous; "
                          "steady state: median of 256 calls after 64 untimed"}
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    # configs[4] fused decode attention over hier records: one sequence's layer at 131072
    # positions x 8 KV heads (K and V from the rows above), 16 query heads (GQA 2)
    NA, NQ5 = 131072, 16
    c6 = S.HierCache(S.config(hd5, 1, H5), pad5, sk, tg, S.band_config(n_sk, [5, 5]), 2, NA, H5,
                     stream=stream.cuda_stream)
    c6.upload_W(Wh.view(np.uint16))
    S.check(L.sp_hip_hier_write_layer(c6.ref, 0, 0, NA, P(x[:NA]), P(x[NA:2 * NA]), H5 * hd5, S.DTYPE_F16))
    q5 = torch.randn((NQ5, hd5), generator=g, device="cuda")
    o5 = torch.empty((NQ5, hd5), device="cuda")
    s5 = torch.empty((NQ5, NA), device="cuda")
    sc5 = C.c_float(1.0 / math.sqrt(hd5))
    t_full = timed(lambda: S.check(L.sp_hip_hier_attn_decode(c6.ref, 0, NA, P(q5), NQ5, sc5, None, P(o5), sp)))
    t_kq = timed(lambda: S.check(L.sp_hip_hier_attn_decode(c6.ref, 0, NA, P(q5), NQ5, sc5, P(s5), None, sp)))
    rec_b = 2 * H5 * NA * B5
    out["cfg5_hier_fused_attn"] = {
        "layer_us": round(t_full * 1e6, 1), "kq_only_layer_us": round(t_kq * 1e6, 1),
        "us_per_token_34_layers": round(34 * t_full * 1e6, 1),
        "record_gbs": round(rec_b / t_full / 1e9, 1),
        "fp16_layer_floor_us": round(2 * H5 * NA * hd5 * 2 / (HBM_PEAK_GBS * 1e3), 1),
        "layout": f"1 layer x {H5} KV heads x {NA} positions, {NQ5} query heads, hd {hd5} (pad {pad5}), "
                  f"K+V hier records of {B5} B; per sequence (a batch of 8 is 8 such calls)"}
    c6.free()
    c5.free()
    # configs[4] sustained: batch-8 decode interleaved with prefill-chunk compression. Eight
    # sequences are the position ranges [131072 i, 131072 (i + 1)) of one cache layer (8 KV heads;
    # K from the rows above, V from their decoded copy); one step of a layer decodes all eight
    # (one batched fused attention call, 16 query heads each) and compresses one 2048-token chunk of a
    # ninth sequence's new K and V into the layer's positions [1048576, 1050624)
    NB, CHK = 8, 2048
    c7 = S.HierCache(S.config(hd5, 1, H5), pad5, sk, tg, S.band_config(n_sk, [5, 5]), 2, NB * NA + CHK, H5,
                     stream=stream.cuda_stream)
    c7.upload_W(Wh.view(np.uint16))
    S.check(L.sp_hip_hier_write_layer(c7.ref, 0, 0, NB * NA, P(x), P(y), H5 * hd5, S.DTYPE_F16))
    q8 = torch.randn((NB, NQ5, hd5), generator=g, device="cuda")
    o8 = torch.empty((NB, NQ5, hd5), device="cuda")
    kc, vc = x[:CHK], x[CHK:2 * CHK]
    st8, ln8 = seq_table([NA * i for i in range(NB)], [NA] * NB)

    def decode8():
        S.check(L.sp_hip_hier_attn_decode_seqs(c7.ref, 0, NB, st8[1], ln8[1], P(q8), NQ5, sc5, None, P(o8), sp))

    def chunk():
        S.check(L.sp_hip_hier_write_layer(c7.ref, 0, NB * NA, CHK, P(kc), P(vc), H5 * hd5, S.DTYPE_F16))

    def step():
        decode8()
        chunk()

    t_dec8, t_chunk, t_step = timed(decode8), timed(chunk), timed(step)
    out["cfg5_batch8_with_prefill_chunk"] = {
        "step_layer_us": round(t_step * 1e6, 1), "decode8_layer_us": round(t_dec8 * 1e6, 1),
        "chunk_layer_us": round(t_chunk * 1e6, 1),
        "chunk_vecs_per_s": round(2 * H5 * CHK / t_chunk, 1),
        "decode_tokens_per_s_34_layers": round(NB / (34 * t_step), 1),
        "decode8_record_gbs": round(NB * rec_b / t_dec8 / 1e9, 1),
        "layout": f"{NB} sequences x {NA} positions x {H5} KV heads, {NQ5} query heads each, hd {hd5} (pad {pad5}); "
                  f"per layer and step: one batched fused attention call (sp_hip_hier_attn_decode_seqs) over "
                  f"{NB} sequences, then one {CHK}-token K+V chunk compressed"}
    c7.free()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--attn-iters", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", choices=["codec", "attn", "variants", "all"], default="all")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run one plain device copy of the K inputs (known bytes) for PMC scaling")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the codec shards by layer or KV head with no exchange between GPUs)", file=sys.stderr)
        sys.exit(2)

    import torch
    import sp_hip as S

    L = S.lib()
    assert torch.cuda.is_available() and L.sp_hip_available() == 1, "needs an MI355X (gfx950)"
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream()
    sptr = C.c_void_p(stream.cuda_stream)
    n_slots = LAYERS * KVH
    cfg = S.config(HD, LAYERS, KVH, k_bits=K_BITS, v_bits=V_BITS)
    cc = S.ShipCache(cfg, POS, stream.cuda_stream)
    kB, vB = cc.c.k_bands.total_bytes, cc.c.v_bands.total_bytes
    log(f"[bench] cache: {n_slots} slots x {POS} pos, K {kB} B, V {vB} B per vector")
    k, v = make_inputs(torch, n_slots, POS, HD)
    kr = torch.empty_like(k)
    vr = torch.empty_like(v)
    torch.cuda.synchronize()
    n_vec = n_slots * POS
    per = algorithmic_bytes(HD, kB, vB)

    def P(t):
        return C.c_void_p(t.data_ptr())

    steps = {
        "k_enc": lambda: L.sp_hip_write_all(cc.ref, 0, POS, P(k), None, S.DTYPE_F16),
        "v_enc": lambda: L.sp_hip_write_all(cc.ref, 0, POS, None, P(v), S.DTYPE_F16),
        "k_dec": lambda: L.sp_hip_read_all(cc.ref, 0, POS, P(kr), None, S.DTYPE_F16, -1),
        "v_dec": lambda: L.sp_hip_read_all(cc.ref, 0, POS, None, P(vr), S.DTYPE_F16, -1),
    }
    result = {}
    if args.copy_calib:
        # one plain copy of n_slots * POS * HD fp16 (reads and writes that many bytes)
        kc = torch.empty_like(k)
        kc.copy_(k)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: {k.numel() * 2} bytes read and written")
        del kc
    if args.only in ("codec", "all"):
        for _ in range(args.warmup):
            for f in steps.values():
                S.check(f(), "codec")
        torch.cuda.synchronize()
        ev = {n: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(args.steps)] for n in steps}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            for n, f in steps.items():
                ev[n][i][0].record(stream)
                S.check(f(), n)
                ev[n][i][1].record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        kern_ms = {n: sum(a.elapsed_time(b) for a, b in ev[n]) / args.steps for n in steps}
        ms_step = wall * 1e3 / args.steps
        step_bytes = n_vec * sum(per.values())
        dom = max(kern_ms, key=kern_ms.get)
        dom_gbs = n_vec * per[dom] / (kern_ms[dom] * 1e-3) / 1e9
        log("[bench] kernel ms: " + ", ".join(f"{n}={t:.3f}" for n, t in kern_ms.items()))
        result.update({
            "metric": "KV vecs/s compress+decompress (HBM GB/s, %roofline); fused dqKQ us/tok @32K",
            "value": round(2 * n_vec / (ms_step * 1e-3), 1),
            "unit": "KV vecs/s",
            "ms_per_step": round(ms_step, 4),
            "hbm_gbs": round(step_bytes / (ms_step * 1e-3) / 1e9, 1),
            "hbm_frac": round(step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "kernel_ms": {n: round(t, 4) for n, t in kern_ms.items()},
            "kernel_gbs": {n: round(n_vec * per[n] / (t * 1e-3) / 1e9, 1) for n, t in kern_ms.items()},
            "roofline": {"kernel": KERNEL_NAMES[dom],
                         "bound": "hbm", "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(dom_gbs / HBM_PEAK_GBS, 4),
                         "traffic": traffic_from_profile(dom),
                         "traffic_source": "profiles/hbm_traffic_ship_codec_cfg1.json (rocprofv3 --pmc "
                                           "FETCH_SIZE/WRITE_SIZE of this kernel, copy-calibrated); "
                                           "read from the committed profile, not measured in this run",
                         "bytes_per_launch": n_vec * per[dom], "avg_ms": round(kern_ms[dom], 4)},
        })
        simds = 4 * torch.cuda.get_device_properties(0).multi_processor_count
        vb = {n: valu_bound_s(n_vec, VALU_PER_TILE[n], simds) * 1e3 for n in steps}
        result["valu_issue"] = {
            "per_tile": {n: VALU_PER_TILE[n] for n in steps},
            "bound_ms": {n: round(t, 4) for n, t in vb.items()},
            "frac": {n: round(vb[n] / kern_ms[n], 3) for n in steps},
            "step_bound_ms": round(sum(vb.values()), 4),
            "note": "VALU-issue bound of each bit-exact codec kernel (instructions per 64-vector tile from "
                    "rocprofv3 SQ_INSTS_VALU, profiles/valu_codec_kernels.md; 4 cycles per wave64 "
                    "instruction per SIMD at 2.4 GHz); the step's sum exceeds its 1.34 ms HBM floor"}
    if args.only in ("attn", "all"):
        # fused decode attention over the compressed 32K cache, all 32 layers per token
        if args.only == "attn":
            S.check(L.sp_hip_write_all(cc.ref, 0, POS, P(k), P(v), S.DTYPE_F16), "write_all")
        q = torch.randn((LAYERS, NQ, HD), dtype=torch.float32, device="cuda")
        out = torch.empty((LAYERS, NQ, HD), dtype=torch.float32, device="cuda")
        scale = C.c_float(1.0 / math.sqrt(HD))

        def fused():
            S.check(L.sp_hip_attn_decode_all_layers(cc.ref, POS, P(q), NQ, scale, P(out), sptr), "attn")

        # scores of every layer, [layer][query head][position]; like the full path, the
        # per-layer launches come from the library's C loop (a Python loop costs ~5 us per
        # call, most of a scores-only layer)
        sc_all = torch.empty((LAYERS, NQ, POS), dtype=torch.float32, device="cuda")

        def fused_kq(mb=-1):
            S.check(L.sp_hip_attn_scores_all_layers(cc.ref, POS, P(q), NQ, scale, P(sc_all), mb, sptr), "kq")

        def fused_bands(want_out, mb=2):
            # band-limited decode (K bands >= mb read as 0; the single V band stays)
            def f():
                if not want_out:
                    return fused_kq(mb)
                for layer in range(LAYERS):
                    S.check(L.sp_hip_attn_decode_bands(cc.ref, layer, POS, P(q[layer]), NQ, scale, None,
                                                       P(out[layer]), mb, sptr), "bands")
            return f

        def fp16():
            for layer in range(LAYERS):
                S.check(L.sp_hip_attn_decode_f16(P(k), P(v), KVH, POS, HD, layer, POS, P(q[layer]), NQ, scale,
                                                 None, P(out[layer]), sptr), "attn_f16")

        def timeit(f):
            for _ in range(3):  # warm-up calls: the first ones after a change of work run slower
                f()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(args.attn_iters):
                f()
            b.record(stream)
            torch.cuda.synchronize()
            return a.elapsed_time(b) / args.attn_iters * 1e3  # us per token

        # uncompressed fp16 attention through torch's batched GEMMs (rocBLAS / hipBLASLt):
        # per layer scores = K . q (KV head-major, contiguous operands), softmax, . V
        kl = k.view(LAYERS, KVH, POS, HD)
        vl = v.view(LAYERS, KVH, POS, HD)
        qh = q.view(LAYERS, KVH, NQ // KVH, HD).transpose(2, 3).contiguous().half()  # [L][KVH][HD][G]

        def torch_kq():
            for layer in range(LAYERS):
                torch.bmm(kl[layer], qh[layer])

        def torch_attn():
            for layer in range(LAYERS):
                s = torch.bmm(kl[layer], qh[layer]).float() * scale.value
                p = torch.softmax(s, dim=1).transpose(1, 2).contiguous().half()
                torch.bmm(p, vl[layer])

        # the compressed-cache variants first, back to back, then the fp16 baselines
        us_fused, us_kq = timeit(fused), timeit(fused_kq)
        us_kq_b2, us_attn_b2 = timeit(fused_bands(False)), timeit(fused_bands(True))
        us_f16, us_tkq, us_tattn = timeit(fp16), timeit(torch_kq), timeit(torch_attn)
        kv_bytes = LAYERS * KVH * POS * (kB + vB)
        result.update({
            "fused_dqkq_us_per_tok": round(us_fused, 1),
            "fused_kq_only_us_per_tok": round(us_kq, 1),
            "fused_kq_only_2bands_us_per_tok": round(us_kq_b2, 1),
            "fused_dqkq_2bands_us_per_tok": round(us_attn_b2, 1),
            "fp16_torch_kq_us_per_tok": round(us_tkq, 1),
            "fp16_torch_attn_us_per_tok": round(us_tattn, 1),
            "fp16_attn_us_per_tok": round(us_f16, 1),
            "fp16_kq_floor_us_per_tok": round(LAYERS * KVH * POS * 2 * HD / (HBM_PEAK_GBS * 1e3), 1),
            "fp16_attn_floor_us_per_tok": round(LAYERS * KVH * POS * 4 * HD / (HBM_PEAK_GBS * 1e3), 1),
            "fused_attn_gbs": round(kv_bytes / (us_fused * 1e-6) / 1e9, 1),
            "fused_attn_floor_us_per_tok": round(kv_bytes / (HBM_PEAK_GBS * 1e3), 1),
        })
        log(f"[bench] fused attn {us_fused:.1f} us/tok, KQ-only {us_kq:.1f}; fp16 torch attn {us_tattn:.1f}, "
            f"torch KQ {us_tkq:.1f}, fp16 lane kernel {us_f16:.1f}; 2 K bands: KQ {us_kq_b2:.1f}, "
            f"attn {us_attn_b2:.1f}")
    if args.only in ("variants", "all"):
        result["variants"] = bench_variants(torch, S, L, stream)
        log("[bench] variants: " + json.dumps(result["variants"]))
    result.update({
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "llama3-8b-shaped KV codec, configs[1]", "layers": LAYERS, "kv_heads": KVH,
                   "q_heads": NQ, "head_dim": HD, "positions": POS, "k_bits": "5,5,4,3", "v_bits": "3",
                   "mobius": True, "vectors_per_step": 2 * n_vec, "io": "fp16 in, fp16 out, records in HBM"},
    })
    if not args.no_cpu:
        if args.only in ("codec", "all"):
            log("[bench] checking a sample of the full-size run against the oracle")
            result["parity_sample_mismatches"] = parity_sample(S, cc, k, v, kr, kB, vB, n_slots)
        log("[bench] timing CPU baseline (oracle, one thread and all cores)")
        result["cpu_baseline"] = cpu_baseline()
    cc.free()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
