"""Exhaustive CPU checks of the band quantizer's short arithmetic forms.

The lane codec divides a band's amax by its largest level with one multiply
and two fmas, takes the reciprocal of the stored fp16 scale with one Newton
step from v_rcp_f32, and sums the code fields into the record words
(shannon-prime-llama_amd/csrc/sp_lane.h: div_by_level, rcp_f16_scale,
rec_add_code). tests/cpp/codec_arith_check.c checks each form against IEEE
division / rint over every fp32 significand (division), every fp16
significand with starts within +-3 ulp (reciprocal) and every half-integer
neighbourhood (codes), so the quantizer stays bit-identical to
kernel_band_quantize_simple (shannon_prime_cuda.cu:131-204).
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def test_quantizer_arithmetic_is_exact(tmp_path):
    exe = str(tmp_path / "codec_arith_check")
    subprocess.run(["gcc", "-std=c11", "-O2", "-ffp-contract=off", "-Wall", "-Wextra", "-Werror",
                    os.path.join(HERE, "cpp", "codec_arith_check.c"), "-o", exe, "-lm"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[-1] == "OK"
    assert sum("div_by_level" in ln for ln in lines) == 7  # m = 1, 3, ..., 127
    assert all(" 0 mismatches" in ln for ln in lines[:-1])


def test_float_reciprocal_division_is_exact():
    """The block transforms of the fused attention's prep and merge kernels
    (shannon-prime-llama_amd/csrc/sp_hier_attn.hip: div_small) take floor(a / d) as
    trunc((a + 0.5) * fl(1 / d)) in fp32. Checked against integer division for every
    a < 4096 and d < 1024 (the transforms use a, d <= 330), and at the stated limits
    a < 2^20 for a spread of divisors."""
    import numpy as np

    a = np.arange(4096, dtype=np.int64)
    for d in range(1, 1024):
        inv = np.float32(1.0) / np.float32(d)
        got = ((a.astype(np.float32) + np.float32(0.5)) * inv).astype(np.int64)
        assert np.array_equal(got, a // d), d
    big = np.arange(0, 1 << 20, 7, dtype=np.int64)
    for d in (1, 2, 3, 5, 7, 11, 330, 1000, 1021, 1023):
        inv = np.float32(1.0) / np.float32(d)
        got = ((big.astype(np.float32) + np.float32(0.5)) * inv).astype(np.int64)
        assert np.array_equal(got, big // d), d
