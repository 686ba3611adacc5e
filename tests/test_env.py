"""The SHANNON_PRIME_* environment as the bridges read it (CPU, no caches made).

sp_llama_resolve_env returns the configuration sp_llama_init_with_role builds
(src/tools/shannon_prime_llama.c:73-307): the kill switch, head-dim defaults,
band lists whose length sets the band count, ternary band masks, the draft
role's precedence and presets, and the backend names.
sp_llama_sqfree_config_from_env is the sqfree bridge's reading
(src/tools/shannon_prime_llama_sqfree.c:48-101)."""
import ctypes as C
import os

import pytest

import sp_hip as S


@pytest.fixture
def env(monkeypatch):
    for k in list(os.environ):
        if k.startswith("SHANNON_PRIME_"):
            monkeypatch.delenv(k)

    def set_(**kw):
        for k, v in kw.items():
            monkeypatch.setenv("SHANNON_PRIME_" + k, v)
    return set_


def resolve(hd=128, role=S.ROLE_DEFAULT, backend=S.BACKEND_CPU):
    p = S.SpLlamaParams(hd, 2, 4, 64, backend, None, None)
    cfg = S.SpConfig()
    be = C.c_int(-7)
    rc = S.lib().sp_llama_resolve_env(C.byref(p), role, C.byref(cfg), C.byref(be))
    return rc, cfg, be.value


def kbits(cfg):
    return list(cfg.k_band_bits[:cfg.k_n_bands])


def vbits(cfg):
    return list(cfg.v_band_bits[:cfg.v_n_bands])


@pytest.mark.parametrize("text,on", [(None, 0), ("0", 0), ("1", 1), ("y", 1), ("Yes", 1), ("", 0), ("true", 0)])
def test_enabled_switch(env, text, on):
    if text is not None:
        env(ENABLED=text)
    assert resolve()[0] == on


def test_head_dim_defaults(env):
    env(ENABLED="1")
    rc, cfg, be = resolve(128)
    assert rc == 1 and kbits(cfg) == [5, 5, 4, 3] and vbits(cfg) == [3]
    assert cfg.use_mobius_mask == 1 and cfg.k_ternary_mask == 0 and cfg.use_fp8 == 0 and be == S.BACKEND_CPU
    for hd in (64, 96):
        rc, cfg, _ = resolve(hd)
        assert kbits(cfg) == [5, 4, 4] and vbits(cfg) == [5]
    assert kbits(resolve(256)[1]) == [5, 5, 4, 3]


@pytest.mark.parametrize("text,want", [
    ("3,3,3,3,3", [3, 3, 3, 3, 3]),   # the count of values sets the band count
    ("5,,4", [5, 0, 4]),              # an empty value reads 0
    ("5,4,", [5, 4]),                 # a trailing comma adds nothing
    (",5", [0, 5]),
    (" 6, 2", [6, 2]),                # leading blanks as atoi skips them
    (",".join(["4"] * 20), [4] * 16),  # at most 16 bands
])
def test_band_lists(env, text, want):
    env(ENABLED="1", K_BITS=text, V_BITS=text)
    _, cfg, _ = resolve()
    assert kbits(cfg) == want and vbits(cfg) == want


def test_empty_band_list_keeps_defaults(env):
    env(ENABLED="1", K_BITS="", V_BITS="")
    _, cfg, _ = resolve()
    assert kbits(cfg) == [5, 5, 4, 3] and vbits(cfg) == [3]


@pytest.mark.parametrize("text,mask", [
    ("3", 1 << 3), ("2,3", 0b1100), (" 1 , x,40,31", (1 << 1) | (1 << 31)), ("-1,2", 1 << 2),
    ("", 0), ("3x", 1 << 3), ("1 2", 1 << 1), (",,\t4", 1 << 4),
])
def test_ternary_masks(env, text, mask):
    env(ENABLED="1", K_TERNARY_BANDS=text, V_TERNARY_BANDS=text)
    _, cfg, _ = resolve()
    assert cfg.k_ternary_mask == mask and cfg.v_ternary_mask == mask


def test_draft_precedence(env):
    env(ENABLED="1", K_BITS="5,5,4,3", DRAFT_K_BITS="2,2", MOBIUS="1", DRAFT_MOBIUS="0")
    _, d, _ = resolve(role=S.ROLE_DRAFT)
    assert kbits(d) == [2, 2] and d.use_mobius_mask == 0
    for role in (S.ROLE_DEFAULT, S.ROLE_TARGET):
        _, c, _ = resolve(role=role)
        assert kbits(c) == [5, 5, 4, 3] and c.use_mobius_mask == 1
    env(DRAFT_K_BITS="")  # an empty draft variable falls back to the global one
    assert kbits(resolve(role=S.ROLE_DRAFT)[1]) == [5, 5, 4, 3]
    env(DRAFT_ENABLED="0")
    assert resolve(role=S.ROLE_DRAFT)[0] == 0 and resolve()[0] == 1


@pytest.mark.parametrize("preset,k,v", [("aggressive", [2, 1], [1]), ("ternary", [2, 2], [2]),
                                        ("ship", [5, 5, 4, 3], [3]), ("nonsense", [5, 5, 4, 3], [3])])
def test_draft_presets(env, preset, k, v):
    env(ENABLED="1", DRAFT_PRESET=preset)
    _, d, _ = resolve(role=S.ROLE_DRAFT)
    assert kbits(d) == k and vbits(d) == v
    _, c, _ = resolve()  # the preset is for draft contexts only
    assert kbits(c) == [5, 5, 4, 3] and vbits(c) == [3]


def test_explicit_bits_override_a_preset(env):
    env(ENABLED="1", DRAFT_PRESET="aggressive", DRAFT_K_BITS="4,4,4")
    _, d, _ = resolve(role=S.ROLE_DRAFT)
    assert kbits(d) == [4, 4, 4] and vbits(d) == [1]


def test_flags_norm_and_backends(env):
    env(ENABLED="1", MOBIUS="0", FP8="1", VHT2_NORM="stage")
    _, cfg, _ = resolve()
    assert cfg.use_mobius_mask == 0 and cfg.use_fp8 == 1 and cfg.vht2_norm == 1
    for name, want in (("cpu", S.BACKEND_CPU), ("hip", S.BACKEND_HIP), ("rocm", S.BACKEND_HIP),
                       ("cuda", S.BACKEND_HIP), ("hexagon", S.BACKEND_HEXAGON), ("adreno", S.BACKEND_ADRENO),
                       ("vulkan", S.BACKEND_VULKAN)):
        env(BACKEND=name)
        assert resolve(backend=S.BACKEND_CPU)[2] == want, name
    env(BACKEND="xyz")  # unknown names leave the caller's backend
    assert resolve(backend=S.BACKEND_HIP)[2] == S.BACKEND_HIP
    env(BACKEND="cpu", DRAFT_BACKEND="hip")
    assert resolve(role=S.ROLE_DRAFT)[2] == S.BACKEND_HIP and resolve()[2] == S.BACKEND_CPU


def sqfree_env():
    out = S.SpLlamaSqfreeConfig()
    S.lib().sp_llama_sqfree_config_from_env(C.byref(out))
    return out


def test_sqfree_bridge_environment(env):
    c = sqfree_env()
    assert (c.sqfree_enabled, c.spinor_enabled, c.residual_bits) == (0, 0, 3)
    assert abs(c.sk_frac - 0.75) < 1e-7 and list(c.k_band_bits[:c.n_k_bands]) == [5, 5, 4, 3]
    assert not S.lib().sp_llama_sqfree_init(128, 2, 2, 16)  # off: NULL, nothing created
    env(SQFREE="yes")  # this bridge wants exactly "1"
    assert sqfree_env().sqfree_enabled == 0
    env(SQFREE="1")
    c = sqfree_env()
    assert c.sqfree_enabled == 1 and list(c.k_band_bits[:c.n_k_bands]) == [5, 4, 4, 4, 5]
    env(SQFREE="0", SPINOR="1")  # the spinor turns the sqfree path on
    c = sqfree_env()
    assert c.sqfree_enabled == 1 and c.spinor_enabled == 1
    for text, want in (("7", 4), ("0", 1), ("", 1), ("2", 2)):
        env(RESIDUAL_BITS=text)
        assert sqfree_env().residual_bits == want
    for text, want in (("0.05", 0.1), ("2", 1.0), ("0.5", 0.5)):
        env(SK_FRAC=text)
        assert abs(sqfree_env().sk_frac - want) < 1e-7
    env(K_BITS="3,3,3,3,3")
    c = sqfree_env()
    assert list(c.k_band_bits[:c.n_k_bands]) == [3] * 5
    env(K_BITS="")
    assert sqfree_env().n_k_bands == 0


@pytest.mark.skipif(os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK),
                    reason="GPU visible: the no-GPU failure path does not apply")
def test_core_variant_caches_need_a_gpu():
    cfg = S.config(128, 1, 1)
    sq = S.SpSqfreeCache()
    assert S.lib().sp_sqfree_cache_init(C.byref(sq), C.byref(cfg), 16, 3, 1) == -1
    hc = S.SpHierCache()
    assert S.lib().sp_hier_cache_init(C.byref(hc), C.byref(cfg), 16, 0, 0, None, 2) == -1
    assert S.lib().sp_hier_cache_init(C.byref(hc), C.byref(cfg), 16, 1, 0, None, 2) == -1
    assert "level" in S.last_error()
    S.lib().sp_sqfree_cache_free(C.byref(sq))
    S.lib().sp_hier_cache_free(C.byref(hc))
