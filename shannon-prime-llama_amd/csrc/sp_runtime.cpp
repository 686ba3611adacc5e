// sp_runtime.cpp -- host runtime of libshannon_prime_hip.so: config and band
// geometry, launch plans, the ship / sqfree / hier device caches, the
// sp_shadow_cache_t host API over the GPU, fused attention wrappers.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <string>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <numeric>
#include <atomic>
#include <mutex>
#include <vector>

#include "../../include/shannon_prime.h"
#include "../../include/sp_hip.h"
#include "sp_internal.h"

// ===========================================================================
// errors
// ===========================================================================
static thread_local char g_err[512];

static void set_err_v(const char *fmt, va_list ap) {
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    if (getenv("SHANNON_PRIME_VERBOSE")) fprintf(stderr, "[Shannon-Prime HIP] %s\n", g_err);
}

static void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    set_err_v(fmt, ap);
    va_end(ap);
}

// The same message slot for the library's other source files.
void sp_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    set_err_v(fmt, ap);
    va_end(ap);
}

static bool hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    set_err("%s: %s", what, hipGetErrorString(e));
    return false;
}

extern "C" const char *sp_hip_last_error(void) { return g_err; }

extern "C" int sp_hip_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
    return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

// ===========================================================================
// core config / geometry (host)
// ===========================================================================
extern "C" void sp_config_init(sp_config_t *cfg, int head_dim, int n_layers, int n_heads_kv) {
    memset(cfg, 0, sizeof(*cfg));
    cfg->head_dim = head_dim;
    cfg->n_layers = n_layers;
    cfg->n_heads_kv = n_heads_kv;
    // ship defaults (shannon_prime_llama.c:238-252): K 5/5/4/3, V flat 3
    cfg->k_n_bands = 4;
    cfg->k_band_bits[0] = 5;
    cfg->k_band_bits[1] = 5;
    cfg->k_band_bits[2] = 4;
    cfg->k_band_bits[3] = 3;
    cfg->v_n_bands = 1;
    cfg->v_band_bits[0] = 3;
    cfg->use_mobius_mask = 1;
    cfg->vht2_norm = SP_VHT2_NORM_FINAL;
}

extern "C" void sp_band_config_init_ext(sp_band_config_t *bc, int head_dim, int n_bands,
                                        const int *band_bits, uint32_t ternary_mask) {
    memset(bc, 0, sizeof(*bc));
    if (n_bands < 1) n_bands = 1;
    if (n_bands > SP_MAX_BANDS) n_bands = SP_MAX_BANDS;
    bc->head_dim = head_dim;
    bc->n_bands = n_bands;
    bc->band_size = head_dim / n_bands;
    bc->ternary_mask = ternary_mask;
    int total = 0;
    for (int b = 0; b < n_bands; b++) {
        const int bits = (ternary_mask & (1u << b)) ? 2 : band_bits[b];
        bc->band_bits[b] = bits;
        const int off = b * bc->band_size;
        const int sz = (b == n_bands - 1) ? head_dim - off : bc->band_size;
        total += 2 + (sz * bits + 7) / 8;
    }
    bc->total_bytes = total;
}

extern "C" void sp_band_config_init(sp_band_config_t *bc, int head_dim, int n_bands,
                                    const int *band_bits) {
    sp_band_config_init_ext(bc, head_dim, n_bands, band_bits, 0u);
}

extern "C" void sp_band_span(const sp_band_config_t *bc, int band, int *offset, int *size) {
    const int off = band * bc->band_size;
    *offset = off;
    *size = (band == bc->n_bands - 1) ? bc->head_dim - off : bc->band_size;
}

static int is_squarefree(int n) {
    if (n < 1) return 0;
    for (int p = 2; p * p <= n; p++)
        if (n % (p * p) == 0) return 0;
    return 1;
}

static int mobius_mu(int n) {
    if (n < 1) return 0;
    int mu = 1;
    for (int p = 2; p * p <= n; p++)
        if (n % p == 0) {
            n /= p;
            if (n % p == 0) return 0;
            mu = -mu;
        }
    return n > 1 ? -mu : mu;
}

// Squarefree-first order: coefficients i with i+1 squarefree (ascending), then
// the rest (ascending). The reference's table builder lives in its absent core
// (sp_mobius_mask_init, used at shannon_prime_cuda.cu:428-445); the kernels
// take the table as data.
static void build_mobius_order(int n, int *order) {
    int r = 0;
    for (int i = 0; i < n; i++) if (is_squarefree(i + 1)) order[r++] = i;
    for (int i = 0; i < n; i++) if (!is_squarefree(i + 1)) order[r++] = i;
}

extern "C" int sp_mobius_mask_init(sp_mobius_mask_t *mask, int n) {
    if (!mask || n <= 0) return -1;
    mask->n = n;
    mask->order = (int *)malloc(sizeof(int) * (size_t)n);
    if (!mask->order) return -1;
    build_mobius_order(n, mask->order);
    return 0;
}

extern "C" void sp_mobius_mask_free(sp_mobius_mask_t *mask) {
    if (!mask) return;
    free(mask->order);
    mask->order = nullptr;
    mask->n = 0;
}

static int is_11_smooth(int n) {
    static const int primes[5] = {2, 3, 5, 7, 11};
    for (int i = 0; i < 5; i++) while (n % primes[i] == 0) n /= primes[i];
    return n == 1;
}

extern "C" int sp_sqfree_pad_dim(int head_dim) {
    if (head_dim <= 0) return -1;
    for (int n = head_dim; n < 16 * head_dim + 64; n++)
        if (is_squarefree(n) && is_11_smooth(n)) return n;
    return -1;
}

extern "C" int sp_hier_default_geometry(int pad_dim, int *skeleton_idx, int *target_idx) {
    if (pad_dim <= 0) return -1;
    const int n_skel = std::max(1, (pad_dim * 9 + 99) / 100);
    if (skeleton_idx || target_idx) {
        std::vector<int> order((size_t)pad_dim);
        build_mobius_order(pad_dim, order.data());
        for (int i = 0; i < pad_dim; i++) {
            if (i < n_skel) { if (skeleton_idx) skeleton_idx[i] = order[i]; }
            else if (target_idx) target_idx[i - n_skel] = order[i];
        }
    }
    return n_skel;
}

static int factor_small(int n, unsigned char *f, int maxf) {
    static const int primes[5] = {2, 3, 5, 7, 11};
    int nf = 0, d = n;
    for (int i = 0; i < 5; i++)
        while (d % primes[i] == 0 && nf < maxf) { f[nf++] = (unsigned char)primes[i]; d /= primes[i]; }
    return d == 1 ? nf : -1;
}

int sp_build_plan(const sp_band_config_t *bc, int n_transform, int norm, int max_bands, SpPlan *P) {
    memset(P, 0, sizeof(*P));
    if (bc->head_dim <= 0 || bc->n_bands < 1 || bc->n_bands > SP_MAX_BANDS) return -1;
    P->hd = bc->head_dim;
    P->n_bands = bc->n_bands;
    P->norm = norm;
    P->inv_sqrt_n = 1.0f / sqrtf((float)n_transform);
    P->max_bands = (max_bands < 0 || max_bands > bc->n_bands) ? bc->n_bands : max_bands;
    int byte_off = 0, chunk_ok = (bc->head_dim % 8 == 0) && (bc->head_dim / 8 <= SP_MAX_CHUNKS);
    for (int b = 0; b < bc->n_bands; b++) {
        const int bits = bc->band_bits[b];
        if (bits < 1 || bits > 8) return -1;
        const int off = b * bc->band_size;
        const int sz = (b == bc->n_bands - 1) ? bc->head_dim - off : bc->band_size;
        if (sz <= 0) return -1;
        P->band_bits[b] = (unsigned char)bits;
        P->band_off[b] = (short)off;
        P->band_sz[b] = (short)sz;
        P->band_byte_off[b] = (short)byte_off;
        byte_off += 2 + (sz * bits + 7) / 8;
        if (off % 8 || sz % 8) chunk_ok = 0;
    }
    P->total_bytes = byte_off;
    P->chunk_ok = chunk_ok;
    if (chunk_ok) {
        for (int b = 0; b < bc->n_bands; b++) {
            P->chunk_first[b] = (unsigned char)(P->band_off[b] / 8);
            P->chunk_last[b] = (unsigned char)((P->band_off[b] + P->band_sz[b]) / 8 - 1);
            for (int c = P->band_off[b] / 8; c <= P->chunk_last[b]; c++) {
                P->chunk_band[c] = (unsigned char)b;
                P->chunk_byte_off[c] =
                    (short)(P->band_byte_off[b] + 2 + (c * 8 - P->band_off[b]) * P->band_bits[b] / 8);
            }
        }
    }
    const int pw2 = n_transform > 0 && (n_transform & (n_transform - 1)) == 0;
    if (!pw2) {
        const int nf = factor_small(n_transform, P->factors, 16);
        if (nf <= 0) return -1;
        P->n_factors = nf;
    }
    static const int primes[5] = {2, 3, 5, 7, 11};
    static const int offs[5] = {SP_CAS_OFF2, SP_CAS_OFF3, SP_CAS_OFF5, SP_CAS_OFF7, SP_CAS_OFF11};
    for (int pi = 0; pi < 5; pi++) {
        const int p = primes[pi];
        for (int k = 0; k < p; k++)
            for (int j = 0; j < p; j++) {
                const double a = 2.0 * M_PI * (double)((k * j) % p) / (double)p;
                P->cas[offs[pi] + k * p + j] = (float)(cos(a) + sin(a));
            }
        P->isp[pi] = 1.0f / sqrtf((float)p);
    }
    return 0;
}

static bool valid_bits(const int *bits, int n) {
    if (n < 1 || n > SP_MAX_BANDS) return false;
    for (int i = 0; i < n; i++)
        if (bits[i] < 1 || bits[i] > 8) return false;
    return true;
}

extern "C" float sp_compression_ratio(const sp_config_t *cfg) {
    sp_band_config_t k, v;
    sp_band_config_init_ext(&k, cfg->head_dim, cfg->k_n_bands, cfg->k_band_bits, cfg->k_ternary_mask);
    sp_band_config_init_ext(&v, cfg->head_dim, cfg->v_n_bands, cfg->v_band_bits, cfg->v_ternary_mask);
    return (float)(4.0 * cfg->head_dim / (double)(k.total_bytes + v.total_bytes));
}

extern "C" void sp_config_print(const sp_config_t *cfg) {
    fprintf(stderr, "  head_dim=%d n_layers=%d n_heads_kv=%d mobius=%d norm=%s\n", cfg->head_dim,
            cfg->n_layers, cfg->n_heads_kv, cfg->use_mobius_mask,
            cfg->vht2_norm == SP_VHT2_NORM_STAGE ? "stage" : "final");
    fprintf(stderr, "  K bands:");
    for (int i = 0; i < cfg->k_n_bands; i++) fprintf(stderr, " %d", cfg->k_band_bits[i]);
    fprintf(stderr, "  V bands:");
    for (int i = 0; i < cfg->v_n_bands; i++) fprintf(stderr, " %d", cfg->v_band_bits[i]);
    fprintf(stderr, "  ratio %.2fx\n", sp_compression_ratio(cfg));
}

extern "C" float sp_correlation_f32(const float *a, const float *b, int n) {
    if (!a || !b || n <= 0) return 0.0f;
    double ma = 0, mb = 0;
    for (int i = 0; i < n; i++) { ma += a[i]; mb += b[i]; }
    ma /= n;
    mb /= n;
    double sab = 0, saa = 0, sbb = 0;
    for (int i = 0; i < n; i++) {
        const double x = a[i] - ma, y = b[i] - mb;
        sab += x * y;
        saa += x * x;
        sbb += y * y;
    }
    if (saa <= 0 || sbb <= 0) return 0.0f;
    return (float)(sab / sqrt(saa * sbb));
}

extern "C" float sp_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, f;
    if (e == 0) {
        if (m == 0) f = sign;
        else {
            int ee = -14;
            while (!(m & 0x400u)) { m <<= 1; ee--; }
            f = sign | ((uint32_t)(ee + 127) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) f = sign | 0x7f800000u | (m << 13);
    else f = sign | ((e + 112u) << 23) | (m << 13);
    float r;
    memcpy(&r, &f, 4);
    return r;
}

extern "C" uint16_t sp_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    int e = (int)(ax >> 23) - 127;
    uint32_t m = ax & 0x7fffffu;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e >= -14) {
        uint32_t keep = m >> 13, rem = m & 0x1fffu, r = ((uint32_t)(e + 15) << 10) | keep;
        if (rem > 0x1000u || (rem == 0x1000u && (keep & 1u))) r += 1;
        return (uint16_t)(sign | r);
    }
    if (ax == 0) return (uint16_t)sign;
    int shift = -e - 1;
    if (shift > 24) return (uint16_t)sign;
    uint32_t mfull = m | 0x800000u, keep = mfull >> shift, rem = mfull & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (keep & 1u))) keep += 1;
    return (uint16_t)(sign | keep);
}

// ===========================================================================
// generic codec entry points
// ===========================================================================
extern "C" int sp_hip_ship_encode(const sp_band_config_t *bc, const int *d_order, int vht2_norm,
                                  const void *d_src, int src_dtype, long long src_outer,
                                  long long src_inner, void *d_dst, long long dst_outer,
                                  int n_outer, int n_inner, void *stream) {
    if (!bc || !d_src || !d_dst || n_outer < 0 || n_inner < 0) { set_err("encode: bad args"); return -1; }
    SpPlan P;
    if (sp_build_plan(bc, bc->head_dim, vht2_norm, -1, &P)) { set_err("encode: bad band config"); return -1; }
    return hip_ok(sp_launch_ship_encode(P, d_order, d_src, src_dtype, src_outer, src_inner,
                                        (unsigned char *)d_dst, dst_outer, n_outer, n_inner,
                                        (hipStream_t)stream), "encode launch") ? 0 : -1;
}

extern "C" int sp_hip_ship_decode(const sp_band_config_t *bc, const int *d_order, int vht2_norm,
                                  int max_bands, const void *d_src, long long src_outer,
                                  void *d_dst, int dst_dtype, long long dst_outer,
                                  long long dst_inner, int n_outer, int n_inner, void *stream) {
    if (!bc || !d_src || !d_dst || n_outer < 0 || n_inner < 0) { set_err("decode: bad args"); return -1; }
    SpPlan P;
    if (sp_build_plan(bc, bc->head_dim, vht2_norm, max_bands, &P)) { set_err("decode: bad band config"); return -1; }
    return hip_ok(sp_launch_ship_decode(P, d_order, (const unsigned char *)d_src, src_outer, d_dst,
                                        dst_dtype, dst_outer, dst_inner, n_outer, n_inner,
                                        (hipStream_t)stream), "decode launch") ? 0 : -1;
}

// test hook: force the generic (one vector per wave) kernels
extern "C" int sp_hip_ship_encode_generic(const sp_band_config_t *bc, const int *d_order,
                                          int vht2_norm, const void *d_src, int src_dtype,
                                          long long src_outer, long long src_inner, void *d_dst,
                                          long long dst_outer, int n_outer, int n_inner,
                                          void *stream) {
    SpPlan P;
    if (!bc || sp_build_plan(bc, bc->head_dim, vht2_norm, -1, &P)) return -1;
    return hip_ok(sp_launch_ship_encode_generic(P, d_order, d_src, src_dtype, src_outer, src_inner,
                                                (unsigned char *)d_dst, dst_outer, n_outer, n_inner,
                                                (hipStream_t)stream), "encode_generic") ? 0 : -1;
}

extern "C" int sp_hip_ship_decode_generic(const sp_band_config_t *bc, const int *d_order,
                                          int vht2_norm, int max_bands, const void *d_src,
                                          long long src_outer, void *d_dst, int dst_dtype,
                                          long long dst_outer, long long dst_inner, int n_outer,
                                          int n_inner, void *stream) {
    SpPlan P;
    if (!bc || sp_build_plan(bc, bc->head_dim, vht2_norm, max_bands, &P)) return -1;
    return hip_ok(sp_launch_ship_decode_generic(P, d_order, (const unsigned char *)d_src, src_outer,
                                                d_dst, dst_dtype, dst_outer, dst_inner, n_outer,
                                                n_inner, (hipStream_t)stream), "decode_generic") ? 0 : -1;
}

extern "C" void sp_hip_vht2_forward(float *d_data, int n, int n_vecs, int vht2_norm, void *stream) {
    sp_band_config_t bc;
    int bits = 8;
    sp_band_config_init(&bc, n, 1, &bits);
    SpPlan P;
    if (!d_data || n <= 0 || sp_build_plan(&bc, n, vht2_norm, -1, &P)) { set_err("vht2: bad dim %d", n); return; }
    hip_ok(sp_launch_transform(P, d_data, n_vecs, (hipStream_t)stream), "vht2");
}

extern "C" void sp_hip_mobius_reorder(float *d_data, const int *d_order, int n, int n_vecs, void *stream) {
    if (!d_data || !d_order || n <= 0) return;
    hip_ok(sp_launch_permute(d_data, d_order, n, n_vecs, 0, (hipStream_t)stream), "reorder");
}

extern "C" void sp_hip_mobius_unreorder(float *d_data, const int *d_order, int n, int n_vecs, void *stream) {
    if (!d_data || !d_order || n <= 0) return;
    hip_ok(sp_launch_permute(d_data, d_order, n, n_vecs, 1, (hipStream_t)stream), "unreorder");
}

// Quantize / dequantize without transform: a plan whose transform is the
// identity is not expressible, so these run the generic kernels on a plan with
// zero transform stages (n_transform = 1).
extern "C" void sp_hip_band_quantize(const float *d_input, void *d_output, const sp_band_config_t *bc,
                                     int n_vecs, void *stream) {
    SpPlan P;
    if (!bc || !d_input || !d_output || sp_build_plan(bc, 1, 0, -1, &P)) return;
    P.chunk_ok = 0;
    P.skip_transform = 1;
    hip_ok(sp_launch_ship_encode_generic(P, nullptr, d_input, SP_DT_F32, 0, bc->head_dim,
                                         (unsigned char *)d_output, 0, 1, n_vecs, (hipStream_t)stream),
           "band_quantize");
}

extern "C" void sp_hip_band_dequantize(const void *d_input, float *d_output, const sp_band_config_t *bc,
                                       int n_vecs, void *stream) {
    SpPlan P;
    if (!bc || !d_input || !d_output || sp_build_plan(bc, 1, 0, -1, &P)) return;
    P.chunk_ok = 0;
    P.skip_transform = 1;
    hip_ok(sp_launch_ship_decode_generic(P, nullptr, (const unsigned char *)d_input, 0, d_output,
                                         SP_DT_F32, 0, bc->head_dim, 1, n_vecs, (hipStream_t)stream),
           "band_dequantize");
}

// ===========================================================================
// ship device cache
// ===========================================================================
struct ShipPriv {
    SpPlan kplan, vplan;
    float *ws = nullptr;
    size_t ws_floats = 0;
    int max_q = 0;
    // batched (multi-sequence) attention workspace, grown on demand
    float *seq_ws = nullptr;
    size_t seq_ws_floats = 0;
    // K coefficient-order calibration: fp64 sums of the fed vectors' transforms
    bool calibrating = false;
    std::vector<double> csum, csum2;
    long long cn = 0;
    // host-pointer calls: persistent device staging and pinned host staging,
    // grown on demand (one caller at a time)
    std::mutex stage_mu;
    float *stage_d = nullptr;
    float *stage_h = nullptr;
    size_t stage_n = 0;  // floats in each
};

// Grow the host-call staging of `pv` to at least n floats (stage_mu held).
static bool stage_reserve(ShipPriv *pv, size_t n) {
    if (n <= pv->stage_n) return true;
    if (pv->stage_d) (void)hipFree(pv->stage_d);
    if (pv->stage_h) (void)hipHostFree(pv->stage_h);
    pv->stage_d = nullptr;
    pv->stage_h = nullptr;
    pv->stage_n = 0;
    const size_t want = n < 4096 * 128 ? (size_t)4096 * 128 : n;
    if (!hip_ok(hipMalloc((void **)&pv->stage_d, want * sizeof(float)), "hipMalloc host-call staging") ||
        !hip_ok(hipHostMalloc((void **)&pv->stage_h, want * sizeof(float), hipHostMallocDefault),
                "hipHostMalloc host-call staging")) {
        if (pv->stage_d) (void)hipFree(pv->stage_d);
        pv->stage_d = nullptr;
        return false;
    }
    pv->stage_n = want;
    return true;
}

static bool check_cfg(const sp_config_t *cfg) {
    if (!cfg || cfg->head_dim <= 0 || cfg->head_dim > SP_MAX_HEAD_DIM || cfg->n_layers <= 0 ||
        cfg->n_heads_kv <= 0) return false;
    if (!valid_bits(cfg->k_band_bits, cfg->k_n_bands) || !valid_bits(cfg->v_band_bits, cfg->v_n_bands))
        return false;
    return true;
}

extern "C" int sp_hip_cache_init(sp_hip_cache_t *cc, const sp_config_t *cfg, int max_seq_len, void *stream) {
    if (!cc) return -1;
    memset(cc, 0, sizeof(*cc));
    if (!check_cfg(cfg) || max_seq_len <= 0) { set_err("cache_init: bad config"); return -1; }
    if (!sp_hip_available()) { set_err("cache_init: no gfx950 device"); return -1; }
    cc->config = *cfg;
    cc->max_seq_len = max_seq_len;
    cc->stream = stream;
    const int hd = cfg->head_dim;
    sp_band_config_init_ext(&cc->k_bands, hd, cfg->k_n_bands, cfg->k_band_bits, cfg->k_ternary_mask);
    sp_band_config_init_ext(&cc->v_bands, hd, cfg->v_n_bands, cfg->v_band_bits, cfg->v_ternary_mask);
    ShipPriv *pv = new ShipPriv();
    if (sp_build_plan(&cc->k_bands, hd, cfg->vht2_norm, -1, &pv->kplan) ||
        sp_build_plan(&cc->v_bands, hd, cfg->vht2_norm, -1, &pv->vplan)) {
        delete pv;
        set_err("cache_init: head_dim %d does not factor over {2,3,5,7,11}", hd);
        return -1;
    }
    if (hd > SP_GEN_MAX_N && !(pv->kplan.chunk_ok && pv->vplan.chunk_ok)) {
        delete pv;
        set_err("cache_init: head_dim %d needs the generic kernels (max %d)", hd, SP_GEN_MAX_N);
        return -1;
    }
    pv->kplan.order_default = 1;  // d_mobius_order below is the default table
    cc->priv = pv;
    const size_t n_slots = (size_t)cfg->n_layers * cfg->n_heads_kv;
    const size_t kb = n_slots * max_seq_len * cc->k_bands.total_bytes;
    const size_t vb = n_slots * max_seq_len * cc->v_bands.total_bytes;
    // SP_CACHE_SLACK bytes after the last record let tile loaders read whole
    // dwords past a record boundary without leaving the allocation.
    bool ok = hip_ok(hipMalloc(&cc->d_k_cache, kb + SP_CACHE_SLACK), "hipMalloc K cache") &&
              hip_ok(hipMalloc(&cc->d_v_cache, vb + SP_CACHE_SLACK), "hipMalloc V cache") &&
              hip_ok(hipMemsetAsync(cc->d_k_cache, 0, kb + SP_CACHE_SLACK, (hipStream_t)stream), "memset K") &&
              hip_ok(hipMemsetAsync(cc->d_v_cache, 0, vb + SP_CACHE_SLACK, (hipStream_t)stream), "memset V");
    if (ok && cfg->use_mobius_mask) {
        std::vector<int> order(hd), inv(hd);
        build_mobius_order(hd, order.data());
        for (int i = 0; i < hd; i++) inv[order[i]] = i;
        ok = hip_ok(hipMalloc((void **)&cc->d_mobius_order, sizeof(int) * hd), "hipMalloc order") &&
             hip_ok(hipMalloc((void **)&cc->d_mobius_inv, sizeof(int) * hd), "hipMalloc inv") &&
             hip_ok(hipMemcpy(cc->d_mobius_order, order.data(), sizeof(int) * hd, hipMemcpyHostToDevice), "order H2D") &&
             hip_ok(hipMemcpy(cc->d_mobius_inv, inv.data(), sizeof(int) * hd, hipMemcpyHostToDevice), "inv H2D");
    }
    if (ok) {
        pv->max_q = cfg->n_heads_kv * 8;
        pv->ws_floats = sp_attn_workspace_floats(pv->max_q, hd, max_seq_len);
        ok = hip_ok(hipMalloc((void **)&pv->ws, pv->ws_floats * sizeof(float)), "hipMalloc attention workspace") &&
             hip_ok(hipMemsetAsync(pv->ws, 0, pv->ws_floats * sizeof(float), (hipStream_t)stream),
                    "attention workspace clear");  // the attention kernel's counters start at zero
    }
    if (ok) ok = hip_ok(hipStreamSynchronize((hipStream_t)stream), "init sync");
    if (!ok) {
        sp_hip_cache_free(cc);
        return -1;
    }
    return 0;
}

extern "C" void sp_hip_cache_free(sp_hip_cache_t *cc) {
    if (!cc) return;
    if (cc->d_k_cache) (void)hipFree(cc->d_k_cache);
    if (cc->d_v_cache) (void)hipFree(cc->d_v_cache);
    if (cc->d_mobius_order) (void)hipFree(cc->d_mobius_order);
    if (cc->d_mobius_inv) (void)hipFree(cc->d_mobius_inv);
    ShipPriv *pv = (ShipPriv *)cc->priv;
    if (pv) {
        if (pv->ws) (void)hipFree(pv->ws);
        if (pv->seq_ws) (void)hipFree(pv->seq_ws);
        if (pv->stage_d) (void)hipFree(pv->stage_d);
        if (pv->stage_h) (void)hipHostFree(pv->stage_h);
        delete pv;
    }
    memset(cc, 0, sizeof(*cc));
}

static inline bool slot_ok(const sp_hip_cache_t *cc, int layer, int head, int pos, int n) {
    return cc && cc->priv && layer >= 0 && layer < cc->config.n_layers && head >= 0 &&
           head < cc->config.n_heads_kv && pos >= 0 && n >= 0 && (long long)pos + n <= cc->max_seq_len;
}

static unsigned char *slot_ptr(const sp_hip_cache_t *cc, int is_v, int layer, int head, int pos) {
    const int B = is_v ? cc->v_bands.total_bytes : cc->k_bands.total_bytes;
    unsigned char *base = (unsigned char *)(is_v ? cc->d_v_cache : cc->d_k_cache);
    const long long slot = (long long)layer * cc->config.n_heads_kv + head;
    return base + (slot * cc->max_seq_len + pos) * B;
}

static int ship_write(sp_hip_cache_t *cc, int is_v, int layer, int head, int pos, int n,
                      const void *src, int dtype) {
    if (!slot_ok(cc, layer, head, pos, n) || !src) { set_err("write: bad slot/pos"); return -1; }
    ShipPriv *pv = (ShipPriv *)cc->priv;
    const SpPlan &P = is_v ? pv->vplan : pv->kplan;
    const int *ord = is_v ? nullptr : cc->d_mobius_order;
    return hip_ok(sp_launch_ship_encode(P, ord, src, dtype, 0, cc->config.head_dim,
                                        slot_ptr(cc, is_v, layer, head, pos), 0, 1, n,
                                        (hipStream_t)cc->stream), "write") ? 0 : -1;
}

static int ship_read(const sp_hip_cache_t *cc, int is_v, int layer, int head, int pos, int n,
                     void *dst, int dtype, int max_bands) {
    if (!slot_ok(cc, layer, head, pos, n) || !dst) { set_err("read: bad slot/pos"); return -1; }
    ShipPriv *pv = (ShipPriv *)cc->priv;
    SpPlan P = is_v ? pv->vplan : pv->kplan;
    if (max_bands >= 0 && max_bands < P.n_bands) P.max_bands = max_bands;
    const int *ord = is_v ? nullptr : cc->d_mobius_order;
    return hip_ok(sp_launch_ship_decode(P, ord, slot_ptr(cc, is_v, layer, head, pos), 0, dst, dtype,
                                        0, cc->config.head_dim, 1, n, (hipStream_t)cc->stream),
                  "read") ? 0 : -1;
}

extern "C" void sp_hip_write_k(sp_hip_cache_t *cc, int l, int h, int p, const float *d) { ship_write(cc, 0, l, h, p, 1, d, SP_DT_F32); }
extern "C" void sp_hip_write_v(sp_hip_cache_t *cc, int l, int h, int p, const float *d) { ship_write(cc, 1, l, h, p, 1, d, SP_DT_F32); }
extern "C" void sp_hip_read_k(const sp_hip_cache_t *cc, int l, int h, int p, float *d) { ship_read(cc, 0, l, h, p, 1, d, SP_DT_F32, -1); }
extern "C" void sp_hip_read_v(const sp_hip_cache_t *cc, int l, int h, int p, float *d) { ship_read(cc, 1, l, h, p, 1, d, SP_DT_F32, -1); }
extern "C" void sp_hip_write_k_batch(sp_hip_cache_t *cc, int l, int h, int s, int n, const float *d) { ship_write(cc, 0, l, h, s, n, d, SP_DT_F32); }
extern "C" void sp_hip_write_v_batch(sp_hip_cache_t *cc, int l, int h, int s, int n, const float *d) { ship_write(cc, 1, l, h, s, n, d, SP_DT_F32); }
extern "C" void sp_hip_read_k_batch(const sp_hip_cache_t *cc, int l, int h, int s, int n, float *d) { ship_read(cc, 0, l, h, s, n, d, SP_DT_F32, -1); }
extern "C" void sp_hip_read_v_batch(const sp_hip_cache_t *cc, int l, int h, int s, int n, float *d) { ship_read(cc, 1, l, h, s, n, d, SP_DT_F32, -1); }
extern "C" void sp_hip_read_k_batch_partial(const sp_hip_cache_t *cc, int l, int h, int s, int n, float *d, int mb) { ship_read(cc, 0, l, h, s, n, d, SP_DT_F32, mb); }
extern "C" void sp_hip_read_v_batch_partial(const sp_hip_cache_t *cc, int l, int h, int s, int n, float *d, int mb) { ship_read(cc, 1, l, h, s, n, d, SP_DT_F32, mb); }
extern "C" void sp_hip_write_k_batch_f16(sp_hip_cache_t *cc, int l, int h, int s, int n, const void *d) { ship_write(cc, 0, l, h, s, n, d, SP_DT_F16); }
extern "C" void sp_hip_write_v_batch_f16(sp_hip_cache_t *cc, int l, int h, int s, int n, const void *d) { ship_write(cc, 1, l, h, s, n, d, SP_DT_F16); }
extern "C" void sp_hip_read_k_batch_f16(const sp_hip_cache_t *cc, int l, int h, int s, int n, void *d) { ship_read(cc, 0, l, h, s, n, d, SP_DT_F16, -1); }
extern "C" void sp_hip_read_v_batch_f16(const sp_hip_cache_t *cc, int l, int h, int s, int n, void *d) { ship_read(cc, 1, l, h, s, n, d, SP_DT_F16, -1); }

extern "C" int sp_hip_write_layer(sp_hip_cache_t *cc, int layer, int start_pos, int n_tok,
                                  const void *d_k, const void *d_v, long long row_stride, int dtype) {
    if (!slot_ok(cc, layer, 0, start_pos, n_tok)) { set_err("write_layer: bad layer/pos"); return -1; }
    const int H = cc->config.n_heads_kv, hd = cc->config.head_dim;
    if (row_stride < (long long)H * hd) { set_err("write_layer: row_stride"); return -1; }
    ShipPriv *pv = (ShipPriv *)cc->priv;
    hipStream_t s = (hipStream_t)cc->stream;
    if (d_k && !hip_ok(sp_launch_ship_encode(pv->kplan, cc->d_mobius_order, d_k, dtype, hd, row_stride,
                                             slot_ptr(cc, 0, layer, 0, start_pos),
                                             (long long)cc->max_seq_len * cc->k_bands.total_bytes, H,
                                             n_tok, s), "write_layer K")) return -1;
    if (d_v && !hip_ok(sp_launch_ship_encode(pv->vplan, nullptr, d_v, dtype, hd, row_stride,
                                             slot_ptr(cc, 1, layer, 0, start_pos),
                                             (long long)cc->max_seq_len * cc->v_bands.total_bytes, H,
                                             n_tok, s), "write_layer V")) return -1;
    return 0;
}

extern "C" int sp_hip_read_layer(const sp_hip_cache_t *cc, int layer, int start_pos, int n_tok,
                                 void *d_k, void *d_v, long long row_stride, int dtype, int max_bands) {
    if (!slot_ok(cc, layer, 0, start_pos, n_tok)) { set_err("read_layer: bad layer/pos"); return -1; }
    const int H = cc->config.n_heads_kv, hd = cc->config.head_dim;
    if (row_stride < (long long)H * hd) { set_err("read_layer: row_stride"); return -1; }
    ShipPriv *pv = (ShipPriv *)cc->priv;
    hipStream_t s = (hipStream_t)cc->stream;
    SpPlan kp = pv->kplan, vp = pv->vplan;
    if (max_bands >= 0) {
        if (max_bands < kp.n_bands) kp.max_bands = max_bands;
        if (max_bands < vp.n_bands) vp.max_bands = max_bands;
    }
    if (d_k && !hip_ok(sp_launch_ship_decode(kp, cc->d_mobius_order, slot_ptr(cc, 0, layer, 0, start_pos),
                                             (long long)cc->max_seq_len * cc->k_bands.total_bytes, d_k,
                                             dtype, hd, row_stride, H, n_tok, s), "read_layer K")) return -1;
    if (d_v && !hip_ok(sp_launch_ship_decode(vp, nullptr, slot_ptr(cc, 1, layer, 0, start_pos),
                                             (long long)cc->max_seq_len * cc->v_bands.total_bytes, d_v,
                                             dtype, hd, row_stride, H, n_tok, s), "read_layer V")) return -1;
    return 0;
}

extern "C" int sp_hip_roundtrip_cells(sp_hip_cache_t *cc, int layer, const int *d_cells, int n_cells,
                                      void *d_k, long long k_cell_stride, void *d_v, long long v_cell_stride,
                                      long long v_elem_stride, int dtype, int max_bands, void *stream) {
    if (!slot_ok(cc, layer, 0, 0, 0) || n_cells < 0 || (n_cells > 0 && !d_cells) ||
        (dtype != SP_DT_F16 && dtype != SP_DT_F32)) { set_err("roundtrip_cells: bad args"); return -1; }
    const int H = cc->config.n_heads_kv, hd = cc->config.head_dim;
    const long long row = (long long)H * hd;
    if (d_k && k_cell_stride < row) { set_err("roundtrip_cells: k_cell_stride"); return -1; }
    if (d_v && !((v_elem_stride == 1 && v_cell_stride >= row) ||
                 (v_cell_stride == 1 && v_elem_stride >= cc->max_seq_len))) {
        set_err("roundtrip_cells: V strides must be rows or the transposed layout"); return -1;
    }
    if (n_cells == 0) return 0;
    ShipPriv *pv = (ShipPriv *)cc->priv;
    hipStream_t s = (hipStream_t)(stream ? stream : cc->stream);
    // The narrow kernel (head_dim/8 lanes per vector, K and V in one launch) wherever
    // its layouts allow: measured faster than the one-vector-per-lane kernel from a
    // single decode cell (7.3 vs 31.6 us per layer, 8 heads) to 2048-cell prefill
    // chunks (20.9 vs 32.7 us). The lane kernel covers hd 96. SP_HIP_RT_KERNEL=narrow|lane
    // forces either.
    const char *force = getenv("SP_HIP_RT_KERNEL");
    const bool f_lane = force && !strcmp(force, "lane"), f_narrow = force && !strcmp(force, "narrow");
    if (!f_lane) {
        const long long kB = cc->k_bands.total_bytes, vB = cc->v_bands.total_bytes;
        const hipError_t e = sp_launch_ship_roundtrip_narrow(
            pv->kplan, cc->d_mobius_order, d_k, k_cell_stride, slot_ptr(cc, 0, layer, 0, 0),
            (long long)cc->max_seq_len * kB, pv->vplan, d_v, v_cell_stride, v_elem_stride,
            slot_ptr(cc, 1, layer, 0, 0), (long long)cc->max_seq_len * vB, dtype, d_cells, n_cells,
            cc->max_seq_len, H, max_bands, s);
        if (e != hipErrorNotSupported) return hip_ok(e, "roundtrip_cells") ? 0 : -1;
        if (f_narrow) { set_err("roundtrip_cells: no narrow kernel for this band layout"); return -1; }
    }
    for (int is_v = 0; is_v < 2; is_v++) {
        void *x = is_v ? d_v : d_k;
        if (!x) continue;
        const SpPlan &P = is_v ? pv->vplan : pv->kplan;
        const int *order = is_v ? nullptr : cc->d_mobius_order;
        if (P.skip_transform || !(order == nullptr || P.order_default)) {
            set_err("roundtrip_cells: needs the default Mobius order"); return -1;
        }
        const long long B = is_v ? cc->v_bands.total_bytes : cc->k_bands.total_bytes;
        const hipError_t e = sp_launch_ship_roundtrip_lane(
            P, order != nullptr, x, dtype, is_v ? v_cell_stride : k_cell_stride, is_v ? v_elem_stride : 1, d_cells,
            n_cells, cc->max_seq_len, slot_ptr(cc, is_v, layer, 0, 0), (long long)cc->max_seq_len * B, H, max_bands, s);
        if (e == hipErrorNotSupported) { set_err("roundtrip_cells: no lane kernel for this band layout"); return -1; }
        if (!hip_ok(e, "roundtrip_cells")) return -1;
    }
    return 0;
}

// ---- calibration --------------------------------------------------------
// Per-coefficient sums of the plan's forward transform (length hd; inputs of
// in_len < hd elements are mean padded) of n device vectors: the kernel's
// per-wave fp64 partials are added here in launch order.
static bool calib_accumulate(const SpPlan &P, int in_len, int hd, const void *d_src, int dtype, long long si, int n,
                             double *sum, double *sum2, hipStream_t s) {
    const int nb = sp_calib_moment_blocks(n);
    const size_t cnt = (size_t)nb * 4 * 2 * hd;
    double *d_part = nullptr;
    if (!hip_ok(hipMalloc((void **)&d_part, cnt * sizeof(double)), "calib alloc")) return false;
    std::vector<double> h(cnt);
    const bool ok = hip_ok(sp_launch_calib_moments(P, in_len, hd, d_src, dtype, si, n, d_part, nb, s), "calib moments") &&
                    hip_ok(hipMemcpyAsync(h.data(), d_part, cnt * sizeof(double), hipMemcpyDeviceToHost, s),
                           "calib D2H") &&
                    hip_ok(hipStreamSynchronize(s), "calib sync");
    (void)hipFree(d_part);
    if (!ok) return false;
    for (size_t w = 0; w < (size_t)nb * 4; w++)
        for (int k = 0; k < hd; k++) {
            sum[k] += h[w * 2 * hd + k];
            sum2[k] += h[w * 2 * hd + hd + k];
        }
    return true;
}

// Coefficients by descending variance sum2/n - (sum/n)^2, ties (and NaN, ranked
// last) by ascending index.
static void rank_by_variance(const double *sum, const double *sum2, long long n, int hd, int *order) {
    std::vector<double> var((size_t)hd);
    for (int k = 0; k < hd; k++) {
        const double m = sum[k] / (double)n, v = sum2[k] / (double)n - m * m;
        var[(size_t)k] = std::isnan(v) ? -INFINITY : v;
    }
    std::vector<int> idx((size_t)hd);
    std::iota(idx.begin(), idx.end(), 0);
    std::stable_sort(idx.begin(), idx.end(), [&](int a, int b) { return var[(size_t)a] > var[(size_t)b]; });
    std::copy(idx.begin(), idx.end(), order);
}

static bool is_default_order(const int *order, int hd) {
    std::vector<int> d((size_t)hd);
    build_mobius_order(hd, d.data());
    return std::equal(d.begin(), d.end(), order);
}

extern "C" int sp_hip_calibrate_begin(sp_hip_cache_t *cc) {
    if (!cc || !cc->priv) { set_err("calibrate_begin: bad cache"); return -1; }
    ShipPriv *pv = (ShipPriv *)cc->priv;
    pv->csum.assign((size_t)cc->config.head_dim, 0.0);
    pv->csum2.assign((size_t)cc->config.head_dim, 0.0);
    pv->cn = 0;
    pv->calibrating = true;
    return 0;
}

extern "C" int sp_hip_calibrate_feed(sp_hip_cache_t *cc, const void *d_vecs, long long row_stride, int n_vecs,
                                     int dtype) {
    if (!cc || !cc->priv || n_vecs < 0 || (n_vecs > 0 && !d_vecs) || row_stride < cc->config.head_dim ||
        (dtype != SP_DT_F16 && dtype != SP_DT_F32)) { set_err("calibrate_feed: bad args"); return -1; }
    ShipPriv *pv = (ShipPriv *)cc->priv;
    if (!pv->calibrating) { set_err("calibrate_feed: no calibrate_begin"); return -1; }
    if (n_vecs == 0) return 0;
    const int hd = cc->config.head_dim;
    if (!calib_accumulate(pv->kplan, hd, hd, d_vecs, dtype, row_stride, n_vecs, pv->csum.data(), pv->csum2.data(),
                          (hipStream_t)cc->stream)) return -1;
    pv->cn += n_vecs;
    return 0;
}

// Make `order` the K coefficient order of the cache (and its inverse table).
static bool install_k_order(sp_hip_cache_t *cc, const int *order) {
    const int hd = cc->config.head_dim;
    std::vector<int> inv((size_t)hd);
    for (int i = 0; i < hd; i++) inv[(size_t)order[i]] = i;
    if (!cc->d_mobius_order &&
        !(hip_ok(hipMalloc((void **)&cc->d_mobius_order, sizeof(int) * hd), "hipMalloc order") &&
          hip_ok(hipMalloc((void **)&cc->d_mobius_inv, sizeof(int) * hd), "hipMalloc inv"))) return false;
    hipStream_t s = (hipStream_t)cc->stream;
    if (!(hip_ok(hipStreamSynchronize(s), "order sync") &&
          hip_ok(hipMemcpy(cc->d_mobius_order, order, sizeof(int) * hd, hipMemcpyHostToDevice), "order H2D") &&
          hip_ok(hipMemcpy(cc->d_mobius_inv, inv.data(), sizeof(int) * hd, hipMemcpyHostToDevice), "inv H2D")))
        return false;
    ShipPriv *pv = (ShipPriv *)cc->priv;
    pv->kplan.order_default = is_default_order(order, hd) ? 1 : 0;
    cc->config.use_mobius_mask = 1;
    return true;
}

extern "C" int sp_hip_calibrate_end(sp_hip_cache_t *cc, int *var_order_out, int apply) {
    if (!cc || !cc->priv) { set_err("calibrate_end: bad cache"); return -1; }
    ShipPriv *pv = (ShipPriv *)cc->priv;
    if (!pv->calibrating || pv->cn <= 0) { set_err("calibrate_end: no data fed"); return -1; }
    const int hd = cc->config.head_dim;
    std::vector<int> order((size_t)hd);
    rank_by_variance(pv->csum.data(), pv->csum2.data(), pv->cn, hd, order.data());
    if (var_order_out) std::copy(order.begin(), order.end(), var_order_out);
    if (apply && !install_k_order(cc, order.data())) return -1;
    pv->calibrating = false;
    return 0;
}

extern "C" int sp_hip_write_all(sp_hip_cache_t *cc, int start_pos, int n_pos, const void *d_k,
                                const void *d_v, int dtype) {
    if (!slot_ok(cc, 0, 0, start_pos, n_pos)) { set_err("write_all: bad pos"); return -1; }
    const int n_slots = cc->config.n_layers * cc->config.n_heads_kv, hd = cc->config.head_dim;
    ShipPriv *pv = (ShipPriv *)cc->priv;
    hipStream_t s = (hipStream_t)cc->stream;
    if (d_k && !hip_ok(sp_launch_ship_encode(pv->kplan, cc->d_mobius_order, d_k, dtype, (long long)n_pos * hd, hd,
                                             slot_ptr(cc, 0, 0, 0, start_pos),
                                             (long long)cc->max_seq_len * cc->k_bands.total_bytes, n_slots,
                                             n_pos, s), "write_all K")) return -1;
    if (d_v && !hip_ok(sp_launch_ship_encode(pv->vplan, nullptr, d_v, dtype, (long long)n_pos * hd, hd,
                                             slot_ptr(cc, 1, 0, 0, start_pos),
                                             (long long)cc->max_seq_len * cc->v_bands.total_bytes, n_slots,
                                             n_pos, s), "write_all V")) return -1;
    return 0;
}

extern "C" int sp_hip_read_all(const sp_hip_cache_t *cc, int start_pos, int n_pos, void *d_k, void *d_v,
                               int dtype, int max_bands) {
    if (!slot_ok(cc, 0, 0, start_pos, n_pos)) { set_err("read_all: bad pos"); return -1; }
    const int n_slots = cc->config.n_layers * cc->config.n_heads_kv, hd = cc->config.head_dim;
    ShipPriv *pv = (ShipPriv *)cc->priv;
    hipStream_t s = (hipStream_t)cc->stream;
    SpPlan kp = pv->kplan, vp = pv->vplan;
    if (max_bands >= 0) {
        if (max_bands < kp.n_bands) kp.max_bands = max_bands;
        if (max_bands < vp.n_bands) vp.max_bands = max_bands;
    }
    if (d_k && !hip_ok(sp_launch_ship_decode(kp, cc->d_mobius_order, slot_ptr(cc, 0, 0, 0, start_pos),
                                             (long long)cc->max_seq_len * cc->k_bands.total_bytes, d_k,
                                             dtype, (long long)n_pos * hd, hd, n_slots, n_pos, s), "read_all K")) return -1;
    if (d_v && !hip_ok(sp_launch_ship_decode(vp, nullptr, slot_ptr(cc, 1, 0, 0, start_pos),
                                             (long long)cc->max_seq_len * cc->v_bands.total_bytes, d_v,
                                             dtype, (long long)n_pos * hd, hd, n_slots, n_pos, s), "read_all V")) return -1;
    return 0;
}

// ===========================================================================
// fused attention
// ===========================================================================
// Sequence table of a (batched) attention call: n_seq ranges [start, start + len) of
// [0, max_seq), each non-empty; scores packed [n_q][len] per sequence. False (error set)
// otherwise.
static bool seq_tab(int n_seq, const int *start, const int *len, int max_seq, int n_q, SpSeqTab *T,
                    const char *who) {
    if (n_seq < 1 || n_seq > SP_ATTN_MAX_SEQ || !start || !len) {
        set_err("%s: 1..%d sequences with start and length arrays", who, SP_ATTN_MAX_SEQ);
        return false;
    }
    memset(T, 0, sizeof(*T));
    T->n_seq = n_seq;
    long long off = 0;
    for (int i = 0; i < n_seq; i++) {
        if (start[i] < 0 || len[i] <= 0 || (long long)start[i] + len[i] > max_seq) {
            set_err("%s: sequence %d [%d, %d + %d) outside [0, %d)", who, i, start[i], start[i], len[i], max_seq);
            return false;
        }
        T->start[i] = start[i];
        T->len[i] = len[i];
        T->soff[i] = off;
        off += (long long)n_q * len[i];
        T->max_len = std::max(T->max_len, len[i]);
    }
    return true;
}

// Grow a stream-ordered workspace to `need` floats (a sync on the stream before freeing).
static bool grow_ws(float **ws, size_t *have, size_t need, hipStream_t s, const char *who) {
    if (need <= *have) return true;
    if (*ws) {
        if (!hip_ok(hipStreamSynchronize(s), who)) return false;
        (void)hipFree(*ws);
        *ws = nullptr;
        *have = 0;
    }
    if (!hip_ok(hipMalloc((void **)ws, need * sizeof(float)), who)) return false;
    *have = need;
    return true;
}

static int cu_count() {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    return cus;
}
// Launch arguments of one layer's decode attention over the cache's records.
int sp_attn_prepare(const sp_hip_cache_t *cc, int layer, int n_kv, const float *d_q, int n_q, float kq_scale,
                    float *d_scores, float *d_out, int max_bands, SpAttnArgs *out_args, SpPlan *out_kp,
                    SpPlan *out_vp) {
    if (!cc || !cc->priv || layer < 0 || layer >= cc->config.n_layers || n_kv <= 0 ||
        n_kv > cc->max_seq_len || !d_q || n_q <= 0) { set_err("attn: bad args"); return -1; }
    ShipPriv *pv = (ShipPriv *)cc->priv;
    SpAttnArgs A;
    const int H = cc->config.n_heads_kv;
    A.kB = cc->k_bands.total_bytes;
    A.vB = cc->v_bands.total_bytes;
    A.k_head_stride = (long long)cc->max_seq_len * A.kB;
    A.v_head_stride = (long long)cc->max_seq_len * A.vB;
    A.kpack = slot_ptr(cc, 0, layer, 0, 0);
    A.vpack = slot_ptr(cc, 1, layer, 0, 0);
    A.n_kv = n_kv;
    A.n_q = n_q;
    A.n_kvh = H;
    A.hd = cc->config.head_dim;
    A.kq_scale = kq_scale;
    A.q = d_q;
    A.scores = d_scores;
    A.out = d_out;
    SpPlan kp = pv->kplan, vp = pv->vplan;
    if (max_bands >= 0) {
        if (max_bands < kp.n_bands) kp.max_bands = max_bands;
        if (max_bands < vp.n_bands) vp.max_bands = max_bands;
    }
    *out_args = A;
    *out_kp = kp;
    *out_vp = vp;
    return 0;
}

extern "C" int sp_hip_attn_decode_bands(const sp_hip_cache_t *cc, int layer, int n_kv, const float *d_q, int n_q,
                                        float kq_scale, float *d_scores, float *d_out, int max_bands, void *stream) {
    SpAttnArgs A;
    SpPlan kp, vp;
    if (sp_attn_prepare(cc, layer, n_kv, d_q, n_q, kq_scale, d_scores, d_out, max_bands, &A, &kp, &vp)) return -1;
    ShipPriv *pv = (ShipPriv *)cc->priv;
    if (n_q > pv->max_q) { set_err("attn: n_q %d > %d", n_q, pv->max_q); return -1; }
    return hip_ok(sp_launch_attn_decode(kp, vp, cc->d_mobius_order, A, pv->ws, pv->ws_floats,
                                        (hipStream_t)(stream ? stream : cc->stream)),
                  "attn launch") ? 0 : -1;
}

extern "C" int sp_hip_attn_decode(const sp_hip_cache_t *cc, int layer, int n_kv, const float *d_q,
                                  int n_q, float kq_scale, float *d_scores, float *d_out, void *stream) {
    return sp_hip_attn_decode_bands(cc, layer, n_kv, d_q, n_q, kq_scale, d_scores, d_out, -1, stream);
}

extern "C" int sp_hip_attn_decode_seqs(const sp_hip_cache_t *cc, int layer, int n_seq, const int *seq_start,
                                       const int *seq_len, const float *d_q, int n_q, float kq_scale, float *d_scores,
                                       float *d_out, void *stream) {
    if (!cc || !cc->priv) { set_err("attn seqs: bad cache"); return -1; }
    SpSeqTab T;
    if (!seq_tab(n_seq, seq_start, seq_len, cc->max_seq_len, n_q, &T, "attn seqs")) return -1;
    SpAttnArgs A;
    SpPlan kp, vp;
    if (sp_attn_prepare(cc, layer, T.max_len, d_q, n_q, kq_scale, d_scores, d_out, -1, &A, &kp, &vp)) return -1;
    if (!d_scores && !d_out) { set_err("attn seqs: no output"); return -1; }
    ShipPriv *pv = (ShipPriv *)cc->priv;
    const hipStream_t s = (hipStream_t)(stream ? stream : cc->stream);
    // the one-position-per-lane layouts (hd 96 / hd 64): every sequence in one launch each of
    // the query preparation, the split kernel and the combine
    const char *off = getenv("SP_HIP_NO_LANE_ATTN");
    int n_runs = (off && off[0] == '1') ? 0 : sp_attn_lane_runs(kp, vp, A, (size_t)1 << 40, n_seq);
    for (int i = 0; i < n_seq && n_runs > 0; i++)  // the lane kernel's dword-aligned record bases, per sequence
        if (((long long)T.start[i] * A.kB) % 4 || ((long long)T.start[i] * A.vB) % 4) n_runs = 0;
    if (n_runs > 0) {
        const size_t rows = (size_t)n_seq * n_q;
        if (!grow_ws(&pv->seq_ws, &pv->seq_ws_floats, rows * A.hd + rows * n_runs * (A.hd + 2), s,
                     "attn seqs workspace")) return -1;
        return hip_ok(sp_launch_attn_lane_seqs(kp, vp, cc->d_mobius_order, A, T, pv->seq_ws, pv->seq_ws_floats, n_runs, s),
                      "attn seqs") ? 0 : -1;
    }
    // otherwise one single-sequence launch sequence per sequence (the matrix-core kernel
    // merges its partials inside its own launch), each over its range of records
    if (n_q > pv->max_q) { set_err("attn seqs: n_q %d > %d", n_q, pv->max_q); return -1; }
    for (int i = 0; i < n_seq; i++) {
        SpAttnArgs Ai = A;
        Ai.kpack += (long long)T.start[i] * A.kB;
        Ai.vpack += (long long)T.start[i] * A.vB;
        Ai.n_kv = T.len[i];
        Ai.q = d_q + (size_t)i * n_q * A.hd;
        Ai.scores = d_scores ? d_scores + T.soff[i] : nullptr;
        Ai.out = d_out ? d_out + (size_t)i * n_q * A.hd : nullptr;
        if (!hip_ok(sp_launch_attn_decode(kp, vp, cc->d_mobius_order, Ai, pv->ws, pv->ws_floats, s), "attn seqs"))
            return -1;
    }
    return 0;
}

extern "C" int sp_hip_attn_decode_all_layers(const sp_hip_cache_t *cc, int n_kv, const float *d_q, int n_q,
                                             float kq_scale, float *d_out, void *stream) {
    if (!cc) return -1;
    const int hd = cc->config.head_dim;
    for (int l = 0; l < cc->config.n_layers; l++)
        if (sp_hip_attn_decode(cc, l, n_kv, d_q + (size_t)l * n_q * hd, n_q, kq_scale, nullptr,
                               d_out + (size_t)l * n_q * hd, stream)) return -1;
    return 0;
}

extern "C" int sp_hip_attn_scores_all_layers(const sp_hip_cache_t *cc, int n_kv, const float *d_q, int n_q,
                                             float kq_scale, float *d_scores, int max_bands, void *stream) {
    if (!cc || !d_scores) return -1;
    const int hd = cc->config.head_dim;
    for (int l = 0; l < cc->config.n_layers; l++)
        if (sp_hip_attn_decode_bands(cc, l, n_kv, d_q + (size_t)l * n_q * hd, n_q, kq_scale,
                                     d_scores + (size_t)l * n_q * n_kv, nullptr, max_bands, stream)) return -1;
    return 0;
}

static std::mutex g_f16ws_mu;
static float *g_f16ws = nullptr;
static size_t g_f16ws_n = 0;

extern "C" int sp_hip_attn_decode_f16(const void *d_k, const void *d_v, int n_heads_kv, int max_seq,
                                      int head_dim, int layer, int n_kv, const float *d_q, int n_q,
                                      float kq_scale, float *d_scores, float *d_out, void *stream) {
    if (!d_k || !d_v || !d_q || n_kv <= 0 || n_kv > max_seq || layer < 0) { set_err("attn_f16: bad args"); return -1; }
    const size_t need = sp_attn_workspace_floats(n_q, head_dim, n_kv);
    std::lock_guard<std::mutex> lk(g_f16ws_mu);
    if (need > g_f16ws_n) {
        if (g_f16ws) (void)hipFree(g_f16ws);
        g_f16ws = nullptr;
        g_f16ws_n = 0;
        if (!hip_ok(hipMalloc((void **)&g_f16ws, need * sizeof(float)), "attn_f16 workspace")) return -1;
        g_f16ws_n = need;
    }
    const long long hs = (long long)max_seq * head_dim;
    const unsigned short *k = (const unsigned short *)d_k + (long long)layer * n_heads_kv * hs;
    const unsigned short *v = (const unsigned short *)d_v + (long long)layer * n_heads_kv * hs;
    return hip_ok(sp_launch_attn_f16(k, v, hs, n_kv, n_q, n_heads_kv, head_dim, kq_scale, d_q,
                                     d_scores, d_out, g_f16ws, g_f16ws_n, (hipStream_t)stream),
                  "attn_f16") ? 0 : -1;
}

// ===========================================================================
// sqfree cache
// ===========================================================================
struct SqPriv {
    SpPlan kplan, vplan;   // bands over sk_k, transform over pad_dim
    bool default_tables = true;  // Knight tables not recalibrated
    // Knight recalibration: fp64 sums of the fed vectors' padded transforms
    bool calibrating = false;
    std::vector<double> csum, csum2;
    long long cn = 0;
    // fused attention workspace (prepared queries, run partials), grown on demand
    float *d_attn_ws = nullptr;
    size_t attn_ws_floats = 0;
};

static SpSqGeo sq_geo(const sp_hip_sqfree_cache_t *cc, int is_v) {
    SpSqGeo G;
    G.hd = cc->config.head_dim;
    G.pad = cc->pad_dim;
    G.sk_k = cc->sk_k;
    G.n_res = cc->n_res;
    G.rbits = cc->residual_bits;
    G.spinor = cc->use_spinor;
    G.bytes = is_v ? cc->bytes_per_pos_v : cc->bytes_per_pos_k;
    G.skel_idx = cc->d_skeleton_idx;
    G.res_idx = cc->d_residual_idx;
    G.csr_off = cc->d_csr_offsets;
    G.csr_slot = cc->d_csr_skel_slot;
    G.csr_mu = cc->d_csr_mu_sign;
    G.default_tables = ((const SqPriv *)cc->priv)->default_tables ? 1 : 0;
    return G;
}

// Knight mask: skeleton = first sk_k entries of the squarefree-first order (or of
// a calibrated ranking) over [0, pad); residuals = the rest; CSR terms of residual c (n = c+1): proper
// divisors d of n whose coefficient d-1 is in the skeleton with mu(n/d) != 0,
// sign mu(n/d). The reference builder (sp_knight_mask_init, called at
// shannon_prime_sqfree.cu:606) is absent; this is the build's documented rule.
static void build_knight(int pad, int sk_k, std::vector<int> &skel, std::vector<int> &res,
                         std::vector<int> &off, std::vector<int> &slot, std::vector<int> &mu,
                         const int *ranking = nullptr) {
    // ranking: a permutation of [0, pad) (calibration's variance ranking); NULL:
    // the squarefree-first order
    std::vector<int> order(pad), slot_of(pad, -1);
    if (ranking) std::copy(ranking, ranking + pad, order.begin());
    else build_mobius_order(pad, order.data());
    skel.assign(order.begin(), order.begin() + sk_k);
    res.assign(order.begin() + sk_k, order.end());
    for (int s = 0; s < sk_k; s++) slot_of[skel[s]] = s;
    off.assign(1, 0);
    slot.clear();
    mu.clear();
    for (size_t r = 0; r < res.size(); r++) {
        const int n = res[r] + 1;
        for (int d = 1; d < n; d++) {
            if (n % d) continue;
            const int m = mobius_mu(n / d);
            if (m == 0 || slot_of[d - 1] < 0) continue;
            slot.push_back(slot_of[d - 1]);
            mu.push_back(m);
        }
        off.push_back((int)slot.size());
    }
}

template <typename T>
static bool upload(T **dptr, const std::vector<T> &h) {
    const size_t n = h.empty() ? 1 : h.size();
    if (!hip_ok(hipMalloc((void **)dptr, n * sizeof(T)), "hipMalloc table")) return false;
    if (h.empty()) return true;
    return hip_ok(hipMemcpy(*dptr, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), "table H2D");
}

extern "C" int sp_hip_sqfree_cache_init_ex(sp_hip_sqfree_cache_t *cc, const sp_config_t *cfg, int max_seq_len,
                                           int residual_bits, int use_spinor, int sk_k, void *stream) {
    if (!cc) return -1;
    memset(cc, 0, sizeof(*cc));
    if (!cfg || cfg->head_dim <= 0 || cfg->n_layers <= 0 || cfg->n_heads_kv <= 0 || max_seq_len <= 0 ||
        residual_bits < 1 || residual_bits > 8) { set_err("sqfree_init: bad config"); return -1; }
    if (!sp_hip_available()) { set_err("sqfree_init: no gfx950 device"); return -1; }
    const int pad = sp_sqfree_pad_dim(cfg->head_dim);
    if (pad <= 0 || pad > SP_GEN_MAX_N) { set_err("sqfree_init: pad %d unsupported", pad); return -1; }
    if (sk_k <= 0) sk_k = pad / 2;
    if (sk_k > pad) sk_k = pad;
    cc->config = *cfg;
    cc->pad_dim = pad;
    cc->sk_k = sk_k;
    cc->n_res = pad - sk_k;
    cc->residual_bits = residual_bits;
    cc->use_spinor = use_spinor ? 1 : 0;
    cc->max_seq_len = max_seq_len;
    cc->n_slots = cfg->n_layers * cfg->n_heads_kv;
    cc->stream = stream;
    // bands over the skeleton; reference defaults 5/4/4/4/5 (shannon_prime_sqfree.cu:615-624)
    static const int defb[5] = {5, 4, 4, 4, 5};
    int kb[SP_MAX_BANDS], vb[SP_MAX_BANDS];
    const int knb = (cfg->k_n_bands > 0 && cfg->k_n_bands <= SP_MAX_BANDS) ? cfg->k_n_bands : 5;
    const int vnb = (cfg->v_n_bands > 0 && cfg->v_n_bands <= SP_MAX_BANDS) ? cfg->v_n_bands : 5;
    for (int i = 0; i < knb; i++) kb[i] = cfg->k_band_bits[i] > 0 ? cfg->k_band_bits[i] : defb[i % 5];
    for (int i = 0; i < vnb; i++) vb[i] = cfg->v_band_bits[i] > 0 ? cfg->v_band_bits[i] : defb[i % 5];
    if (!valid_bits(kb, knb) || !valid_bits(vb, vnb)) { set_err("sqfree_init: band bits"); return -1; }
    sp_band_config_init(&cc->k_bands, sk_k, knb, kb);
    sp_band_config_init(&cc->v_bands, sk_k, vnb, vb);
    SqPriv *pv = new SqPriv();
    cc->priv = pv;
    if (sp_build_plan(&cc->k_bands, pad, 0, -1, &pv->kplan) || sp_build_plan(&cc->v_bands, pad, 0, -1, &pv->vplan)) {
        set_err("sqfree_init: plan");
        sp_hip_sqfree_cache_free(cc);
        return -1;
    }
    std::vector<int> skel, res, off, slot, mu;
    build_knight(pad, sk_k, skel, res, off, slot, mu);
    cc->n_terms = (int)slot.size();
    const int res_bytes = (cc->n_res * residual_bits + 7) / 8;
    const int sheet = cc->use_spinor ? (cc->n_res + 7) / 8 : 0;
    cc->bytes_per_pos_k = cc->k_bands.total_bytes + 4 + res_bytes + sheet;
    cc->bytes_per_pos_v = cc->v_bands.total_bytes + 4 + res_bytes + sheet;
    if (cc->bytes_per_pos_k + 8 > SP_GEN_MAX_REC || cc->bytes_per_pos_v + 8 > SP_GEN_MAX_REC) {
        set_err("sqfree_init: record too large");
        sp_hip_sqfree_cache_free(cc);
        return -1;
    }
    // SP_CACHE_SLACK bytes past the last record: per-lane record loaders read the
    // dwords covering a record
    const size_t kbytes = (size_t)cc->n_slots * max_seq_len * cc->bytes_per_pos_k + SP_CACHE_SLACK;
    const size_t vbytes = (size_t)cc->n_slots * max_seq_len * cc->bytes_per_pos_v + SP_CACHE_SLACK;
    bool ok = upload(&cc->d_skeleton_idx, skel) && upload(&cc->d_residual_idx, res) &&
              upload(&cc->d_csr_offsets, off) && upload(&cc->d_csr_skel_slot, slot) &&
              upload(&cc->d_csr_mu_sign, mu) &&
              hip_ok(hipMalloc((void **)&cc->d_k_cache, kbytes), "hipMalloc sqfree K") &&
              hip_ok(hipMalloc((void **)&cc->d_v_cache, vbytes), "hipMalloc sqfree V") &&
              hip_ok(hipMemsetAsync(cc->d_k_cache, 0, kbytes, (hipStream_t)stream), "memset") &&
              hip_ok(hipMemsetAsync(cc->d_v_cache, 0, vbytes, (hipStream_t)stream), "memset") &&
              hip_ok(hipStreamSynchronize((hipStream_t)stream), "sync");
    if (!ok) {
        sp_hip_sqfree_cache_free(cc);
        return -1;
    }
    return 0;
}

extern "C" int sp_hip_sqfree_cache_init(sp_hip_sqfree_cache_t *cc, const sp_config_t *cfg, int max_seq_len,
                                        int residual_bits, int use_spinor, void *stream) {
    return sp_hip_sqfree_cache_init_ex(cc, cfg, max_seq_len, residual_bits, use_spinor, 0, stream);
}

extern "C" void sp_hip_sqfree_cache_free(sp_hip_sqfree_cache_t *cc) {
    if (!cc) return;
    void *ptrs[] = {cc->d_skeleton_idx, cc->d_residual_idx, cc->d_csr_offsets, cc->d_csr_skel_slot,
                    cc->d_csr_mu_sign, cc->d_k_cache, cc->d_v_cache};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    if (cc->priv && ((SqPriv *)cc->priv)->d_attn_ws) (void)hipFree(((SqPriv *)cc->priv)->d_attn_ws);
    delete (SqPriv *)cc->priv;
    memset(cc, 0, sizeof(*cc));
}

static bool sq_slot_ok(const sp_hip_sqfree_cache_t *cc, int layer, int head, int pos, int n) {
    return cc && cc->priv && layer >= 0 && layer < cc->config.n_layers && head >= 0 &&
           head < cc->config.n_heads_kv && pos >= 0 && n >= 0 && (long long)pos + n <= cc->max_seq_len;
}

extern "C" int sp_hip_sqfree_write_batch(sp_hip_sqfree_cache_t *cc, int is_v, int layer, int head,
                                         int start_pos, int n_pos, const void *d_src, int dtype) {
    if (!sq_slot_ok(cc, layer, head, start_pos, n_pos) || !d_src) { set_err("sqfree write: bad args"); return -1; }
    SqPriv *pv = (SqPriv *)cc->priv;
    const SpSqGeo G = sq_geo(cc, is_v);
    unsigned char *base = is_v ? cc->d_v_cache : cc->d_k_cache;
    const long long slot = (long long)layer * cc->config.n_heads_kv + head;
    unsigned char *dst = base + (slot * cc->max_seq_len + start_pos) * G.bytes;
    return hip_ok(sp_launch_sqfree_encode(is_v ? pv->vplan : pv->kplan, G, d_src, dtype, 0,
                                          cc->config.head_dim, dst, 0, 1, n_pos, (hipStream_t)cc->stream),
                  "sqfree encode") ? 0 : -1;
}

extern "C" int sp_hip_sqfree_read_batch(const sp_hip_sqfree_cache_t *cc, int is_v, int layer, int head,
                                        int start_pos, int n_pos, void *d_dst, int dtype) {
    if (!sq_slot_ok(cc, layer, head, start_pos, n_pos) || !d_dst) { set_err("sqfree read: bad args"); return -1; }
    SqPriv *pv = (SqPriv *)cc->priv;
    const SpSqGeo G = sq_geo(cc, is_v);
    const unsigned char *base = is_v ? cc->d_v_cache : cc->d_k_cache;
    const long long slot = (long long)layer * cc->config.n_heads_kv + head;
    const unsigned char *src = base + (slot * cc->max_seq_len + start_pos) * G.bytes;
    return hip_ok(sp_launch_sqfree_decode(is_v ? pv->vplan : pv->kplan, G, src, 0, d_dst, dtype, 0,
                                          cc->config.head_dim, 1, n_pos, (hipStream_t)cc->stream),
                  "sqfree decode") ? 0 : -1;
}

extern "C" int sp_hip_sqfree_write_layer(sp_hip_sqfree_cache_t *cc, int layer, int start_pos, int n_tok,
                                         const void *d_k, const void *d_v, long long row_stride, int dtype) {
    if (!sq_slot_ok(cc, layer, 0, start_pos, n_tok)) { set_err("sqfree write_layer: bad layer/pos"); return -1; }
    const int H = cc->config.n_heads_kv, hd = cc->config.head_dim;
    if (row_stride < (long long)H * hd) { set_err("sqfree write_layer: row_stride"); return -1; }
    SqPriv *pv = (SqPriv *)cc->priv;
    for (int is_v = 0; is_v < 2; is_v++) {
        const void *src = is_v ? d_v : d_k;
        if (!src) continue;
        const SpSqGeo G = sq_geo(cc, is_v);
        unsigned char *dst = (is_v ? cc->d_v_cache : cc->d_k_cache) +
                             ((long long)layer * H * cc->max_seq_len + start_pos) * G.bytes;
        if (!hip_ok(sp_launch_sqfree_encode(is_v ? pv->vplan : pv->kplan, G, src, dtype, hd, row_stride, dst,
                                            (long long)cc->max_seq_len * G.bytes, H, n_tok, (hipStream_t)cc->stream),
                    "sqfree write_layer")) return -1;
    }
    return 0;
}

extern "C" int sp_hip_sqfree_read_layer(const sp_hip_sqfree_cache_t *cc, int layer, int start_pos, int n_tok,
                                        void *d_k, void *d_v, long long row_stride, int dtype) {
    if (!sq_slot_ok(cc, layer, 0, start_pos, n_tok)) { set_err("sqfree read_layer: bad layer/pos"); return -1; }
    const int H = cc->config.n_heads_kv, hd = cc->config.head_dim;
    if (row_stride < (long long)H * hd) { set_err("sqfree read_layer: row_stride"); return -1; }
    SqPriv *pv = (SqPriv *)cc->priv;
    for (int is_v = 0; is_v < 2; is_v++) {
        void *dst = is_v ? d_v : d_k;
        if (!dst) continue;
        const SpSqGeo G = sq_geo(cc, is_v);
        const unsigned char *src = (is_v ? cc->d_v_cache : cc->d_k_cache) +
                                   ((long long)layer * H * cc->max_seq_len + start_pos) * G.bytes;
        if (!hip_ok(sp_launch_sqfree_decode(is_v ? pv->vplan : pv->kplan, G, src, (long long)cc->max_seq_len * G.bytes,
                                            dst, dtype, hd, row_stride, H, n_tok, (hipStream_t)cc->stream),
                    "sqfree read_layer")) return -1;
    }
    return 0;
}

extern "C" int sp_hip_sqfree_attn_decode_seqs(const sp_hip_sqfree_cache_t *cc, int layer, int n_seq,
                                              const int *seq_start, const int *seq_len, const float *d_q, int n_q,
                                              float kq_scale, float *d_scores, float *d_out, void *stream) {
    if (!cc || !cc->priv || layer < 0 || layer >= cc->config.n_layers || !d_q || n_q <= 0 || (!d_scores && !d_out)) {
        set_err("sqfree attn: bad args");
        return -1;
    }
    SpSeqTab T;
    if (!seq_tab(n_seq, seq_start, seq_len, cc->max_seq_len, n_q, &T, "sqfree attn")) return -1;
    const int H = cc->config.n_heads_kv;
    if (n_q % H || n_q / H > 8) { set_err("sqfree attn: n_q must be a multiple of n_heads_kv, at most 8 per KV head"); return -1; }
    SqPriv *pv = (SqPriv *)cc->priv;
    const SpSqGeo GK = sq_geo(cc, 0);
    if (!sp_sqfree_attn_kind(pv->kplan, pv->vplan, GK)) {
        set_err("sqfree attn: no fused kernel for this geometry (needs head_dim 128, pad 154, skeleton 77 or 115 "
                "with K bands 5/4/4/4/5, V 5/4/4/4/5 or one 3-bit band at 115, 3-bit residuals, spinor, "
                "default Knight tables)");
        return -1;
    }
    const long long slot0 = (long long)layer * H;
    SpHierAttnArgs HA;
    memset(&HA, 0, sizeof(HA));
    HA.W = nullptr;  // no predictor: the skeleton and residual coefficients are both stored
    HA.skel_idx = cc->d_skeleton_idx;
    HA.tgt_idx = cc->d_residual_idx;
    HA.q = d_q;
    HA.kq_scale = kq_scale;
    HA.scores = d_scores;
    HA.out = d_out;
    HA.n_q = n_q;
    HA.n_kvh = H;
    HA.n_kv = T.max_len;
    HA.hd = cc->config.head_dim;
    HA.pad = cc->pad_dim;
    HA.n_skel = cc->sk_k;
    HA.n_target = cc->n_res;
    HA.rbits = cc->residual_bits;
    HA.B = cc->bytes_per_pos_k;
    HA.ps = sp_hier_attn_prep_floats(HA.n_skel, HA.n_target);
    HA.pp = (4 + HA.n_skel + HA.n_target + 3) & ~3;
    SpSqAttnArgs A;
    A.kcache = cc->d_k_cache + slot0 * cc->max_seq_len * cc->bytes_per_pos_k;
    A.vcache = cc->d_v_cache + slot0 * cc->max_seq_len * cc->bytes_per_pos_v;
    A.k_slot_bytes = (long long)cc->max_seq_len * cc->bytes_per_pos_k;
    A.v_slot_bytes = (long long)cc->max_seq_len * cc->bytes_per_pos_v;
    A.scores = d_scores;
    A.out = d_out;
    A.n_q = n_q;
    A.n_kvh = H;
    A.n_kv = T.max_len;
    A.ps = HA.ps;
    A.qo = (HA.n_skel + 3) & ~3;  // the prepared query's residual part
    A.pp = HA.pp;
    int n_runs = sp_sqfree_attn_runs(pv->kplan, pv->vplan, GK, n_q, H, T.max_len, cu_count(), n_seq, d_out != nullptr);
    // SP_HIP_SQFREE_ATTN_RUNS=n caps the runs per KV head (read at each call; tests use it
    // to give every run several tiles at small context lengths)
    if (const char *e = getenv("SP_HIP_SQFREE_ATTN_RUNS")) {
        const int r = atoi(e);
        if (r > 0) n_runs = std::min(n_runs, r);
    }
    const hipStream_t s = (hipStream_t)(stream ? stream : cc->stream);
    if (!grow_ws(&pv->d_attn_ws, &pv->attn_ws_floats, sp_hier_attn_workspace_floats(HA, n_runs, n_seq), s,
                 "sqfree attn workspace")) return -1;
    return hip_ok(sp_launch_sqfree_attn(pv->kplan, pv->vplan, GK, HA, A, T, pv->d_attn_ws, pv->attn_ws_floats,
                                        n_runs, s), "sqfree attn") ? 0 : -1;
}

extern "C" int sp_hip_sqfree_attn_decode(const sp_hip_sqfree_cache_t *cc, int layer, int n_kv, const float *d_q,
                                         int n_q, float kq_scale, float *d_scores, float *d_out, void *stream) {
    const int start = 0;
    return sp_hip_sqfree_attn_decode_seqs(cc, layer, 1, &start, &n_kv, d_q, n_q, kq_scale, d_scores, d_out, stream);
}

extern "C" void sp_hip_sqfree_write_k(sp_hip_sqfree_cache_t *cc, int l, int h, int p, const float *d) { sp_hip_sqfree_write_batch(cc, 0, l, h, p, 1, d, SP_DT_F32); }
extern "C" void sp_hip_sqfree_write_v(sp_hip_sqfree_cache_t *cc, int l, int h, int p, const float *d) { sp_hip_sqfree_write_batch(cc, 1, l, h, p, 1, d, SP_DT_F32); }
extern "C" void sp_hip_sqfree_read_k(const sp_hip_sqfree_cache_t *cc, int l, int h, int p, float *d) { sp_hip_sqfree_read_batch(cc, 0, l, h, p, 1, d, SP_DT_F32); }
extern "C" void sp_hip_sqfree_read_v(const sp_hip_sqfree_cache_t *cc, int l, int h, int p, float *d) { sp_hip_sqfree_read_batch(cc, 1, l, h, p, 1, d, SP_DT_F32); }
extern "C" void sp_hip_sqfree_read_k_batch(const sp_hip_sqfree_cache_t *cc, int l, int h, int s, int n, float *d) { sp_hip_sqfree_read_batch(cc, 0, l, h, s, n, d, SP_DT_F32); }
extern "C" void sp_hip_sqfree_read_v_batch(const sp_hip_sqfree_cache_t *cc, int l, int h, int s, int n, float *d) { sp_hip_sqfree_read_batch(cc, 1, l, h, s, n, d, SP_DT_F32); }

extern "C" int sp_hip_sqfree_calibrate_begin(sp_hip_sqfree_cache_t *cc) {
    if (!cc || !cc->priv) { set_err("sqfree calibrate_begin: bad cache"); return -1; }
    SqPriv *pv = (SqPriv *)cc->priv;
    pv->csum.assign((size_t)cc->pad_dim, 0.0);
    pv->csum2.assign((size_t)cc->pad_dim, 0.0);
    pv->cn = 0;
    pv->calibrating = true;
    return 0;
}

extern "C" int sp_hip_sqfree_calibrate_feed(sp_hip_sqfree_cache_t *cc, const void *d_vecs, long long row_stride,
                                            int n_vecs, int dtype) {
    if (!cc || !cc->priv || n_vecs < 0 || (n_vecs > 0 && !d_vecs) || row_stride < cc->config.head_dim ||
        (dtype != SP_DT_F16 && dtype != SP_DT_F32)) { set_err("sqfree calibrate_feed: bad args"); return -1; }
    SqPriv *pv = (SqPriv *)cc->priv;
    if (!pv->calibrating) { set_err("sqfree calibrate_feed: no calibrate_begin"); return -1; }
    if (n_vecs == 0) return 0;
    if (!calib_accumulate(pv->kplan, cc->config.head_dim, cc->pad_dim, d_vecs, dtype, row_stride, n_vecs,
                          pv->csum.data(), pv->csum2.data(), (hipStream_t)cc->stream)) return -1;
    pv->cn += n_vecs;
    return 0;
}

extern "C" int sp_hip_sqfree_calibrate_end(sp_hip_sqfree_cache_t *cc, int *ranking_out, int apply) {
    if (!cc || !cc->priv) { set_err("sqfree calibrate_end: bad cache"); return -1; }
    SqPriv *pv = (SqPriv *)cc->priv;
    if (!pv->calibrating || pv->cn <= 0) { set_err("sqfree calibrate_end: no data fed"); return -1; }
    const int pad = cc->pad_dim;
    std::vector<int> rank((size_t)pad);
    rank_by_variance(pv->csum.data(), pv->csum2.data(), pv->cn, pad, rank.data());
    if (ranking_out) std::copy(rank.begin(), rank.end(), ranking_out);
    if (apply) {
        std::vector<int> skel, res, off, slot, mu;
        build_knight(pad, cc->sk_k, skel, res, off, slot, mu, rank.data());
        int *old[5] = {cc->d_skeleton_idx, cc->d_residual_idx, cc->d_csr_offsets, cc->d_csr_skel_slot,
                       cc->d_csr_mu_sign};
        cc->d_skeleton_idx = cc->d_residual_idx = cc->d_csr_offsets = cc->d_csr_skel_slot = cc->d_csr_mu_sign = nullptr;
        const bool ok = hip_ok(hipStreamSynchronize((hipStream_t)cc->stream), "sqfree calib sync") &&
                        upload(&cc->d_skeleton_idx, skel) && upload(&cc->d_residual_idx, res) &&
                        upload(&cc->d_csr_offsets, off) && upload(&cc->d_csr_skel_slot, slot) &&
                        upload(&cc->d_csr_mu_sign, mu);
        if (!ok) {
            int *now[5] = {cc->d_skeleton_idx, cc->d_residual_idx, cc->d_csr_offsets, cc->d_csr_skel_slot,
                           cc->d_csr_mu_sign};
            for (int *q : now)
                if (q) (void)hipFree(q);
            cc->d_skeleton_idx = old[0], cc->d_residual_idx = old[1], cc->d_csr_offsets = old[2];
            cc->d_csr_skel_slot = old[3], cc->d_csr_mu_sign = old[4];
            return -1;
        }
        for (int *q : old)
            if (q) (void)hipFree(q);
        cc->n_terms = (int)slot.size();
        std::vector<int> dflt((size_t)pad);
        build_mobius_order(pad, dflt.data());
        pv->default_tables = std::equal(dflt.begin(), dflt.begin() + cc->sk_k, rank.begin()) &&
                             std::equal(dflt.begin() + cc->sk_k, dflt.end(), rank.begin() + cc->sk_k);
    }
    pv->calibrating = false;
    return 0;
}

extern "C" int sp_hip_sqfree_get_tables(const sp_hip_sqfree_cache_t *cc, int *skeleton_idx, int *residual_idx,
                                        int *csr_offsets, int *csr_skel_slot, int *csr_mu_sign) {
    if (!cc || !cc->priv) return -1;
    bool ok = true;
    if (skeleton_idx) ok &= hip_ok(hipMemcpy(skeleton_idx, cc->d_skeleton_idx, sizeof(int) * cc->sk_k, hipMemcpyDeviceToHost), "D2H");
    if (residual_idx && cc->n_res) ok &= hip_ok(hipMemcpy(residual_idx, cc->d_residual_idx, sizeof(int) * cc->n_res, hipMemcpyDeviceToHost), "D2H");
    if (csr_offsets) ok &= hip_ok(hipMemcpy(csr_offsets, cc->d_csr_offsets, sizeof(int) * (cc->n_res + 1), hipMemcpyDeviceToHost), "D2H");
    if (csr_skel_slot && cc->n_terms) ok &= hip_ok(hipMemcpy(csr_skel_slot, cc->d_csr_skel_slot, sizeof(int) * cc->n_terms, hipMemcpyDeviceToHost), "D2H");
    if (csr_mu_sign && cc->n_terms) ok &= hip_ok(hipMemcpy(csr_mu_sign, cc->d_csr_mu_sign, sizeof(int) * cc->n_terms, hipMemcpyDeviceToHost), "D2H");
    return ok ? 0 : -1;
}

// ===========================================================================
// hierarchical cache
// ===========================================================================
struct HierPriv {
    SpPlan plan;
    bool default_geo;  // skeleton/targets equal sp_hier_default_geometry(pad_dim)
    // predictor fit: per-slot fp64 Gram accumulators on the device
    bool calibrating = false;
    double *d_acc = nullptr;   // [n_slots][n_ent]
    double *d_part = nullptr;  // [256][n_ent] block partials of one feed
    std::vector<long long> n_fed;
    // fused attention: prepared queries and the runs' partials (grown on demand)
    float *d_attn_ws = nullptr;
    size_t attn_ws_floats = 0;
};

static void hier_calib_release(HierPriv *pv) {
    if (pv->d_acc) (void)hipFree(pv->d_acc);
    if (pv->d_part) (void)hipFree(pv->d_part);
    pv->d_acc = pv->d_part = nullptr;
    pv->n_fed.clear();
    pv->calibrating = false;
}

extern "C" int sp_hip_hier_cache_init(sp_hip_hier_cache_t *hc, const sp_config_t *cfg, int pad_dim,
                                      int n_skeleton, int n_target, int target_res_bits,
                                      const int *skeleton_idx, const int *target_idx,
                                      const sp_band_config_t *skel_bands, int max_seq_len, int n_slots,
                                      void *stream) {
    if (!hc) return -1;
    memset(hc, 0, sizeof(*hc));
    if (!cfg || !skeleton_idx || !target_idx || !skel_bands || pad_dim <= 0 || pad_dim > SP_GEN_MAX_N ||
        n_skeleton <= 0 || n_target <= 0 || n_skeleton + n_target > pad_dim || target_res_bits < 1 ||
        target_res_bits > 8 || max_seq_len <= 0 || n_slots <= 0 || cfg->head_dim > pad_dim ||
        skel_bands->head_dim != n_skeleton) { set_err("hier_init: bad args"); return -1; }
    for (int i = 0; i < n_skeleton; i++) if (skeleton_idx[i] < 0 || skeleton_idx[i] >= pad_dim) { set_err("hier_init: skeleton idx"); return -1; }
    for (int i = 0; i < n_target; i++) if (target_idx[i] < 0 || target_idx[i] >= pad_dim) { set_err("hier_init: target idx"); return -1; }
    if (!sp_hip_available()) { set_err("hier_init: no gfx950 device"); return -1; }
    hc->config = *cfg;
    hc->pad_dim = pad_dim;
    hc->n_skeleton = n_skeleton;
    hc->n_target = n_target;
    hc->target_res_bits = target_res_bits;
    hc->n_slots = n_slots;
    hc->max_seq_len = max_seq_len;
    hc->skel_bands = *skel_bands;
    hc->stream = stream;
    HierPriv *pv = new HierPriv();
    hc->priv = pv;
    if (sp_build_plan(skel_bands, pad_dim, 0, -1, &pv->plan)) { set_err("hier_init: plan"); sp_hip_hier_cache_free(hc); return -1; }
    {
        std::vector<int> ds((size_t)pad_dim), dt((size_t)pad_dim);
        const int ns = sp_hier_default_geometry(pad_dim, ds.data(), dt.data());
        pv->default_geo = ns == n_skeleton && n_target == pad_dim - ns &&
                          std::equal(skeleton_idx, skeleton_idx + n_skeleton, ds.begin()) &&
                          std::equal(target_idx, target_idx + n_target, dt.begin());
    }
    const int res_bytes = (n_target * target_res_bits + 7) / 8;
    hc->bytes_per_pos_k = hc->bytes_per_pos_v = skel_bands->total_bytes + 4 + res_bytes;
    if (hc->bytes_per_pos_k + 8 > SP_GEN_MAX_REC) { set_err("hier_init: record too large"); sp_hip_hier_cache_free(hc); return -1; }
    const size_t cb = (size_t)n_slots * max_seq_len * hc->bytes_per_pos_k + SP_CACHE_SLACK;
    const size_t wb = (size_t)n_slots * n_target * n_skeleton * sizeof(uint16_t);
    std::vector<int> sk(skeleton_idx, skeleton_idx + n_skeleton), tg(target_idx, target_idx + n_target);
    bool ok = upload(&hc->d_skeleton_idx, sk) && upload(&hc->d_target_idx, tg) &&
              hip_ok(hipMalloc((void **)&hc->d_k_cache, cb), "hipMalloc hier K") &&
              hip_ok(hipMalloc((void **)&hc->d_v_cache, cb), "hipMalloc hier V") &&
              hip_ok(hipMalloc((void **)&hc->d_W, wb), "hipMalloc W") &&
              hip_ok(hipMemsetAsync(hc->d_k_cache, 0, cb, (hipStream_t)stream), "memset") &&
              hip_ok(hipMemsetAsync(hc->d_v_cache, 0, cb, (hipStream_t)stream), "memset") &&
              hip_ok(hipMemsetAsync(hc->d_W, 0, wb, (hipStream_t)stream), "memset") &&
              hip_ok(hipStreamSynchronize((hipStream_t)stream), "sync");
    if (!ok) {
        sp_hip_hier_cache_free(hc);
        return -1;
    }
    return 0;
}

extern "C" void sp_hip_hier_cache_free(sp_hip_hier_cache_t *hc) {
    if (!hc) return;
    void *ptrs[] = {hc->d_W, hc->d_skeleton_idx, hc->d_target_idx, hc->d_k_cache, hc->d_v_cache};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    if (hc->priv) {
        hier_calib_release((HierPriv *)hc->priv);
        if (((HierPriv *)hc->priv)->d_attn_ws) (void)hipFree(((HierPriv *)hc->priv)->d_attn_ws);
    }
    delete (HierPriv *)hc->priv;
    memset(hc, 0, sizeof(*hc));
}

extern "C" int sp_hip_hier_cache_upload_W(sp_hip_hier_cache_t *hc, const uint16_t *W_all) {
    if (!hc || !hc->priv || !W_all) return -1;
    const size_t wb = (size_t)hc->n_slots * hc->n_target * hc->n_skeleton * sizeof(uint16_t);
    return hip_ok(hipMemcpy(hc->d_W, W_all, wb, hipMemcpyHostToDevice), "upload_W") ? 0 : -1;
}

static SpHierGeo hier_geo(const sp_hip_hier_cache_t *hc, int slot) {
    SpHierGeo G;
    G.hd = hc->config.head_dim;
    G.pad = hc->pad_dim;
    G.n_skel = hc->n_skeleton;
    G.n_target = hc->n_target;
    G.rbits = hc->target_res_bits;
    G.bytes = hc->bytes_per_pos_k;
    G.skel_idx = hc->d_skeleton_idx;
    G.target_idx = hc->d_target_idx;
    G.W = hc->d_W + (size_t)slot * hc->n_target * hc->n_skeleton;
    G.w_outer = (long long)hc->n_target * hc->n_skeleton;
    G.default_geo = ((const HierPriv *)hc->priv)->default_geo ? 1 : 0;
    return G;
}

static bool hier_slot_ok(const sp_hip_hier_cache_t *hc, int layer, int head, int pos, int n) {
    if (!hc || !hc->priv || layer < 0 || head < 0 || head >= hc->config.n_heads_kv || pos < 0 || n < 0 ||
        (long long)pos + n > hc->max_seq_len) return false;
    const long long slot = (long long)layer * hc->config.n_heads_kv + head;
    return slot < hc->n_slots;
}

extern "C" int sp_hip_hier_write_batch(sp_hip_hier_cache_t *hc, int is_v, int layer, int head, int start_pos,
                                       int n_pos, const void *d_src, int dtype) {
    if (!hier_slot_ok(hc, layer, head, start_pos, n_pos) || !d_src) { set_err("hier write: bad args"); return -1; }
    const int slot = layer * hc->config.n_heads_kv + head;
    const SpHierGeo G = hier_geo(hc, slot);
    unsigned char *base = is_v ? hc->d_v_cache : hc->d_k_cache;
    unsigned char *dst = base + ((long long)slot * hc->max_seq_len + start_pos) * G.bytes;
    return hip_ok(sp_launch_hier_encode(((HierPriv *)hc->priv)->plan, G, d_src, dtype, 0, hc->config.head_dim,
                                        dst, 0, 1, n_pos, (hipStream_t)hc->stream), "hier encode") ? 0 : -1;
}

extern "C" int sp_hip_hier_read_batch(const sp_hip_hier_cache_t *hc, int is_v, int layer, int head, int start_pos,
                                      int n_pos, void *d_dst, int dtype) {
    if (!hier_slot_ok(hc, layer, head, start_pos, n_pos) || !d_dst) { set_err("hier read: bad args"); return -1; }
    const int slot = layer * hc->config.n_heads_kv + head;
    const SpHierGeo G = hier_geo(hc, slot);
    const unsigned char *base = is_v ? hc->d_v_cache : hc->d_k_cache;
    const unsigned char *src = base + ((long long)slot * hc->max_seq_len + start_pos) * G.bytes;
    return hip_ok(sp_launch_hier_decode(((HierPriv *)hc->priv)->plan, G, src, 0, d_dst, dtype, 0,
                                        hc->config.head_dim, 1, n_pos, (hipStream_t)hc->stream),
                  "hier decode") ? 0 : -1;
}

extern "C" int sp_hip_hier_write_layer(sp_hip_hier_cache_t *hc, int layer, int start_pos, int n_tok,
                                       const void *d_k, const void *d_v, long long row_stride, int dtype) {
    if (!hier_slot_ok(hc, layer, 0, start_pos, n_tok) ||
        (long long)(layer + 1) * hc->config.n_heads_kv > hc->n_slots) { set_err("hier write_layer: bad layer/pos"); return -1; }
    const int H = hc->config.n_heads_kv, hd = hc->config.head_dim;
    if (row_stride < (long long)H * hd) { set_err("hier write_layer: row_stride"); return -1; }
    const SpHierGeo G = hier_geo(hc, layer * H);
    const long long rec0 = ((long long)layer * H * hc->max_seq_len + start_pos) * G.bytes;
    const long long hs = (long long)hc->max_seq_len * G.bytes;
    const SpPlan &plan = ((HierPriv *)hc->priv)->plan;
    if (d_k && d_v)  // one launch for both sides: twice the tiles in flight for short chunks
        return hip_ok(sp_launch_hier_encode_kv(plan, G, d_k, d_v, dtype, hd, row_stride, hc->d_k_cache + rec0,
                                               hc->d_v_cache + rec0, hs, H, n_tok, (hipStream_t)hc->stream),
                      "hier write_layer") ? 0 : -1;
    for (int is_v = 0; is_v < 2; is_v++) {
        const void *src = is_v ? d_v : d_k;
        if (!src) continue;
        unsigned char *dst = (is_v ? hc->d_v_cache : hc->d_k_cache) + rec0;
        if (!hip_ok(sp_launch_hier_encode(plan, G, src, dtype, hd, row_stride, dst, hs, H, n_tok,
                                          (hipStream_t)hc->stream),
                    "hier write_layer")) return -1;
    }
    return 0;
}

extern "C" int sp_hip_hier_read_layer(const sp_hip_hier_cache_t *hc, int layer, int start_pos, int n_tok,
                                      void *d_k, void *d_v, long long row_stride, int dtype) {
    if (!hier_slot_ok(hc, layer, 0, start_pos, n_tok) ||
        (long long)(layer + 1) * hc->config.n_heads_kv > hc->n_slots) { set_err("hier read_layer: bad layer/pos"); return -1; }
    const int H = hc->config.n_heads_kv, hd = hc->config.head_dim;
    if (row_stride < (long long)H * hd) { set_err("hier read_layer: row_stride"); return -1; }
    const SpHierGeo G = hier_geo(hc, layer * H);
    for (int is_v = 0; is_v < 2; is_v++) {
        void *dst = is_v ? d_v : d_k;
        if (!dst) continue;
        const unsigned char *src = (is_v ? hc->d_v_cache : hc->d_k_cache) +
                                   ((long long)layer * H * hc->max_seq_len + start_pos) * G.bytes;
        if (!hip_ok(sp_launch_hier_decode(((HierPriv *)hc->priv)->plan, G, src, (long long)hc->max_seq_len * G.bytes,
                                          dst, dtype, hd, row_stride, H, n_tok, (hipStream_t)hc->stream),
                    "hier read_layer")) return -1;
    }
    return 0;
}

extern "C" int sp_hip_hier_attn_decode_seqs(const sp_hip_hier_cache_t *hc, int layer, int n_seq, const int *seq_start,
                                            const int *seq_len, const float *d_q, int n_q, float kq_scale,
                                            float *d_scores, float *d_out, void *stream) {
    if (!hc || !hc->priv || layer < 0 || layer >= hc->config.n_layers || !d_q || n_q <= 0 || (!d_scores && !d_out) ||
        (long long)(layer + 1) * hc->config.n_heads_kv > hc->n_slots) {
        set_err("hier attn: bad args");
        return -1;
    }
    SpSeqTab T;
    if (!seq_tab(n_seq, seq_start, seq_len, hc->max_seq_len, n_q, &T, "hier attn")) return -1;
    const int H = hc->config.n_heads_kv;
    if (n_q % H || n_q / H > 8) { set_err("hier attn: n_q must be a multiple of n_heads_kv, at most 8 per KV head"); return -1; }
    HierPriv *pv = (HierPriv *)hc->priv;
    const SpHierGeo G = hier_geo(hc, layer * H);
    SpHierAttnArgs A;
    A.kcache = hc->d_k_cache + (long long)layer * H * hc->max_seq_len * G.bytes;
    A.vcache = hc->d_v_cache + (long long)layer * H * hc->max_seq_len * G.bytes;
    A.slot_bytes = (long long)hc->max_seq_len * G.bytes;
    A.W = G.W;
    A.w_outer = G.w_outer;
    A.skel_idx = G.skel_idx;
    A.tgt_idx = G.target_idx;
    A.q = d_q;
    A.kq_scale = kq_scale;
    A.scores = d_scores;
    A.out = d_out;
    A.n_q = n_q;
    A.n_kvh = H;
    A.n_kv = T.max_len;
    A.hd = hc->config.head_dim;
    A.pad = hc->pad_dim;
    A.n_skel = hc->n_skeleton;
    A.n_target = hc->n_target;
    A.rbits = hc->target_res_bits;
    A.B = G.bytes;
    A.ps = sp_hier_attn_prep_floats(A.n_skel, A.n_target);
    A.pp = (4 + A.n_skel + A.n_target + 3) & ~3;
    const int cus = cu_count();
    // The 256-position chunk kernel serves every geometry up to its LDS limit (at pad 330,
    // at most 4 query heads per KV head). Past it, the one-position-per-lane split kernel
    // serves the configs[4] geometry (hd 256, pad 330, skeleton 30 at 5/5 bits, 300 targets
    // at 2 bits) with up to 8; it is the slower of the two where both fit (measured at
    // 189 vs 169 us per layer), and SP_HIP_HIER_ATTN_LANE=1 (read at each call)
    // selects it wherever it fits, for tests.
    const char *lane_on = getenv("SP_HIP_HIER_ATTN_LANE");
    const bool lane = sp_hier_attn_lane_ok(pv->plan, A) &&
                      ((lane_on && lane_on[0] == '1') || (A.pad == 330 && n_q / H > 4));
    int n_runs = lane ? sp_hier_attn_lane_runs(A, cus, n_seq) : sp_hier_attn_runs(A, cus, n_seq);
    // SP_HIP_HIER_ATTN_RUNS=n caps the runs per KV head (read at each call; tests use it to
    // give every run several chunks or tiles at small context lengths)
    if (const char *e = getenv("SP_HIP_HIER_ATTN_RUNS")) {
        const int r = atoi(e);
        if (r > 0) n_runs = std::min(n_runs, r);
    }
    const hipStream_t s = (hipStream_t)(stream ? stream : hc->stream);
    if (!grow_ws(&pv->d_attn_ws, &pv->attn_ws_floats, sp_hier_attn_workspace_floats(A, n_runs, n_seq), s,
                 "hier attn workspace")) return -1;
    if (lane)
        return hip_ok(sp_launch_hier_attn_lane(pv->plan, A, T, pv->d_attn_ws, pv->attn_ws_floats, n_runs, s),
                      "hier attn (lane)") ? 0 : -1;
    return hip_ok(sp_launch_hier_attn(pv->plan, A, T, pv->d_attn_ws, pv->attn_ws_floats, n_runs, s), "hier attn") ? 0 : -1;
}

extern "C" int sp_hip_hier_attn_decode(const sp_hip_hier_cache_t *hc, int layer, int n_kv, const float *d_q,
                                       int n_q, float kq_scale, float *d_scores, float *d_out, void *stream) {
    const int start = 0;
    return sp_hip_hier_attn_decode_seqs(hc, layer, 1, &start, &n_kv, d_q, n_q, kq_scale, d_scores, d_out, stream);
}

extern "C" int sp_hip_hier_calibrate_begin(sp_hip_hier_cache_t *hc) {
    if (!hc || !hc->priv) { set_err("hier calibrate_begin: bad cache"); return -1; }
    HierPriv *pv = (HierPriv *)hc->priv;
    hier_calib_release(pv);
    const size_t n_ent = (size_t)sp_calib_gram_entries(hc->n_skeleton, hc->n_target);
    const size_t acc_b = (size_t)hc->n_slots * n_ent * sizeof(double);
    if (!(hip_ok(hipMalloc((void **)&pv->d_acc, acc_b), "hipMalloc gram") &&
          hip_ok(hipMalloc((void **)&pv->d_part, 256 * n_ent * sizeof(double)), "hipMalloc gram partials") &&
          hip_ok(hipMemsetAsync(pv->d_acc, 0, acc_b, (hipStream_t)hc->stream), "memset gram"))) {
        hier_calib_release(pv);
        return -1;
    }
    pv->n_fed.assign((size_t)hc->n_slots, 0);
    pv->calibrating = true;
    return 0;
}

extern "C" int sp_hip_hier_calibrate_feed(sp_hip_hier_cache_t *hc, int slot, const void *d_vecs, long long row_stride,
                                          int n_vecs, int dtype) {
    if (!hc || !hc->priv || slot < 0 || slot >= hc->n_slots || n_vecs < 0 || (n_vecs > 0 && !d_vecs) ||
        row_stride < hc->config.head_dim || (dtype != SP_DT_F16 && dtype != SP_DT_F32)) {
        set_err("hier calibrate_feed: bad args"); return -1;
    }
    HierPriv *pv = (HierPriv *)hc->priv;
    if (!pv->calibrating) { set_err("hier calibrate_feed: no calibrate_begin"); return -1; }
    if (n_vecs == 0) return 0;
    const SpHierGeo G = hier_geo(hc, slot);
    const int n_ent = sp_calib_gram_entries(hc->n_skeleton, hc->n_target);
    const int nb = sp_calib_moment_blocks(n_vecs);
    if (!hip_ok(sp_launch_calib_hier_gram(pv->plan, G, d_vecs, dtype, row_stride, n_vecs, pv->d_part, nb,
                                          pv->d_acc + (size_t)slot * n_ent, (hipStream_t)hc->stream),
                "hier gram")) return -1;
    pv->n_fed[(size_t)slot] += n_vecs;
    return 0;
}

// W = G_ts (G_ss + lambda I)^-1 for one slot: Cholesky of the ns x ns system,
// then one forward / back substitution per target row. False when the system
// is not positive definite.
static bool hier_solve(const double *acc, int ns, int nt, double ridge, std::vector<double> &W) {
    const double *Gts = acc, *Gss = acc + (size_t)nt * ns;
    double tr = 0.0;
    for (int i = 0; i < ns; i++) tr += Gss[(size_t)i * ns + i];
    const double lam = ridge * (tr > 0.0 ? tr / ns : 1.0);
    std::vector<double> Lm((size_t)ns * ns, 0.0);
    for (int i = 0; i < ns; i++)
        for (int j = 0; j <= i; j++) {
            double v = 0.5 * (Gss[(size_t)i * ns + j] + Gss[(size_t)j * ns + i]) + (i == j ? lam : 0.0);
            for (int k = 0; k < j; k++) v -= Lm[(size_t)i * ns + k] * Lm[(size_t)j * ns + k];
            if (i == j) {
                if (!(v > 0.0)) return false;
                Lm[(size_t)i * ns + i] = std::sqrt(v);
            } else {
                Lm[(size_t)i * ns + j] = v / Lm[(size_t)j * ns + j];
            }
        }
    W.assign((size_t)nt * ns, 0.0);
    std::vector<double> y((size_t)ns);
    for (int t = 0; t < nt; t++) {
        for (int i = 0; i < ns; i++) {
            double v = Gts[(size_t)t * ns + i];
            for (int k = 0; k < i; k++) v -= Lm[(size_t)i * ns + k] * y[(size_t)k];
            y[(size_t)i] = v / Lm[(size_t)i * ns + i];
        }
        for (int i = ns - 1; i >= 0; i--) {
            double v = y[(size_t)i];
            for (int k = i + 1; k < ns; k++) v -= Lm[(size_t)k * ns + i] * W[(size_t)t * ns + k];
            W[(size_t)t * ns + i] = v / Lm[(size_t)i * ns + i];
        }
    }
    return true;
}

// Solves every fed slot and uploads W = keep * W_old + (1 - keep) * W_fit (keep = 0:
// plain replacement), rounded to fp16 via fp32; a slot whose system is not
// positive definite fits W_fit = 0.
static int hier_calib_finish(sp_hip_hier_cache_t *hc, double ridge, double keep) {
    if (!hc || !hc->priv || !(ridge >= 0.0) || !(keep >= 0.0 && keep <= 1.0)) {
        set_err("hier calibrate_end: bad args"); return -1;
    }
    HierPriv *pv = (HierPriv *)hc->priv;
    if (!pv->calibrating) { set_err("hier calibrate_end: no calibrate_begin"); return -1; }
    const int ns = hc->n_skeleton, nt = hc->n_target;
    const size_t n_ent = (size_t)sp_calib_gram_entries(ns, nt), w_slot = (size_t)nt * ns;
    std::vector<double> acc((size_t)hc->n_slots * n_ent);
    std::vector<uint16_t> W_all((size_t)hc->n_slots * w_slot);
    hipStream_t s = (hipStream_t)hc->stream;
    bool ok = hip_ok(hipMemcpyAsync(acc.data(), pv->d_acc, acc.size() * sizeof(double), hipMemcpyDeviceToHost, s),
                     "gram D2H") &&
              hip_ok(hipMemcpyAsync(W_all.data(), hc->d_W, W_all.size() * sizeof(uint16_t), hipMemcpyDeviceToHost,
                                    s), "W D2H") &&
              hip_ok(hipStreamSynchronize(s), "gram sync");
    if (ok) {
        std::vector<double> W;
        for (int slot = 0; slot < hc->n_slots; slot++) {
            if (pv->n_fed[(size_t)slot] <= 0) continue;
            uint16_t *dst = W_all.data() + (size_t)slot * w_slot;
            if (!hier_solve(acc.data() + (size_t)slot * n_ent, ns, nt, ridge, W))
                W.assign(w_slot, 0.0);  // degenerate data: no prediction
            for (size_t e = 0; e < w_slot; e++) {
                const double w = keep > 0.0 ? keep * (double)sp_f16_to_f32(dst[e]) + (1.0 - keep) * W[e] : W[e];
                dst[e] = sp_f32_to_f16((float)w);
            }
        }
        ok = hip_ok(hipMemcpy(hc->d_W, W_all.data(), W_all.size() * sizeof(uint16_t), hipMemcpyHostToDevice),
                    "W upload");
    }
    hier_calib_release(pv);
    return ok ? 0 : -1;
}

extern "C" int sp_hip_hier_calibrate_end(sp_hip_hier_cache_t *hc, double ridge) {
    return hier_calib_finish(hc, ridge, 0.0);
}

extern "C" int sp_hip_hier_calibrate_end_ema(sp_hip_hier_cache_t *hc, double ridge, float keep_frac) {
    return hier_calib_finish(hc, ridge, (double)keep_frac);
}

extern "C" void sp_hip_hier_write_k(sp_hip_hier_cache_t *hc, int l, int h, int p, const float *d) { sp_hip_hier_write_batch(hc, 0, l, h, p, 1, d, SP_DT_F32); }
extern "C" void sp_hip_hier_write_v(sp_hip_hier_cache_t *hc, int l, int h, int p, const float *d) { sp_hip_hier_write_batch(hc, 1, l, h, p, 1, d, SP_DT_F32); }
extern "C" void sp_hip_hier_read_k(const sp_hip_hier_cache_t *hc, int l, int h, int p, float *d) { sp_hip_hier_read_batch(hc, 0, l, h, p, 1, d, SP_DT_F32); }
extern "C" void sp_hip_hier_read_v(const sp_hip_hier_cache_t *hc, int l, int h, int p, float *d) { sp_hip_hier_read_batch(hc, 1, l, h, p, 1, d, SP_DT_F32); }

// ===========================================================================
// events / streams
// ===========================================================================
extern "C" void *sp_hip_event_create(void) {
    hipEvent_t e = nullptr;
    if (!hip_ok(hipEventCreate(&e), "event create")) return nullptr;
    return (void *)e;
}
extern "C" void sp_hip_event_destroy(void *ev) {
    if (ev) (void)hipEventDestroy((hipEvent_t)ev);
}
extern "C" int sp_hip_event_record(void *ev, void *stream) {
    return hip_ok(hipEventRecord((hipEvent_t)ev, (hipStream_t)stream), "event record") ? 0 : -1;
}
extern "C" float sp_hip_event_elapsed_ms(void *a, void *b) {
    float ms = -1.0f;
    if (!hip_ok(hipEventSynchronize((hipEvent_t)b), "event sync")) return -1.0f;
    if (!hip_ok(hipEventElapsedTime(&ms, (hipEvent_t)a, (hipEvent_t)b), "elapsed")) return -1.0f;
    return ms;
}
extern "C" int sp_hip_memset(void *d_ptr, int value, size_t bytes, void *stream) {
    if (!d_ptr) return -1;
    return hip_ok(hipMemsetAsync(d_ptr, value, bytes, (hipStream_t)stream), "memset") ? 0 : -1;
}
extern "C" int sp_hip_stream_sync(void *stream) {
    return hip_ok(hipStreamSynchronize((hipStream_t)stream), "stream sync") ? 0 : -1;
}

// ===========================================================================
// host-buffer staging over a device cache
// ===========================================================================
// Host API calls stage through one device buffer per cache (not reentrant per
// cache, like the reference's per-context scratch) and return after the copy
// back completes.
struct HostStage {
    float *d_vec = nullptr;          // [cap][hd] fp32
    unsigned char *d_rec = nullptr;  // [cap][max(kB, vB)]
    int cap = 0, hd = 0, rec = 0;
    hipStream_t stream = nullptr;
    int order_n = 0;
    int *d_order = nullptr;
};

static HostStage *stage_create(int hd, int rec_bytes, int cap, const int *h_order) {
    HostStage *st = new HostStage();
    st->cap = cap;
    st->hd = hd;
    st->rec = rec_bytes;
    bool ok = hip_ok(hipStreamCreate(&st->stream), "stream create") &&
              hip_ok(hipMalloc((void **)&st->d_vec, sizeof(float) * (size_t)cap * hd), "stage vec") &&
              hip_ok(hipMalloc((void **)&st->d_rec, (size_t)cap * rec_bytes), "stage rec");
    if (ok && h_order) {
        st->order_n = hd;
        ok = hip_ok(hipMalloc((void **)&st->d_order, sizeof(int) * hd), "stage order") &&
             hip_ok(hipMemcpy(st->d_order, h_order, sizeof(int) * hd, hipMemcpyHostToDevice), "order H2D");
    }
    if (!ok) {
        if (st->d_vec) (void)hipFree(st->d_vec);
        if (st->d_rec) (void)hipFree(st->d_rec);
        if (st->d_order) (void)hipFree(st->d_order);
        if (st->stream) (void)hipStreamDestroy(st->stream);
        delete st;
        return nullptr;
    }
    return st;
}

static void stage_destroy(HostStage *st) {
    if (!st) return;
    (void)hipStreamSynchronize(st->stream);
    (void)hipFree(st->d_vec);
    (void)hipFree(st->d_rec);
    if (st->d_order) (void)hipFree(st->d_order);
    (void)hipStreamDestroy(st->stream);
    delete st;
}

// ===========================================================================
// sp_shadow_cache_t over the GPU
// ===========================================================================
struct ShadowDev {
    HostStage *st;
    SpPlan kplan, vplan;
    int slot_capacity = 0;  // positions each caller-owned slot buffer holds (0: not told)
};

extern "C" int sp_shadow_cache_set_slot_capacity(sp_shadow_cache_t *sc, int n_positions) {
    if (!sc || !sc->dev || n_positions <= 0) { set_err("set_slot_capacity: bad args"); return -1; }
    ((ShadowDev *)sc->dev)->slot_capacity = n_positions;
    return 0;
}

extern "C" int sp_shadow_cache_init(sp_shadow_cache_t *sc, const sp_config_t *cfg) {
    if (!sc) return -1;
    memset(sc, 0, sizeof(*sc));
    if (!check_cfg(cfg)) { set_err("shadow_init: bad config"); return -1; }
    if (!sp_hip_available()) { set_err("shadow_init: no gfx950 device"); return -1; }
    sc->config = *cfg;
    const int hd = cfg->head_dim;
    sp_band_config_init_ext(&sc->k_bands, hd, cfg->k_n_bands, cfg->k_band_bits, cfg->k_ternary_mask);
    sp_band_config_init_ext(&sc->v_bands, hd, cfg->v_n_bands, cfg->v_band_bits, cfg->v_ternary_mask);
    if (cfg->use_mobius_mask && sp_mobius_mask_init(&sc->mobius_mask, hd)) return -1;
    ShadowDev *dv = new ShadowDev();
    if (sp_build_plan(&sc->k_bands, hd, cfg->vht2_norm, -1, &dv->kplan) ||
        sp_build_plan(&sc->v_bands, hd, cfg->vht2_norm, -1, &dv->vplan)) {
        delete dv;
        sp_mobius_mask_free(&sc->mobius_mask);
        set_err("shadow_init: head_dim %d unsupported", hd);
        return -1;
    }
    dv->kplan.order_default = 1;
    const int rec = sc->k_bands.total_bytes > sc->v_bands.total_bytes ? sc->k_bands.total_bytes : sc->v_bands.total_bytes;
    dv->st = stage_create(hd, rec, 4096, cfg->use_mobius_mask ? sc->mobius_mask.order : nullptr);
    if (!dv->st) {
        delete dv;
        sp_mobius_mask_free(&sc->mobius_mask);
        return -1;
    }
    sc->dev = dv;
    return 0;
}

extern "C" void sp_shadow_cache_free(sp_shadow_cache_t *sc) {
    if (!sc) return;
    ShadowDev *dv = (ShadowDev *)sc->dev;
    if (dv) {
        stage_destroy(dv->st);
        delete dv;
    }
    sp_mobius_mask_free(&sc->mobius_mask);
    free(sc->calib_sum);
    free(sc->calib_sum2);
    free(sc->var_order);
    sc->calib_sum = sc->calib_sum2 = nullptr;
    sc->var_order = nullptr;
    sc->calibrating = sc->use_var_reorder = 0;
    sc->dev = nullptr;
}

extern "C" int sp_shadow_calibrate_begin(sp_shadow_cache_t *sc) {
    if (!sc || !sc->dev) return -1;
    const size_t hd = (size_t)sc->config.head_dim;
    if (!sc->calib_sum) sc->calib_sum = (double *)malloc(hd * sizeof(double));
    if (!sc->calib_sum2) sc->calib_sum2 = (double *)malloc(hd * sizeof(double));
    if (!sc->calib_sum || !sc->calib_sum2) { set_err("calibrate_begin: out of memory"); return -1; }
    memset(sc->calib_sum, 0, hd * sizeof(double));
    memset(sc->calib_sum2, 0, hd * sizeof(double));
    sc->calib_n = 0;
    sc->calibrating = 1;
    return 0;
}

extern "C" void sp_shadow_calibrate_feed(sp_shadow_cache_t *sc, const float *vec) {
    if (!sc || !sc->dev || !sc->calibrating || !vec || !sc->calib_sum || !sc->calib_sum2) return;
    ShadowDev *dv = (ShadowDev *)sc->dev;
    HostStage *st = dv->st;
    const int hd = sc->config.head_dim;
    if (!hip_ok(hipMemcpyAsync(st->d_vec, vec, sizeof(float) * hd, hipMemcpyHostToDevice, st->stream), "calib H2D"))
        return;
    if (calib_accumulate(dv->kplan, hd, hd, st->d_vec, SP_DT_F32, hd, 1, sc->calib_sum, sc->calib_sum2, st->stream))
        sc->calib_n++;
}

extern "C" int sp_shadow_calibrate_end(sp_shadow_cache_t *sc) {
    if (!sc || !sc->dev || !sc->calib_sum || !sc->calib_sum2 || sc->calib_n <= 0) return -1;
    const int hd = sc->config.head_dim;
    if (!sc->var_order) sc->var_order = (int *)malloc(sizeof(int) * (size_t)hd);
    if (!sc->var_order) { set_err("calibrate_end: out of memory"); return -1; }
    rank_by_variance(sc->calib_sum, sc->calib_sum2, sc->calib_n, hd, sc->var_order);
    // var_order becomes the K coefficient order of later writes and reads
    ShadowDev *dv = (ShadowDev *)sc->dev;
    HostStage *st = dv->st;
    if (!st->d_order) {
        if (!hip_ok(hipMalloc((void **)&st->d_order, sizeof(int) * hd), "hipMalloc order")) return -1;
        st->order_n = hd;
    }
    if (!hip_ok(hipStreamSynchronize(st->stream), "order sync") ||
        !hip_ok(hipMemcpy(st->d_order, sc->var_order, sizeof(int) * hd, hipMemcpyHostToDevice), "order H2D"))
        return -1;
    dv->kplan.order_default = is_default_order(sc->var_order, hd) ? 1 : 0;
    sc->use_var_reorder = 1;
    sc->calibrating = 0;
    return 0;
}

static uint8_t *shadow_rec(const sp_shadow_cache_t *sc, int is_v, int layer, int head, int pos) {
    if (!sc || !sc->dev || layer < 0 || layer >= sc->config.n_layers || head < 0 ||
        head >= sc->config.n_heads_kv || pos < 0) return nullptr;
    uint8_t **slots = is_v ? sc->v_cache : sc->k_cache;
    if (!slots) return nullptr;
    uint8_t *s = slots[layer * sc->config.n_heads_kv + head];
    if (!s) return nullptr;
    return s + (size_t)pos * (is_v ? sc->v_bands.total_bytes : sc->k_bands.total_bytes);
}

static void shadow_write(sp_shadow_cache_t *sc, int is_v, int layer, int head, int start, int n,
                         const float *vecs) {
    uint8_t *dst = shadow_rec(sc, is_v, layer, head, start);
    if (!dst || !vecs || n <= 0) return;
    ShadowDev *dv = (ShadowDev *)sc->dev;
    HostStage *st = dv->st;
    const int hd = sc->config.head_dim, B = is_v ? sc->v_bands.total_bytes : sc->k_bands.total_bytes;
    const int *ord = is_v ? nullptr : st->d_order;
    for (int done = 0; done < n; done += st->cap) {
        const int m = (n - done) < st->cap ? (n - done) : st->cap;
        if (!hip_ok(hipMemcpyAsync(st->d_vec, vecs + (size_t)done * hd, sizeof(float) * (size_t)m * hd,
                                   hipMemcpyHostToDevice, st->stream), "shadow H2D") ||
            !hip_ok(sp_launch_ship_encode(is_v ? dv->vplan : dv->kplan, ord, st->d_vec, SP_DT_F32, 0, hd,
                                          st->d_rec, 0, 1, m, st->stream), "shadow encode") ||
            !hip_ok(hipMemcpyAsync(dst + (size_t)done * B, st->d_rec, (size_t)m * B, hipMemcpyDeviceToHost,
                                   st->stream), "shadow D2H") ||
            !hip_ok(hipStreamSynchronize(st->stream), "shadow sync"))
            return;
    }
}

static void shadow_read(const sp_shadow_cache_t *sc, int is_v, int layer, int head, int start, int n,
                        float *out, int max_bands) {
    const uint8_t *src = shadow_rec(sc, is_v, layer, head, start);
    if (!src || !out || n <= 0) return;
    ShadowDev *dv = (ShadowDev *)sc->dev;
    HostStage *st = dv->st;
    const int hd = sc->config.head_dim, B = is_v ? sc->v_bands.total_bytes : sc->k_bands.total_bytes;
    SpPlan P = is_v ? dv->vplan : dv->kplan;
    if (max_bands >= 0 && max_bands < P.n_bands) P.max_bands = max_bands;
    const int *ord = is_v ? nullptr : st->d_order;
    for (int done = 0; done < n; done += st->cap) {
        const int m = (n - done) < st->cap ? (n - done) : st->cap;
        if (!hip_ok(hipMemcpyAsync(st->d_rec, src + (size_t)done * B, (size_t)m * B, hipMemcpyHostToDevice,
                                   st->stream), "shadow H2D") ||
            !hip_ok(sp_launch_ship_decode(P, ord, st->d_rec, 0, st->d_vec, SP_DT_F32, 0, hd, 1, m, st->stream),
                    "shadow decode") ||
            !hip_ok(hipMemcpyAsync(out + (size_t)done * hd, st->d_vec, sizeof(float) * (size_t)m * hd,
                                   hipMemcpyDeviceToHost, st->stream), "shadow D2H") ||
            !hip_ok(hipStreamSynchronize(st->stream), "shadow sync"))
            return;
    }
}

extern "C" void sp_shadow_write_k(sp_shadow_cache_t *sc, int l, int h, int p, const float *v) { shadow_write(sc, 0, l, h, p, 1, v); }
extern "C" void sp_shadow_write_v(sp_shadow_cache_t *sc, int l, int h, int p, const float *v) { shadow_write(sc, 1, l, h, p, 1, v); }
extern "C" void sp_shadow_write_k_batch(sp_shadow_cache_t *sc, int l, int h, int s, int n, const float *v) { shadow_write(sc, 0, l, h, s, n, v); }
extern "C" void sp_shadow_write_v_batch(sp_shadow_cache_t *sc, int l, int h, int s, int n, const float *v) { shadow_write(sc, 1, l, h, s, n, v); }
extern "C" void sp_shadow_read_k(const sp_shadow_cache_t *sc, int l, int h, int p, float *o) { shadow_read(sc, 0, l, h, p, 1, o, -1); }
extern "C" void sp_shadow_read_v(const sp_shadow_cache_t *sc, int l, int h, int p, float *o) { shadow_read(sc, 1, l, h, p, 1, o, -1); }
extern "C" void sp_shadow_read_k_partial(const sp_shadow_cache_t *sc, int l, int h, int p, float *o, int mb) { shadow_read(sc, 0, l, h, p, 1, o, mb); }
extern "C" void sp_shadow_read_v_partial(const sp_shadow_cache_t *sc, int l, int h, int p, float *o, int mb) { shadow_read(sc, 1, l, h, p, 1, o, mb); }
extern "C" void sp_shadow_read_k_batch(const sp_shadow_cache_t *sc, int l, int h, int s, int n, float *o) { shadow_read(sc, 0, l, h, s, n, o, -1); }
extern "C" void sp_shadow_read_v_batch(const sp_shadow_cache_t *sc, int l, int h, int s, int n, float *o) { shadow_read(sc, 1, l, h, s, n, o, -1); }

// ===========================================================================
// host-buffer I/O on a device cache (bridge HIP backend)
// ===========================================================================
extern "C" int sp_hip_write_host(sp_hip_cache_t *cc, int is_v, int layer, int head, int start_pos,
                                 int n_pos, const float *h_vecs) {
    if (!slot_ok(cc, layer, head, start_pos, n_pos) || !h_vecs) { set_err("write_host: bad args"); return -1; }
    if (n_pos == 0) return 0;
    ShipPriv *pv = (ShipPriv *)cc->priv;
    const size_t n = (size_t)n_pos * cc->config.head_dim;
    std::lock_guard<std::mutex> lk(pv->stage_mu);
    if (!stage_reserve(pv, n)) return -1;
    memcpy(pv->stage_h, h_vecs, n * sizeof(float));
    const bool ok =
        hip_ok(hipMemcpyAsync(pv->stage_d, pv->stage_h, n * sizeof(float), hipMemcpyHostToDevice, (hipStream_t)cc->stream),
               "H2D") &&
        ship_write(cc, is_v, layer, head, start_pos, n_pos, pv->stage_d, SP_DT_F32) == 0 &&
        hip_ok(hipStreamSynchronize((hipStream_t)cc->stream), "sync");
    return ok ? 0 : -1;
}

extern "C" int sp_hip_read_host(const sp_hip_cache_t *cc, int is_v, int layer, int head, int start_pos,
                                int n_pos, float *h_out, int max_bands) {
    if (!slot_ok(cc, layer, head, start_pos, n_pos) || !h_out) { set_err("read_host: bad args"); return -1; }
    if (n_pos == 0) return 0;
    ShipPriv *pv = (ShipPriv *)cc->priv;
    const size_t n = (size_t)n_pos * cc->config.head_dim;
    std::lock_guard<std::mutex> lk(pv->stage_mu);
    if (!stage_reserve(pv, n)) return -1;
    const bool ok =
        ship_read(cc, is_v, layer, head, start_pos, n_pos, pv->stage_d, SP_DT_F32, max_bands) == 0 &&
        hip_ok(hipMemcpyAsync(pv->stage_h, pv->stage_d, n * sizeof(float), hipMemcpyDeviceToHost, (hipStream_t)cc->stream),
               "D2H") &&
        hip_ok(hipStreamSynchronize((hipStream_t)cc->stream), "sync");
    if (ok) memcpy(h_out, pv->stage_h, n * sizeof(float));
    return ok ? 0 : -1;
}

// ===========================================================================
// System 1/2 dual cache (DualKvCache, kv_cache.cpp:1593-1877)
// ===========================================================================
// A per-position route table chooses the owner of each position: System 1 (the
// ship cache) or System 2 (a sqfree or hier cache). Writes go to the owner only;
// the merged read decodes System 1 over the whole range and then System 2 over
// the sorted list of its positions only (the general kernels' listed-position
// form), writing those rows over System 1's output on the same stream.
struct DualPriv {
    std::vector<unsigned char> route;  // 1: System 2
    int n2 = 0;                        // positions routed to System 2
    bool dirty = true;                 // device list out of date
    int *d_list = nullptr;             // System 2 positions, ascending
    // pinned staging for the list upload, double-buffered: a buffer is refilled
    // only after the copy issued from it last time has run (its event)
    int *h_list[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool ev_used[2] = {false, false};
    int cur = 0;
    int n_list = 0;
};

static bool dual_dims(const sp_hip_dual_cache_t *dc, int *L, int *H, int *hd, int *ms) {
    if (!dc || !dc->priv || !dc->sys1 || !dc->sys2) return false;
    *L = dc->sys1->config.n_layers, *H = dc->sys1->config.n_heads_kv, *hd = dc->sys1->config.head_dim;
    *ms = dc->max_seq_len;
    return true;
}

extern "C" int sp_hip_dual_init(sp_hip_dual_cache_t *dc, sp_hip_cache_t *sys1, int sys2_kind, void *sys2,
                                float entropy_threshold) {
    if (!dc || !sys1 || !sys1->priv || !sys2 || (sys2_kind != SP_DUAL_SQFREE && sys2_kind != SP_DUAL_HIER)) {
        set_err("dual_init: bad args"); return -1;
    }
    memset(dc, 0, sizeof(*dc));
    const sp_config_t *c2;
    int ms2;
    void *st2;
    if (sys2_kind == SP_DUAL_SQFREE) {
        const sp_hip_sqfree_cache_t *q = (const sp_hip_sqfree_cache_t *)sys2;
        c2 = &q->config, ms2 = q->max_seq_len, st2 = q->stream;
    } else {
        const sp_hip_hier_cache_t *q = (const sp_hip_hier_cache_t *)sys2;
        c2 = &q->config, ms2 = q->max_seq_len, st2 = q->stream;
        if (q->n_slots < q->config.n_layers * q->config.n_heads_kv) { set_err("dual_init: hier slots"); return -1; }
    }
    const sp_config_t &c1 = sys1->config;
    if (c1.head_dim != c2->head_dim || c1.n_layers != c2->n_layers || c1.n_heads_kv != c2->n_heads_kv ||
        sys1->max_seq_len != ms2) {
        set_err("dual_init: System 1 and 2 shapes differ"); return -1;
    }
    if (sys1->stream != st2) { set_err("dual_init: System 1 and 2 must share a stream"); return -1; }
    DualPriv *pv = new DualPriv();
    pv->route.assign((size_t)ms2, 0);
    bool ok = hip_ok(hipMalloc((void **)&pv->d_list, (size_t)ms2 * sizeof(int)), "dual list");
    for (int b = 0; b < 2 && ok; b++)
        ok = hip_ok(hipHostMalloc((void **)&pv->h_list[b], (size_t)ms2 * sizeof(int), hipHostMallocDefault),
                    "dual list staging") &&
             hip_ok(hipEventCreateWithFlags(&pv->ev[b], hipEventDisableTiming), "dual list event");
    if (!ok) {
        if (pv->d_list) (void)hipFree(pv->d_list);
        for (int b = 0; b < 2; b++) {
            if (pv->h_list[b]) (void)hipHostFree(pv->h_list[b]);
            if (pv->ev[b]) (void)hipEventDestroy(pv->ev[b]);
        }
        delete pv;
        return -1;
    }
    dc->sys1 = sys1;
    dc->sys2 = sys2;
    dc->sys2_kind = sys2_kind;
    dc->entropy_threshold = entropy_threshold;
    dc->max_seq_len = ms2;
    dc->priv = pv;
    return 0;
}

extern "C" void sp_hip_dual_free(sp_hip_dual_cache_t *dc) {
    if (!dc || !dc->priv) return;
    DualPriv *pv = (DualPriv *)dc->priv;
    (void)hipStreamSynchronize((hipStream_t)dc->sys1->stream);  // a list upload may be in flight
    (void)hipFree(pv->d_list);
    for (int b = 0; b < 2; b++) {
        (void)hipHostFree(pv->h_list[b]);
        (void)hipEventDestroy(pv->ev[b]);
    }
    delete pv;
    dc->priv = nullptr;
}

extern "C" int sp_hip_dual_route_position(sp_hip_dual_cache_t *dc, int pos, float entropy) {
    if (!dc || !dc->priv || pos < 0 || pos >= dc->max_seq_len) return 0;
    DualPriv *pv = (DualPriv *)dc->priv;
    const unsigned char r = entropy >= dc->entropy_threshold ? 1 : 0;
    if (pv->route[(size_t)pos] != r) {
        pv->n2 += r ? 1 : -1;
        pv->route[(size_t)pos] = r;
        pv->dirty = true;
    }
    return r;
}

extern "C" int sp_hip_dual_owner_of(const sp_hip_dual_cache_t *dc, int pos) {
    if (!dc || !dc->priv || pos < 0 || pos >= dc->max_seq_len) return 1;
    return ((const DualPriv *)dc->priv)->route[(size_t)pos] ? 2 : 1;
}

extern "C" int sp_hip_dual_sys1_count(const sp_hip_dual_cache_t *dc) {
    return (dc && dc->priv) ? dc->max_seq_len - ((const DualPriv *)dc->priv)->n2 : 0;
}

extern "C" int sp_hip_dual_sys2_count(const sp_hip_dual_cache_t *dc) {
    return (dc && dc->priv) ? ((const DualPriv *)dc->priv)->n2 : 0;
}

extern "C" int sp_hip_dual_write_layer(sp_hip_dual_cache_t *dc, int layer, int start_pos, int n_tok, const void *d_k,
                                       const void *d_v, long long row_stride, int dtype) {
    int L, H, hd, ms;
    if (!dual_dims(dc, &L, &H, &hd, &ms) || layer < 0 || layer >= L || start_pos < 0 || n_tok < 0 ||
        (long long)start_pos + n_tok > ms || row_stride < (long long)H * hd || (dtype != SP_DT_F16 && dtype != SP_DT_F32)) {
        set_err("dual write_layer: bad args"); return -1;
    }
    const DualPriv *pv = (const DualPriv *)dc->priv;
    const long long esz = dtype == SP_DT_F16 ? 2 : 4;
    // one layer-wide write per run of positions with the same owner
    for (int t = 0; t < n_tok;) {
        const unsigned char r = pv->route[(size_t)(start_pos + t)];
        int e = t + 1;
        while (e < n_tok && pv->route[(size_t)(start_pos + e)] == r) e++;
        const long long off = (long long)t * row_stride * esz;
        const void *k = d_k ? (const unsigned char *)d_k + off : nullptr;
        const void *v = d_v ? (const unsigned char *)d_v + off : nullptr;
        int rc;
        if (!r)
            rc = sp_hip_write_layer(dc->sys1, layer, start_pos + t, e - t, k, v, row_stride, dtype);
        else if (dc->sys2_kind == SP_DUAL_SQFREE)
            rc = sp_hip_sqfree_write_layer((sp_hip_sqfree_cache_t *)dc->sys2, layer, start_pos + t, e - t, k, v,
                                           row_stride, dtype);
        else
            rc = sp_hip_hier_write_layer((sp_hip_hier_cache_t *)dc->sys2, layer, start_pos + t, e - t, k, v,
                                         row_stride, dtype);
        if (rc) return -1;
        t = e;
    }
    return 0;
}

extern "C" int sp_hip_dual_read_merged(sp_hip_dual_cache_t *dc, int layer, int kv_len, void *d_k, void *d_v,
                                       long long row_stride, int dtype) {
    int L, H, hd, ms;
    if (!dual_dims(dc, &L, &H, &hd, &ms) || layer < 0 || layer >= L || kv_len <= 0 || kv_len > ms ||
        row_stride < (long long)H * hd || (dtype != SP_DT_F16 && dtype != SP_DT_F32)) {
        set_err("dual read_merged: bad args"); return -1;
    }
    DualPriv *pv = (DualPriv *)dc->priv;
    hipStream_t s = (hipStream_t)dc->sys1->stream;
    if (sp_hip_read_layer(dc->sys1, layer, 0, kv_len, d_k, d_v, row_stride, dtype, -1)) return -1;
    if (pv->n2 == 0) return 0;
    if (pv->dirty) {
        // refill the other staging buffer once the copy last issued from it has run
        // (stream order keeps the device list from changing under earlier kernels)
        const int b = pv->cur ^ 1;
        if (pv->ev_used[b] && !hip_ok(hipEventSynchronize(pv->ev[b]), "dual list staging wait")) return -1;
        int n = 0;
        for (int p = 0; p < ms; p++)
            if (pv->route[(size_t)p]) pv->h_list[b][n++] = p;
        if (n && !(hip_ok(hipMemcpyAsync(pv->d_list, pv->h_list[b], (size_t)n * sizeof(int), hipMemcpyHostToDevice, s),
                          "dual list upload") &&
                   hip_ok(hipEventRecord(pv->ev[b], s), "dual list event"))) return -1;
        pv->ev_used[b] = n > 0;
        pv->cur = b;
        pv->n_list = n;
        pv->dirty = false;
    }
    // System 2 positions below kv_len: a prefix of the ascending list
    const int *hl = pv->h_list[pv->cur];
    const int n2 = (int)(std::lower_bound(hl, hl + pv->n_list, kv_len) - hl);
    if (n2 == 0) return 0;
    for (int is_v = 0; is_v < 2; is_v++) {
        void *dst = is_v ? d_v : d_k;
        if (!dst) continue;
        hipError_t e;
        if (dc->sys2_kind == SP_DUAL_SQFREE) {
            const sp_hip_sqfree_cache_t *q = (const sp_hip_sqfree_cache_t *)dc->sys2;
            const SqPriv *qp = (const SqPriv *)q->priv;
            const SpSqGeo G = sq_geo(q, is_v);
            const unsigned char *src = (is_v ? q->d_v_cache : q->d_k_cache) + (long long)layer * H * ms * G.bytes;
            e = sp_launch_sqfree_decode(is_v ? qp->vplan : qp->kplan, G, src, (long long)ms * G.bytes, dst, dtype, hd,
                                        row_stride, H, n2, s, pv->d_list);
        } else {
            const sp_hip_hier_cache_t *q = (const sp_hip_hier_cache_t *)dc->sys2;
            const SpHierGeo G = hier_geo(q, layer * H);
            const unsigned char *src = (is_v ? q->d_v_cache : q->d_k_cache) + (long long)layer * H * ms * G.bytes;
            e = sp_launch_hier_decode(((const HierPriv *)q->priv)->plan, G, src, (long long)ms * G.bytes, dst, dtype,
                                      hd, row_stride, H, n2, s, pv->d_list);
        }
        if (!hip_ok(e, "dual read_merged System 2")) return -1;
    }
    return 0;
}

// ===========================================================================
// disk serialisation, formats v2 and v3 (KvCache::save_to_disk / load_from_disk,
// kv_cache.h:132-146, kv_cache.cpp:1533-1585; band-major v3, partial load, and
// v2 files staying readable: the disk-tier notes of CHANGELOG.md)
// ===========================================================================
// One file per layer, {prefix}.L{layer}.bin: a 64-byte header, then the K
// segments and the V segments, each [n_heads][n_pos][segment bytes] (sp_disk.hip).
// v3 (the ship caches) cuts each record into its bands (+ the sqfree/hier tail);
// v2 (the sqfree and hier caches, which the reference has not moved to v3) keeps
// each record whole: one segment of B bytes, i.e. the records in cache order.
// Every loader reads both; a partial load of a v2 file reads every band.

extern "C" uint64_t sp_fnv1a64(const void *data, size_t n) {
    const unsigned char *p = (const unsigned char *)data;
    uint64_t h = 0xcbf29ce484222325ULL;  // FNV-1a 64: offset basis, prime 2^40 + 2^8 + 0xb3
    for (size_t i = 0; i < n; i++) {
        h ^= p[i];
        h *= 0x100000001b3ULL;
    }
    return h;
}

namespace {

constexpr uint32_t DISK_V2 = 2, DISK_V3 = 3;
enum { DISK_SHIP = 0, DISK_SQFREE = 1, DISK_HIER = 2, DISK_HIER_W = 3 };

struct DiskHeader {  // 64 bytes, little-endian
    char magic[4];        // "VHT2"
    uint32_t version;     // 3
    uint64_t model_hash;  // FNV-1a of the model path (the caller's)
    int32_t n_pos, layer, n_heads, head_dim, kind, k_bytes, v_bytes, k_segs, v_segs;
    uint32_t order_check; // low 32 bits of FNV-1a of the K coefficient order (ship), else 0
    uint64_t check;       // FNV-1a of bytes [0, 56)
};
static_assert(sizeof(DiskHeader) == 64, "the disk header is 64 bytes");

// A record's segments: each band's [fp16 scale][codes], then the bytes after the
// last band (sqfree/hier: magnitude, residual codes, spinor sheet) as one more.
SpDiskSegs disk_segs(const sp_band_config_t *bc, int B, long long n_rec) {
    SpDiskSegs S{};
    int byte = 0, n = 0;
    for (int b = 0; b < bc->n_bands; b++) {
        int off, sz;
        sp_band_span(bc, b, &off, &sz);
        S.off[n] = (short)byte;
        S.len[n] = (short)(2 + (sz * bc->band_bits[b] + 7) / 8);
        byte += S.len[n++];
    }
    if (byte < B) {
        S.off[n] = (short)byte;
        S.len[n++] = (short)(B - byte);
    }
    S.n = n;
    long long base = 0;
    for (int s = 0; s < n; s++) {
        S.base[s] = base;
        base += n_rec * S.len[s];
    }
    return S;
}

// A file's segments: v3 per band (disk_segs), v2 one whole-record segment.
SpDiskSegs file_segs(uint32_t version, const sp_band_config_t *bc, int B, long long n_rec) {
    if (version == DISK_V3) return disk_segs(bc, B, n_rec);
    SpDiskSegs S{};
    S.n = 1;
    S.off[0] = 0;
    S.len[0] = (short)B;
    S.base[0] = 0;
    return S;
}

long long segs_bytes(const SpDiskSegs &S, int n_seg, long long n_rec) {
    long long b = 0;
    for (int s = 0; s < n_seg && s < S.n; s++) b += n_rec * S.len[s];
    return b;
}

struct DiskCache {  // what save/load need of any of the three cache kinds
    int kind, n_layers, H, hd, max_seq, kB, vB;
    uint32_t version;  // the format this kind writes
    unsigned char *kc, *vc;
    const sp_band_config_t *kbc, *vbc;
    uint32_t order_check;
    hipStream_t s;
};

std::string layer_path(const char *prefix, int l) { return std::string(prefix) + ".L" + std::to_string(l) + ".bin"; }

void header_seal(DiskHeader &h) { h.check = sp_fnv1a64(&h, 56); }

bool hash_ok(uint64_t got, uint64_t want, const char *what) {
    if (got == want) return true;
    const char *e = getenv("SP_DISK_HASH_STRICT");
    if (e && e[0] == '0') {
        fprintf(stderr, "[sp-hip] %s: model hash mismatch (file %016llx, expected %016llx); loading anyway "
                        "(SP_DISK_HASH_STRICT=0)\n", what, (unsigned long long)got, (unsigned long long)want);
        return true;
    }
    set_err("%s: model hash mismatch (file %016llx, expected %016llx)", what, (unsigned long long)got,
            (unsigned long long)want);
    return false;
}

int disk_save(const DiskCache &D, const char *prefix, int n_pos, uint64_t model_hash) {
    if (!prefix || n_pos <= 0 || n_pos > D.max_seq) { set_err("save: bad n_pos %d", n_pos); return -1; }
    const long long n_rec = (long long)D.H * n_pos;
    const SpDiskSegs Sk = file_segs(D.version, D.kbc, D.kB, n_rec), Sv = file_segs(D.version, D.vbc, D.vB, n_rec);
    const size_t kbytes = (size_t)n_rec * D.kB, body = kbytes + (size_t)n_rec * D.vB;
    unsigned char *d_stage = nullptr, *h_stage = nullptr;
    if (!(hip_ok(hipMalloc((void **)&d_stage, body), "save staging") &&
          hip_ok(hipHostMalloc((void **)&h_stage, body, hipHostMallocDefault), "save host staging"))) {
        if (d_stage) (void)hipFree(d_stage);
        return -1;
    }
    int rc = 0;
    for (int l = 0; l < D.n_layers && rc == 0; l++) {
        const long long ks = (long long)D.max_seq * D.kB, vs = (long long)D.max_seq * D.vB;
        if (!(hip_ok(sp_launch_disk_pack(D.kc + (long long)l * D.H * ks, ks, D.kB, D.H, n_pos, Sk, d_stage, D.s),
                     "save pack K") &&
              hip_ok(sp_launch_disk_pack(D.vc + (long long)l * D.H * vs, vs, D.vB, D.H, n_pos, Sv, d_stage + kbytes, D.s),
                     "save pack V") &&
              hip_ok(hipMemcpyAsync(h_stage, d_stage, body, hipMemcpyDeviceToHost, D.s), "save D2H") &&
              hip_ok(hipStreamSynchronize(D.s), "save sync"))) { rc = -1; break; }
        DiskHeader h{};
        memcpy(h.magic, "VHT2", 4);
        h.version = D.version;
        h.model_hash = model_hash;
        h.n_pos = n_pos, h.layer = l, h.n_heads = D.H, h.head_dim = D.hd, h.kind = D.kind;
        h.k_bytes = D.kB, h.v_bytes = D.vB, h.k_segs = Sk.n, h.v_segs = Sv.n, h.order_check = D.order_check;
        header_seal(h);
        const std::string path = layer_path(prefix, l);
        FILE *f = fopen(path.c_str(), "wb");
        if (!f) { set_err("save: cannot open %s", path.c_str()); rc = -1; break; }
        const bool ok = fwrite(&h, sizeof(h), 1, f) == 1 && fwrite(h_stage, 1, body, f) == body;
        if (fclose(f) != 0 || !ok) { set_err("save: write failed for %s", path.c_str()); rc = -1; }
    }
    (void)hipFree(d_stage);
    (void)hipHostFree(h_stage);
    return rc;
}

// Opens layer l's file and checks its header against the cache D (shape, n_pos
// within D.max_seq and equal to n_pos_all when that is >= 0, coefficient order,
// model hash, segment layout) and the file's length against the body the header
// announces. Returns the file positioned after the header, or nullptr with the
// error set.
FILE *open_layer_file(const DiskCache &D, const char *prefix, int l, uint64_t expected_hash, int n_pos_all,
                      DiskHeader &h) {
    const std::string path = layer_path(prefix, l);
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) { set_err("load: cannot open %s", path.c_str()); return nullptr; }
    h = DiskHeader{};
    bool ok = fread(&h, sizeof(h), 1, f) == 1;
    if (!ok || memcmp(h.magic, "VHT2", 4) != 0 || h.check != sp_fnv1a64(&h, 56)) {
        set_err("load: %s is not a VHT2 cache file", path.c_str());
        ok = false;
    } else if (h.version != DISK_V2 && h.version != DISK_V3) {
        set_err("load: %s has format version %u (this build reads 2 and 3)", path.c_str(), h.version);
        ok = false;
    } else if (h.kind != D.kind || h.layer != l || h.n_heads != D.H || h.head_dim != D.hd || h.k_bytes != D.kB ||
               h.v_bytes != D.vB || h.n_pos <= 0 || (n_pos_all >= 0 && h.n_pos != n_pos_all)) {
        set_err("load: %s does not match this cache's shape", path.c_str());
        ok = false;
    } else if (h.n_pos > D.max_seq) {
        set_err("load: %s holds %d positions, the cache has room for %d", path.c_str(), h.n_pos, D.max_seq);
        ok = false;
    } else if (h.order_check != D.order_check) {
        set_err("load: %s was written with another coefficient order", path.c_str());
        ok = false;
    } else {
        ok = hash_ok(h.model_hash, expected_hash, "load");
    }
    if (ok) {
        const long long n_rec = (long long)D.H * h.n_pos;
        const SpDiskSegs Sk = file_segs(h.version, D.kbc, D.kB, n_rec), Sv = file_segs(h.version, D.vbc, D.vB, n_rec);
        if (Sk.n != h.k_segs || Sv.n != h.v_segs) {
            set_err("load: %s band layout differs", path.c_str());
            ok = false;
        } else {
            const long long want = (long long)sizeof(h) + n_rec * (D.kB + D.vB);
            ok = fseek(f, 0, SEEK_END) == 0 && ftell(f) >= want && fseek(f, (long)sizeof(h), SEEK_SET) == 0;
            if (!ok) set_err("load: %s is truncated", path.c_str());
        }
    }
    if (!ok) {
        fclose(f);
        return nullptr;
    }
    return f;
}

// Checks every layer's file before anything is loaded, so a bad file at layer l
// leaves the records of layers < l untouched. Returns the common n_pos or -1.
int check_layer_files(const DiskCache &D, const char *prefix, uint64_t expected_hash) {
    if (!prefix) { set_err("load: no prefix"); return -1; }
    int n_pos_all = -1;
    for (int l = 0; l < D.n_layers; l++) {
        DiskHeader h;
        FILE *f = open_layer_file(D, prefix, l, expected_hash, n_pos_all, h);
        if (!f) return -1;
        fclose(f);
        n_pos_all = h.n_pos;
    }
    return n_pos_all;
}

// Loads positions [0, n_pos) of every layer; segments past max_segs (< 0: all)
// are cleared instead of read (v3 files; a v2 file is read whole). Returns n_pos.
int disk_load(const DiskCache &D, const char *prefix, uint64_t expected_hash, int max_segs) {
    int n_pos_all = check_layer_files(D, prefix, expected_hash);
    if (n_pos_all < 0) return -1;
    unsigned char *d_stage = nullptr, *h_stage = nullptr;
    size_t cap = 0;
    int rc = 0;
    for (int l = 0; l < D.n_layers && rc == 0; l++) {
        DiskHeader h;
        FILE *f = open_layer_file(D, prefix, l, expected_hash, n_pos_all, h);
        if (!f) { rc = -1; break; }
        const std::string path = layer_path(prefix, l);
        const long long n_rec = (long long)D.H * h.n_pos;
        const SpDiskSegs Sk = file_segs(h.version, D.kbc, D.kB, n_rec), Sv = file_segs(h.version, D.vbc, D.vB, n_rec);
        const int ms = h.version == DISK_V3 ? max_segs : -1;
        const int nk = ms < 0 ? Sk.n : std::min(ms, Sk.n), nv = ms < 0 ? Sv.n : std::min(ms, Sv.n);
        const size_t kfull = (size_t)n_rec * D.kB, body = kfull + (size_t)n_rec * D.vB;
        const size_t kread = (size_t)segs_bytes(Sk, nk, n_rec), vread = (size_t)segs_bytes(Sv, nv, n_rec);
        if (body > cap) {
            if (d_stage) (void)hipFree(d_stage);
            if (h_stage) (void)hipHostFree(h_stage);
            d_stage = nullptr, h_stage = nullptr, cap = 0;
            if (!(hip_ok(hipMalloc((void **)&d_stage, body), "load staging") &&
                  hip_ok(hipHostMalloc((void **)&h_stage, body, hipHostMallocDefault), "load host staging"))) {
                fclose(f); rc = -1; break;
            }
            cap = body;
        }
        // the K segments to load, skip the rest of K, the V segments to load
        const bool ok = fread(h_stage, 1, kread, f) == kread && fseek(f, (long)(kfull - kread), SEEK_CUR) == 0 &&
                        fread(h_stage + kfull, 1, vread, f) == vread;
        fclose(f);
        if (!ok) { set_err("load: %s is truncated", path.c_str()); rc = -1; break; }
        const long long ks = (long long)D.max_seq * D.kB, vs = (long long)D.max_seq * D.vB;
        if (!(hip_ok(hipMemcpyAsync(d_stage, h_stage, body, hipMemcpyHostToDevice, D.s), "load H2D") &&
              hip_ok(sp_launch_disk_unpack(d_stage, ks, D.kB, D.H, h.n_pos, Sk, nk, D.kc + (long long)l * D.H * ks, D.s),
                     "load unpack K") &&
              hip_ok(sp_launch_disk_unpack(d_stage + kfull, vs, D.vB, D.H, h.n_pos, Sv, nv,
                                           D.vc + (long long)l * D.H * vs, D.s), "load unpack V") &&
              hip_ok(hipStreamSynchronize(D.s), "load sync"))) { rc = -1; break; }
    }
    if (d_stage) (void)hipFree(d_stage);
    if (h_stage) (void)hipHostFree(h_stage);
    return rc == 0 ? n_pos_all : -1;
}

bool ship_disk(const sp_hip_cache_t *cc, DiskCache &D) {
    if (!cc || !cc->priv) { set_err("disk: bad cache"); return false; }
    D.kind = DISK_SHIP, D.version = DISK_V3, D.n_layers = cc->config.n_layers, D.H = cc->config.n_heads_kv,
    D.hd = cc->config.head_dim;
    D.max_seq = cc->max_seq_len, D.kB = cc->k_bands.total_bytes, D.vB = cc->v_bands.total_bytes;
    D.kc = (unsigned char *)cc->d_k_cache, D.vc = (unsigned char *)cc->d_v_cache;
    D.kbc = &cc->k_bands, D.vbc = &cc->v_bands, D.s = (hipStream_t)cc->stream;
    D.order_check = 0;
    if (cc->d_mobius_order) {
        std::vector<int> ord((size_t)D.hd);
        if (!hip_ok(hipMemcpy(ord.data(), cc->d_mobius_order, ord.size() * sizeof(int), hipMemcpyDeviceToHost),
                    "disk order")) return false;
        D.order_check = (uint32_t)sp_fnv1a64(ord.data(), ord.size() * sizeof(int));
    }
    return true;
}

bool sqfree_disk(const sp_hip_sqfree_cache_t *cc, DiskCache &D) {
    if (!cc || !cc->priv) { set_err("disk: bad sqfree cache"); return false; }
    const int H = cc->config.n_heads_kv;
    if (cc->n_slots < cc->config.n_layers * H) { set_err("disk: sqfree slots"); return false; }
    D.kind = DISK_SQFREE, D.version = DISK_V2, D.n_layers = cc->config.n_layers, D.H = H, D.hd = cc->config.head_dim;
    D.max_seq = cc->max_seq_len, D.kB = cc->bytes_per_pos_k, D.vB = cc->bytes_per_pos_v;
    D.kc = cc->d_k_cache, D.vc = cc->d_v_cache, D.kbc = &cc->k_bands, D.vbc = &cc->v_bands;
    D.s = (hipStream_t)cc->stream, D.order_check = 0;
    return true;
}

bool hier_disk(const sp_hip_hier_cache_t *hc, DiskCache &D) {
    if (!hc || !hc->priv) { set_err("disk: bad hier cache"); return false; }
    const int H = hc->config.n_heads_kv;
    if (hc->n_slots < hc->config.n_layers * H) { set_err("disk: hier slots"); return false; }
    D.kind = DISK_HIER, D.version = DISK_V2, D.n_layers = hc->config.n_layers, D.H = H, D.hd = hc->config.head_dim;
    D.max_seq = hc->max_seq_len, D.kB = hc->bytes_per_pos_k, D.vB = hc->bytes_per_pos_v;
    D.kc = hc->d_k_cache, D.vc = hc->d_v_cache, D.kbc = &hc->skel_bands, D.vbc = &hc->skel_bands;
    D.s = (hipStream_t)hc->stream, D.order_check = 0;
    return true;
}

}  // namespace

extern "C" int sp_hip_cache_save(const sp_hip_cache_t *cc, const char *prefix, int n_pos, uint64_t model_hash) {
    DiskCache D;
    return ship_disk(cc, D) ? disk_save(D, prefix, n_pos, model_hash) : -1;
}

extern "C" int sp_hip_cache_load(sp_hip_cache_t *cc, const char *prefix, uint64_t expected_hash) {
    DiskCache D;
    return ship_disk(cc, D) ? disk_load(D, prefix, expected_hash, -1) : -1;
}

extern "C" int sp_hip_cache_load_partial(sp_hip_cache_t *cc, const char *prefix, uint64_t expected_hash,
                                         int max_bands) {
    DiskCache D;
    if (max_bands < 0) { set_err("load_partial: max_bands < 0"); return -1; }
    return ship_disk(cc, D) ? disk_load(D, prefix, expected_hash, max_bands) : -1;
}

extern "C" int sp_hip_sqfree_cache_save(const sp_hip_sqfree_cache_t *cc, const char *prefix, int n_pos,
                                        uint64_t model_hash) {
    DiskCache D;
    return sqfree_disk(cc, D) ? disk_save(D, prefix, n_pos, model_hash) : -1;
}

extern "C" int sp_hip_sqfree_cache_load(sp_hip_sqfree_cache_t *cc, const char *prefix, uint64_t expected_hash) {
    DiskCache D;
    return sqfree_disk(cc, D) ? disk_load(D, prefix, expected_hash, -1) : -1;
}

// The hier cache also writes {prefix}.hier_w.bin: a header (kind 3, n_heads =
// n_slots, head_dim = n_target, k_bytes = n_skeleton) and every slot's fp16 W.
extern "C" int sp_hip_hier_cache_save(const sp_hip_hier_cache_t *hc, const char *prefix, int n_pos,
                                      uint64_t model_hash) {
    DiskCache D;
    if (!hier_disk(hc, D) || disk_save(D, prefix, n_pos, model_hash)) return -1;
    const size_t nw = (size_t)hc->n_slots * hc->n_target * hc->n_skeleton;
    std::vector<uint16_t> W(nw);
    if (!hip_ok(hipMemcpy(W.data(), hc->d_W, nw * sizeof(uint16_t), hipMemcpyDeviceToHost), "save W")) return -1;
    DiskHeader h{};
    memcpy(h.magic, "VHT2", 4);
    h.version = D.version;
    h.model_hash = model_hash;
    h.n_heads = hc->n_slots, h.head_dim = hc->n_target, h.k_bytes = hc->n_skeleton, h.kind = DISK_HIER_W;
    header_seal(h);
    const std::string path = std::string(prefix) + ".hier_w.bin";
    FILE *f = fopen(path.c_str(), "wb");
    if (!f) { set_err("save: cannot open %s", path.c_str()); return -1; }
    const bool ok = fwrite(&h, sizeof(h), 1, f) == 1 && fwrite(W.data(), sizeof(uint16_t), nw, f) == nw;
    if (fclose(f) != 0 || !ok) { set_err("save: write failed for %s", path.c_str()); return -1; }
    return 0;
}

extern "C" int sp_hip_hier_cache_load(sp_hip_hier_cache_t *hc, const char *prefix, uint64_t expected_hash) {
    DiskCache D;
    if (!hier_disk(hc, D) || !prefix) { if (!prefix) set_err("load: no prefix"); return -1; }
    const std::string path = std::string(prefix) + ".hier_w.bin";
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) { set_err("load: cannot open %s", path.c_str()); return -1; }
    DiskHeader h{};
    const size_t nw = (size_t)hc->n_slots * hc->n_target * hc->n_skeleton;
    std::vector<uint16_t> W(nw);
    bool ok = fread(&h, sizeof(h), 1, f) == 1 && memcmp(h.magic, "VHT2", 4) == 0 && h.check == sp_fnv1a64(&h, 56) &&
              (h.version == DISK_V2 || h.version == DISK_V3) && h.kind == DISK_HIER_W && h.n_heads == hc->n_slots &&
              h.head_dim == hc->n_target && h.k_bytes == hc->n_skeleton;
    if (!ok) set_err("load: %s does not match this hier cache", path.c_str());
    ok = ok && hash_ok(h.model_hash, expected_hash, "load");
    if (ok && fread(W.data(), sizeof(uint16_t), nw, f) != nw) { set_err("load: %s is truncated", path.c_str()); ok = false; }
    fclose(f);
    if (!ok) return -1;
    const int n = disk_load(D, prefix, expected_hash, -1);
    if (n < 0) return -1;
    return sp_hip_hier_cache_upload_W(hc, W.data()) == 0 ? n : -1;
}

// Memory report of a ship cache (sp_cuda_print_memory, shannon_prime_cuda.cu:663-677):
// record bytes against an fp16 K+V cache of the same shape.
extern "C" void sp_hip_print_memory(const sp_hip_cache_t *cc) {
    if (!cc) return;
    const double slots = (double)cc->config.n_layers * cc->config.n_heads_kv * cc->max_seq_len;
    const double k = slots * cc->k_bands.total_bytes, v = slots * cc->v_bands.total_bytes;
    const double fp16 = slots * cc->config.head_dim * 2.0 * 2.0, mib = 1024.0 * 1024.0;
    fprintf(stderr, "[sp-hip] cache memory: %.2f MiB of records (K %.2f + V %.2f), fp16 K+V %.2f MiB, %.1fx smaller\n",
            (k + v) / mib, k / mib, v / mib, fp16 / mib, (k + v) > 0 ? fp16 / (k + v) : 0.0);
}

// Shadow cache save / load (sp_shadow_cache_save / _load / _load_partial, called
// at kv_cache.cpp:1549, 1572): the shadow cache's records are host buffers
// (k_cache[slot], v_cache[slot], slot = layer * n_heads + head), so the same v3
// files are written and read here with a host-side band-major repack. Files are
// interchangeable with sp_hip_cache_save / _load for the same config and order.
namespace {

uint32_t shadow_order_check(const sp_shadow_cache_t *sc) {
    const int hd = sc->config.head_dim;
    const int *ord = sc->use_var_reorder && sc->var_order ? sc->var_order
                   : sc->config.use_mobius_mask ? sc->mobius_mask.order : nullptr;
    return ord ? (uint32_t)sp_fnv1a64(ord, (size_t)hd * sizeof(int)) : 0u;
}

int shadow_disk(sp_shadow_cache_t *sc, const char *prefix, int n_pos, uint64_t hash, int max_segs, bool save) {
    if (!sc || !sc->dev || !sc->k_cache || !sc->v_cache || !prefix) { set_err("shadow disk: bad cache"); return -1; }
    const int cap = ((ShadowDev *)sc->dev)->slot_capacity;
    if (cap <= 0) {
        set_err("shadow disk: slot capacity unknown (sp_shadow_cache_set_slot_capacity)");
        return -1;
    }
    const int H = sc->config.n_heads_kv, hd = sc->config.head_dim, Lyr = sc->config.n_layers;
    const int kB = sc->k_bands.total_bytes, vB = sc->v_bands.total_bytes;
    DiskCache D{};
    D.kind = DISK_SHIP, D.version = DISK_V3, D.n_layers = Lyr, D.H = H, D.hd = hd, D.max_seq = cap, D.kB = kB, D.vB = vB;
    D.kbc = &sc->k_bands, D.vbc = &sc->v_bands, D.order_check = shadow_order_check(sc);
    for (int l = 0; l < Lyr; l++)
        for (int hh = 0; hh < H; hh++)
            if (!sc->k_cache[l * H + hh] || !sc->v_cache[l * H + hh]) {
                set_err("shadow disk: slot %d has no buffer", l * H + hh);
                return -1;
            }
    if (save && (n_pos <= 0 || n_pos > cap)) { set_err("shadow save: n_pos %d outside 1..%d", n_pos, cap); return -1; }
    if (!save) {
        n_pos = check_layer_files(D, prefix, hash);  // every file checked before any record changes
        if (n_pos < 0) return -1;
    }
    std::vector<unsigned char> body;
    for (int l = 0; l < Lyr; l++) {
        const std::string path = layer_path(prefix, l);
        DiskHeader h{};
        FILE *f = save ? fopen(path.c_str(), "wb") : open_layer_file(D, prefix, l, hash, n_pos, h);
        if (!f) {
            if (save) set_err("shadow disk: cannot open %s", path.c_str());
            return -1;
        }
        const long long n_rec = (long long)H * n_pos;
        const uint32_t ver = save ? DISK_V3 : h.version;
        const SpDiskSegs Sk = file_segs(ver, &sc->k_bands, kB, n_rec), Sv = file_segs(ver, &sc->v_bands, vB, n_rec);
        const size_t kfull = (size_t)n_rec * kB;
        body.assign(kfull + (size_t)n_rec * vB, 0);
        bool ok = true;
        if (!save) {
            const int ms = ver == DISK_V3 ? max_segs : -1;  // a v2 file is read whole
            const int nk = ms < 0 ? Sk.n : std::min(ms, Sk.n), nv = ms < 0 ? Sv.n : std::min(ms, Sv.n);
            const size_t kread = (size_t)segs_bytes(Sk, nk, n_rec), vread = (size_t)segs_bytes(Sv, nv, n_rec);
            ok = fread(body.data(), 1, kread, f) == kread && fseek(f, (long)(kfull - kread), SEEK_CUR) == 0 &&
                 fread(body.data() + kfull, 1, vread, f) == vread;
            if (!ok) set_err("load: %s is truncated", path.c_str());
            // segments past the loaded ones stay zero in `body` and clear the records
        }
        for (int side = 0; side < 2 && ok; side++) {
            const SpDiskSegs &Sg = side ? Sv : Sk;
            const int B = side ? vB : kB;
            unsigned char *base = body.data() + (side ? kfull : 0);
            for (int hh = 0; hh < H; hh++) {
                uint8_t *rec = (side ? sc->v_cache : sc->k_cache)[l * H + hh];
                for (int p = 0; p < n_pos; p++)
                    for (int sg = 0; sg < Sg.n; sg++) {
                        unsigned char *seg = base + Sg.base[sg] + ((long long)hh * n_pos + p) * Sg.len[sg];
                        unsigned char *r = rec + (size_t)p * B + Sg.off[sg];
                        if (save) memcpy(seg, r, (size_t)Sg.len[sg]);
                        else memcpy(r, seg, (size_t)Sg.len[sg]);
                    }
            }
        }
        if (ok && save) {
            memcpy(h.magic, "VHT2", 4);
            h.version = DISK_V3;
            h.model_hash = hash;
            h.n_pos = n_pos, h.layer = l, h.n_heads = H, h.head_dim = hd, h.kind = DISK_SHIP;
            h.k_bytes = kB, h.v_bytes = vB, h.k_segs = Sk.n, h.v_segs = Sv.n, h.order_check = D.order_check;
            header_seal(h);
            ok = fwrite(&h, sizeof(h), 1, f) == 1 && fwrite(body.data(), 1, body.size(), f) == body.size();
            if (!ok) set_err("save: write failed for %s", path.c_str());
        }
        if (fclose(f) != 0 && save) { set_err("save: write failed for %s", path.c_str()); ok = false; }
        if (!ok) return -1;
    }
    return save ? 0 : n_pos;
}

}  // namespace

extern "C" int sp_shadow_cache_save(const sp_shadow_cache_t *sc, const char *prefix, int n_pos, uint64_t model_hash) {
    if (n_pos <= 0) { set_err("shadow save: bad n_pos"); return -1; }
    return shadow_disk(const_cast<sp_shadow_cache_t *>(sc), prefix, n_pos, model_hash, -1, true);
}

extern "C" int sp_shadow_cache_load(sp_shadow_cache_t *sc, const char *prefix, uint64_t expected_hash) {
    return shadow_disk(sc, prefix, 0, expected_hash, -1, false);
}

extern "C" int sp_shadow_cache_load_partial(sp_shadow_cache_t *sc, const char *prefix, uint64_t expected_hash,
                                            int max_bands) {
    if (max_bands < 0) { set_err("load_partial: max_bands < 0"); return -1; }
    return shadow_disk(sc, prefix, 0, expected_hash, max_bands, false);
}

// ===========================================================================
// host-pointer forms of the core's per-vector calls: sp_vht2_forward_f32 (called
// at llama_sp_fused_kq.cpp:33, kv_cache.cpp:399) and sp_band_quantize /
// sp_band_dequantize(_partial) (the absent core's band codec): one round trip
// through a device staging buffer, computed by the same kernels as the caches
// ===========================================================================
static std::mutex g_core_mu;
static float *g_core_f = nullptr;
static unsigned char *g_core_b = nullptr;
static size_t g_core_nf = 0, g_core_nb = 0;

static bool core_stage(size_t nf, size_t nb) {
    if (nf > g_core_nf) {
        if (g_core_f) (void)hipFree(g_core_f);
        g_core_f = nullptr, g_core_nf = 0;
        if (!hip_ok(hipMalloc((void **)&g_core_f, nf * sizeof(float)), "core staging")) return false;
        g_core_nf = nf;
    }
    if (nb > g_core_nb) {
        if (g_core_b) (void)hipFree(g_core_b);
        g_core_b = nullptr, g_core_nb = 0;
        if (!hip_ok(hipMalloc((void **)&g_core_b, nb + SP_CACHE_SLACK), "core staging")) return false;
        g_core_nb = nb;
    }
    return true;
}

// A configuration these calls cannot run leaves the caller's output untouched
// and says so once on stderr (the message stays in sp_hip_last_error()).
static void core_refuse(const char *what) {
    static std::atomic<int> said{0};
    if (!said.exchange(1)) fprintf(stderr, "[Shannon-Prime HIP] %s: %s; output left unchanged\n", what, g_err);
}

extern "C" void sp_vht2_forward_f32(float *data, int n) {
    if (!data || n <= 0) return;
    sp_band_config_t bc;
    int bits = 8;
    sp_band_config_init(&bc, n, 1, &bits);
    SpPlan P;
    if (sp_build_plan(&bc, n, SP_VHT2_NORM_FINAL, -1, &P)) {
        set_err("sp_vht2_forward_f32: length %d does not factor over 2, 3, 5, 7, 11", n);
        core_refuse("sp_vht2_forward_f32");
        return;
    }
    std::lock_guard<std::mutex> lk(g_core_mu);
    if (!core_stage((size_t)n, 0) ||
        !hip_ok(hipMemcpy(g_core_f, data, (size_t)n * sizeof(float), hipMemcpyHostToDevice), "vht2 H2D") ||
        !hip_ok(sp_launch_transform(P, g_core_f, 1, nullptr), "vht2") ||
        !hip_ok(hipMemcpy(data, g_core_f, (size_t)n * sizeof(float), hipMemcpyDeviceToHost), "vht2 D2H"))
        core_refuse("sp_vht2_forward_f32");
}

// Plan of the band codec with no transform (the core's sp_band_quantize works on
// coefficients already transformed).
static bool band_plan(const sp_band_config_t *bc, SpPlan &P, const char *what) {
    if (sp_build_plan(bc, 1, 0, -1, &P)) {
        set_err("%s: band configuration rejected", what);
        core_refuse(what);
        return false;
    }
    P.chunk_ok = 0;
    P.skip_transform = 1;
    return true;
}

extern "C" void sp_band_quantize(const float *in, uint8_t *out, const sp_band_config_t *bc) {
    if (!in || !out || !bc) return;
    SpPlan P;
    if (!band_plan(bc, P, "sp_band_quantize")) return;
    std::lock_guard<std::mutex> lk(g_core_mu);
    const size_t n = (size_t)bc->head_dim, B = (size_t)bc->total_bytes;
    if (!core_stage(n, B) || !hip_ok(hipMemcpy(g_core_f, in, n * sizeof(float), hipMemcpyHostToDevice), "quantize H2D") ||
        !hip_ok(sp_launch_ship_encode_generic(P, nullptr, g_core_f, SP_DT_F32, 0, bc->head_dim, g_core_b, 0, 1, 1,
                                              nullptr), "band_quantize") ||
        !hip_ok(hipMemcpy(out, g_core_b, B, hipMemcpyDeviceToHost), "quantize D2H"))
        core_refuse("sp_band_quantize");
}

// bands >= max_bands read as 0; max_bands < 0 (or >= n_bands) reads every band
extern "C" void sp_band_dequantize_partial(const uint8_t *in, float *out, const sp_band_config_t *bc, int max_bands) {
    if (!in || !out || !bc) return;
    SpPlan P;
    if (!band_plan(bc, P, "sp_band_dequantize")) return;
    if (max_bands >= 0 && max_bands < P.n_bands) P.max_bands = max_bands;
    std::lock_guard<std::mutex> lk(g_core_mu);
    const size_t n = (size_t)bc->head_dim, B = (size_t)bc->total_bytes;
    if (!core_stage(n, B) || !hip_ok(hipMemcpy(g_core_b, in, B, hipMemcpyHostToDevice), "dequantize H2D") ||
        !hip_ok(sp_launch_ship_decode_generic(P, nullptr, g_core_b, 0, g_core_f, SP_DT_F32, 0, bc->head_dim, 1, 1,
                                              nullptr), "band_dequantize") ||
        !hip_ok(hipMemcpy(out, g_core_f, n * sizeof(float), hipMemcpyDeviceToHost), "dequantize D2H"))
        core_refuse("sp_band_dequantize");
}

extern "C" void sp_band_dequantize(const uint8_t *in, float *out, const sp_band_config_t *bc) {
    sp_band_dequantize_partial(in, out, bc, -1);
}

// Knight mask tables on the host (sp_knight_mask_init / _free, called at
// shannon_prime_sqfree.cu:606-657): the same tables the sqfree caches build.
extern "C" int sp_knight_mask_init(sp_knight_mask_t *m, int pad_dim, int sk_k, const int *ranking) {
    if (!m || pad_dim <= 0 || sk_k <= 0 || sk_k > pad_dim) { set_err("knight_mask_init: bad args"); return -1; }
    memset(m, 0, sizeof(*m));
    std::vector<int> skel, res, off, slot, mu;
    build_knight(pad_dim, sk_k, skel, res, off, slot, mu, ranking);
    const int nr = (int)res.size(), nt = (int)slot.size();
    m->skeleton_idx = (int *)malloc(sizeof(int) * (size_t)sk_k);
    m->residual_idx = (int *)malloc(sizeof(int) * (size_t)(nr > 0 ? nr : 1));
    m->csr_offsets = (int *)malloc(sizeof(int) * (size_t)(nr + 1));
    m->csr_skel_slot = (int *)malloc(sizeof(int) * (size_t)(nt > 0 ? nt : 1));
    m->csr_mu_sign = (int8_t *)malloc((size_t)(nt > 0 ? nt : 1));
    if (!m->skeleton_idx || !m->residual_idx || !m->csr_offsets || !m->csr_skel_slot || !m->csr_mu_sign) {
        sp_knight_mask_free(m);
        set_err("knight_mask_init: out of memory");
        return -1;
    }
    std::copy(skel.begin(), skel.end(), m->skeleton_idx);
    std::copy(res.begin(), res.end(), m->residual_idx);
    std::copy(off.begin(), off.end(), m->csr_offsets);
    std::copy(slot.begin(), slot.end(), m->csr_skel_slot);
    for (int t = 0; t < nt; t++) m->csr_mu_sign[t] = (int8_t)mu[(size_t)t];
    m->pad_dim = pad_dim, m->sk_k = sk_k, m->n_res = nr, m->n_terms = nt;
    return 0;
}

extern "C" void sp_knight_mask_free(sp_knight_mask_t *m) {
    if (!m) return;
    free(m->skeleton_idx);
    free(m->residual_idx);
    free(m->csr_offsets);
    free(m->csr_skel_slot);
    free(m->csr_mu_sign);
    memset(m, 0, sizeof(*m));
}
