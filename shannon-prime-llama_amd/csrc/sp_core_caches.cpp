// sp_core_caches.cpp -- the core's sqfree and hierarchical caches on host
// vectors (sp_sqfree_cache_t, sp_hier_cache_t in shannon_prime.h).
//
// Each host cache owns a device cache (sp_hip_sqfree_cache_t /
// sp_hip_hier_cache_t) on a stream of its own, plus one vector of pinned host
// staging and one of device staging. A write copies the caller's vector into the
// pinned buffer, sends it to the device and runs the device cache's write; a read
// runs the device read and brings the vector back. Every call ends with a stream
// synchronisation, so the staging is free again when it returns; a mutex per
// cache serialises callers that share one cache.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/shannon_prime.h"
#include "../../include/sp_hip.h"
#include "sp_internal.h"

namespace {

// Device vector staging shared by both host caches.
struct Staging {
    hipStream_t stream = nullptr;
    float *h_vec = nullptr;  // pinned, max(head_dim, pad_dim) floats
    float *d_vec = nullptr;
    int n = 0;
    std::mutex mu;

    bool open(int floats) {
        n = floats;
        if (hipStreamCreate(&stream) != hipSuccess) { stream = nullptr; return false; }
        if (hipHostMalloc((void **)&h_vec, sizeof(float) * (size_t)n, hipHostMallocDefault) != hipSuccess) {
            h_vec = nullptr;
            return false;
        }
        if (hipMalloc((void **)&d_vec, sizeof(float) * (size_t)n) != hipSuccess) {
            d_vec = nullptr;
            return false;
        }
        return true;
    }
    void close() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (d_vec) (void)hipFree(d_vec);
        if (h_vec) (void)hipHostFree(h_vec);
        if (stream) (void)hipStreamDestroy(stream);
        d_vec = nullptr;
        h_vec = nullptr;
        stream = nullptr;
    }
    // host vector -> d_vec (the caller then launches on `stream`)
    bool send(const float *v, int count) {
        memcpy(h_vec, v, sizeof(float) * (size_t)count);
        return hipMemcpyAsync(d_vec, h_vec, sizeof(float) * (size_t)count, hipMemcpyHostToDevice, stream) ==
               hipSuccess;
    }
    // d_vec -> host vector, after the launches queued on `stream`
    bool receive(float *v, int count) {
        if (hipMemcpyAsync(h_vec, d_vec, sizeof(float) * (size_t)count, hipMemcpyDeviceToHost, stream) !=
                hipSuccess ||
            hipStreamSynchronize(stream) != hipSuccess)
            return false;
        memcpy(v, h_vec, sizeof(float) * (size_t)count);
        return true;
    }
    bool finish() { return hipStreamSynchronize(stream) == hipSuccess; }
};

struct SqfreeHost {
    sp_hip_sqfree_cache_t dc;
    Staging st;
};

struct HierHost {
    sp_hip_hier_cache_t dc;
    Staging st;
};

bool slot_in_range(const sp_config_t &cfg, int max_seq, int layer, int head, int pos) {
    return layer >= 0 && layer < cfg.n_layers && head >= 0 && head < cfg.n_heads_kv && pos >= 0 && pos < max_seq;
}

// Host copy of the device cache's Knight tables (replaces m's arrays).
bool sync_mask(const sp_hip_sqfree_cache_t &dc, sp_knight_mask_t *m) {
    sp_knight_mask_free(m);
    m->pad_dim = dc.pad_dim;
    m->sk_k = dc.sk_k;
    m->n_res = dc.n_res;
    m->n_terms = dc.n_terms;
    m->skeleton_idx = (int *)malloc(sizeof(int) * (size_t)(dc.sk_k > 0 ? dc.sk_k : 1));
    m->residual_idx = (int *)malloc(sizeof(int) * (size_t)(dc.n_res > 0 ? dc.n_res : 1));
    m->csr_offsets = (int *)malloc(sizeof(int) * (size_t)(dc.n_res + 1));
    m->csr_skel_slot = (int *)malloc(sizeof(int) * (size_t)(dc.n_terms > 0 ? dc.n_terms : 1));
    m->csr_mu_sign = (int8_t *)malloc((size_t)(dc.n_terms > 0 ? dc.n_terms : 1));
    std::vector<int> sign((size_t)(dc.n_terms > 0 ? dc.n_terms : 1));
    if (!m->skeleton_idx || !m->residual_idx || !m->csr_offsets || !m->csr_skel_slot || !m->csr_mu_sign ||
        sp_hip_sqfree_get_tables(&dc, m->skeleton_idx, m->residual_idx, m->csr_offsets, m->csr_skel_slot,
                                 sign.data()) != 0) {
        sp_knight_mask_free(m);
        return false;
    }
    for (int i = 0; i < dc.n_terms; i++) m->csr_mu_sign[i] = (int8_t)sign[(size_t)i];
    return true;
}

}  // namespace

// ===========================================================================
// sqfree + spinor
// ===========================================================================
extern "C" int sp_sqfree_cache_init(sp_sqfree_cache_t *c, const sp_config_t *cfg, int max_seq_len,
                                    int residual_bits, int use_spinor) {
    if (!c) return -1;
    memset(c, 0, sizeof(*c));
    if (!cfg || max_seq_len <= 0) { sp_set_error("sqfree_cache_init: bad args"); return -1; }
    SqfreeHost *h = new SqfreeHost();
    memset(&h->dc, 0, sizeof(h->dc));
    const int pad = sp_sqfree_pad_dim(cfg->head_dim);
    if (pad <= 0 || !h->st.open(pad > cfg->head_dim ? pad : cfg->head_dim) ||
        sp_hip_sqfree_cache_init(&h->dc, cfg, max_seq_len, residual_bits, use_spinor, h->st.stream) != 0 ||
        !sync_mask(h->dc, &c->mask)) {
        if (h->dc.priv) sp_hip_sqfree_cache_free(&h->dc);
        h->st.close();
        delete h;
        memset(c, 0, sizeof(*c));
        return -1;
    }
    c->config = *cfg;
    c->pad_dim = h->dc.pad_dim;
    c->k_bands = h->dc.k_bands;
    c->v_bands = h->dc.v_bands;
    c->residual_bits = h->dc.residual_bits;
    c->use_spinor = h->dc.use_spinor;
    c->max_seq_len = max_seq_len;
    c->bytes_per_pos_k = h->dc.bytes_per_pos_k;
    c->bytes_per_pos_v = h->dc.bytes_per_pos_v;
    c->dev = h;
    return 0;
}

extern "C" void sp_sqfree_cache_free(sp_sqfree_cache_t *c) {
    if (!c) return;
    SqfreeHost *h = (SqfreeHost *)c->dev;
    if (h) {
        h->st.finish();
        sp_hip_sqfree_cache_free(&h->dc);
        h->st.close();
        delete h;
    }
    sp_knight_mask_free(&c->mask);
    memset(c, 0, sizeof(*c));
}

static void sqfree_write(sp_sqfree_cache_t *c, int is_v, int layer, int head, int pos, const float *vec) {
    if (!c || !c->dev || !vec || !slot_in_range(c->config, c->max_seq_len, layer, head, pos)) return;
    SqfreeHost *h = (SqfreeHost *)c->dev;
    std::lock_guard<std::mutex> lk(h->st.mu);
    if (!h->st.send(vec, c->config.head_dim)) return;
    if (is_v) sp_hip_sqfree_write_v(&h->dc, layer, head, pos, h->st.d_vec);
    else sp_hip_sqfree_write_k(&h->dc, layer, head, pos, h->st.d_vec);
    h->st.finish();
}

static void sqfree_read(const sp_sqfree_cache_t *c, int is_v, int layer, int head, int pos, float *out) {
    if (!c || !c->dev || !out || !slot_in_range(c->config, c->max_seq_len, layer, head, pos)) return;
    SqfreeHost *h = (SqfreeHost *)c->dev;
    std::lock_guard<std::mutex> lk(h->st.mu);
    if (is_v) sp_hip_sqfree_read_v(&h->dc, layer, head, pos, h->st.d_vec);
    else sp_hip_sqfree_read_k(&h->dc, layer, head, pos, h->st.d_vec);
    h->st.receive(out, c->config.head_dim);
}

extern "C" void sp_sqfree_write_k(sp_sqfree_cache_t *c, int l, int h, int p, const float *v) { sqfree_write(c, 0, l, h, p, v); }
extern "C" void sp_sqfree_write_v(sp_sqfree_cache_t *c, int l, int h, int p, const float *v) { sqfree_write(c, 1, l, h, p, v); }
extern "C" void sp_sqfree_read_k(const sp_sqfree_cache_t *c, int l, int h, int p, float *o) { sqfree_read(c, 0, l, h, p, o); }
extern "C" void sp_sqfree_read_v(const sp_sqfree_cache_t *c, int l, int h, int p, float *o) { sqfree_read(c, 1, l, h, p, o); }

extern "C" int sp_sqfree_calibrate_begin(sp_sqfree_cache_t *c) {
    if (!c || !c->dev) return -1;
    return sp_hip_sqfree_calibrate_begin(&((SqfreeHost *)c->dev)->dc);
}

extern "C" void sp_sqfree_calibrate_feed(sp_sqfree_cache_t *c, const float *vec) {
    if (!c || !c->dev || !vec) return;
    SqfreeHost *h = (SqfreeHost *)c->dev;
    std::lock_guard<std::mutex> lk(h->st.mu);
    const int hd = c->config.head_dim;
    if (h->st.send(vec, hd)) (void)sp_hip_sqfree_calibrate_feed(&h->dc, h->st.d_vec, hd, 1, SP_DT_F32);
    h->st.finish();
}

extern "C" int sp_sqfree_calibrate_end(sp_sqfree_cache_t *c) {
    if (!c || !c->dev) return -1;
    SqfreeHost *h = (SqfreeHost *)c->dev;
    if (sp_hip_sqfree_calibrate_end(&h->dc, nullptr, 1) != 0) return -1;
    return sync_mask(h->dc, &c->mask) ? 0 : -1;
}

extern "C" int sp_sqfree_cache_save(const sp_sqfree_cache_t *c, const char *prefix, int n_pos, uint64_t model_hash) {
    if (!c || !c->dev) return -1;
    return sp_hip_sqfree_cache_save(&((SqfreeHost *)c->dev)->dc, prefix, n_pos, model_hash);
}

extern "C" int sp_sqfree_cache_load(sp_sqfree_cache_t *c, const char *prefix, uint64_t expected_hash) {
    if (!c || !c->dev) return -1;
    return sp_hip_sqfree_cache_load(&((SqfreeHost *)c->dev)->dc, prefix, expected_hash);
}

// ===========================================================================
// hierarchical
// ===========================================================================
// predictors[s].W <- the device cache's W of every slot
static bool hier_pull_W(sp_hier_cache_t *hc) {
    HierHost *h = (HierHost *)hc->dev;
    const size_t per = (size_t)h->dc.n_target * h->dc.n_skeleton;
    if (hipStreamSynchronize(h->st.stream) != hipSuccess) return false;
    return hipMemcpy(hc->predictors[0].W, h->dc.d_W, per * hc->n_slots * sizeof(uint16_t), hipMemcpyDeviceToHost) ==
           hipSuccess;
}

extern "C" int sp_hier_cache_init(sp_hier_cache_t *hc, const sp_config_t *cfg, int max_seq_len, int level,
                                  int n_skel_bands, const int *skel_bits, int res_bits) {
    if (!hc) return -1;
    memset(hc, 0, sizeof(*hc));
    if (!cfg || max_seq_len <= 0 || cfg->n_layers <= 0 || cfg->n_heads_kv <= 0) {
        sp_set_error("hier_cache_init: bad args");
        return -1;
    }
    if (level != 0) {
        sp_set_error("hier_cache_init: level %d: only level 0 (the default geometry) is built", level);
        return -1;
    }
    if (res_bits < 1 || res_bits > 4) { sp_set_error("hier_cache_init: res_bits %d outside 1..4", res_bits); return -1; }
    static const int k_default_skel[2] = {5, 5};
    if (n_skel_bands <= 0 || !skel_bits) {
        n_skel_bands = 2;
        skel_bits = k_default_skel;
    }
    if (n_skel_bands > SP_MAX_BANDS) { sp_set_error("hier_cache_init: %d skeleton bands", n_skel_bands); return -1; }
    const int pad = sp_sqfree_pad_dim(cfg->head_dim);
    if (pad <= 0) { sp_set_error("hier_cache_init: head_dim %d has no pad", cfg->head_dim); return -1; }
    std::vector<int> skel((size_t)pad), tgt((size_t)pad);
    const int ns = sp_hier_default_geometry(pad, skel.data(), tgt.data());
    if (ns <= 0) { sp_set_error("hier_cache_init: geometry"); return -1; }
    const int nt = pad - ns;
    const int n_slots = cfg->n_layers * cfg->n_heads_kv;
    sp_band_config_t sb;
    sp_band_config_init(&sb, ns, n_skel_bands, skel_bits);

    HierHost *h = new HierHost();
    memset(&h->dc, 0, sizeof(h->dc));
    hc->predictors = (sp_hier_predictor_t *)calloc((size_t)n_slots, sizeof(sp_hier_predictor_t));
    int *idx = (int *)malloc(sizeof(int) * (size_t)pad);
    uint16_t *W = (uint16_t *)calloc((size_t)n_slots * nt * ns, sizeof(uint16_t));
    if (!hc->predictors || !idx || !W || !h->st.open(pad) ||
        sp_hip_hier_cache_init(&h->dc, cfg, pad, ns, nt, res_bits, skel.data(), tgt.data(), &sb, max_seq_len,
                               n_slots, h->st.stream) != 0) {
        if (h->dc.priv) sp_hip_hier_cache_free(&h->dc);
        h->st.close();
        delete h;
        free(hc->predictors);
        free(idx);
        free(W);
        memset(hc, 0, sizeof(*hc));
        return -1;
    }
    memcpy(idx, skel.data(), sizeof(int) * (size_t)ns);
    memcpy(idx + ns, tgt.data(), sizeof(int) * (size_t)nt);
    for (int s = 0; s < n_slots; s++) {
        sp_hier_predictor_t *p = &hc->predictors[s];
        p->pad_dim = pad;
        p->n_skeleton = ns;
        p->n_target = nt;
        p->skeleton_idx = idx;
        p->target_idx = idx + ns;
        p->skel_bands = sb;
        p->target_res_bits = res_bits;
        p->W = W + (size_t)s * nt * ns;
    }
    hc->config = *cfg;
    hc->pad_dim = pad;
    hc->n_slots = n_slots;
    hc->max_seq_len = max_seq_len;
    hc->level = level;
    hc->bytes_per_pos = h->dc.bytes_per_pos_k;
    hc->dev = h;
    return 0;
}

extern "C" void sp_hier_cache_free(sp_hier_cache_t *hc) {
    if (!hc) return;
    HierHost *h = (HierHost *)hc->dev;
    if (h) {
        h->st.finish();
        sp_hip_hier_cache_free(&h->dc);
        h->st.close();
        delete h;
    }
    if (hc->predictors) {
        free(hc->predictors[0].skeleton_idx);  // one table: skeleton then targets
        free(hc->predictors[0].W);             // one block: every slot's W
        free(hc->predictors);
    }
    memset(hc, 0, sizeof(*hc));
}

static void hier_write(sp_hier_cache_t *hc, int is_v, int layer, int head, int pos, const float *vec) {
    if (!hc || !hc->dev || !vec || !slot_in_range(hc->config, hc->max_seq_len, layer, head, pos)) return;
    HierHost *h = (HierHost *)hc->dev;
    std::lock_guard<std::mutex> lk(h->st.mu);
    if (!h->st.send(vec, hc->config.head_dim)) return;
    if (is_v) sp_hip_hier_write_v(&h->dc, layer, head, pos, h->st.d_vec);
    else sp_hip_hier_write_k(&h->dc, layer, head, pos, h->st.d_vec);
    h->st.finish();
}

static void hier_read(const sp_hier_cache_t *hc, int is_v, int layer, int head, int pos, float *out) {
    if (!hc || !hc->dev || !out || !slot_in_range(hc->config, hc->max_seq_len, layer, head, pos)) return;
    HierHost *h = (HierHost *)hc->dev;
    std::lock_guard<std::mutex> lk(h->st.mu);
    if (is_v) sp_hip_hier_read_v(&h->dc, layer, head, pos, h->st.d_vec);
    else sp_hip_hier_read_k(&h->dc, layer, head, pos, h->st.d_vec);
    h->st.receive(out, hc->config.head_dim);
}

extern "C" void sp_hier_cache_write_k(sp_hier_cache_t *c, int l, int h, int p, const float *v) { hier_write(c, 0, l, h, p, v); }
extern "C" void sp_hier_cache_write_v(sp_hier_cache_t *c, int l, int h, int p, const float *v) { hier_write(c, 1, l, h, p, v); }
extern "C" void sp_hier_cache_read_k(const sp_hier_cache_t *c, int l, int h, int p, float *o) { hier_read(c, 0, l, h, p, o); }
extern "C" void sp_hier_cache_read_v(const sp_hier_cache_t *c, int l, int h, int p, float *o) { hier_read(c, 1, l, h, p, o); }

extern "C" int sp_hier_cache_calibrate_begin(sp_hier_cache_t *hc) {
    if (!hc || !hc->dev) return -1;
    return sp_hip_hier_calibrate_begin(&((HierHost *)hc->dev)->dc);
}

extern "C" void sp_hier_cache_calibrate_feed(sp_hier_cache_t *hc, int slot, const float *vec) {
    if (!hc || !hc->dev || !vec || slot < 0 || slot >= hc->n_slots) return;
    HierHost *h = (HierHost *)hc->dev;
    std::lock_guard<std::mutex> lk(h->st.mu);
    const int hd = hc->config.head_dim;
    if (h->st.send(vec, hd)) (void)sp_hip_hier_calibrate_feed(&h->dc, slot, h->st.d_vec, hd, 1, SP_DT_F32);
    h->st.finish();
}

static constexpr double k_hier_ridge = 1e-6;

extern "C" int sp_hier_cache_calibrate_end(sp_hier_cache_t *hc) {
    if (!hc || !hc->dev) return -1;
    if (sp_hip_hier_calibrate_end(&((HierHost *)hc->dev)->dc, k_hier_ridge) != 0) return -1;
    return hier_pull_W(hc) ? 0 : -1;
}

extern "C" int sp_hier_cache_calibrate_end_ema(sp_hier_cache_t *hc, float keep_frac) {
    if (!hc || !hc->dev) return -1;
    if (sp_hip_hier_calibrate_end_ema(&((HierHost *)hc->dev)->dc, k_hier_ridge, keep_frac) != 0) return -1;
    return hier_pull_W(hc) ? 0 : -1;
}

extern "C" int sp_hier_cache_save(const sp_hier_cache_t *hc, const char *prefix, int n_pos, uint64_t model_hash) {
    if (!hc || !hc->dev) return -1;
    return sp_hip_hier_cache_save(&((HierHost *)hc->dev)->dc, prefix, n_pos, model_hash);
}

extern "C" int sp_hier_cache_load(sp_hier_cache_t *hc, const char *prefix, uint64_t expected_hash) {
    if (!hc || !hc->dev) return -1;
    const int rc = sp_hip_hier_cache_load(&((HierHost *)hc->dev)->dc, prefix, expected_hash);
    if (rc < 0) return rc;
    return hier_pull_W(hc) ? rc : -1;
}
