/* sp_kv_cache.hpp -- C++ host-side mirror of the reference engine's KvCache for
 * GPU-resident caches (src/engine/kv_cache.h:23-147: create_gpu, write_gpu,
 * read_gpu, calibration, disk), header-only over the C-ABI of sp_hip.h.
 * Layouts as in the reference: write_gpu takes d_K_flat / d_V_flat fp32 rows of
 * n_tokens x (n_head_kv * head_dim) (element (t, h, d) at t*n_head_kv*head_dim +
 * h*head_dim + d), read_gpu writes positions [0, kv_len) in the same layout.
 * The composition is picked by the config like the reference's Config switches
 * (engine.h: sqfree, spinor, mobius, residual_bits, k/v bits, hierarchical,
 * hier_res_bits, hier_skel_bits). Methods return false / -1 on error;
 * sp_hip_last_error() has the reason. */
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "sp_hip.h"

namespace sp::hip {

struct KvCacheConfig {
    bool sqfree = false;            // sqfree + Knight skeleton (+ spinor)
    bool spinor = false;
    bool mobius = true;             // ship-path Mobius reorder
    int residual_bits = 3;          // sqfree residual depth
    int sqfree_skeleton = 0;        // sqfree skeleton size; 0: half the padded length
    std::vector<int> k_bits{5, 5, 4, 3};
    std::vector<int> v_bits{3};
    bool hierarchical = false;      // hierarchical Vilenkin (default geometry; W from calibration)
    int hier_res_bits = 2;
    std::vector<int> hier_skel_bits{5, 5};
};

class KvCache {
public:
    static std::unique_ptr<KvCache> create_gpu(int n_layer, int n_head_kv, int head_dim, int max_seq,
                                               const KvCacheConfig &cfg, void *stream) {
        std::unique_ptr<KvCache> kv(new KvCache());
        sp_config_t c;
        sp_config_init(&c, head_dim, n_layer, n_head_kv);
        c.k_n_bands = (int)cfg.k_bits.size();
        for (int b = 0; b < c.k_n_bands && b < 16; b++) c.k_band_bits[b] = cfg.k_bits[(size_t)b];
        c.v_n_bands = (int)cfg.v_bits.size();
        for (int b = 0; b < c.v_n_bands && b < 16; b++) c.v_band_bits[b] = cfg.v_bits[(size_t)b];
        c.use_mobius_mask = cfg.mobius ? 1 : 0;
        kv->n_layer_ = n_layer, kv->n_head_kv_ = n_head_kv, kv->head_dim_ = head_dim, kv->max_seq_ = max_seq;
        if (cfg.hierarchical) {
            const int pad = sp_sqfree_pad_dim(head_dim);
            const int ns = sp_hier_default_geometry(pad, nullptr, nullptr);
            if (pad <= 0 || ns <= 0) return nullptr;
            std::vector<int> sk((size_t)ns), tg((size_t)(pad - ns));
            sp_hier_default_geometry(pad, sk.data(), tg.data());
            sp_band_config_t sbc;
            sp_band_config_init(&sbc, ns, (int)cfg.hier_skel_bits.size(), cfg.hier_skel_bits.data());
            if (sp_hip_hier_cache_init(&kv->hier_, &c, pad, ns, pad - ns, cfg.hier_res_bits, sk.data(), tg.data(),
                                       &sbc, max_seq, n_layer * n_head_kv, stream)) return nullptr;
            kv->kind_ = HIER;
        } else if (cfg.sqfree) {
            if (sp_hip_sqfree_cache_init_ex(&kv->sq_, &c, max_seq, cfg.residual_bits, cfg.spinor ? 1 : 0,
                                            cfg.sqfree_skeleton, stream)) return nullptr;
            kv->kind_ = SQFREE;
        } else {
            if (sp_hip_cache_init(&kv->ship_, &c, max_seq, stream)) return nullptr;
            kv->kind_ = SHIP;
        }
        return kv;
    }

    ~KvCache() {
        if (kind_ == SHIP) sp_hip_cache_free(&ship_);
        if (kind_ == SQFREE) sp_hip_sqfree_cache_free(&sq_);
        if (kind_ == HIER) sp_hip_hier_cache_free(&hier_);
    }
    KvCache(const KvCache &) = delete;
    KvCache &operator=(const KvCache &) = delete;

    bool write_gpu(int layer, int pos_offset, int n_tokens, const float *d_K_flat, const float *d_V_flat) {
        const long long rs = row();
        if (kind_ == SHIP) return !sp_hip_write_layer(&ship_, layer, pos_offset, n_tokens, d_K_flat, d_V_flat, rs, SP_DTYPE_F32);
        if (kind_ == SQFREE)
            return !sp_hip_sqfree_write_layer(&sq_, layer, pos_offset, n_tokens, d_K_flat, d_V_flat, rs, SP_DTYPE_F32);
        return !sp_hip_hier_write_layer(&hier_, layer, pos_offset, n_tokens, d_K_flat, d_V_flat, rs, SP_DTYPE_F32);
    }

    bool read_gpu(int layer, int kv_len, float *d_K_out, float *d_V_out) const {
        const long long rs = row();
        if (kind_ == SHIP) return !sp_hip_read_layer(&ship_, layer, 0, kv_len, d_K_out, d_V_out, rs, SP_DTYPE_F32, -1);
        if (kind_ == SQFREE) return !sp_hip_sqfree_read_layer(&sq_, layer, 0, kv_len, d_K_out, d_V_out, rs, SP_DTYPE_F32);
        return !sp_hip_hier_read_layer(&hier_, layer, 0, kv_len, d_K_out, d_V_out, rs, SP_DTYPE_F32);
    }

    bool is_gpu() const { return true; }
    bool is_hierarchical() const { return kind_ == HIER; }
    bool is_calibrated() const { return calibrated_; }

    // calibration (KvCache::calibrate_begin / feed / end / end_ema): the feeds take
    // device batches of n fp32 vectors of head_dim (row stride head_dim); the
    // hierarchical cache is fed per slot (layer * n_head_kv + head)
    bool calibrate_begin() {
        if (kind_ == SHIP) return !sp_hip_calibrate_begin(&ship_);
        if (kind_ == SQFREE) return !sp_hip_sqfree_calibrate_begin(&sq_);
        return !sp_hip_hier_calibrate_begin(&hier_);
    }
    bool calibrate_feed(const float *d_vecs, int n) {
        if (kind_ == SHIP) return !sp_hip_calibrate_feed(&ship_, d_vecs, head_dim_, n, SP_DTYPE_F32);
        if (kind_ == SQFREE) return !sp_hip_sqfree_calibrate_feed(&sq_, d_vecs, head_dim_, n, SP_DTYPE_F32);
        return false;  // the hierarchical predictor is fed per slot
    }
    bool calibrate_feed(int slot, const float *d_vecs, int n) {
        if (kind_ != HIER) return calibrate_feed(d_vecs, n);
        return !sp_hip_hier_calibrate_feed(&hier_, slot, d_vecs, head_dim_, n, SP_DTYPE_F32);
    }
    bool calibrate_end(double hier_ridge = 1e-6) { return calibrate_end_ema(0.0f, hier_ridge); }
    bool calibrate_end_ema(float keep_frac, double hier_ridge = 1e-6) {
        int rc;
        if (kind_ == SHIP) rc = sp_hip_calibrate_end(&ship_, nullptr, 1);
        else if (kind_ == SQFREE) rc = sp_hip_sqfree_calibrate_end(&sq_, nullptr, 1);
        else rc = sp_hip_hier_calibrate_end_ema(&hier_, hier_ridge, keep_frac);
        if (!rc) calibrated_ = true;
        return !rc;
    }

    // disk (KvCache::save_to_disk / load_from_disk / load_from_disk_partial)
    int save_to_disk(const std::string &prefix, int n_pos, uint64_t model_hash) const {
        if (kind_ == SHIP) return sp_hip_cache_save(&ship_, prefix.c_str(), n_pos, model_hash);
        if (kind_ == SQFREE) return sp_hip_sqfree_cache_save(&sq_, prefix.c_str(), n_pos, model_hash);
        return sp_hip_hier_cache_save(&hier_, prefix.c_str(), n_pos, model_hash);
    }
    int load_from_disk(const std::string &prefix, uint64_t expected_hash) {
        if (kind_ == SHIP) return sp_hip_cache_load(&ship_, prefix.c_str(), expected_hash);
        if (kind_ == SQFREE) return sp_hip_sqfree_cache_load(&sq_, prefix.c_str(), expected_hash);
        return sp_hip_hier_cache_load(&hier_, prefix.c_str(), expected_hash);
    }
    int load_from_disk_partial(const std::string &prefix, uint64_t expected_hash, int max_bands) {
        return kind_ == SHIP ? sp_hip_cache_load_partial(&ship_, prefix.c_str(), expected_hash, max_bands) : -1;
    }

    int n_layer() const { return n_layer_; }
    int n_head_kv() const { return n_head_kv_; }
    int head_dim() const { return head_dim_; }
    int max_seq() const { return max_seq_; }
    std::string describe() const {
        return std::string("Shannon-Prime MI355X KvCache: ") + (kind_ == SHIP ? "ship" : kind_ == SQFREE ? "sqfree" : "hierarchical") +
               ", " + std::to_string(n_layer_) + " layers x " + std::to_string(n_head_kv_) + " heads x " +
               std::to_string(max_seq_) + " positions, head_dim " + std::to_string(head_dim_);
    }
    // the underlying C caches (for the attention, round-trip and dual-cache calls)
    sp_hip_cache_t *ship() { return kind_ == SHIP ? &ship_ : nullptr; }
    sp_hip_sqfree_cache_t *sqfree() { return kind_ == SQFREE ? &sq_ : nullptr; }
    sp_hip_hier_cache_t *hier() { return kind_ == HIER ? &hier_ : nullptr; }

private:
    enum Kind { NONE, SHIP, SQFREE, HIER };
    KvCache() = default;
    long long row() const { return (long long)n_head_kv_ * head_dim_; }
    Kind kind_ = NONE;
    bool calibrated_ = false;
    int n_layer_ = 0, n_head_kv_ = 0, head_dim_ = 0, max_seq_ = 0;
    mutable sp_hip_cache_t ship_{};
    mutable sp_hip_sqfree_cache_t sq_{};
    mutable sp_hip_hier_cache_t hier_{};
};

}  // namespace sp::hip
