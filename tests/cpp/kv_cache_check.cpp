// kv_cache_check.cpp -- drives include/sp_kv_cache.hpp (the C++ KvCache mirror)
// on the GPU for the ship, sqfree and hier compositions: write_gpu, read_gpu,
// calibration (hier: per-slot predictor fit), save_to_disk / load_from_disk into
// a fresh cache. It dumps inputs, outputs and the hier W to <dir> for the Python
// test to check against the oracle, and exits non-zero when a reloaded cache
// reads back differently.
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "sp_kv_cache.hpp"

static bool dump(const std::string &path, const void *p, size_t n) {
    FILE *f = fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = fwrite(p, 1, n, f) == n;
    return fclose(f) == 0 && ok;
}

int main(int argc, char **argv) {
    if (argc != 2) { fprintf(stderr, "usage: kv_cache_check <out dir>\n"); return 2; }
    const std::string dir = argv[1];
    const int L = 2, H = 2, hd = 128, S = 96, n = 80;
    const size_t row = (size_t)H * hd, elems = (size_t)n * row;
    // fp16-representable values (k / 512 with |k| < 2048) from a fixed LCG
    std::vector<float> x(elems * L);
    uint32_t s = 12345u;
    for (auto &v : x) {
        s = s * 1664525u + 1013904223u;
        v = (float)((int)((s >> 8) % 4095u) - 2047) / 512.0f;
    }
    if (!dump(dir + "/x.bin", x.data(), x.size() * 4)) return 3;
    float *d_x = nullptr, *d_y = nullptr, *d_z = nullptr;
    if (hipMalloc((void **)&d_x, x.size() * 4) || hipMalloc((void **)&d_y, elems * 4) ||
        hipMalloc((void **)&d_z, elems * 4)) return 4;
    if (hipMemcpy(d_x, x.data(), x.size() * 4, hipMemcpyHostToDevice)) return 4;
    const char *names[3] = {"ship", "sqfree", "hier"};
    for (int kind = 0; kind < 3; kind++) {
        sp::hip::KvCacheConfig cfg;
        if (kind == 1) cfg.sqfree = cfg.spinor = true, cfg.k_bits = cfg.v_bits = {5, 4, 4, 4, 5};
        if (kind == 2) cfg.hierarchical = true;
        auto kv = sp::hip::KvCache::create_gpu(L, H, hd, S, cfg, nullptr);
        if (!kv) { fprintf(stderr, "%s: create_gpu: %s\n", names[kind], sp_hip_last_error()); return 5; }
        printf("%s\n", kv->describe().c_str());
        if (kind == 2) {  // fit each slot's predictor on that head's vectors (rows of the layer)
            bool ok = kv->calibrate_begin();
            for (int l = 0; l < L && ok; l++)
                for (int h = 0; h < H && ok; h++) {
                    // head h of layer l: n rows at stride row; gather them contiguous
                    std::vector<float> v((size_t)n * hd);
                    for (int t = 0; t < n; t++)
                        memcpy(&v[(size_t)t * hd], &x[(size_t)l * elems + (size_t)t * row + (size_t)h * hd], hd * 4);
                    float *d_v = nullptr;
                    ok = !hipMalloc((void **)&d_v, v.size() * 4) &&
                         !hipMemcpy(d_v, v.data(), v.size() * 4, hipMemcpyHostToDevice) &&
                         kv->calibrate_feed(l * H + h, d_v, n) && !hipDeviceSynchronize();
                    (void)hipFree(d_v);
                }
            if (!ok || !kv->calibrate_end() || !kv->is_calibrated()) {
                fprintf(stderr, "hier calibration: %s\n", sp_hip_last_error());
                return 6;
            }
            std::vector<uint16_t> W((size_t)L * H * kv->hier()->n_target * kv->hier()->n_skeleton);
            if (hipMemcpy(W.data(), kv->hier()->d_W, W.size() * 2, hipMemcpyDeviceToHost) ||
                !dump(dir + "/hier_W.bin", W.data(), W.size() * 2)) return 6;
        }
        const std::string prefix = dir + "/" + names[kind];
        for (int l = 0; l < L; l++) {
            if (!kv->write_gpu(l, 0, n, d_x + (size_t)l * elems, d_x + (size_t)l * elems) ||
                !kv->read_gpu(l, n, d_y, nullptr)) {
                fprintf(stderr, "%s: write/read: %s\n", names[kind], sp_hip_last_error());
                return 7;
            }
            std::vector<float> y(elems);
            if (hipMemcpy(y.data(), d_y, elems * 4, hipMemcpyDeviceToHost) ||
                !dump(dir + "/" + names[kind] + "_y" + std::to_string(l) + ".bin", y.data(), elems * 4)) return 7;
        }
        if (kv->save_to_disk(prefix, n, 77) != 0) { fprintf(stderr, "%s: save: %s\n", names[kind], sp_hip_last_error()); return 8; }
        auto kv2 = sp::hip::KvCache::create_gpu(L, H, hd, S, cfg, nullptr);
        if (!kv2 || kv2->load_from_disk(prefix, 77) != n) {
            fprintf(stderr, "%s: load: %s\n", names[kind], sp_hip_last_error());
            return 9;
        }
        for (int l = 0; l < L; l++) {
            std::vector<float> a(elems), b(elems);
            if (!kv->read_gpu(l, n, d_y, d_y) || !kv2->read_gpu(l, n, d_z, d_z) ||
                hipMemcpy(a.data(), d_y, elems * 4, hipMemcpyDeviceToHost) ||
                hipMemcpy(b.data(), d_z, elems * 4, hipMemcpyDeviceToHost)) return 10;
            if (memcmp(a.data(), b.data(), elems * 4) != 0) {
                fprintf(stderr, "%s: layer %d reads back differently after load\n", names[kind], l);
                return 11;
            }
        }
        printf("%s ok\n", names[kind]);
    }
    (void)hipFree(d_x);
    (void)hipFree(d_y);
    (void)hipFree(d_z);
    return 0;
}
