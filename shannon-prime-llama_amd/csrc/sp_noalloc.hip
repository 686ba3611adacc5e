// sp_noalloc.hip -- decode attention that allocates nothing.
//
// sp_hip_attn_decode_bands_noalloc is sp_hip_attn_decode_bands with the
// attention workspace (the general kernel's rotated queries and the per-split
// partials [m, l, o[hd]] the merge reads) taken from one fixed array in device
// memory instead of the workspace the cache allocated at init. A call makes no
// hipMalloc or hipFree and calls no allocating routine, for callers that cannot
// allocate (code under HIP graph capture, allocation-free serving loops).
//
// The array is a file-scope __device__ variable, so every GPU the library runs
// on holds its own copy until the process ends. Its device address is looked up
// once per device with hipGetSymbolAddress and kept per device; host code uses
// only that address. The array's last lines hold the matrix-core kernel's
// per-KV-head arrival counters, which must be zero when a call starts: the
// array is zero-initialised, and every completed call leaves the counters at
// zero (the last block of each KV head resets its counter). The kernels write
// every other scratch word before reading it in the same call. All calls on one
// GPU share the array: calls that overlap on one GPU (two streams, or two host
// threads) race on it.
#include <mutex>

#include "sp_internal.h"

namespace {

constexpr size_t SCRATCH_BYTES = 16u << 20;  // 16 MiB per GPU
constexpr size_t SCRATCH_FLOATS = SCRATCH_BYTES / sizeof(float);
constexpr int MAX_DEVICES = 64;

static __device__ __align__(256) float scratch[SCRATCH_FLOATS];

std::mutex g_scratch_mu;
float *g_scratch_ptr[MAX_DEVICES] = {};

// Device address of `scratch` on the device that runs stream s (the current
// device, which s must belong to); nullptr with the error set on failure.
float *scratch_for_stream(hipStream_t s) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        sp_set_error("attn_noalloc: no current device (%s)", hipGetErrorString(e));
        return nullptr;
    }
    if (s) {
        hipDevice_t sd = -1;
        e = hipStreamGetDevice(s, &sd);
        if (e != hipSuccess) {
            sp_set_error("attn_noalloc: stream device: %s", hipGetErrorString(e));
            return nullptr;
        }
        if (sd != dev) {
            sp_set_error("attn_noalloc: the stream belongs to device %d, the current device is %d", (int)sd, dev);
            return nullptr;
        }
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            sp_set_error("attn_noalloc: scratch address on device %d: %s", dev, hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = static_cast<float *>(ptr);
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" size_t sp_hip_attn_noalloc_max_floats(void) { return SCRATCH_FLOATS; }

extern "C" int sp_hip_attn_decode_bands_noalloc(const sp_hip_cache_t *cc, int layer, int n_kv, const float *d_q,
                                                int n_q, float kq_scale, float *d_scores, float *d_out, int max_bands,
                                                void *stream) {
    SpAttnArgs A;
    SpPlan kp, vp;
    if (sp_attn_prepare(cc, layer, n_kv, d_q, n_q, kq_scale, d_scores, d_out, max_bands, &A, &kp, &vp)) return -1;
    const size_t need = sp_attn_workspace_floats(n_q, A.hd, n_kv);
    if (need > SCRATCH_FLOATS) {
        sp_set_error("attn_noalloc: %d query heads over %d positions at head_dim %d need %zu floats of workspace; "
                     "the fixed scratch holds %zu",
                     n_q, n_kv, A.hd, need, SCRATCH_FLOATS);
        return -1;
    }
    const hipStream_t s = (hipStream_t)(stream ? stream : cc->stream);
    float *ws = scratch_for_stream(s);
    if (!ws) return -1;
    const hipError_t e = sp_launch_attn_decode(kp, vp, cc->d_mobius_order, A, ws, SCRATCH_FLOATS, s);
    if (e != hipSuccess) {
        sp_set_error("attn_noalloc launch: %s", hipGetErrorString(e));
        return -1;
    }
    return 0;
}
