// sp_disk.hip -- repacking between the caches' position-major records and the
// band-major disk layout (format v3 of the reference's disk tier, CHANGELOG.md
// "Disk-tier scaffold", kv_cache.h:132-146): a record is cut into segments (its
// bands, plus for sqfree/hier the residual tail), and segment s of every (slot,
// position) is stored contiguously, [segment][slot][position][segment bytes], so a
// partial load reads the first bands' regions only. Format v2 is the same with one
// segment, the whole record.
// One thread per record: it reads its record's bytes in one contiguous run and
// writes each segment at its place in the segment's region; consecutive threads
// handle consecutive positions, so both sides move through memory in order.
#include "sp_internal.h"

namespace {

__global__ void __launch_bounds__(256)
k_disk_pack(const unsigned char *__restrict__ rec, long long slot_stride, int B, int n_pos, long long n_rec,
            const SpDiskSegs S, unsigned char *__restrict__ out) {
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n_rec) return;
    const long long slot = idx / n_pos, pos = idx - slot * n_pos;
    const unsigned char *r = rec + slot * slot_stride + pos * B;
    for (int s = 0; s < S.n; s++) {
        unsigned char *o = out + S.base[s] + idx * S.len[s];
        const unsigned char *i = r + S.off[s];
        for (int k = 0; k < S.len[s]; k++) o[k] = i[k];
    }
}

// Segments s < n_load come from `in` (which holds only those regions); the bytes
// of the others are cleared, so they decode as 0.
__global__ void __launch_bounds__(256)
k_disk_unpack(const unsigned char *__restrict__ in, long long slot_stride, int B, int n_pos, long long n_rec,
              const SpDiskSegs S, int n_load, unsigned char *__restrict__ rec) {
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n_rec) return;
    const long long slot = idx / n_pos, pos = idx - slot * n_pos;
    unsigned char *r = rec + slot * slot_stride + pos * B;
    for (int s = 0; s < S.n; s++) {
        unsigned char *o = r + S.off[s];
        if (s < n_load) {
            const unsigned char *i = in + S.base[s] + idx * S.len[s];
            for (int k = 0; k < S.len[s]; k++) o[k] = i[k];
        } else {
            for (int k = 0; k < S.len[s]; k++) o[k] = 0;
        }
    }
}

}  // namespace

hipError_t sp_launch_disk_pack(const unsigned char *rec, long long slot_stride, int B, int n_slots, int n_pos,
                               const SpDiskSegs &S, unsigned char *out, hipStream_t s) {
    const long long n_rec = (long long)n_slots * n_pos;
    if (n_rec <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_disk_pack, dim3((unsigned)((n_rec + 255) / 256)), dim3(256), 0, s, rec, slot_stride, B, n_pos,
                       n_rec, S, out);
    return hipGetLastError();
}

hipError_t sp_launch_disk_unpack(const unsigned char *in, long long slot_stride, int B, int n_slots, int n_pos,
                                 const SpDiskSegs &S, int n_load, unsigned char *rec, hipStream_t s) {
    const long long n_rec = (long long)n_slots * n_pos;
    if (n_rec <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_disk_unpack, dim3((unsigned)((n_rec + 255) / 256)), dim3(256), 0, s, in, slot_stride, B,
                       n_pos, n_rec, S, n_load, rec);
    return hipGetLastError();
}
