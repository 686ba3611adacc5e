// sp_attn_mfma.hip -- fused decompress-attention decode on the matrix cores for
// the shipping layout: head_dim 128, K bands 5/5/4/3 (any coefficient order),
// V one 3-bit band (records of 76 and 50 bytes).
//
// Same algebra as the general kernel (sp_attn.hip), replacing the CPU op
// llama_sp_kq_compute (src/engine/llama_sp_fused_kq.cpp:83-165): with
// q~ = kq_scale * reorder(VHT2(q)),
//   score_t = sum_b scale_b[t] * sum_{k in b} q~[k] (u_k - m_b),
//   sum_t p_t V~_t = VHT2(sum_t p_t dq(V_t)).
//
// One 256-thread block per (KV head, 256-position split):
//   * the query rows go out first, then the chunk's K (and V) records as
//     straight-line coalesced dword loads into registers; q~ for the block's
//     GQA group is formed while they are in flight (two in-register radix
//     passes over LDS), scaled by a power of two per head so its largest entry
//     lies in [2^11, 2^12), and split into fp16 hi + lo parts: B columns
//     (2h, 2h+1) of v_mfma_f32_16x16x32_f16 carry head h, ~22 bits together.
//   * scores: lane (row, q4) of a 16-position tile takes a contiguous run of 8
//     codes of every band from one 64-bit window of its record (the B operand
//     uses the matching coefficient permutation); a shift/or/mask makes a code
//     pair 1024 + u in fp16 and one packed subtract centres it (u - m_b,
//     exact); per-position band scales are applied to the fp32 MFMA results.
//   * softmax over the chunk; w = p * scale_v is scaled per head by a power of
//     two and split hi + lo the same way.
//   * values in two halves: V codes are unpacked into a transposed byte tile
//     (element-major, overlaying the dead K records); the value MFMA's B
//     operand is one byte permute (1024 + u in fp16) and one packed subtract
//     (-> u - 3) per pair.
// Partials [m, l, o~[128]] per (query head, split) go to the workspace in the
// layout k_attn_combine (sp_attn.hip) merges.
#include "sp_internal.h"

#include <cstdlib>

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int HD = 128, KB = 76, VB = 50;
constexpr int CHUNK = 256;                   // positions per block (the general kernel's split)
constexpr int KDW = CHUNK * KB / 4;          // 4864 dwords of K records
constexpr int VDW = CHUNK * VB / 4;          // 3200 dwords of V records
constexpr int KREG = KDW / 256;              // 19
constexpr int VREG = (VDW + 1 + 255) / 256;  // 13 (one more dword when the V chunk is shifted)
constexpr int DVT_STRIDE = 128 + 8;          // bytes per element row of the transposed V code tile (128 positions)
constexpr int SC_STRIDE = CHUNK + 8;         // floats per head row of scores / weights
constexpr int QS_STRIDE = HD + 4;            // floats per head row of the query transform
constexpr float INV_SQRT_HD = 0.08838834764831845f;

// LDS layout (bytes). U holds the K records until the scores are done, then the
// transposed V code tile of one half chunk.
constexpr int OFF_U = 0;
constexpr int SZ_U = CHUNK * KB + 16;                  // >= 128 * DVT_STRIDE
constexpr int OFF_KS = SZ_U;                           // ks[4][CHUNK]: K band scales
constexpr int OFF_SC = OFF_KS + 4 * CHUNK * 4;         // sc[8][SC_STRIDE]; during set-up qs[8][QS_STRIDE]
constexpr int OFF_QB = OFF_SC + 8 * SC_STRIDE * 4;     // bop[16][128] fp16 B operand, cb[16][4][4], fh[8]
constexpr int OFF_CB = OFF_QB + 16 * HD * 2;
constexpr int OFF_FH = OFF_CB + 16 * 4 * 4 * 4;
constexpr int OFF_VS = OFF_FH + 8 * 4;                 // vs[CHUNK]: V scales
constexpr int OFF_VREC = OFF_VS + CHUNK * 4;           // V records (+ shift, + one dword)
constexpr int OFF_ST = OFF_VREC + CHUNK * VB + 16;     // st[8][4]: per head max, sum, 1/w-scale
constexpr int LDS_FULL = OFF_ST + 8 * 4 * 4;
constexpr int LDS_KQ = OFF_VS;
static_assert(SZ_U >= 128 * DVT_STRIDE, "V code tile must fit the K record area");
static_assert(8 * QS_STRIDE <= 8 * SC_STRIDE, "query staging must fit the score area");
static_assert(OFF_KS % 16 == 0 && OFF_SC % 16 == 0 && OFF_QB % 16 == 0 && OFF_CB % 16 == 0 && OFF_VS % 16 == 0 &&
                  OFF_VREC % 16 == 0 && OFF_ST % 16 == 0,
              "LDS regions 16-byte aligned");
constexpr uint32_t BUF_WORD3 = 0x00020000u;  // raw buffer resource, dword data (gfx9 family)
constexpr int BUF_NT = 2;                    // non-temporal load policy

__device__ __forceinline__ constexpr int kbits(int b) { return b < 2 ? 5 : (b == 2 ? 4 : 3); }
__device__ __forceinline__ constexpr int kbyte(int b) { return b == 0 ? 0 : b == 1 ? 22 : b == 2 ? 44 : 62; }

// Code pairs as fp16 (1024 + u, exact): the MFMA accumulator starts at
// -(1024 + m_b) * sum(B column over the band), which centres the codes.
// Two adjacent BITS-bit codes at bit `off` of x: the 2*BITS-bit field times
// (1 + 2^(16-BITS)) copies the second code to bit 16, the mask keeps both slots.
// The mask and the 0x6400 bits arrive in registers (kmask, kbias) so one
// three-input bit operation, (a & b) | c, finishes the pair.
template <int BITS>
__device__ __forceinline__ uint32_t code_pair(uint32_t x, uint32_t off, uint32_t kmask, uint32_t kbias) {
    const uint32_t y = __builtin_amdgcn_ubfe(x, off, 2 * BITS);
    return __builtin_amdgcn_bitop3_b32(y * (1u + (1u << (16 - BITS))), kmask, kbias, 0xEA);
}

__device__ __forceinline__ half8_t as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const u32x4 v = {a, b, c, d};
    return __builtin_bit_cast(half8_t, v);
}

// Eight consecutive codes of one band (bits [sh, sh + 8*BITS) of d1:d0) -> the
// lane's 8-slot A operand of v_mfma_f32_16x16x32_f16. 5- and 3-bit bands: slot
// e holds code e. 4-bit band: codes i and i + 4 sit 16 bits apart already, so
// the slots hold codes (0,4,1,5,2,6,3,7).
template <int BITS>
__device__ __forceinline__ half8_t band_codes(uint32_t d0, uint32_t d1, uint32_t sh, uint32_t kmask, uint32_t kbias) {
    const uint32_t lo = __builtin_amdgcn_alignbit(d1, d0, sh);  // window bits 0..31
    if (BITS == 4)
        return as_half8(__builtin_amdgcn_bitop3_b32(lo, kmask, kbias, 0xEA),
                        __builtin_amdgcn_bitop3_b32(lo >> 4, kmask, kbias, 0xEA),
                        __builtin_amdgcn_bitop3_b32(lo >> 8, kmask, kbias, 0xEA),
                        __builtin_amdgcn_bitop3_b32(lo >> 12, kmask, kbias, 0xEA));
    uint32_t p67;
    if (BITS == 5) p67 = code_pair<5>(__builtin_amdgcn_alignbit(d1 >> sh, lo, 30), 0, kmask, kbias);  // bits 30..39
    else p67 = code_pair<BITS>(lo, 6 * BITS, kmask, kbias);
    return as_half8(code_pair<BITS>(lo, 0, kmask, kbias), code_pair<BITS>(lo, 2 * BITS, kmask, kbias),
                    code_pair<BITS>(lo, 4 * BITS, kmask, kbias), p67);
}

// Slot (0..7) of a lane's band operand for code c (0..7) of its run in band b.
__device__ __forceinline__ int code_slot(int b, int c) {
    return b == 2 ? ((((c & 3) >> 1) << 2) | ((c & 1) << 1) | (c >> 2)) : c;
}

// Eight 3-bit V codes (one per byte) -> fp16 (u - 3): bytes are spread into
// 16-bit lanes under a 0x64 high byte (1024 + u), then 1027 is subtracted.
__device__ __forceinline__ half8_t vcodes8(uint32_t c0, uint32_t c1) {
    const _Float16 k = (_Float16)1027.0f;
    const half2_t b = {k, k};
    const half2_t x0 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, c0, 0x04010400u)) - b;
    const half2_t x1 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, c0, 0x04030402u)) - b;
    const half2_t x2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, c1, 0x04010400u)) - b;
    const half2_t x3 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, c1, 0x04030402u)) - b;
    return as_half8(__builtin_bit_cast(uint32_t, x0), __builtin_bit_cast(uint32_t, x1), __builtin_bit_cast(uint32_t, x2),
                    __builtin_bit_cast(uint32_t, x3));
}

// v -> (hi, lo) fp16 bit patterns with hi + lo ~= v to ~22 bits.
__device__ __forceinline__ void split_hl(float v, uint32_t &hi, uint32_t &lo) {
    const _Float16 h = (_Float16)v;
    hi = (uint32_t)__builtin_bit_cast(unsigned short, h);
    const _Float16 l = (_Float16)(v - (float)h);
    lo = (uint32_t)__builtin_bit_cast(unsigned short, l);
}

// Power of two p with amax * p in [2^11, 2^12) (1 when amax is 0 or not finite).
__device__ __forceinline__ float pow2_norm(float amax) {
    if (!(amax > 0.0f) || !(amax < INFINITY)) return 1.0f;
    int e;
    (void)frexpf(amax, &e);  // amax = f * 2^e, f in [0.5, 1)
    return ldexpf(1.0f, 12 - e);
}

// fp16 scale bits -> float; a non-finite scale dequantizes to 0.
__device__ __forceinline__ float scale_of(unsigned short h) {
    const float f = (float)__builtin_bit_cast(_Float16, h);
    return ((h & 0x7c00u) == 0x7c00u) ? 0.0f : f;
}

// v + the value of the lane with index lane ^ 1 (DPP quad permute [1,0,3,2]).
__device__ __forceinline__ float add_xor1(float v) {
    return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
}

// radix-2 Sylvester butterflies over every index bit of x (natural order)
template <int N>
__device__ __forceinline__ void hadamard_regs(float (&x)[N]) {
#pragma unroll
    for (int len = 1; len < N; len <<= 1)
#pragma unroll
        for (int i = 0; i < N; i++)
            if ((i & len) == 0) {
                const float u = x[i], v = x[i + len];
                x[i] = u + v;
                x[i + len] = u - v;
            }
}

}  // namespace

// One 256-thread block per (KV head, 256-position split).
template <bool WANT_OUT>
__global__ void __launch_bounds__(256, WANT_OUT ? 3 : 4)
k_attn_mfma_split(const SpAttnArgs A, const int *__restrict__ order, float *__restrict__ ws, int n_splits) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[WANT_OUT ? LDS_FULL : LDS_KQ];
    unsigned char *krec = smem + OFF_U;
    unsigned char *dvt = smem + OFF_U;
    float *ks = reinterpret_cast<float *>(smem + OFF_KS);
    float *sc = reinterpret_cast<float *>(smem + OFF_SC);
    float *qs = sc;  // natural-order query transform [8][QS_STRIDE] during set-up
    unsigned short *bop = reinterpret_cast<unsigned short *>(smem + OFF_QB);  // [16 columns][128 slots] fp16
    float *cb = reinterpret_cast<float *>(smem + OFF_CB);                       // [16 columns][4 bands][4 copies]
    float *fh = reinterpret_cast<float *>(smem + OFF_FH);                       // [8] power-of-two query scale

    const int kvh = blockIdx.x, split = blockIdx.y, tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63, q4 = lane >> 4, c16 = lane & 15;
    const int G = A.n_q / A.n_kvh, h0 = kvh * G;
    const int c0 = split * CHUNK;
    const int n_chunk = min(CHUNK, A.n_kv - c0);

    // ---- 1. the query (4 elements per thread) and the order entry, loaded first ----
    float qv[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int idx = tid + 256 * r, h = idx >> 7;
        qv[r] = A.q[(long long)(h0 + min(h, G - 1)) * HD + (idx & (HD - 1))];
    }
    // Without an order table, read (and ignore) an in-bounds word of q: both
    // candidates are kernel-argument pointers, so this stays a global load (a
    // flat load here would make every later wait drain all loads).
    const int *op = order ? order : reinterpret_cast<const int *>(A.q);
    const int ordv = op[tid & (HD - 1)];
    const int ord = order ? ordv : (tid & (HD - 1));
    __asm__ volatile("" ::: "memory");  // keep the query loads ahead of the record loads

    // ---- 2. the chunk's records: dword buffer loads (out-of-range dwords read as 0) ----
    uint32_t kr[KREG];
    {
        const unsigned char *kg = A.kpack + (long long)kvh * A.k_head_stride + (long long)c0 * KB;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)kg, (short)0, n_chunk * KB, BUF_WORD3);
#pragma unroll
        for (int i = 0; i < KREG; i++) kr[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, 4 * tid, 1024 * i, BUF_NT);
    }
    // A V chunk may start 2 bytes past a dword boundary (odd max_seq): its dwords
    // are read from 2 bytes before it and the staged records start at vshift. The
    // last dword may run 2 bytes past the last record; the packed caches carry
    // slack bytes after their last record for this.
    uint32_t vr[WANT_OUT ? VREG : 1];
    int vshift = 0;
    if (WANT_OUT) {
        const unsigned char *vg = A.vpack + (long long)kvh * A.v_head_stride + (long long)c0 * VB;
        vshift = (int)((uintptr_t)vg & 3);
        const int nbytes = (n_chunk * VB + vshift + 3) & ~3;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)(vg - vshift), (short)0, nbytes, BUF_WORD3);
#pragma unroll
        for (int i = 0; i < VREG; i++) vr[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, 4 * tid, 1024 * i, BUF_NT);
    }

    // ---- 3. q~ = kq_scale * reorder(VHT2(q)) while the records are in flight ----
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int idx = tid + 256 * r, h = idx >> 7;
        if (h < G) qs[h * QS_STRIDE + (idx & (HD - 1))] = qv[r];
    }
    __syncthreads();
    if (tid < G * 16) {  // butterflies over element bits 4..6
        const int h = tid >> 4, k = tid & 15;
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; i++) x[i] = qs[h * QS_STRIDE + k + 16 * i];
        hadamard_regs(x);
#pragma unroll
        for (int i = 0; i < 8; i++) qs[h * QS_STRIDE + k + 16 * i] = x[i];
    }
    __syncthreads();
    if (tid < G * 8) {  // butterflies over element bits 0..3, then the scale
        const int h = tid >> 3, m = tid & 7;
        float4 *row = reinterpret_cast<float4 *>(qs + h * QS_STRIDE + 16 * m);
        float x[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 v = row[i];
            x[4 * i] = v.x;
            x[4 * i + 1] = v.y;
            x[4 * i + 2] = v.z;
            x[4 * i + 3] = v.w;
        }
        hadamard_regs(x);
        const float s = A.kq_scale * INV_SQRT_HD;
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            x[i] *= s;
            amax = fmaxf(amax, fabsf(x[i]));
        }
#pragma unroll
        for (int i = 0; i < 4; i++) row[i] = make_float4(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
        // the 8 threads of a head are 8 aligned lanes of one wave
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
        if (m == 0) fh[h] = pow2_norm(amax);
    }
    __syncthreads();
    // B operand in LDS: column 2h + part (0: hi, 1: lo) of q~ * fh[h] in record
    // order, laid out so lane (c16, q4) reads the 8 slots of band b as one
    // 16-byte word at (4b + q4) * 8. Record coefficient kr = 32b + 8*q4 + c.
    {
        const int kr = tid & (HD - 1), b = kr >> 5, lq = (kr >> 3) & 3;
        const int idx = (4 * b + lq) * 8 + code_slot(b, kr & 7);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int h = (tid >> 7) + 2 * r;
            if (h < G) {
                uint32_t hi, lo;
                split_hl(qs[h * QS_STRIDE + ord] * fh[h], hi, lo);
                bop[(2 * h) * HD + idx] = (unsigned short)hi;
                bop[(2 * h + 1) * HD + idx] = (unsigned short)lo;
            }
        }
    }
    // records -> LDS
#pragma unroll
    for (int i = 0; i < KREG; i++) reinterpret_cast<uint32_t *>(krec)[tid + 256 * i] = kr[i];
    if (WANT_OUT) {
        unsigned char *vrec = smem + OFF_VREC;
#pragma unroll
        for (int i = 0; i < VREG; i++) {
            const int k = tid + 256 * i;
            if (k <= VDW) reinterpret_cast<uint32_t *>(vrec)[k] = vr[i];
        }
    }
    __syncthreads();

    // ---- 4. per (column, band): (1024 + m_b) * sum of the column's slots; per-position scales ----
    if (tid < 64) {
        const int col = tid >> 2, b = tid & 3;
        if ((col >> 1) < G) {
            float tp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const half8_t v = __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4 *>(bop + col * HD + 32 * b + 8 * i));
#pragma unroll
                for (int e = 0; e < 8; e++) tp[e & 3] += (float)v[e];
            }
            const float t = (tp[0] + tp[1]) + (tp[2] + tp[3]);
            // minus, four copies: read back as an MFMA accumulator start
            const float c = -(1024.0f + (float)((1 << (kbits(b) - 1)) - 1)) * t;
            *reinterpret_cast<float4 *>(cb + (col * 4 + b) * 4) = make_float4(c, c, c, c);
        }
    }
    {
        const unsigned char *r = krec + tid * KB;
        const bool live = tid < n_chunk;
#pragma unroll
        for (int b = 0; b < 4; b++)
            ks[b * CHUNK + tid] = live ? scale_of(*reinterpret_cast<const unsigned short *>(r + kbyte(b))) : 0.0f;
        if (WANT_OUT) {
            const unsigned char *v = smem + OFF_VREC + vshift + tid * VB;
            reinterpret_cast<float *>(smem + OFF_VS)[tid] = live ? scale_of(*reinterpret_cast<const unsigned short *>(v)) : 0.0f;
            if (tid < 8) {
                float *st = reinterpret_cast<float *>(smem + OFF_ST);
                st[4 * tid] = -INFINITY;
                st[4 * tid + 1] = 0.0f;
                st[4 * tid + 2] = 1.0f;
            }
        }
    }
    __syncthreads();

    // ---- 5. B operand, accumulator start and unscale of this lane's column c16 = 2h + part ----
    half8_t bq[4];
    float4_t cinit[4];
    float q_unscale = 1.0f;
    {
        const int h = c16 >> 1;
        const bool live = h < G;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const u32x4 v = live ? *reinterpret_cast<const u32x4 *>(bop + c16 * HD + (4 * b + q4) * 8) : u32x4{0u, 0u, 0u, 0u};
            bq[b] = __builtin_bit_cast(half8_t, v);
        }
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const float4 c4 = live ? *reinterpret_cast<const float4 *>(cb + (c16 * 4 + b) * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
            cinit[b] = float4_t{c4.x, c4.y, c4.z, c4.w};
        }
        if (live) q_unscale = 1.0f / fh[h];  // exact: a power of two
    }

    // ---- 6. scores: wave w owns positions [64w, 64w + 64) as four 16-row tiles ----
    int wofs[4], wsh[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const int p = 8 * (kbyte(b) + 2) + 8 * q4 * kbits(b);
        wofs[b] = 4 * (p >> 5);
        wsh[b] = p & 31;
    }
    const bool vec_store = A.scores && ((A.n_kv & 3) == 0);
    // code-slot masks and the fp16 1024 bits, kept in registers for bitop3
    const uint32_t kbias = __builtin_amdgcn_readfirstlane(0x64006400u);
    uint32_t kmask5 = 0x001f001fu, kmask4 = 0x000f000fu, kmask3 = 0x00070007u;
    __asm__("" : "+v"(kmask5), "+v"(kmask4), "+v"(kmask3));
#pragma unroll
    for (int sub = 0; sub < 4; sub++) {
        const int tb = 64 * w + 16 * sub;
        const unsigned char *rec = krec + (tb + c16) * KB;  // A row = position tb + c16
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t d0 = *reinterpret_cast<const uint32_t *>(rec + wofs[b]);
            const uint32_t d1 = *reinterpret_cast<const uint32_t *>(rec + wofs[b] + 4);
            half8_t a;
            if (b < 2) a = band_codes<5>(d0, d1, wsh[b], kmask5, kbias);
            else if (b == 2) a = band_codes<4>(d0, d1, wsh[b], kmask4, kbias);
            else a = band_codes<3>(d0, d1, wsh[b], kmask3, kbias);
            const float4_t d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[b], cinit[b], 0, 0, 0);
            // D rows 4*q4 + j (positions), column c16
            const float4 s4 = *reinterpret_cast<const float4 *>(ks + b * CHUNK + tb + 4 * q4);
            acc[0] = fmaf(s4.x, d[0], acc[0]);
            acc[1] = fmaf(s4.y, d[1], acc[1]);
            acc[2] = fmaf(s4.z, d[2], acc[2]);
            acc[3] = fmaf(s4.w, d[3], acc[3]);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) acc[j] = add_xor1(acc[j]) * q_unscale;  // hi + lo columns
        const int h = c16 >> 1;
        if ((c16 & 1) == 0 && h < G) {
            const int t = tb + 4 * q4;
            if (WANT_OUT) *reinterpret_cast<float4 *>(sc + h * SC_STRIDE + t) = make_float4(acc[0], acc[1], acc[2], acc[3]);
            if (A.scores) {
                float *dst = A.scores + (long long)(h0 + h) * A.n_kv + c0 + t;
                if (vec_store && t + 3 < n_chunk) {
                    *reinterpret_cast<float4 *>(dst) = make_float4(acc[0], acc[1], acc[2], acc[3]);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        if (t + j < n_chunk) dst[j] = acc[j];
                }
            }
        }
    }
    if (!WANT_OUT) return;
    __syncthreads();

    float *vs = reinterpret_cast<float *>(smem + OFF_VS);
    float *st = reinterpret_cast<float *>(smem + OFF_ST);
    // ---- 7. softmax over the chunk (wave w: heads w, w + 4); sc <- scaled w = p * scale_v ----
    for (int h = w; h < G; h += 4) {
        float sv[4];
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = lane + 64 * i;
            sv[i] = t < n_chunk ? sc[h * SC_STRIDE + t] : -INFINITY;
            m = fmaxf(m, sv[i]);
        }
        m = sp_wave_max(m);
        float l = 0.0f, wm = 0.0f, wv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = lane + 64 * i;
            const float p = t < n_chunk ? __expf(sv[i] - m) : 0.0f;
            wv[i] = p * vs[t];
            l += p;
            wm = fmaxf(wm, wv[i]);
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            l += __shfl_xor(l, o, 64);
            wm = fmaxf(wm, __shfl_xor(wm, o, 64));
        }
        const float f = pow2_norm(wm);
#pragma unroll
        for (int i = 0; i < 4; i++) sc[h * SC_STRIDE + lane + 64 * i] = wv[i] * f;
        if (lane == 0) {
            st[4 * h] = m;
            st[4 * h + 1] = l;
            st[4 * h + 2] = 1.0f / f;
        }
    }

    // ---- 8. values, in two halves of 128 positions:
    // D[(h, part)][i] = sum_t w_part[h][t] * (u[t][i] - 3) ----
    float4_t d0 = {0.f, 0.f, 0.f, 0.f}, d1 = {0.f, 0.f, 0.f, 0.f};
    const unsigned char *vrecs = smem + OFF_VREC + vshift;
    const int hrow = c16 >> 1, part = c16 & 1;  // A row = c16
    const bool live = hrow < G;
    const int n0 = 32 * w + c16;
#pragma unroll
    for (int half = 0; half < 2; half++) {
        __syncthreads();  // K records (first half) or the previous V tile are no longer read
        {
            // thread: elements 16g .. 16g+15 (48 bits at byte 2 + 6g) of positions 4pq .. 4pq+3
            const int g = tid & 7, pq = tid >> 3;
            unsigned long long bits[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const unsigned short *p = reinterpret_cast<const unsigned short *>(
                    vrecs + (128 * half + 4 * pq + i) * VB + 2 + 6 * g);
                bits[i] = (unsigned long long)p[0] | ((unsigned long long)p[1] << 16) | ((unsigned long long)p[2] << 32);
            }
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t u0 = (uint32_t)(bits[0] >> (3 * e)) & 7u, u1 = (uint32_t)(bits[1] >> (3 * e)) & 7u;
                const uint32_t u2 = (uint32_t)(bits[2] >> (3 * e)) & 7u, u3 = (uint32_t)(bits[3] >> (3 * e)) & 7u;
                *reinterpret_cast<uint32_t *>(dvt + (16 * g + e) * DVT_STRIDE + 4 * pq) =
                    u0 | (u1 << 8) | (u2 << 16) | (u3 << 24);
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const int tb = 32 * kk + 8 * q4;  // A row c16, k-slots 8*q4 + e: positions tb + e
            uint32_t wd[4];
            {
                float wv[8];
                if (live) {
                    const float4 x = *reinterpret_cast<const float4 *>(sc + hrow * SC_STRIDE + 128 * half + tb);
                    const float4 y = *reinterpret_cast<const float4 *>(sc + hrow * SC_STRIDE + 128 * half + tb + 4);
                    wv[0] = x.x; wv[1] = x.y; wv[2] = x.z; wv[3] = x.w;
                    wv[4] = y.x; wv[5] = y.y; wv[6] = y.z; wv[7] = y.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) wv[e] = 0.0f;
                }
                uint32_t h16[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    uint32_t hi, lo;
                    split_hl(wv[e], hi, lo);
                    h16[e] = part ? lo : hi;
                }
#pragma unroll
                for (int e = 0; e < 4; e++) wd[e] = h16[2 * e] | (h16[2 * e + 1] << 16);
            }
            const half8_t a = as_half8(wd[0], wd[1], wd[2], wd[3]);
            const u32x2 v0 = *reinterpret_cast<const u32x2 *>(dvt + n0 * DVT_STRIDE + tb);
            const u32x2 v1 = *reinterpret_cast<const u32x2 *>(dvt + (n0 + 16) * DVT_STRIDE + tb);
            d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, vcodes8(v0[0], v0[1]), d0, 0, 0, 0);
            d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, vcodes8(v1[0], v1[1]), d1, 0, 0, 0);
        }
    }
    // ---- 9. partials: D rows 4*q4 + j are head 2*q4 + (j >> 1), part j & 1 ----
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const int h = 2 * q4 + hh;
        if (h < G) {
            const float un = st[4 * h + 2];
            float *dst = ws + ((long long)(h0 + h) * n_splits + split) * (HD + 2) + 2;
            dst[32 * w + c16] = (d0[2 * hh] + d0[2 * hh + 1]) * un;
            dst[32 * w + 16 + c16] = (d1[2 * hh] + d1[2 * hh + 1]) * un;
        }
    }
    if (tid < G) {
        float *dst = ws + ((long long)(h0 + tid) * n_splits + split) * (HD + 2);
        dst[0] = st[4 * tid];
        dst[1] = st[4 * tid + 1];
    }
}

// SP_HIP_NO_MFMA_ATTN=1 sends every layout to the general kernel (read at each
// call so tests can cross-check both paths in one process).
hipError_t sp_launch_attn_mfma_split(const SpPlan &KP, const SpPlan &VP, const int *order, const SpAttnArgs &A,
                                     float *part, int n_splits, hipStream_t s) {
    static const int kb[4] = {5, 5, 4, 3};
    const char *off = getenv("SP_HIP_NO_MFMA_ATTN");
    if (off && off[0] == '1') return hipErrorNotSupported;
    if (A.hd != HD || A.kB != KB || A.vB != VB || KP.hd != HD || VP.hd != HD || KP.n_bands != 4 ||
        KP.skip_transform || VP.n_bands != 1 || VP.band_bits[0] != 3 || VP.skip_transform)
        return hipErrorNotSupported;
    for (int b = 0; b < 4; b++)
        if (KP.band_bits[b] != kb[b] || KP.band_off[b] != 32 * b || KP.band_sz[b] != 32 ||
            KP.band_byte_off[b] != (b == 0 ? 0 : b == 1 ? 22 : b == 2 ? 44 : 62))
            return hipErrorNotSupported;
    if (A.n_q % A.n_kvh || A.n_q / A.n_kvh > 8 || (long long)n_splits * CHUNK < A.n_kv) return hipErrorNotSupported;
    if (((uintptr_t)A.kpack % 4) || ((uintptr_t)A.vpack % 2) || (A.k_head_stride % 4) || (A.v_head_stride % 2))
        return hipErrorNotSupported;
    if (A.out)
        hipLaunchKernelGGL(k_attn_mfma_split<true>, dim3(A.n_kvh, n_splits), dim3(256), 0, s, A, order, part, n_splits);
    else
        hipLaunchKernelGGL(k_attn_mfma_split<false>, dim3(A.n_kvh, n_splits), dim3(256), 0, s, A, order, part, n_splits);
    return hipGetLastError();
}
