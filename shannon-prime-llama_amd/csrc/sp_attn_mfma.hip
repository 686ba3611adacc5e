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
//     uses the matching coefficient permutation); a shift/multiply/mask puts a
//     code pair at the top of two fp16 mantissas, 2^BITS + u (exact), and the
//     MFMA accumulator starts at -(2^BITS + m_b) * sum(q~ over the band), which
//     centres the codes; per-position band scales are applied to the fp32 MFMA
//     results.
//   * softmax over the chunk; w = p * scale_v is scaled per head by a power of
//     two and split hi + lo the same way.
//   * values in two halves: V codes are unpacked into a transposed byte tile
//     (element-major, overlaying the dead K records); the value MFMA's B
//     operand is one byte permute (1024 + u in fp16) and one packed subtract
//     (-> u - 3) per pair.
// Partials [m, l, o~[128]] per (query head, split) go to the workspace in the
// layout k_attn_combine (sp_attn.hip) merges.
#include "sp_internal.h"
#include "sp_mfma_codes.h"

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
constexpr int W_LO = CHUNK + 8;              // fp16 offset of a weight row's lo part (bank-shifted from the hi part)
constexpr int SC_STRIDE = CHUNK + 8;         // floats per head row of scores / weights
constexpr float INV_SQRT_HD = 0.08838834764831845f;

// LDS layout (bytes). U holds the K records until the scores are done, then the
// transposed V code tile of one half chunk.
constexpr int OFF_U = 0;
constexpr int SZ_U = CHUNK * KB + 16;                  // >= HD * DVT_STRIDE (V code tile of a half chunk)
constexpr int OFF_KS = SZ_U;                           // ks[CHUNK][4]: K band scales
constexpr int OFF_SC = OFF_KS + 4 * CHUNK * 4;         // sc[8][SC_STRIDE]
constexpr int OFF_QB = OFF_SC + 8 * SC_STRIDE * 4;     // qop[16][128] fp16 query operand, cb[4][16], fu[8]
constexpr int OFF_CB = OFF_QB + 16 * HD * 2;
constexpr int OFF_FH = OFF_CB + 4 * 16 * 4;
constexpr int OFF_VS = OFF_FH + 16 * 4;                // vs[CHUNK]: V scales
constexpr int OFF_VREC = OFF_VS + CHUNK * 4;           // V records (+ shift, + one dword)
constexpr int OFF_ST = OFF_VREC + CHUNK * VB + 16;     // st[8][4]: per head max, sum, 1/w-scale
constexpr int LDS_FULL = OFF_ST + 8 * 4 * 4;
constexpr int LDS_KQ = OFF_VS;
static_assert(SZ_U >= HD * DVT_STRIDE, "V code tile must fit the K record area");
static_assert(W_LO + CHUNK <= 2 * SC_STRIDE, "a head's hi and lo weight parts must fit its score row");
static_assert(OFF_KS % 16 == 0 && OFF_SC % 16 == 0 && OFF_QB % 16 == 0 && OFF_CB % 16 == 0 && OFF_VS % 16 == 0 &&
                  OFF_VREC % 16 == 0 && OFF_ST % 16 == 0,
              "LDS regions 16-byte aligned");
constexpr uint32_t BUF_WORD3 = 0x00020000u;  // raw buffer resource, dword data (gfx9 family)
constexpr int BUF_NT = 2;                    // non-temporal load policy

__device__ __forceinline__ constexpr int kbits(int b) { return b < 2 ? 5 : (b == 2 ? 4 : 3); }
__device__ __forceinline__ constexpr int kbyte(int b) { return b == 0 ? 0 : b == 1 ? 22 : b == 2 ? 44 : 62; }

// Slot (0..7) of a lane's band operand for code c (0..7) of its run in band b.
__device__ __forceinline__ int code_slot(int b, int c) { return code_slot_bits(kbits(b), c); }

// Eight 3-bit V codes (one per byte) -> fp16 (u - 3): a byte permute spreads a
// pair under a 0x64 high byte (1024 + u, exact) and a packed subtract of 1027
// centres it (exact).
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

// Value of lane (lane ^ M) for M a power of two below 64: quad permutes and a
// row rotate via DPP, the others via swizzle / permute (no LDS memory traffic).
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
    const int x = __float_as_int(v);
    int r;
    if (M == 1) r = __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true);        // quad_perm [1,0,3,2]
    else if (M == 2) r = __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true);   // quad_perm [2,3,0,1]
    else if (M == 4) r = __builtin_amdgcn_ds_swizzle(x, 0x101F);              // xor 4 within 32 lanes
    else if (M == 8) r = __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true);  // row_ror:8 (xor 8 in a row of 16)
    else if (M == 16) r = __builtin_amdgcn_ds_swizzle(x, 0x401F);             // xor 16 within 32 lanes
    else r = __builtin_amdgcn_ds_bpermute(((int)(__lane_id() ^ 32)) << 2, x);
    return __int_as_float(r);
}

// One Sylvester stage across lane bit M: x' = x + p (bit clear) or p - x (bit set).
template <int M>
__device__ __forceinline__ float lane_butterfly(float x, int lane) {
    const float p = lane_xor<M>(x);
    return fmaf(x, (lane & M) ? -1.0f : 1.0f, p);
}

template <int M>
__device__ __forceinline__ float wave_max_step(float v) { return fmaxf(v, lane_xor<M>(v)); }
template <int M>
__device__ __forceinline__ float wave_sum_step(float v) { return v + lane_xor<M>(v); }

}  // namespace

// Records of one 256-position split into registers: dword buffer loads, out-of-
// range dwords read as 0. A V split may start 2 bytes past a dword boundary
// (odd max_seq): its dwords are read from 2 bytes before it and the staged
// records start at vshift; the last dword may run 2 bytes past the last record,
// which the packed caches' slack bytes after their last record cover.
template <bool WANT_V>
__device__ __forceinline__ void load_split(const SpAttnArgs &A, int kvh, int split, int vshift, int tid,
                                           uint32_t (&kr)[KREG], uint32_t (&vr)[WANT_V ? VREG : 1]) {
    const int c0 = split * CHUNK, n_chunk = min(CHUNK, A.n_kv - c0);
    const unsigned char *kg = A.kpack + (long long)kvh * A.k_head_stride + (long long)c0 * KB;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void *)kg, (short)0, n_chunk * KB, BUF_WORD3);
#pragma unroll
    for (int i = 0; i < KREG; i++) kr[i] = __builtin_amdgcn_raw_buffer_load_b32(rk, 4 * tid, 1024 * i, BUF_NT);
    if (WANT_V) {
        const unsigned char *vg = A.vpack + (long long)kvh * A.v_head_stride + (long long)c0 * VB - vshift;
        const int nbytes = (n_chunk * VB + vshift + 3) & ~3;
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void *)vg, (short)0, nbytes, BUF_WORD3);
#pragma unroll
        for (int i = 0; i < (WANT_V ? VREG : 1); i++)
            vr[i] = __builtin_amdgcn_raw_buffer_load_b32(rv, 4 * tid, 1024 * i, BUF_NT);
    }
}

// One 256-thread block per (KV head, run of `rounds` consecutive 256-position
// splits). The query operand is prepared once per block; each round stages one
// split's records from registers into LDS and prefetches the next split's
// while it computes. Every split writes its own partial.
// The full kernel is bounded for the two blocks per CU its grid places (up to 256
// registers: the compiler then hoists more LDS reads, 3-4% faster than a bound of three).
template <bool WANT_OUT, bool ALL_BANDS>
__global__ void __launch_bounds__(256, WANT_OUT ? 2 : 4)
k_attn_mfma_split(const SpAttnArgs A, const int *__restrict__ order, float *__restrict__ ws, int n_splits,
                  int rounds, int kbands, int vbands) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[WANT_OUT ? LDS_FULL : LDS_KQ];
    unsigned char *krec = smem + OFF_U;
    unsigned char *dvt = smem + OFF_U;
    float *ks = reinterpret_cast<float *>(smem + OFF_KS);
    float *sc = reinterpret_cast<float *>(smem + OFF_SC);
    unsigned short *bop = reinterpret_cast<unsigned short *>(smem + OFF_QB);  // [16 rows][128 slots] fp16
    float *cb = reinterpret_cast<float *>(smem + OFF_CB);                       // [4 bands][16 rows]
    float *fu = reinterpret_cast<float *>(smem + OFF_FH);                       // [8] inverse query scale

    const int kvh = blockIdx.x, tid = threadIdx.x;
    const int split0 = blockIdx.y * rounds;
    const int w = tid >> 6, lane = tid & 63, q4 = lane >> 4, c16 = lane & 15;
    const int G = A.n_q / A.n_kvh, h0 = kvh * G;

    // ---- 1. wave w prepares heads w and w + 4: their query rows and the order
    // entries of record coefficients lane and lane + 64 are loaded first ----
    float qx[2][2];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const float *qg = A.q + (long long)(h0 + min(w + 4 * r, G - 1)) * HD;
        qx[r][0] = qg[lane];
        qx[r][1] = qg[lane + 64];
    }
    // Without an order table, read (and ignore) in-bounds words of q: both
    // candidates are kernel-argument pointers, so these stay global loads (a
    // flat load here would make every later wait drain all loads).
    const int *op = order ? order : reinterpret_cast<const int *>(A.q);
    const int ov0 = op[lane], ov1 = op[lane + 64];
    const int ord0 = order ? ov0 : lane, ord1 = order ? ov1 : lane + 64;
    __asm__ volatile("" ::: "memory");  // keep the query loads ahead of the record loads

    // ---- 2. the first split's records ----
    const int vshift = WANT_OUT ? (int)((uintptr_t)(A.vpack + (long long)kvh * A.v_head_stride) & 3) : 0;
    uint32_t kr[KREG];
    uint32_t vr[WANT_OUT ? VREG : 1];
    load_split<WANT_OUT>(A, kvh, split0, vshift, tid, kr, vr);

    // ---- 3. while the records are in flight: q~ = kq_scale * reorder(VHT2(q)) per
    // head, in registers (lane holds elements lane and lane + 64), scaled by a power
    // of two fh so its largest entry lies in [2^11, 2^12) and split into fp16 hi + lo:
    // the query operand rows 2h (hi) and 2h + 1 (lo) in LDS, laid out so lane
    // (c16, q4) of the score MFMA reads the 8 slots of band b as one 16-byte word
    // at (4b + q4) * 8 (record coefficient k = 32b + 8*q4 + c). Also per (row,
    // band) -(2^BITS + m_b) * sum of the row's slots: the MFMA accumulator start. ----
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int h = w + 4 * r;
        if (h >= G) break;
        float x0 = qx[r][0], x1 = qx[r][1];
        x0 = lane_butterfly<1>(x0, lane);   x1 = lane_butterfly<1>(x1, lane);
        x0 = lane_butterfly<2>(x0, lane);   x1 = lane_butterfly<2>(x1, lane);
        x0 = lane_butterfly<4>(x0, lane);   x1 = lane_butterfly<4>(x1, lane);
        x0 = lane_butterfly<8>(x0, lane);   x1 = lane_butterfly<8>(x1, lane);
        x0 = lane_butterfly<16>(x0, lane);  x1 = lane_butterfly<16>(x1, lane);
        x0 = lane_butterfly<32>(x0, lane);  x1 = lane_butterfly<32>(x1, lane);
        const float sq = A.kq_scale * INV_SQRT_HD;
        const float y0 = (x0 + x1) * sq, y1 = (x0 - x1) * sq;  // elements lane, lane + 64
        float amax = fmaxf(fabsf(y0), fabsf(y1));
        amax = wave_max_step<1>(amax);
        amax = wave_max_step<2>(amax);
        amax = wave_max_step<4>(amax);
        amax = wave_max_step<8>(amax);
        amax = wave_max_step<16>(amax);
        amax = wave_max_step<32>(amax);
        const float f = pow2_norm(amax);
        // record coefficients lane (bands 0, 1) and lane + 64 (bands 2, 3)
        float va, vb;
        {
            const float a0 = __int_as_float(__builtin_amdgcn_ds_bpermute((ord0 & 63) << 2, __float_as_int(y0)));
            const float a1 = __int_as_float(__builtin_amdgcn_ds_bpermute((ord0 & 63) << 2, __float_as_int(y1)));
            const float b0 = __int_as_float(__builtin_amdgcn_ds_bpermute((ord1 & 63) << 2, __float_as_int(y0)));
            const float b1 = __int_as_float(__builtin_amdgcn_ds_bpermute((ord1 & 63) << 2, __float_as_int(y1)));
            va = ((ord0 & 64) ? a1 : a0) * f;
            vb = ((ord1 & 64) ? b1 : b0) * f;
        }
        uint32_t ha, la, hb, lb;
        split_hl(va, ha, la);
        split_hl(vb, hb, lb);
        const int ka = lane, kb = lane + 64;
        const int ia = (4 * (ka >> 5) + ((ka >> 3) & 3)) * 8 + code_slot(ka >> 5, ka & 7);
        const int ib = (4 * (kb >> 5) + ((kb >> 3) & 3)) * 8 + code_slot(kb >> 5, kb & 7);
        bop[(2 * h) * HD + ia] = (unsigned short)ha;
        bop[(2 * h + 1) * HD + ia] = (unsigned short)la;
        bop[(2 * h) * HD + ib] = (unsigned short)hb;
        bop[(2 * h + 1) * HD + ib] = (unsigned short)lb;
        // band sums over each 32-lane half (band of ka: lane >> 5; of kb: 2 + (lane >> 5))
        float sha = (float)__builtin_bit_cast(_Float16, (unsigned short)ha);
        float sla = (float)__builtin_bit_cast(_Float16, (unsigned short)la);
        float shb = (float)__builtin_bit_cast(_Float16, (unsigned short)hb);
        float slb = (float)__builtin_bit_cast(_Float16, (unsigned short)lb);
        sha = wave_sum_step<1>(sha); sla = wave_sum_step<1>(sla); shb = wave_sum_step<1>(shb); slb = wave_sum_step<1>(slb);
        sha = wave_sum_step<2>(sha); sla = wave_sum_step<2>(sla); shb = wave_sum_step<2>(shb); slb = wave_sum_step<2>(slb);
        sha = wave_sum_step<4>(sha); sla = wave_sum_step<4>(sla); shb = wave_sum_step<4>(shb); slb = wave_sum_step<4>(slb);
        sha = wave_sum_step<8>(sha); sla = wave_sum_step<8>(sla); shb = wave_sum_step<8>(shb); slb = wave_sum_step<8>(slb);
        sha = wave_sum_step<16>(sha); sla = wave_sum_step<16>(sla); shb = wave_sum_step<16>(shb); slb = wave_sum_step<16>(slb);
        if ((lane & 31) == 0) {
            const int ba = lane >> 5, bb = 2 + (lane >> 5);
            const float ca = -(float)((1 << kbits(ba)) + (1 << (kbits(ba) - 1)) - 1);  // -(2^BITS + m_b)
            const float cbb = -(float)((1 << kbits(bb)) + (1 << (kbits(bb) - 1)) - 1);
            cb[ba * 16 + 2 * h] = ca * sha;
            cb[ba * 16 + 2 * h + 1] = ca * sla;
            cb[bb * 16 + 2 * h] = cbb * shb;
            cb[bb * 16 + 2 * h + 1] = cbb * slb;
        }
        if (lane == 0) fu[h] = 1.0f / f;  // exact: a power of two
    }
    __syncthreads();
    // query operand of row c16 = 2h + part; accumulator start of rows 4*q4 + j
    // (rows of heads >= G hold whatever the LDS holds and are never stored)
    half8_t qop[4];
    float4_t cinit[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
        qop[b] = __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4 *>(bop + c16 * HD + (4 * b + q4) * 8));
        const float4 c4 = *reinterpret_cast<const float4 *>(cb + b * 16 + 4 * q4);
        cinit[b] = float4_t{c4.x, c4.y, c4.z, c4.w};
    }
    const int hq0 = 2 * q4, hq1 = 2 * q4 + 1;  // heads of this lane's D rows (j = 0,1 and 2,3)
    const float un0 = fu[hq0], un1 = fu[hq1];
    int wofs[4], wsh[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const int p = 8 * (kbyte(b) + 2) + 8 * q4 * kbits(b);
        wofs[b] = 4 * (p >> 5);
        wsh[b] = p & 31;
    }
    // code-slot masks and the fp16 2^BITS exponent bits, kept in registers for bitop3
    const uint32_t kbias5 = __builtin_amdgcn_readfirstlane(code_bias<5>());
    const uint32_t kbias4 = __builtin_amdgcn_readfirstlane(code_bias<4>());
    const uint32_t kbias3 = __builtin_amdgcn_readfirstlane(code_bias<3>());
    uint32_t kmask5 = code_mask<5>(), kmask4 = code_mask<4>(), kmask3 = code_mask<3>();
    __asm__("" : "+v"(kmask5), "+v"(kmask4), "+v"(kmask3));

    // running softmax state of this lane's heads 2*q4 + hh over the block's rounds
    float om[2] = {-INFINITY, -INFINITY}, ol[2] = {0.0f, 0.0f}, orun[2][2] = {{0.f, 0.f}, {0.f, 0.f}};

    for (int round = 0; round < rounds; round++) {
        const int split = split0 + round;
        if (split >= n_splits) break;
        const int c0 = split * CHUNK;
        const int n_chunk = min(CHUNK, A.n_kv - c0);
        if (round > 0) __syncthreads();  // the previous round is done with the LDS
        // ---- stage this split's records; prefetch the next split's ----
#pragma unroll
        for (int i = 0; i < KREG; i++) reinterpret_cast<uint32_t *>(krec)[tid + 256 * i] = kr[i];
        if (WANT_OUT) {
            unsigned char *vrec = smem + OFF_VREC;
#pragma unroll
            for (int i = 0; i < (WANT_OUT ? VREG : 1); i++) {
                const int k = tid + 256 * i;
                if (k <= VDW) reinterpret_cast<uint32_t *>(vrec)[k] = vr[i];
            }
        }
        if (round + 1 < rounds && split + 1 < n_splits) load_split<WANT_OUT>(A, kvh, split + 1, vshift, tid, kr, vr);
        __syncthreads();
        // ---- per-position scales ----
        {
            const unsigned char *r = krec + tid * KB;
            const bool live = tid < n_chunk;
#pragma unroll
            for (int b = 0; b < 4; b++)
                ks[tid * 4 + b] = live && (ALL_BANDS || b < kbands) ? scale_of(*reinterpret_cast<const unsigned short *>(r + kbyte(b))) : 0.0f;
            if (WANT_OUT) {
                const unsigned char *v = smem + OFF_VREC + vshift + tid * VB;
                reinterpret_cast<float *>(smem + OFF_VS)[tid] = live && (ALL_BANDS || vbands > 0) ? scale_of(*reinterpret_cast<const unsigned short *>(v)) : 0.0f;
            }
        }
        __syncthreads();

        // ---- scores: wave w owns positions [64w, 64w + 64) as four 16-column tiles;
        // D[row (h, part)][position]: lane (c16, q4) holds position tb + c16, rows 4*q4 + j ----
#pragma unroll
        for (int sub = 0; sub < 4; sub++) {
            const int t = 64 * w + 16 * sub + c16;  // this lane's position (column)
            const unsigned char *rec = krec + t * KB;
            const float4 s4 = *reinterpret_cast<const float4 *>(ks + 4 * t);
            const float sb[4] = {s4.x, s4.y, s4.z, s4.w};
            float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                if (!ALL_BANDS && b >= kbands) break;  // bands past the limit read as 0 (kernel-uniform)
                const uint32_t d0 = *reinterpret_cast<const uint32_t *>(rec + wofs[b]);
                const uint32_t d1 = *reinterpret_cast<const uint32_t *>(rec + wofs[b] + 4);
                half8_t code;
                if (b < 2) code = band_codes<5>(d0, d1, wsh[b], kmask5, kbias5);
                else if (b == 2) code = band_codes<4>(d0, d1, wsh[b], kmask4, kbias4);
                else code = band_codes<3>(d0, d1, wsh[b], kmask3, kbias3);
                const float4_t d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qop[b], code, cinit[b], 0, 0, 0);
                acc0 = fmaf(sb[b], d[0] + d[1], acc0);  // hi + lo rows of head hq0
                acc1 = fmaf(sb[b], d[2] + d[3], acc1);
            }
            acc0 *= un0;
            acc1 *= un1;
            if (t < n_chunk) {
                if (hq0 < G) {
                    if (WANT_OUT) sc[hq0 * SC_STRIDE + t] = acc0;
                    if (A.scores) A.scores[(long long)(h0 + hq0) * A.n_kv + c0 + t] = acc0;
                }
                if (hq1 < G) {
                    if (WANT_OUT) sc[hq1 * SC_STRIDE + t] = acc1;
                    if (A.scores) A.scores[(long long)(h0 + hq1) * A.n_kv + c0 + t] = acc1;
                }
            }
        }
        if (!WANT_OUT) continue;
        __syncthreads();

        float *vs = reinterpret_cast<float *>(smem + OFF_VS);
        float *st = reinterpret_cast<float *>(smem + OFF_ST);
        // ---- softmax over the split (wave w: heads w, w + 4); sc <- scaled w = p * scale_v ----
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
            // the value MFMA's A operand rows 2h (hi) and 2h + 1 (lo), fp16, written over
            // this head's score row (all of which this wave has already read)
            unsigned short *wrow = reinterpret_cast<unsigned short *>(sc + h * SC_STRIDE);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                // lo part scaled by 2^11 (exact) so it stays a normal fp16 value
                const float v = wv[i] * f;
                const _Float16 hh = (_Float16)v;
                const uint32_t hi = (uint32_t)__builtin_bit_cast(unsigned short, hh);
                const uint32_t lo = (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)((v - (float)hh) * 2048.0f));
                wrow[lane + 64 * i] = (unsigned short)hi;
                wrow[W_LO + lane + 64 * i] = (unsigned short)lo;
            }
            if (lane == 0) {
                st[4 * h] = m;
                st[4 * h + 1] = l;
                st[4 * h + 2] = 1.0f / f;
            }
        }

        // ---- values, in two halves of 128 positions:
        // D[(h, part)][i] = sum_t w_part[h][t] * (u[t][i] - 3) ----
        __syncthreads();  // st complete; K records no longer read
        float4_t d0 = {0.f, 0.f, 0.f, 0.f}, d1 = {0.f, 0.f, 0.f, 0.f};
        const unsigned char *vrecs = smem + OFF_VREC + vshift;
        const int hrow = c16 >> 1, part = c16 & 1;  // A row = c16 (rows of heads >= G are never stored)
        const int n0 = 32 * w + c16;
#pragma unroll
        for (int half = 0; half < 2; half++) {
            if (half) __syncthreads();  // the previous V tile is no longer read
            {
                // thread: elements 16g .. 16g+15 (48 bits at byte 2 + 6g) of positions
                // 4pq .. 4pq+3 (a, b, c, d) -> dvt[element][position] bytes. Per group of
                // four elements, two positions' 12-bit chunks share a dword (16 bits
                // apart), so one shift and mask yields both positions' codes of an
                // element and a byte permute lines up all four positions. Element rows
                // 32s .. 32s + 31 store their 32-byte position blocks XOR-swizzled by s,
                // so each wave's tile writes fall in 64 distinct banks.
                const int g = tid & 7, pq = tid >> 3;
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const unsigned short *p = reinterpret_cast<const unsigned short *>(
                        vrecs + (128 * half + 4 * pq + i) * VB + 2 + 6 * g);
                    lo[i] = (uint32_t)p[0] | ((uint32_t)p[1] << 16);
                    hi[i] = p[2];
                }
#pragma unroll
                for (int sg = 0; sg < 4; sg++) {
                    uint32_t c[4];
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        c[i] = sg < 2 ? __builtin_amdgcn_ubfe(lo[i], 12 * sg, 12)
                                      : (sg == 2 ? (__builtin_amdgcn_alignbit(hi[i], lo[i], 24) & 0xfffu)
                                                 : __builtin_amdgcn_ubfe(hi[i], 4, 12));
                    const uint32_t wab = c[0] | (c[1] << 16), wcd = c[2] | (c[3] << 16);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const uint32_t x = (wab >> (3 * e)) & 0x00070007u, y = (wcd >> (3 * e)) & 0x00070007u;
                        *reinterpret_cast<uint32_t *>(dvt + (16 * g + 4 * sg + e) * DVT_STRIDE + ((4 * pq) ^ (32 * (g >> 1)))) =
                            __builtin_amdgcn_perm(y, x, 0x06040200u);
                    }
                }
            }
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int tb = 32 * kk + 8 * q4;  // A row c16, k-slots 8*q4 + e: positions tb + e
                const half8_t a = __builtin_bit_cast(
                    half8_t, *reinterpret_cast<const u32x4 *>(reinterpret_cast<const unsigned short *>(sc + hrow * SC_STRIDE) +
                                                              part * W_LO + 128 * half + tb));
                const u32x2 v0 = *reinterpret_cast<const u32x2 *>(dvt + n0 * DVT_STRIDE + (tb ^ (32 * w)));
                const u32x2 v1 = *reinterpret_cast<const u32x2 *>(dvt + (n0 + 16) * DVT_STRIDE + (tb ^ (32 * w)));
                d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, vcodes8(v0[0], v0[1]), d0, 0, 0, 0);
                d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, vcodes8(v1[0], v1[1]), d1, 0, 0, 0);
            }
        }
        // ---- fold this split into the running state: D rows 4*q4 + j are head
        // 2*q4 + (j >> 1), part j & 1 (rows of heads >= G carry junk, never stored) ----
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const int h = 2 * q4 + hh;
            const float mr = st[4 * h], lr = st[4 * h + 1], un = st[4 * h + 2];  // un: 1/w-scale
            const float o0 = fmaf(d0[2 * hh + 1], 1.0f / 2048.0f, d0[2 * hh]) * un;
            const float o1 = fmaf(d1[2 * hh + 1], 1.0f / 2048.0f, d1[2 * hh]) * un;
            const float mx = fmaxf(om[hh], mr);
            const float a = __expf(om[hh] - mx), b = __expf(mr - mx);
            orun[hh][0] = fmaf(orun[hh][0], a, o0 * b);
            orun[hh][1] = fmaf(orun[hh][1], a, o1 * b);
            ol[hh] = fmaf(ol[hh], a, lr * b);
            om[hh] = mx;
        }
    }
    if (!WANT_OUT) return;

    // ---- the block's partial [m, l, o[128]] per head, o in the natural domain
    // (inverse VHT2 in registers: wave w transforms heads w and w + 4) ----
    __syncthreads();  // the last round is done with the LDS
    float *st = reinterpret_cast<float *>(smem + OFF_ST);
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const int h = 2 * q4 + hh;
        if (h < G) {
            sc[h * SC_STRIDE + 32 * w + c16] = orun[hh][0];
            sc[h * SC_STRIDE + 32 * w + 16 + c16] = orun[hh][1];
            if (w == 0 && c16 == 0) {
                st[4 * h] = om[hh];
                st[4 * h + 1] = ol[hh];
            }
        }
    }
    __syncthreads();
    const int n_parts = gridDim.y;
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int h = w + 4 * r;
        if (h >= G) break;
        float x0 = sc[h * SC_STRIDE + lane], x1 = sc[h * SC_STRIDE + lane + 64];
        x0 = lane_butterfly<1>(x0, lane);   x1 = lane_butterfly<1>(x1, lane);
        x0 = lane_butterfly<2>(x0, lane);   x1 = lane_butterfly<2>(x1, lane);
        x0 = lane_butterfly<4>(x0, lane);   x1 = lane_butterfly<4>(x1, lane);
        x0 = lane_butterfly<8>(x0, lane);   x1 = lane_butterfly<8>(x1, lane);
        x0 = lane_butterfly<16>(x0, lane);  x1 = lane_butterfly<16>(x1, lane);
        x0 = lane_butterfly<32>(x0, lane);  x1 = lane_butterfly<32>(x1, lane);
        float *dst = ws + ((long long)(h0 + h) * n_parts + blockIdx.y) * (HD + 2);
        dst[2 + lane] = (x0 + x1) * INV_SQRT_HD;
        dst[2 + lane + 64] = (x0 - x1) * INV_SQRT_HD;
        if (lane == 0) {
            dst[0] = st[4 * h];
            dst[1] = st[4 * h + 1];
        }
    }
}

// Compute units of the current device (cached per device).
static int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] <= 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// SP_HIP_NO_MFMA_ATTN=1 sends every layout to the general kernel (read at each
// call so tests can cross-check both paths in one process).
hipError_t sp_launch_attn_mfma_split(const SpPlan &KP, const SpPlan &VP, const int *order, const SpAttnArgs &A,
                                     float *part, int n_splits, int *n_parts, hipStream_t s) {
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
    // Runs of consecutive splits per block: aim for ~2 blocks per CU so each
    // block prefetches its next split while computing the current one.
    const int total = A.n_kvh * n_splits;
    const int target = 2 * device_cus();
    const int rounds = total > target ? (total + target - 1) / target : 1;
    const int nb = (n_splits + rounds - 1) / rounds;
    *n_parts = nb;
    // every band: a branch-free score loop (the band-limited one schedules worse)
    const bool all = KP.max_bands >= 4 && VP.max_bands >= 1;
    const dim3 grid(A.n_kvh, nb);
    const int kb_lim = KP.max_bands, vb_lim = VP.max_bands;
    if (A.out) {
        if (all) hipLaunchKernelGGL((k_attn_mfma_split<true, true>), grid, dim3(256), 0, s, A, order, part, n_splits, rounds, kb_lim, vb_lim);
        else hipLaunchKernelGGL((k_attn_mfma_split<true, false>), grid, dim3(256), 0, s, A, order, part, n_splits, rounds, kb_lim, vb_lim);
    } else {
        if (all) hipLaunchKernelGGL((k_attn_mfma_split<false, true>), grid, dim3(256), 0, s, A, order, part, n_splits, rounds, kb_lim, vb_lim);
        else hipLaunchKernelGGL((k_attn_mfma_split<false, false>), grid, dim3(256), 0, s, A, order, part, n_splits, rounds, kb_lim, vb_lim);
    }
    return hipGetLastError();
}
