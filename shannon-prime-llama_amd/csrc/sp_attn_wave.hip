// sp_attn_wave.hip -- fused decompress-attention decode on the matrix cores for
// the shipping layout: head_dim 128, K bands 5/5/4/3 (any coefficient order),
// V one 3-bit band (records of 76 and 50 bytes). One 64-position tile per wave.
//
// Same algebra as the general kernel (sp_attn.hip), replacing the CPU op
// llama_sp_kq_compute (src/engine/llama_sp_fused_kq.cpp:83-165) and the ggml
// softmax . V after it: with q~ = kq_scale * reorder(VHT2(q)),
//   score_t = sum_b scale_b[t] * sum_{k in b} q~[k] (u_k - m_b),
//   sum_t p_t V~_t = VHT2(sum_t p_t dq(V_t)).
//
// Block = 16 waves on one CU, one KV head, a run of consecutive 64-position
// tiles; each wave works its own tiles with no block barrier:
//   * the tile's K and V records arrive as 16-byte buffer loads (range-checked,
//     so a partial tile reads zeros) and are staged in the wave's LDS region;
//     lane t then holds record t of the K tile in registers.
//   * scores on v_mfma_f32_4x4x4_16b_f16 (16 blocks of 4 x 4 x 4): block b's
//     rows are positions 4b .. 4b+3 (A: lane 4b + i gives 4 codes of its own
//     record, as fp16 2^BITS + u, sp_mfma_codes.h), its columns 4 query heads
//     (B: the query's fp16 hi and lo parts from LDS, two MFMAs into the same
//     accumulator), K = 4 coefficients of one band; 8 steps per band, one
//     accumulator per band started at -(2^BITS + m_b) * sum(q~ over the band).
//     Every code field sits at a compile-time bit of the record. Lane 4b + j
//     ends with head j's scores for positions 4b .. 4b+3; band scales come from
//     the quad's records by DPP broadcast.
//   * softmax over the tile in that layout (4 positions of one head per lane);
//     the weights w = p * scale_v, scaled per head by a power of two, go to LDS
//     as fp16 hi + lo rows.
//   * values on v_mfma_f32_16x16x32_f16, A = weights, B = V codes: a lane's
//     column n covers elements 8n .. 8n+7 (24 bits at record byte 2 + 3n) and
//     its two K slots per dword are two positions, so one byte permute puts
//     both positions' codes of an element pair in one dword; a shift and an
//     and-or land each at the top of an fp16 mantissa (8 + u), and a packed
//     subtract centres it (u - 3, exact).
//   * the block's waves merge their (m, l, o~) in LDS; each block writes one
//     spectral-domain partial [m, l, o~[128]] per query head with agent-scope
//     atomic stores, waits for them to complete and counts itself on its KV
//     head's counter; the block that arrives last reads the partials back with
//     agent-scope atomic loads, merges them and applies one inverse VHT2 per head.
#include "sp_internal.h"
#include "sp_mfma_codes.h"

#include <algorithm>
#include <cstdlib>

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int HD = 128, KB = 76, VB = 50;
constexpr int TILE = 64;   // positions per wave and tile
constexpr int NW = 16;     // waves per block
constexpr int NT = 64 * NW;
constexpr float INV_SQRT_HD = 0.08838834764831845f;

// Per-wave LDS region (bytes). Once every lane holds its K record in registers
// the K area carries the weight rows and the per-head softmax state.
constexpr int R_K = 0;                  // K records, 64 x 76 B
constexpr int R_WT = 0;                 // weight rows [16][WT_STRIDE] fp16
constexpr int WT_STRIDE = 72;           // fp16 per weight row: 64 slots + 8 (bank shift)
constexpr int R_ST = R_WT + 16 * WT_STRIDE * 2;  // per head [m, l, 1/f, -] f32
constexpr int R_V = 4880;               // V records: vshift + 64 x 50 B (+ slack for the window reads)
constexpr int R_SIZE = R_V + 3216;
// Block-shared region after the wave regions.
constexpr int QS_STRIDE = HD + 4;       // fp16 per (part, head) query row: the 4 heads of a read fall in distinct banks
constexpr int S_QS = NW * R_SIZE;       // query operand [part][head 8][QS_STRIDE: band 4 x slot 32] fp16
constexpr int S_CB = S_QS + 2 * 8 * QS_STRIDE * 2;  // accumulator starts [head 8][band 4] f32
constexpr int S_FU = S_CB + 8 * 4 * 4;       // inverse query scale [head 8] f32
constexpr int S_FLAG = S_FU + 8 * 4;         // [0] the block arrived last for its KV head, [1] query operand ready
constexpr int LDS_BYTES = S_FLAG + 16;
constexpr int MB_STRIDE = 132;          // floats per (wave, head) in the in-block merge: m, l, -, -, o~[128]
static_assert(R_ST + 8 * 16 <= R_V && R_V >= TILE * KB, "K area holds the records, then the weights and state");
static_assert(R_SIZE - R_V >= 2 + TILE * VB + 14, "V area with slack for the window reads");
static_assert(NW * 8 * MB_STRIDE * 4 <= S_QS, "merge records fit the wave regions");
constexpr int MAX_PARTS = 256;          // partials per KV head (blocks per KV head)
static_assert(R_V % 16 == 0 && R_SIZE % 16 == 0 && S_QS % 16 == 0 && S_CB % 16 == 0 && S_FU % 16 == 0,
              "LDS regions 16-byte aligned");
static_assert(LDS_BYTES <= 160 * 1024, "LDS of one CU");
constexpr int K_LOADS = (TILE * KB + 1023) / 1024;          // 5 x 16 B per lane
constexpr int V_LOADS = (TILE * VB + 2 + 3 + 1023) / 1024;  // 4 x 16 B per lane
constexpr uint32_t BUF_WORD3 = 0x00020000u;  // raw buffer resource, dword data (gfx9 family)
constexpr int BUF_NT = 2;                    // non-temporal load policy
constexpr uint32_t VMASK = 0x03800380u;      // fp16 mantissa bits 7..9 of both halves
constexpr uint32_t VBIAS = 0x48004800u;      // fp16 2^3 in both halves: 8 + u with u at bits 7..9

__device__ __forceinline__ constexpr int kbits(int b) { return b < 2 ? 5 : (b == 2 ? 4 : 3); }
__device__ __forceinline__ constexpr int kbyte(int b) { return b == 0 ? 0 : b == 1 ? 22 : b == 2 ? 44 : 62; }

// Score MFMA slots. Step s of a band takes slots 4s .. 4s+3, i.e. the band's
// code pairs 2s and 2s + 1, each pair one dword of two fp16 (pair p: slots
// 2p, 2p + 1). A pair built with one shift and one masked OR needs its two
// codes about 16 bits apart:
//   5-bit band: pairs (6g + i, 6g + i + 3), g < 5, i < 3, are 15 bits apart:
//     the first code at mantissa bits 5..9 (2^5 + c), the second at bits
//     4..8 of the high half (2^5 + c/2: half gain, so its query slot holds 2q~);
//     codes 30 and 31 form an ordinary pair (both 2^5 + c).
//   3-bit band: likewise pairs (10g + i, 10g + i + 5), g < 3, i < 5 (2^3 + c,
//     2^3 + c/2), and the ordinary pair (30, 31).
//   4-bit band: a dword of 8 codes 8d + 4a + i yields pairs (i, i + 4) already
//     16 bits apart (both 2^4 + c), steps 2d and 2d + 1.
// slot_of(b, c) = slot of code c; the high bit of the result marks half gain.
__device__ __forceinline__ int score_slot(int b, int c) {
    if (b == 2) {
        const int d = c >> 3, a = (c >> 2) & 1, i = c & 3;
        return 8 * d + 4 * (i >> 1) + 2 * (i & 1) + a;
    }
    const int span = b < 2 ? 6 : 10, half = span / 2;  // codes per group, pairs per group
    if (c >= 30) return 30 + (c - 30);                 // pair 15, ordinary
    const int g = c / span, i = c % span;
    const int pr = half * g + (i < half ? i : i - half);
    return i < half ? 2 * pr : (2 * pr + 1) | 0x100;
}

// The 32 record bits starting at bit p (p compile-time after unrolling; bits past
// the record's 19 dwords read from the zero dword r[19]).
__device__ __forceinline__ uint32_t rec_window(const uint32_t (&r)[20], int p) {
    const int d = p >> 5, o = p & 31;
    return o == 0 ? r[d] : __builtin_amdgcn_alignbit(r[d + 1], r[d], o);
}

// v -> (hi, lo) fp16 bit patterns with hi + lo ~= v to ~22 bits.
__device__ __forceinline__ void split_hl(float v, uint32_t &hi, uint32_t &lo) {
    const _Float16 h = (_Float16)v;
    hi = (uint32_t)__builtin_bit_cast(unsigned short, h);
    const _Float16 l = (_Float16)(v - (float)h);
    lo = (uint32_t)__builtin_bit_cast(unsigned short, l);
}

// Power of two p with amax * p in [2^11, 2^12) (1 when amax is 0 or not finite),
// and its reciprocal (exact).
__device__ __forceinline__ float pow2_norm(float amax, float &inv) {
    if (!(amax > 0.0f) || !(amax < INFINITY)) {
        inv = 1.0f;
        return 1.0f;
    }
    int e;
    (void)frexpf(amax, &e);  // amax = f * 2^e, f in [0.5, 1)
    inv = ldexpf(1.0f, e - 12);
    return ldexpf(1.0f, 12 - e);
}

// fp16 scale bits -> float; a non-finite scale dequantizes to 0.
__device__ __forceinline__ float scale_of(uint32_t h) {
    const float f = (float)__builtin_bit_cast(_Float16, (unsigned short)h);
    return ((h & 0x7c00u) == 0x7c00u) ? 0.0f : f;
}

// Value of lane (lane ^ M) for M a power of two below 64, all on the VALU (no
// LDS crossbar round trip): quad permutes and row shifts / rotates via DPP,
// 16 and 32 via the gfx950 row swaps (permlane16/32_swap(x, x) leave lane l
// with lane l ^ 16 (^ 32) in one result or the other, by that lane bit).
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
    const int x = __float_as_int(v);
    const int lane = (int)__lane_id();
    int r;
    if (M == 1) r = __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true);        // quad_perm [1,0,3,2]
    else if (M == 2) r = __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true);   // quad_perm [2,3,0,1]
    else if (M == 4) {                                                        // row_shr:4 / row_shl:4
        const int dn = __builtin_amdgcn_mov_dpp(x, 0x114, 0xF, 0xF, true), up = __builtin_amdgcn_mov_dpp(x, 0x104, 0xF, 0xF, true);
        r = (lane & 4) ? dn : up;
    } else if (M == 8) r = __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true);  // row_ror:8 (xor 8 in a row of 16)
    else if (M == 16) {
        const u32x2 t = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
        r = (int)((lane & 16) ? t[0] : t[1]);
    } else {
        const u32x2 t = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
        r = (int)((lane & 32) ? t[0] : t[1]);
    }
    return __int_as_float(r);
}

// Value of lane I of this lane's quad (DPP quad_perm [I, I, I, I]).
template <int I>
__device__ __forceinline__ float quad_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), I * 0x55, 0xF, 0xF, true));
}

// One Sylvester stage across lane bit M: x' = x + p (bit clear) or p - x (bit set).
template <int M>
__device__ __forceinline__ float lane_butterfly(float x, int lane) {
    const float p = lane_xor<M>(x);
    return fmaf(x, (lane & M) ? -1.0f : 1.0f, p);
}

// max(a, b) of finite or infinite values as one v_med3 (fmaxf would first quiet
// the exchanged operand, an extra instruction per step)
__device__ __forceinline__ float max_ninf(float a, float b) { return __builtin_amdgcn_fmed3f(a, b, INFINITY); }

template <int M>
__device__ __forceinline__ float wave_max_step(float v) { return max_ninf(v, lane_xor<M>(v)); }
template <int M>
__device__ __forceinline__ float wave_sum_step(float v) { return v + lane_xor<M>(v); }

// Max / sum over the 16 lanes with the same lane & 3 (one head's quads).
__device__ __forceinline__ float head_max(float v) {
    v = wave_max_step<4>(v);
    v = wave_max_step<8>(v);
    v = wave_max_step<16>(v);
    return wave_max_step<32>(v);
}
__device__ __forceinline__ float head_sum(float v) {
    v = wave_sum_step<4>(v);
    v = wave_sum_step<8>(v);
    v = wave_sum_step<16>(v);
    return wave_sum_step<32>(v);
}

// Bits [p, p + w) of a K record held as 19 dwords (p, w compile-time after unrolling).
__device__ __forceinline__ uint32_t rec_bits(const uint32_t (&r)[20], int p, int w) {
    const int d = p >> 5, o = p & 31;
    if (o + w <= 32) return __builtin_amdgcn_ubfe(r[d], o, w);
    return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(r[d + 1], r[d], o), 0, w);
}

// Two adjacent BITS-bit codes y = c0 | c1 << BITS -> fp16 pair (2^BITS + c0, 2^BITS + c1)
// (the multiply-and-mask of sp_mfma_codes.h on a field already extracted).
template <int BITS>
__device__ __forceinline__ uint32_t pair_fp16(uint32_t y, uint32_t kmask, uint32_t kbias) {
    return __builtin_amdgcn_bitop3_b32(y * ((1u << (10 - BITS)) + (1u << (26 - 2 * BITS))), kmask, kbias, 0xEA);
}

// Pair p (0..15) of a 5- or 3-bit band as one dword of two fp16 (see score_slot).
template <int BITS>
__device__ __forceinline__ uint32_t band_pair(const uint32_t (&r)[20], int b0, int p, uint32_t kmask, uint32_t kbias,
                                              uint32_t kmask15) {
    constexpr int span = BITS == 5 ? 6 : 10, half = span / 2;
    if (p == 15) return pair_fp16<BITS>(rec_bits(r, b0 + 30 * BITS, 2 * BITS), kmask, kbias);
    const int a = span * (p / half) + p % half;  // first code of the pair
    // the first code lands at mantissa bits 10-BITS .. 9, the second 15 bits above it
    return __builtin_amdgcn_bitop3_b32(rec_window(r, b0 + BITS * a - (10 - BITS)), kmask15, kbias, 0xEA);
}

// The score MFMA's A operand for band b, step s: 4 codes of the lane's record
// as fp16 in slots 4s .. 4s+3 (see score_slot).
__device__ __forceinline__ half4_t score_codes(const uint32_t (&r)[20], int b, int s, uint32_t kmask5, uint32_t kbias5,
                                               uint32_t kmask4, uint32_t kbias4, uint32_t kmask3, uint32_t kbias3,
                                               uint32_t kmask5p, uint32_t kmask3p) {
    uint32_t x0, x1;
    if (b < 2) {
        const int b0 = 8 * (kbyte(b) + 2);
        x0 = band_pair<5>(r, b0, 2 * s, kmask5, kbias5, kmask5p);
        x1 = band_pair<5>(r, b0, 2 * s + 1, kmask5, kbias5, kmask5p);
    } else if (b == 2) {
        // the dword of codes 8d .. 8d+7 starts at bit 368 + 32d = 32 (11 + d) + 16
        const int d = s >> 1;
        const uint32_t x = __builtin_amdgcn_alignbit(r[12 + d], r[11 + d], 16);
        if ((s & 1) == 0) {
            x0 = __builtin_amdgcn_bitop3_b32(x << 6, kmask4, kbias4, 0xEA);  // codes 0, 4
            x1 = __builtin_amdgcn_bitop3_b32(x << 2, kmask4, kbias4, 0xEA);  // codes 1, 5
        } else {
            x0 = __builtin_amdgcn_bitop3_b32(x >> 2, kmask4, kbias4, 0xEA);  // codes 2, 6
            x1 = __builtin_amdgcn_bitop3_b32(x >> 6, kmask4, kbias4, 0xEA);  // codes 3, 7
        }
    } else {
        const int b0 = 8 * (kbyte(3) + 2);
        x0 = band_pair<3>(r, b0, 2 * s, kmask3, kbias3, kmask3p);
        x1 = band_pair<3>(r, b0, 2 * s + 1, kmask3, kbias3, kmask3p);
    }
    return __builtin_bit_cast(half4_t, u32x2{x0, x1});
}

// The 32 bits at byte offset sh/8 past the dword-aligned p (a V window's 24 bits and one more byte).
__device__ __forceinline__ uint32_t v_window(const unsigned char *p, uint32_t sh) {
    const uint32_t *d = reinterpret_cast<const uint32_t *>(p);
    return __builtin_amdgcn_alignbit(d[1], d[0], sh);
}

// Code j (0..7) of two positions' windows as two fp16 u - 3 (exact): a shift
// and an and-or put each code at the top of an fp16 mantissa under the
// exponent of 2^3 (8 + u), one packed subtract centres it. pa = bytes 0,1 of
// both windows, pb = bytes 1,2. (Centring here rather than subtracting
// 11 * sum(w) after the MFMA keeps the offset's rounding out of the sums: that
// rounding would be the same for every coefficient and the inverse VHT2 would
// gather it into output element 0.)
template <int J>
__device__ __forceinline__ uint32_t v_pair(uint32_t pa, uint32_t pb, uint32_t vmask, uint32_t vbias) {
    uint32_t x;
    if (J == 0) x = pa << 7;
    else if (J == 1) x = pa << 4;
    else if (J == 2) x = pa << 1;
    else if (J == 3) x = pa >> 2;
    else if (J == 4) x = pa >> 5;
    else if (J == 5) x = pb;
    else if (J == 6) x = pb >> 3;
    else x = pb >> 6;
    const _Float16 k11 = (_Float16)11.0f;
    const half2_t c = __builtin_bit_cast(half2_t, __builtin_amdgcn_bitop3_b32(x, vmask, vbias, 0xEA)) - half2_t{k11, k11};
    return __builtin_bit_cast(uint32_t, c);
}

// Records of one tile in registers: 16-byte buffer loads, out-of-range dwords
// read as 0. The V stream starts vshift (0 or 2) bytes before its first record.
struct TileRegs {
    u32x4 k[K_LOADS];
    u32x4 v[V_LOADS];
};

template <bool WANT_V>
__device__ __forceinline__ void load_tile(const SpAttnArgs &A, int kvh, int c0, int n_chunk, int vshift, int lane,
                                          TileRegs &r) {
    const unsigned char *kg = A.kpack + (long long)kvh * A.k_head_stride + (long long)c0 * KB;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void *)kg, (short)0, n_chunk * KB, BUF_WORD3);
#pragma unroll
    for (int i = 0; i < K_LOADS; i++) r.k[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, 16 * lane, 1024 * i, BUF_NT);
    if (WANT_V) {
        const unsigned char *vg = A.vpack + (long long)kvh * A.v_head_stride + (long long)c0 * VB - vshift;
        const int nbytes = (n_chunk * VB + vshift + 3) & ~3;
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void *)vg, (short)0, nbytes, BUF_WORD3);
#pragma unroll
        for (int i = 0; i < V_LOADS; i++) r.v[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, 16 * lane, 1024 * i, BUF_NT);
    }
}

template <bool WANT_V>
__device__ __forceinline__ void stage_tile(unsigned char *wl, const TileRegs &r, int lane) {
#pragma unroll
    for (int i = 0; i < K_LOADS; i++) {
        const int off = 16 * lane + 1024 * i;
        if (off < R_V - R_K) *reinterpret_cast<u32x4 *>(wl + R_K + off) = r.k[i];
    }
    if (WANT_V) {
#pragma unroll
        for (int i = 0; i < V_LOADS; i++) {
            const int off = 16 * lane + 1024 * i;
            if (off < R_SIZE - R_V) *reinterpret_cast<u32x4 *>(wl + R_V + off) = r.v[i];
        }
    }
}

}  // namespace

// One block of 16 waves per (KV head, run of tiles); wave w works tiles
// w * tpw .. w * tpw + tpw - 1 of the block's run. Partials go to
// part[(query head) * n_parts + blockIdx.y] as [m, l, o~[128]]. NH = 1 serves
// up to 4 query heads per KV head, NH = 2 up to 8 (a second set of columns).
// MULTI = false: one tile per wave (tpw = 1), so no running state is carried.
// Band limits: K bands b >= kbands and the V band when vbands == 0 take a zero
// scale (a finite sum times 0 adds exactly nothing, so the scores and outputs
// equal those with the bands read as 0, at the cost of the all-band loop).
template <bool WANT_OUT, int NH, bool MULTI>
__global__ void __launch_bounds__(NT, 1)
k_attn_wave(const SpAttnArgs A, const int *__restrict__ order, float *__restrict__ part, int n_parts, int tpw,
            int kbands, int vbands, int *__restrict__ counters) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[LDS_BYTES];
    const int kvh = blockIdx.x, blk = blockIdx.y, tid = threadIdx.x;
    // the wave index is wave-uniform: a scalar, so the buffer resources and LDS bases built from it are too
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, q4 = lane >> 4, c16 = lane & 15;
    const int G = A.n_q / A.n_kvh, h0 = kvh * G;
    unsigned char *wl = smem + w * R_SIZE;
    unsigned short *qs = reinterpret_cast<unsigned short *>(smem + S_QS);  // [part][head][band][slot] fp16
    float *cb = reinterpret_cast<float *>(smem + S_CB);                    // [head][band]
    float *fu = reinterpret_cast<float *>(smem + S_FU);                    // [head]

    // ---- 1. the waves w >= G issue their first tile's record loads at once;
    // wave w < G prepares head w first: its query row and the order entries of
    // record coefficients lane and lane + 64 ----
    int *ready = reinterpret_cast<int *>(smem + S_FLAG + 4);  // query-operand waves done
    if (tid == 0) *ready = 0;
    __syncthreads();
    const int vshift = WANT_OUT ? (int)((uintptr_t)(A.vpack + (long long)kvh * A.v_head_stride) & 3) : 0;
    const int tile0 = (blk * NW + w) * tpw;  // tile index of the wave's first tile within the KV head
    const int c00 = tile0 * TILE;
    const int n_chunk0 = c00 < A.n_kv ? min(TILE, A.n_kv - c00) : 0;
    TileRegs regs;
    if (w >= G) load_tile<WANT_OUT>(A, kvh, c00, n_chunk0, vshift, lane, regs);
    float qx0 = 0.0f, qx1 = 0.0f;
    int ord0 = lane, ord1 = lane + 64;
    if (w < G) {
        const float *qg = A.q + (long long)(h0 + w) * HD;
        qx0 = qg[lane];
        qx1 = qg[lane + 64];
        // Without an order table, read (and ignore) in-bounds words of q: both
        // candidates are kernel-argument pointers, so these stay global loads.
        const int *op = order ? order : reinterpret_cast<const int *>(A.q);
        const int ov0 = op[lane], ov1 = op[lane + 64];
        ord0 = order ? ov0 : lane;
        ord1 = order ? ov1 : lane + 64;
    }

    // ---- 2. q~ = kq_scale * reorder(VHT2(q)) for head w, in registers (lane
    // holds elements lane and lane + 64), scaled by a power of two fh so its
    // largest entry lies in [2^11, 2^12) and split into fp16 hi + lo, stored in
    // the score MFMA's slot order. Per band, -(2^BITS + m_b) * sum(hi + lo over
    // the band): the accumulator start. ----
    if (w < G) {
        const int h = w;
        float x0 = qx0, x1 = qx1;
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
        float finv;
        const float f = pow2_norm(amax, finv);
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
        const int ba = lane >> 5, bb = 2 + (lane >> 5);  // bands of coefficients lane and lane + 64
        const int sa_ = score_slot(ba, lane & 31), sb_ = score_slot(bb, lane & 31);
        const int ia = 32 * ba + (sa_ & 0xff), ib = 32 * bb + (sb_ & 0xff);
        // a half-gain slot (its code stored as 2^BITS + c/2) holds 2q~: exact in fp16
        const float ga = (sa_ & 0x100) ? 2.0f : 1.0f, gb = (sb_ & 0x100) ? 2.0f : 1.0f;
        const float fha = (float)__builtin_bit_cast(_Float16, (unsigned short)ha), fla = (float)__builtin_bit_cast(_Float16, (unsigned short)la);
        const float fhb = (float)__builtin_bit_cast(_Float16, (unsigned short)hb), flb = (float)__builtin_bit_cast(_Float16, (unsigned short)lb);
        qs[(0 * 8 + h) * QS_STRIDE + ia] = __builtin_bit_cast(unsigned short, (_Float16)(fha * ga));
        qs[(1 * 8 + h) * QS_STRIDE + ia] = __builtin_bit_cast(unsigned short, (_Float16)(fla * ga));
        qs[(0 * 8 + h) * QS_STRIDE + ib] = __builtin_bit_cast(unsigned short, (_Float16)(fhb * gb));
        qs[(1 * 8 + h) * QS_STRIDE + ib] = __builtin_bit_cast(unsigned short, (_Float16)(flb * gb));
        // centring: sum over the band of q~ (offset / gain + m_b), the slot's fp16
        // value being offset + gain * code with offset 2^BITS
        const float wa = ga * (float)(1 << kbits(ba)) + (float)((1 << (kbits(ba) - 1)) - 1);
        const float wb = gb * (float)(1 << kbits(bb)) + (float)((1 << (kbits(bb) - 1)) - 1);
        float sa = (fha + fla) * wa;
        float sb = (fhb + flb) * wb;
        sa = wave_sum_step<1>(sa); sb = wave_sum_step<1>(sb);
        sa = wave_sum_step<2>(sa); sb = wave_sum_step<2>(sb);
        sa = wave_sum_step<4>(sa); sb = wave_sum_step<4>(sb);
        sa = wave_sum_step<8>(sa); sb = wave_sum_step<8>(sb);
        sa = wave_sum_step<16>(sa); sb = wave_sum_step<16>(sb);
        if ((lane & 31) == 0) {
            cb[h * 4 + ba] = -sa;
            cb[h * 4 + bb] = -sb;
        }
        if (lane == 0) fu[h] = finv;
        // publish: this wave's LDS writes are complete before it counts itself
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) __hip_atomic_fetch_add(ready, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }

    // ---- 3. the preparing waves' first tile. No block barrier here: each wave
    // checks `ready` just before its first query read ----
    if (w < G) load_tile<WANT_OUT>(A, kvh, c00, n_chunk0, vshift, lane, regs);
    // score rows 16-byte aligned at every tile: one 16-byte non-temporal store per lane
    const bool sc_vec = ((uintptr_t)A.scores & 15) == 0 && (A.n_kv & 3) == 0;

    // code-slot masks and the fp16 2^BITS exponent bits, kept in registers for bitop3
    const uint32_t kbias5 = __builtin_amdgcn_readfirstlane(code_bias<5>());
    const uint32_t kbias4 = __builtin_amdgcn_readfirstlane(code_bias<4>());
    const uint32_t kbias3 = __builtin_amdgcn_readfirstlane(code_bias<3>());
    const uint32_t vbias = __builtin_amdgcn_readfirstlane(VBIAS);
    uint32_t kmask5 = code_mask<5>(), kmask4 = code_mask<4>(), kmask3 = code_mask<3>(), vmask = VMASK;
    uint32_t kmask5p = 0x01F003E0u, kmask3p = 0x01C00380u;  // 15-bit pairs: bits 5..9 + 20..24, 7..9 + 22..24
    __asm__("" : "+v"(kmask5), "+v"(kmask4), "+v"(kmask3), "+v"(vmask), "+v"(kmask5p), "+v"(kmask3p));

    // running state of this lane's value heads 2*q4 + hh over the wave's tiles
    float om[2] = {-INFINITY, -INFINITY}, ol[2] = {0.0f, 0.0f};
    float oo[2][8];
#pragma unroll
    for (int hh = 0; hh < 2; hh++)
#pragma unroll
        for (int j = 0; j < 8; j++) oo[hh][j] = 0.0f;

    for (int it = 0; it < (MULTI ? tpw : 1); it++) {
        const int c0 = (tile0 + it) * TILE;
        if (c0 >= A.n_kv) break;  // wave-uniform
        const int n_chunk = min(TILE, A.n_kv - c0);
        // LDS addresses below derive from an opaque per-tile copy of the lane
        // index: loop-invariant, they would otherwise be hoisted out of the tile
        // loop and held (or spilled) through it.
        int ln = lane;
        __asm__ volatile("" : "+v"(ln));
        const int c16i = ln & 15, q4i = ln >> 4, hj = ln & 3, qd = ln >> 2;
        if (it > 0) load_tile<WANT_OUT>(A, kvh, c0, n_chunk, vshift, lane, regs);
        __asm__ volatile("" ::: "memory");  // the previous tile's LDS reads are issued before the new records land
        stage_tile<WANT_OUT>(wl, regs, lane);
        __asm__ volatile("" ::: "memory");
        // ---- lane t takes record t of the K tile into registers, and the scale of its V record ----
        uint32_t r[20];
        {
            const uint32_t *kr = reinterpret_cast<const uint32_t *>(wl + R_K + ln * KB);
#pragma unroll
            for (int m = 0; m < 19; m++) r[m] = kr[m];
            r[19] = 0;
        }
        float sv_own = 0.0f;
        if (WANT_OUT)
            // (a lane past the tile's end takes whatever scale lies there: its weight is p = 0)
            sv_own = vbands > 0
                         ? scale_of(*reinterpret_cast<const unsigned short *>(wl + R_V + vshift + ln * VB))
                         : 0.0f;
        __asm__ volatile("" ::: "memory");  // every lane has read its record before the K area is reused

        // ---- the query operand is in LDS once the G preparing waves have counted
        // themselves (each sets the count once, unconditionally, so this ends) ----
        if (it == 0) {
            while (__hip_atomic_load(ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < G) __builtin_amdgcn_s_sleep(1);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        }
        // ---- scores: accumulator (set, band) starts at the band's centring ----
        float4_t acc[NH][4];
#pragma unroll
        for (int st = 0; st < NH; st++) {
            const float4 c4 = *reinterpret_cast<const float4 *>(cb + (4 * st + hj) * 4);
            const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
            for (int b = 0; b < 4; b++) acc[st][b] = float4_t{cv[b], cv[b], cv[b], cv[b]};
        }
#pragma unroll
        for (int s = 0; s < 8; s++) {  // step s of every band: slots 4s .. 4s+3
            half4_t a[4];
#pragma unroll
            for (int b = 0; b < 4; b++) {
                a[b] = score_codes(r, b, s, kmask5, kbias5, kmask4, kbias4, kmask3, kbias3, kmask5p, kmask3p);
            }
#pragma unroll
            for (int st = 0; st < NH; st++)
#pragma unroll
                for (int part = 0; part < 2; part++)
#pragma unroll
                    for (int b = 0; b < 4; b++) {
                        const half4_t qv = __builtin_bit_cast(
                            half4_t, *reinterpret_cast<const u32x2 *>(qs + (part * 8 + 4 * st + hj) * QS_STRIDE + 32 * b + 4 * s));
                        acc[st][b] = __builtin_amdgcn_mfma_f32_4x4x4f16(a[b], qv, acc[st][b], 0, 0, 0);
                    }
        }
        // band scales of the lane's own record; position 4*qd + i's come from quad lane i
        // (a lane past the tile's end holds a zero record: scale 0)
        float ks[4];
#pragma unroll
        for (int b = 0; b < 4; b++)
            ks[b] = b < kbands ? scale_of(rec_bits(r, 8 * kbyte(b), 16)) : 0.0f;
        float sc[NH][4];
#pragma unroll
        for (int st = 0; st < NH; st++) {
            const float un = fu[4 * st + hj];
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const float s0 = quad_bcast<0>(ks[b]), s1 = quad_bcast<1>(ks[b]);
                const float s2 = quad_bcast<2>(ks[b]), s3 = quad_bcast<3>(ks[b]);
                if (b == 0) {
                    sc[st][0] = s0 * acc[st][b][0];
                    sc[st][1] = s1 * acc[st][b][1];
                    sc[st][2] = s2 * acc[st][b][2];
                    sc[st][3] = s3 * acc[st][b][3];
                } else {
                    sc[st][0] = fmaf(s0, acc[st][b][0], sc[st][0]);
                    sc[st][1] = fmaf(s1, acc[st][b][1], sc[st][1]);
                    sc[st][2] = fmaf(s2, acc[st][b][2], sc[st][2]);
                    sc[st][3] = fmaf(s3, acc[st][b][3], sc[st][3]);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++) sc[st][i] *= un;
            if (A.scores && 4 * st + hj < G) {
                float *dst = A.scores + (long long)(h0 + 4 * st + hj) * A.n_kv + c0 + 4 * qd;
                if (n_chunk == TILE && sc_vec) {
                    __builtin_nontemporal_store(float4_t{sc[st][0], sc[st][1], sc[st][2], sc[st][3]}, reinterpret_cast<float4_t *>(dst));
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (4 * qd + i < n_chunk) dst[i] = sc[st][i];
                }
            }
        }
        if (!WANT_OUT) continue;

        // ---- softmax over the tile, lane (quad qd, head hj) holding positions 4*qd + i;
        // weights w = p * scale_v as fp16 hi / lo rows 2h / 2h + 1 (slot = position) ----
        unsigned short *wt = reinterpret_cast<unsigned short *>(wl + R_WT);
        float *stt = reinterpret_cast<float *>(wl + R_ST);
        const float sv[4] = {quad_bcast<0>(sv_own), quad_bcast<1>(sv_own), quad_bcast<2>(sv_own), quad_bcast<3>(sv_own)};
#pragma unroll
        for (int st = 0; st < NH; st++) {
            float v[4] = {sc[st][0], sc[st][1], sc[st][2], sc[st][3]};
            if (n_chunk < TILE) {  // positions past the tile's end take no weight
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = 4 * qd + i < n_chunk ? v[i] : -INFINITY;
            }
            float m = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
            m = head_max(m);  // finite: the tile holds at least one position
            float l = 0.0f, wm = 0.0f, wv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float p = __expf(v[i] - m);
                l = i == 0 ? p : l + p;
                wv[i] = p * sv[i];
                wm = fmaxf(wm, wv[i]);
            }
            wm = head_max(wm);
            float finv;
            const float f = pow2_norm(wm, finv);
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                // lo part scaled by 2^11 (exact) so it stays a normal fp16 value
                const float x = wv[i] * f;
                const _Float16 hv = (_Float16)x;
                hi[i] = (uint32_t)__builtin_bit_cast(unsigned short, hv);
                lo[i] = (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)((x - (float)hv) * 2048.0f));
            }
            const int row = 2 * (4 * st + hj);
            *reinterpret_cast<u32x2 *>(wt + row * WT_STRIDE + 4 * qd) = u32x2{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16)};
            *reinterpret_cast<u32x2 *>(wt + (row + 1) * WT_STRIDE + 4 * qd) = u32x2{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
            l = head_sum(l);
            if (qd == 0) *reinterpret_cast<float4 *>(stt + 4 * (4 * st + hj)) = float4{m, l, finv, 0.0f};
        }
        __asm__ volatile("" ::: "memory");

        // ---- values: D[(h, part)][n] over K slots 32k + 8*q4 + e (positions
        // 32k + 8*q4 + e); B column n = element 8n + j of MFMA j ----
        float4_t vacc[8];
#pragma unroll
        for (int j = 0; j < 8; j++) vacc[j] = float4_t{0.f, 0.f, 0.f, 0.f};
        // lane (c16, q4)'s window of position t starts at byte vshift + 50t + 2 + 3*c16 of
        // the V region; its positions 32k + 8*q4 + e keep one alignment for even e and
        // one for odd e (steps of 100 and 1600 bytes), so each has a dword-aligned base
        // and a shift
        const int xw0 = vshift + (8 * q4i) * VB + 2 + 3 * c16i, xw1 = xw0 + VB;
        const unsigned char *vb0 = wl + R_V + (xw0 & ~3), *vb1 = wl + R_V + (xw1 & ~3);
        const uint32_t vsh0 = (uint32_t)(xw0 & 3) * 8u, vsh1 = (uint32_t)(xw1 & 3) * 8u;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const half8_t a =
                __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4 *>(wt + c16i * WT_STRIDE + 32 * k + 8 * q4i));
            // K slot pair p (slots 2p, 2p + 1): both positions' bytes 0,1 (pa) and 1,2 (pb)
            uint32_t pa[4], pb[4];
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const uint32_t we = v_window(vb0 + 32 * k * VB + 2 * p * VB, vsh0);
                const uint32_t wo = v_window(vb1 + 32 * k * VB + 2 * p * VB, vsh1);
                pa[p] = __builtin_amdgcn_perm(wo, we, 0x05040100u);
                pb[p] = __builtin_amdgcn_perm(wo, we, 0x06050201u);
            }
#define SP_V_MFMA(J)                                                                                              \
    vacc[J] = __builtin_amdgcn_mfma_f32_16x16x32_f16(                                                             \
        a,                                                                                                        \
        __builtin_bit_cast(half8_t, u32x4{v_pair<J>(pa[0], pb[0], vmask, vbias), v_pair<J>(pa[1], pb[1], vmask, vbias), \
                                          v_pair<J>(pa[2], pb[2], vmask, vbias), v_pair<J>(pa[3], pb[3], vmask, vbias)}), \
        vacc[J], 0, 0, 0)
            SP_V_MFMA(0);
            SP_V_MFMA(1);
            SP_V_MFMA(2);
            SP_V_MFMA(3);
            SP_V_MFMA(4);
            SP_V_MFMA(5);
            SP_V_MFMA(6);
            SP_V_MFMA(7);
#undef SP_V_MFMA
        }
        // ---- fold the tile into the running state: D rows 4*q4 + 2hh (+1) are
        // head 2*q4 + hh's hi (lo) weights; o~[8*c16 + j] = sum p * scale_v * (u - 3) ----
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const float4 t4 = *reinterpret_cast<const float4 *>(stt + 4 * (2 * q4i + hh));  // m, l, 1/f of the head
            float o[8];
#pragma unroll
            for (int j = 0; j < 8; j++) o[j] = fmaf(vacc[j][2 * hh + 1], 1.0f / 2048.0f, vacc[j][2 * hh]) * t4.z;
            if (!MULTI || it == 0) {
#pragma unroll
                for (int j = 0; j < 8; j++) oo[hh][j] = o[j];
                ol[hh] = t4.y;
                om[hh] = t4.x;
            } else {
                const float mx = fmaxf(om[hh], t4.x);
                const float ea = __expf(om[hh] - mx), eb = __expf(t4.x - mx);
#pragma unroll
                for (int j = 0; j < 8; j++) oo[hh][j] = fmaf(oo[hh][j], ea, o[j] * eb);
                ol[hh] = fmaf(ol[hh], ea, t4.y * eb);
                om[hh] = mx;
            }
        }
        __asm__ volatile("" ::: "memory");  // this tile's LDS reads are issued before the next tile is staged
    }
    if (!WANT_OUT) return;

    // ---- merge the block's waves: record (wave, head) = [m, l, -, -, o~[128]] ----
    __syncthreads();  // every wave is done with its LDS region
    float *mb = reinterpret_cast<float *>(smem);
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const int h = 2 * q4 + hh;
        if (h < G) {
            float *rec = mb + (w * 8 + h) * MB_STRIDE;
            *reinterpret_cast<float4 *>(rec + 4 + 8 * c16) = float4{oo[hh][0], oo[hh][1], oo[hh][2], oo[hh][3]};
            *reinterpret_cast<float4 *>(rec + 8 + 8 * c16) = float4{oo[hh][4], oo[hh][5], oo[hh][6], oo[hh][7]};
            if (c16 == 0) {
                rec[0] = om[hh];
                rec[1] = ol[hh];
            }
        }
    }
    __syncthreads();
    if (tid < G * HD) {
        const int h = tid >> 7, i = tid & (HD - 1);
        float M = -INFINITY;
#pragma unroll
        for (int v = 0; v < NW; v++) M = fmaxf(M, mb[(v * 8 + h) * MB_STRIDE]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int v = 0; v < NW; v++) {
            const float *rec = mb + (v * 8 + h) * MB_STRIDE;
            const float e = __expf(rec[0] - M);  // a wave without tiles: m = -inf, e = 0
            L = fmaf(rec[1], e, L);
            O = fmaf(rec[4 + i], e, O);
        }
        // agent-scope atomic stores: written through to where every CU's
        // agent-scope loads read, with no cache writeback needed before the count
        float *dst = part + ((long long)(h0 + h) * n_parts + blk) * (HD + 2);
        __hip_atomic_store(dst + 2 + i, O, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (i == 0) {
            __hip_atomic_store(dst, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(dst + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // ---- the last block of the KV head to arrive merges every block's partial:
    // each block's stores have completed before it counts itself ----
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    int *flag = reinterpret_cast<int *>(smem + S_FLAG);
    if (tid == 0) {
        int *cnt = counters + kvh * SP_ATTN_COUNTER_STRIDE;
        const int arrived = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = arrived == n_parts - 1;
        if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // ready for the next call
        *flag = last;
    }
    __syncthreads();
    if (!*flag) return;
    // Two halves of the block (G <= 4) take half the partials each: thread
    // (half, h, i) loads o~[i] of its partials, and lane k of each 16-lane row
    // the m and l of partial p0 + k, shared across the row (one m, l load per
    // partial and lane instead of one per element)
    float *vec = reinterpret_cast<float *>(smem);   // [G][HD] merged o~ / L
    float *xo = vec + 8 * HD;                       // second half's o~ [G][HD]
    float *xml = xo + 8 * HD;                       // second half's (M, L) [G][2]
    const int GH = G * HD, halves = 2 * GH <= NT ? 2 : 1;
    const int half = tid >= GH ? 1 : 0, r = tid - half * GH, h = r >> 7, i = r & (HD - 1);
    const int per = (n_parts + halves - 1) / halves, pb = half * per, pe = min(n_parts, pb + per);
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    if (tid < halves * GH) {
        const float *src = part + (long long)(h0 + h) * n_parts * (HD + 2);
        for (int p0 = pb; p0 < pe; p0 += 16) {
            const int pk = min(p0 + (lane & 15), pe - 1);
            const float mk0 = __hip_atomic_load(src + (long long)pk * (HD + 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float lk = __hip_atomic_load(src + (long long)pk * (HD + 2) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            float po[16];
#pragma unroll
            for (int k = 0; k < 16; k++)
                po[k] = __hip_atomic_load(src + (long long)min(p0 + k, pe - 1) * (HD + 2) + 2 + i, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
            const float mk = p0 + (lane & 15) < pe ? mk0 : -INFINITY;  // a repeated last partial counts once
            float cm = mk;
            cm = wave_max_step<1>(cm);
            cm = wave_max_step<2>(cm);
            cm = wave_max_step<4>(cm);
            cm = wave_max_step<8>(cm);
            cm = fmaxf(cm, M);
            const float ek = mk == -INFINITY ? 0.0f : __expf(mk - cm);
            float ls = lk * ek;
            ls = wave_sum_step<1>(ls);
            ls = wave_sum_step<2>(ls);
            ls = wave_sum_step<4>(ls);
            ls = wave_sum_step<8>(ls);
            const float a = M == -INFINITY ? 0.0f : __expf(M - cm);  // rescale of the running sums
            L = fmaf(L, a, ls);
            O *= a;
#pragma unroll
            for (int k = 0; k < 16; k++)
                O = fmaf(po[k], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ek), k)), O);
            M = cm;
        }
    }
    if (halves == 2 && half == 1) {
        xo[r] = O;
        if (i == 0) {
            xml[2 * h] = M;
            xml[2 * h + 1] = L;
        }
    }
    __syncthreads();
    if (tid < GH) {
        if (halves == 2) {
            const float m2 = xml[2 * h], l2 = xml[2 * h + 1], o2 = xo[r];
            const float cm = fmaxf(M, m2);
            const float a = M == -INFINITY ? 0.0f : __expf(M - cm), b = m2 == -INFINITY ? 0.0f : __expf(m2 - cm);
            L = fmaf(L, a, l2 * b);
            O = fmaf(O, a, o2 * b);
        }
        vec[r] = O / L;
    }
    __syncthreads();
    // ---- one inverse VHT2 per query head: wave h, lane holds elements lane and lane + 64 ----
    if (w < G) {
        float x0 = vec[w * HD + lane], x1 = vec[w * HD + lane + 64];
        x0 = lane_butterfly<1>(x0, lane);   x1 = lane_butterfly<1>(x1, lane);
        x0 = lane_butterfly<2>(x0, lane);   x1 = lane_butterfly<2>(x1, lane);
        x0 = lane_butterfly<4>(x0, lane);   x1 = lane_butterfly<4>(x1, lane);
        x0 = lane_butterfly<8>(x0, lane);   x1 = lane_butterfly<8>(x1, lane);
        x0 = lane_butterfly<16>(x0, lane);  x1 = lane_butterfly<16>(x1, lane);
        x0 = lane_butterfly<32>(x0, lane);  x1 = lane_butterfly<32>(x1, lane);
        float *o = A.out + (long long)(h0 + w) * HD;
        o[lane] = (x0 + x1) * INV_SQRT_HD;
        o[lane + 64] = (x0 - x1) * INV_SQRT_HD;
    }
}

// Compute units of the current device (cached per device).
static int wave_device_cus() {
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

template <int NH, bool MULTI>
static void launch_wave(const SpAttnArgs &A, const int *order, float *part, int nb, int tpw, int kb_lim, int vb_lim,
                        int *cnt, hipStream_t s) {
    const dim3 grid(A.n_kvh, nb);
    if (A.out) hipLaunchKernelGGL((k_attn_wave<true, NH, MULTI>), grid, dim3(NT), 0, s, A, order, part, nb, tpw, kb_lim, vb_lim, cnt);
    else hipLaunchKernelGGL((k_attn_wave<false, NH, MULTI>), grid, dim3(NT), 0, s, A, order, part, nb, tpw, kb_lim, vb_lim, cnt);
}

hipError_t sp_launch_attn_wave(const SpPlan &KP, const SpPlan &VP, const int *order, const SpAttnArgs &A, float *part,
                               size_t part_floats, int *counters, hipStream_t s) {
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
    if (A.n_q % A.n_kvh || A.n_q / A.n_kvh > 8 || A.n_kvh > SP_ATTN_MAX_KVH) return hipErrorNotSupported;
    if (((uintptr_t)A.kpack % 4) || ((uintptr_t)A.vpack % 2) || (A.k_head_stride % 4) || (A.v_head_stride % 2))
        return hipErrorNotSupported;
    // Tiles per wave: one round of blocks (one per CU) when the context allows.
    const long long n_tiles = (A.n_kv + TILE - 1) / TILE;
    const long long waves = (long long)wave_device_cus() * NW;
    int tpw = (int)std::max(1LL, ((long long)A.n_kvh * n_tiles + waves - 1) / waves);
    tpw = (int)std::max<long long>(tpw, (n_tiles + (long long)NW * MAX_PARTS - 1) / ((long long)NW * MAX_PARTS));
    const int nb = (int)((n_tiles + (long long)NW * tpw - 1) / ((long long)NW * tpw));
    if (!part || !counters || (size_t)A.n_q * nb * (HD + 2) > part_floats) return hipErrorInvalidValue;
    const bool multi = tpw > 1;
    if (A.n_q / A.n_kvh <= 4) {
        if (multi) launch_wave<1, true>(A, order, part, nb, tpw, KP.max_bands, VP.max_bands, counters, s);
        else launch_wave<1, false>(A, order, part, nb, tpw, KP.max_bands, VP.max_bands, counters, s);
    } else {
        if (multi) launch_wave<2, true>(A, order, part, nb, tpw, KP.max_bands, VP.max_bands, counters, s);
        else launch_wave<2, false>(A, order, part, nb, tpw, KP.max_bands, VP.max_bands, counters, s);
    }
    return hipGetLastError();
}
