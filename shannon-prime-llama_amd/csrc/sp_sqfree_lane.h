// sp_sqfree_lane.h -- compile-time pieces of the one-vector-per-lane sqfree
// kernels shared by the codec (sp_sqfree_lane.hip) and the fused attention
// (sp_sqfree_attn.hip): the Knight mask as a compile-time table, the record
// layout, and the CSR Mobius prediction.
#pragma once
#include "sp_lane.h"

namespace {

constexpr int c_mu(int n) {
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

// Knight mask (the host's build_knight rule): skeleton = first SK entries of the
// squarefree-first order over [0, PAD), residuals = the rest in that order; the
// CSR terms of residual coefficient c (n = c + 1) are the proper divisors d of n
// whose coefficient d - 1 is in the skeleton and mu(n/d) != 0, with sign mu(n/d).
template <int PAD, int SK>
struct Knight {
    static constexpr int NR = PAD - SK, MAXT = PAD * 16;
    int skel[SK];
    int res[NR > 0 ? NR : 1];
    int off[NR + 1];
    int slot[MAXT];
    int mu[MAXT];
    int n_terms;
    constexpr Knight() : skel(), res(), off(), slot(), mu(), n_terms(0) {
        const MobOrder<PAD> mo{};
        int slot_of[PAD] = {};
        for (int i = 0; i < PAD; i++) slot_of[i] = -1;
        for (int s = 0; s < SK; s++) {
            skel[s] = mo.v[s];
            slot_of[mo.v[s]] = s;
        }
        for (int r = 0; r < NR; r++) res[r] = mo.v[SK + r];
        off[0] = 0;
        for (int r = 0; r < NR; r++) {
            const int n = res[r] + 1;
            for (int d = 1; d < n; d++) {
                if (n % d) continue;
                const int m = c_mu(n / d);
                if (m == 0 || slot_of[d - 1] < 0) continue;
                slot[n_terms] = slot_of[d - 1];
                mu[n_terms] = m;
                n_terms++;
            }
            off[r + 1] = n_terms;
        }
    }
};
template <int PAD, int SK>
__device__ constexpr Knight<PAD, SK> kKnight{};

// Record [skeleton bands][mag f32 LE][residual levels][sheet bits]
// (shannon_prime_sqfree.cu:683-686).
template <int PAD, int SK, int RBITS, bool SPIN, class SL>
struct SqRec {
    static constexpr int NR = PAD - SK;
    static constexpr int mag_byte = SL::total;
    static constexpr int res_bit = 8 * (SL::total + 4);
    static constexpr int res_bytes = (NR * RBITS + 7) / 8;
    static constexpr int sheet_bit = 8 * (SL::total + 4 + res_bytes);
    static constexpr int total = SL::total + 4 + res_bytes + (SPIN ? (NR + 7) / 8 : 0);
    static constexpr int dwords = (total + 3) / 4;
};

// pred[r] = sum over the CSR row of mu * skel[slot], from 0.0f in CSR order
// (kernel_mobius_predict, shannon_prime_sqfree.cu:179-203); mu = +-1, so each
// term is +-skel exactly and p + (-s) is p - s.
template <int PAD, int SK>
__device__ __forceinline__ float csr_predict(const float (&sk)[SK], int r) {
    constexpr auto &KN = kKnight<PAD, SK>;
    float p = 0.0f;
#pragma unroll
    for (int j = KN.off[r]; j < KN.off[r + 1]; j++) p = KN.mu[j] > 0 ? p + sk[KN.slot[j]] : p - sk[KN.slot[j]];
    return p;
}

}  // namespace
