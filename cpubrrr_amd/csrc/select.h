// select.h -- top-k expert selection from certified router logits (one
// wavefront, no LDS, no cross-workgroup synchronisation).
//
// Inputs per expert e: Ls[e] = exact (fp64) sum of the reference's fp32
// router products plus bias, Bs[e] = bound on |reference serial fp32 sum -
// Ls[e]| (k_route).  The reference selects by descending value with the
// lowest index winning ties (engine_gpt2.rs:852-867 insertion with strict
// comparisons; engine_qwen2.rs:403-410 stable sort), then takes a softmax
// over the k selected logits.  If every selected expert's interval lies
// strictly above the intervals of all experts ranked after it, the choice
// and its order are the reference's for any values inside the bounds.
// Otherwise the candidates that could reach the top-k are recomputed in the
// reference's serial order (acc = b; acc += W[j]*xn[j]) and selected exactly.
#pragma once
#include "moe_common.h"

namespace cpb {

struct Selection {
    int ids[8];
    float logit[8];     // fp32 logits of the selected experts, in rank order
    float wts[8];       // softmax over them (reference order of operations)
    int fallback;       // 1 when the exact serial logits were needed
};

// Executed by one wavefront (64 lanes).  lds: 4*NE doubles of scratch.
// Lane l handles experts l, l+64, ...: rank_e = #{j : L_j > L_e or
// (L_j == L_e and j < e)} from LDS broadcast reads, so every expert is ranked
// in one pass with no dependent cross-lane steps.  Outputs ids/logit/wts in
// rank order (written by lane 0 into `out`).
CPB_DEV void select_experts_wave(const double* __restrict__ Ls, const double* __restrict__ Bs, int NE, int K,
                                 const float* __restrict__ router_w, const float* __restrict__ router_b,
                                 const float* __restrict__ xn, int d, double* lds, Selection* out) {
    const int lane = threadIdx.x & 63;
    double* sL = lds;            // [NE] values used for ranking
    double* sH = lds + NE;       // [NE] upper bounds
    int* sR = (int*)(lds + 2 * NE);          // [NE] ranks
    int* sSel = (int*)(lds + 3 * NE);        // [8] expert at rank i
    for (int e = lane; e < NE; e += 64) { const double l = ld_dev(Ls + e); sL[e] = l; sH[e] = l + ld_dev(Bs + e); }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int e = lane; e < NE; e += 64) {
        const double v = sL[e];
        int r = 0;
#pragma unroll 16
        for (int j = 0; j < NE; j++) { const double o = sL[j]; r += (o > v) || (o == v && j < e); }
        sR[e] = r;
        if (r < K) sSel[r] = e;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // certification: the expert at rank r < K must lie strictly above every
    // expert ranked after it
    bool bad = false;
    for (int e = lane; e < NE; e += 64) {
        const int r = sR[e];
        if (r < K) {
            const double lo = sL[e] - (sH[e] - sL[e]);
#pragma unroll 16
            for (int j = 0; j < NE; j++) bad |= (sR[j] > r) & (sH[j] >= lo);
        }
    }
    const bool ok = !__any(bad);
    if (!ok) {
        // candidates: intervals reaching the lowest lower bound of the selected
        double tau = 1e300;
        for (int i = 0; i < K; i++) { const int e = sSel[i]; tau = fmin(tau, sL[e] - (sH[e] - sL[e])); }
        __builtin_amdgcn_wave_barrier();
        for (int e = lane; e < NE; e += 64) {
            double v = -1e300;
            if (sH[e] >= tau) {
                float acc = router_b ? router_b[e] : 0.0f;
                const float* Wr = router_w + (size_t)e * d;
                for (int j = 0; j < d; j++) acc = __fadd_rn(acc, __fmul_rn(Wr[j], ld_dev(xn + j)));
                v = (double)acc;
            }
            sL[e] = v;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int e = lane; e < NE; e += 64) {
            const double v = sL[e];
            int r = 0;
            for (int j = 0; j < NE; j++) { const double o = sL[j]; r += (o > v) || (o == v && j < e); }
            if (r < K) sSel[r] = e;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (lane == 0) {
        // softmax over the k selected, reference order: ex_i = exp(l_i - l_0), serial sum
        float e8[8], wsum = 0.0f;
        for (int i = 0; i < K; i++) { out->ids[i] = sSel[i]; out->logit[i] = (float)sL[sSel[i]]; }
        for (int i = 0; i < K; i++) { e8[i] = expf(out->logit[i] - out->logit[0]); wsum += e8[i]; }
        for (int i = 0; i < K; i++) out->wts[i] = e8[i] / wsum;
        out->fallback = ok ? 0 : 1;
    }
}

}  // namespace cpb
