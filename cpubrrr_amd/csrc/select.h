// select.h -- top-k expert selection from certified router logits (one
// wavefront, LDS scratch, no cross-workgroup synchronisation).
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

// Executed by one wavefront (64 lanes).  lds: 4*NE doubles + d floats of
// scratch (the floats only for the exact fallback).
// Lane l holds experts l, l+64, ... (NE <= 256) in registers; the top-k come
// from k rounds of wave-wide argmax (cross-lane shuffles, no LDS round
// trips), the certification from one wave-wide max.  logits_out (optional)
// receives the fp32 value of every expert's exact logit.  Outputs ids / logit
// / wts in rank order into `out` (valid in every lane after the call).
CPB_DEV void select_experts_wave(const double* __restrict__ Ls, const double* __restrict__ Bs, int NE, int K,
                                 const float* __restrict__ router_w, const float* __restrict__ router_b,
                                 const float* __restrict__ xn, int d, double* lds, Selection* out,
                                 float* logits_out = nullptr, unsigned long long* stamps = nullptr) {
#ifdef CPB_DECODE_STAMPS
#define SSTAMP(i) do { if (stamps && (threadIdx.x & 63) == 0) stamps[i] = wall_clock64(); } while (0)
#else
#define SSTAMP(i) do { (void)stamps; } while (0)
#endif
    const int lane = threadIdx.x & 63;
    double* sL = lds;            // [NE] values used for ranking
    double* sH = lds + NE;       // [NE] upper bounds
    int* sSel = (int*)(lds + 3 * NE);        // [8] expert at rank i
    // one coherent round trip for all values
    double lv[4], bv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int e = lane + 64 * k;
        lv[k] = e < NE ? ld_dev(Ls + e) : 0.0;
        bv[k] = e < NE ? ld_dev(Bs + e) : 0.0;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int e = lane + 64 * k;
        if (e < NE) {
            sL[e] = lv[k];
            sH[e] = lv[k] + bv[k];
            if (logits_out) logits_out[e] = (float)lv[k];
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    SSTAMP(0);
    // K rounds of wave-wide argmax over the register values: descending,
    // lowest index first among equal values (the reference's strict insertion)
    unsigned taken = 0;                    // bit k: expert lane + 64k already selected
    for (int i = 0; i < K; i++) {
        double best = -__builtin_inf();
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (lane + 64 * k < NE && !((taken >> k) & 1u)) best = fmax(best, lv[k]);
        best = wave_max_f64(best);
        int bi = 0x7fffffff;
#pragma unroll
        for (int k = 3; k >= 0; k--) {
            const uint64_t m = __ballot(lane + 64 * k < NE && !((taken >> k) & 1u) && lv[k] == best);
            if (m) bi = 64 * k + __builtin_ctzll(m);
        }
        if (lane == 0) sSel[i] = bi;
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    }
    SSTAMP(1);
    // certification: the expert at rank r < K must lie strictly above every
    // expert ranked after it, i.e. lo_r > max(hi of ranks r+1..K-1, hi of
    // every unselected expert)
    double mu = -1e300;
#pragma unroll
    for (int k = 0; k < 4; k++)
        if (lane + 64 * k < NE && !((taken >> k) & 1u)) mu = fmax(mu, lv[k] + bv[k]);
    mu = wave_max_f64(mu);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    bool bad = false;
    {
        double suffix = mu;
        for (int i = K - 1; i >= 0; i--) {
            const int e = __builtin_amdgcn_readfirstlane(sSel[i]);
            const int src = e & 63, kk = e >> 6;
            const double l = readlane_f64(kk == 0 ? lv[0] : kk == 1 ? lv[1] : kk == 2 ? lv[2] : lv[3], src);
            const double b = readlane_f64(kk == 0 ? bv[0] : kk == 1 ? bv[1] : kk == 2 ? bv[2] : bv[3], src);
            if (!(l - b > suffix)) bad = true;
            suffix = fmax(suffix, l + b);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const bool ok = !__any(bad);
    SSTAMP(2);
    if (!ok) {
        // candidates: intervals reaching the lowest lower bound of the selected
        double tau = 1e300;
        for (int i = 0; i < K; i++) { const int e = sSel[i]; tau = fmin(tau, sL[e] - (sH[e] - sL[e])); }
        __builtin_amdgcn_wave_barrier();
        // xn staged in LDS with coherent 16-byte loads (it may have been written
        // by other workgroups of this launch), then each candidate lane runs the
        // reference's serial chain with its router row fetched 64 weights ahead
        float* xst = (float*)(lds + 4 * NE);
        {
            const __amdgpu_buffer_rsrc_t r = buf_rsrc(xn, (uint32_t)d * 4);
            for (int i = lane; i < d / 4; i += 64) ((u32x4*)xst)[i] = ld_dev16(r, (uint32_t)i * 16);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int e = lane; e < NE; e += 64) {
            double v = -1e300;
            if (sH[e] >= tau) {
                float acc = router_b ? router_b[e] : 0.0f;
                const float* Wr = router_w + (size_t)e * d;
                float4 w4[16], n4[16];
#pragma unroll
                for (int u = 0; u < 16; u++) w4[u] = 4 * u < d ? *(const float4*)(Wr + 4 * u) : float4{0, 0, 0, 0};
                for (int j0 = 0; j0 < d; j0 += 64) {
                    // next chunk requested before this one is consumed
#pragma unroll
                    for (int u = 0; u < 16; u++)
                        n4[u] = j0 + 64 + 4 * u < d ? *(const float4*)(Wr + j0 + 64 + 4 * u) : float4{0, 0, 0, 0};
#pragma unroll
                    for (int u = 0; u < 16; u++) {
                        if (j0 + 4 * u >= d) break;
                        const float* w = (const float*)&w4[u];
#pragma unroll
                        for (int c = 0; c < 4; c++) acc = __fadd_rn(acc, __fmul_rn(w[c], xst[j0 + 4 * u + c]));
                    }
#pragma unroll
                    for (int u = 0; u < 16; u++) w4[u] = n4[u];
                }
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
    SSTAMP(3);
    // softmax over the k selected, reference order: ex_i = exp(l_i - l_0)
    // (lane i), then the serial sum ex_0 + ex_1 + ... (every lane)
    const int mi = lane < K ? lane : 0;
    const int me = sSel[mi];
    const float ml = (float)sL[me];
    const float l0 = (float)sL[sSel[0]];
    const float ex = expf(ml - l0);
    float wsum = 0.0f;
    for (int i = 0; i < K; i++) wsum += __shfl(ex, i);
    const float wt = ex / wsum;
    if (lane < K) {
        out->ids[lane] = me;
        out->logit[lane] = ml;
        out->wts[lane] = wt;
    }
    if (lane == 0) out->fallback = ok ? 0 : 1;
    SSTAMP(4);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace cpb
