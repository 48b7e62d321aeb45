// select.h -- top-k expert selection from certified router logits (one
// wavefront, registers; LDS only on the exact path).
//
// Inputs per expert e: Ls[e] = fp64 logit, Bs[e] = bound on |reference serial
// fp32 logit - Ls[e]| (k_route).  The reference selects by descending value with the
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

// candidates whose exact serial logits are computed side by side: four in
// the decode kernels (their LDS budget), eight in the batched selection
constexpr int kExactGroup = 4;
constexpr int kExactGroupWide = 8;
CPB_DEV_HOST_INLINE constexpr int exact_group(int cand) { return cand > 1 ? kExactGroupWide : kExactGroup; }
// LDS floats per candidate's product row: d plus the chain's look-ahead slack
// (64 floats), a multiple of 4 (16-byte reads) that spreads the chain lanes
// over the banks
CPB_DEV_HOST_INLINE int exact_stride(int d) { return d + 68; }
// acc += v in order, 32 products, fp32 round to nearest (the reference's
// serial chain)
CPB_DEV float serial_add32(const f32x4 (&v)[8], float acc) {
#pragma unroll
    for (int u = 0; u < 8; u++) {
        acc = __fadd_rn(acc, v[u][0]);
        acc = __fadd_rn(acc, v[u][1]);
        acc = __fadd_rn(acc, v[u][2]);
        acc = __fadd_rn(acc, v[u][3]);
    }
    return acc;
}

struct Selection {
    int ids[8];
    float logit[8];     // fp32 logits of the selected experts, in rank order
    float wts[8];       // softmax over them (reference order of operations)
    int fallback;       // 1 when the exact serial logits were needed
};

// The exact path of the selection: recompute, in the reference's serial order
// (acc = b; acc += W[j]*xn[j]), the logit of every expert whose interval
// reaches the lowest lower bound of the provisional top-k, then rank those
// exactly (descending, lowest index first).  sL / sH: LDS values and upper
// bounds of all NE experts; sSel: LDS [K] provisional choice, overwritten;
// pst: LDS scratch of exact_group(CAND) * exact_stride(d) floats, then NE
// ints.  One wavefront.
template <int CAND, int CHUNK>
CPB_DEV void exact_reselect(double* sL, const double* sH, int* sSel, int NE, int K, const float* __restrict__ router_w,
                            const float* __restrict__ router_b, const float* __restrict__ xn, int d, float* pst) {
    const int lane = threadIdx.x & 63;
    constexpr int NG = exact_group(CAND);
    int* sList = (int*)(pst + NG * exact_stride(d));   // [NE] every candidate, ascending
    // candidates: intervals reaching the lowest lower bound of the selected
    double tau = 1e300;
    for (int i = 0; i < K; i++) { const int e = sSel[i]; tau = fmin(tau, sL[e] - (sH[e] - sL[e])); }
    // the others can never reach the top k
    for (int e = lane; e < NE; e += 64)
        if (!(sH[e] >= tau)) sL[e] = -1e300;
    // the candidates in ascending order, 64 experts per ballot
    int nl = 0;
    {
        const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
        for (int base = 0; base < NE; base += 64) {
            const int e = base + lane;
            const bool c = e < NE && sH[e] >= tau;
            const uint64_t m = __ballot(c);
            if (c) sList[nl + __popcll(m & below)] = e;
            nl += __popcll(m);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(xn, (uint32_t)d * 4);
    const int stride = exact_stride(d);
    // candidates in groups of kExactGroup: the wave writes each candidate's
    // fp32 products W[j]*xn[j] to LDS (coalesced row loads), then lane c runs
    // candidate c's serial chain acc = b; acc += p_j over them
    for (int g0 = 0; g0 < nl; g0 += NG) {
        // the group's candidates
        const int ng = min(NG, nl - g0);
        const int* sCand = sList + g0;
        if constexpr (CAND == 1) {
            // one 16-byte load pair per lane in flight (few registers)
            for (int c = 0; c < ng; c++) {
                const int ec = sCand[c];
                const __amdgpu_buffer_rsrc_t rw = buf_rsrc(router_w + (size_t)ec * d, (uint32_t)d * 4);
                for (int j = 4 * lane; j < d; j += 256) {
                    const u32x4 w4 = __builtin_amdgcn_raw_buffer_load_b128(rw, (uint32_t)j * 4, 0, 0);
                    const u32x4 x4 = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)j * 4, 0, 0);
                    float4 p4;
                    p4.x = __fmul_rn(__uint_as_float(w4[0]), __uint_as_float(x4[0]));
                    p4.y = __fmul_rn(__uint_as_float(w4[1]), __uint_as_float(x4[1]));
                    p4.z = __fmul_rn(__uint_as_float(w4[2]), __uint_as_float(x4[2]));
                    p4.w = __fmul_rn(__uint_as_float(w4[3]), __uint_as_float(x4[3]));
                    *(float4*)(pst + c * stride + j) = p4;
                }
            }
        } else {
            // CAND candidates' rows (CHUNK 16-byte loads per lane each) in flight per round
            for (int c0 = 0; c0 < ng; c0 += CAND) {
                for (int j0 = 0; j0 < d; j0 += 256 * CHUNK) {
                    u32x4 x4[CHUNK], w4[CAND][CHUNK];
    #pragma unroll
                    for (int k = 0; k < CHUNK; k++) {
                        const int j = j0 + 256 * k + 4 * lane;
                        x4[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, j < d ? (uint32_t)j * 4 : kOffNone, 0, 0);
                    }
    #pragma unroll
                    for (int ci = 0; ci < CAND; ci++) {
                        const int c = c0 + ci;
                        const int ec = sCand[c < ng ? c : 0];
                        const __amdgpu_buffer_rsrc_t rw = buf_rsrc(router_w + (size_t)ec * d, c < ng ? (uint32_t)d * 4 : 0u);
    #pragma unroll
                        for (int k = 0; k < CHUNK; k++) {
                            const int j = j0 + 256 * k + 4 * lane;
                            w4[ci][k] = __builtin_amdgcn_raw_buffer_load_b128(rw, j < d ? (uint32_t)j * 4 : kOffNone, 0, 0);
                        }
                    }
    #pragma unroll
                    for (int ci = 0; ci < CAND; ci++) {
                        const int c = c0 + ci;
    #pragma unroll
                        for (int k = 0; k < CHUNK; k++) {
                            const int j = j0 + 256 * k + 4 * lane;
                            if (c < ng && j < d) {
                                float4 p4;
                                p4.x = __fmul_rn(__uint_as_float(w4[ci][k][0]), __uint_as_float(x4[k][0]));
                                p4.y = __fmul_rn(__uint_as_float(w4[ci][k][1]), __uint_as_float(x4[k][1]));
                                p4.z = __fmul_rn(__uint_as_float(w4[ci][k][2]), __uint_as_float(x4[k][2]));
                                p4.w = __fmul_rn(__uint_as_float(w4[ci][k][3]), __uint_as_float(x4[k][3]));
                                *(float4*)(pst + c * stride + j) = p4;
                            }
                        }
                    }
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < ng) {
            const int e = sCand[lane];
            const float* pr = pst + lane * stride;
            float acc = router_b ? router_b[e] : 0.0f;
            int j = 0;
            if constexpr (CAND > 1) {
                // full groups of 32 products streamed from LDS (the next
                // group's reads issued before the current group's adds; the
                // look-ahead reads at most 64 floats past d, inside the
                // stride's slack).  64 registers: the wide variant only.
                const int nfull = d / 32;
                uint32_t ra = lds_addr(pr);
                f32x4 ga[8], gb[8];
                lds_read8(ga, ra);
                for (int m = 0;; m += 2) {
                    lds_read8(gb, ra + 128);
                    lds_wait_older8(ga);
                    if (m >= nfull) break;
                    acc = serial_add32(ga, acc);
                    lds_read8(ga, ra + 256);
                    lds_wait_older8(gb);
                    if (m + 1 >= nfull) break;
                    acc = serial_add32(gb, acc);
                    ra += 256;
                }
                lds_wait_all();
                j = nfull * 32;
            } else {
                for (; j + 32 <= d; j += 32) {
                    f32x4 v[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) v[u] = *(const f32x4*)(pr + j + 4 * u);
                    acc = serial_add32(v, acc);
                }
            }
            for (; j < d; j++) acc = __fadd_rn(acc, pr[j]);
            sL[e] = (double)acc;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // exact ranking among the candidates (every other expert is below them
    // all, and the candidates include the k provisional choices)
    for (int i = lane; i < nl; i += 64) {
        const int e = sList[i];
        const double v = sL[e];
        int r = 0;
        for (int j = 0; j < nl; j++) {
            const int oe = sList[j];
            const double o = sL[oe];
            r += (o > v) || (o == v && oe < e);
        }
        if (r < K) sSel[r] = e;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Selection inputs and outputs for a kernel that selects at its own start
// (the routing kernel published lstar / lbound before this launch began, so
// plain loads see them).
struct SelectIn {
    const double* lstar;     // [ne] null: ids / wts were selected elsewhere
    const double* lbound;    // [ne]
    const float* router_w;   // exact fallback only
    const float* router_b;
    const float* xn;
    int ne, k, d;
    int32_t* ids;            // [k]  written by workgroup 0
    float* wts;              // [k]
    float* logits;           // [ne]
    int32_t* fallback;       // [1]
};
// LDS bytes select_topk_wave may use (its exact fallback)
CPB_DEV_HOST_INLINE size_t select_lds_bytes(int ne, int d, int group = kExactGroup) {
    return sizeof(double) * 2 * ne + 64 + sizeof(float) * group * exact_stride(d) + sizeof(int) * ne;
}

// Wave-wide maximum of a 32-bit unsigned value via DPP (quad swaps, half-row
// and row mirrors, row broadcasts 15 / 31), returned wave-uniform.
CPB_DEV uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
// Order-preserving map of a float onto unsigned integers (-0 < +0).
CPB_DEV uint32_t float_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
CPB_DEV float key_float(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k); }
// fp32 bounds of a double: lo <= x <= hi
// (finite x; one ulp outward when the nearest float lies on the wrong side)
CPB_DEV float f32_up(double x) {
    const float f = (float)x;
    if (!((double)f < x)) return f;
    const uint32_t u = __float_as_uint(f);
    return (u & 0x7fffffffu) == 0 ? __uint_as_float(1u) : __uint_as_float(f > 0.0f ? u + 1 : u - 1);
}
CPB_DEV float f32_down(double x) {
    const float f = (float)x;
    if (!((double)f > x)) return f;
    const uint32_t u = __float_as_uint(f);
    return (u & 0x7fffffffu) == 0 ? __uint_as_float(0x80000001u) : __uint_as_float(f > 0.0f ? u - 1 : u + 1);
}

// Rare path of select_topk_wave (pointer and scalar
// arguments only, so the caller needs no stack): exact_reselect over the LDS
// image the caller wrote.
template <int CAND, int CHUNK>
CPB_DEV void select_exact_path(unsigned char* lds, int NE, int K, const float* router_w,
                                                            const float* router_b, const float* xn, int d) {
    double* sL = (double*)lds;
    double* sH = sL + NE;
    int* sSel = (int*)(sH + NE);
    float* xst = (float*)(lds + sizeof(double) * 2 * NE + 64);
    exact_reselect<CAND, CHUNK>(sL, sH, sSel, NE, K, router_w, router_b, xn, d, xst);
}

// One wavefront's LDS writes visible to its later LDS reads (a wave's LDS
// operations complete in order; unlike a fence this does not wait for the
// wave's outstanding global loads).
CPB_DEV void wave_lds_order() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Top-k by one wavefront with every value in registers: lane l holds experts
// l + 64j (j < 4).  The provisional ranking uses 32-bit keys (the logit
// rounded to fp32, its top 24 bits, then 255 - index so that equal keys pick
// the lowest index): K rounds of a DPP wave max.  Lane i < K collects rank i's
// expert, fp32 logit and fp32 bounds rounded outwards.  Certification: rank i
// must lie strictly above every later rank and every unselected expert; a
// ranking that truncation made wrong cannot pass it, and then the exact path
// (the reference's serial logits) decides.  Softmax over the k in the
// reference's order.  Writes *out (LDS) from lanes < K.
// The intervals of a <= 64-expert selection, one per lane, loaded ahead (a
// caller issues these before its other loads so that the selection does not
// wait for them: a wave's loads complete in order).
struct SelectPre {
    double lv, bv;
};
CPB_DEV SelectPre select_preload(const SelectIn& s) {
    const int lane = threadIdx.x & 63;
    const bool ok = s.ne <= 64 && lane < s.ne;
    return SelectPre{ok ? s.lstar[lane] : 0.0, ok ? s.lbound[lane] : 0.0};
}

// Workgroup pre-pass of the selection for up to 256 experts (one thread per
// expert; blockDim.x >= ne): every thread ranks its expert's 32-bit key
// against all keys in LDS (rank = number of larger keys), the top k write
// their id, fp32 logit and outward-rounded bounds to LDS by rank, the others
// fold their upper bound into an LDS maximum.  Thread e also publishes its
// fp32 logit when logits_out is set.  Ends with a barrier; select_topk_wave
// (called with ranked = true by one wavefront) then certifies and finishes
// from the LDS state.  LDS: the first select_ranked_bytes bytes of lds.
constexpr size_t select_ranked_bytes = 256 * 4 + 8 * 4 * 4 + 16 + 256 * 4;
// Thread e's interval, loaded by the caller ahead of its other loads (a
// wavefront's loads complete in order).
CPB_DEV SelectPre select_preload_wg(const SelectIn& s) {
    const int tid = threadIdx.x;
    const bool ok = tid < s.ne;
    return SelectPre{ok ? s.lstar[tid] : 0.0, ok ? s.lbound[tid] : 0.0};
}
CPB_DEV void select_rank_wg(const SelectIn& s, unsigned char* lds, float* logits_out, const SelectPre& pre) {
    const int tid = threadIdx.x, NE = s.ne, K = s.k;
    uint32_t* skey = (uint32_t*)lds;                   // [256]
    int* sE = (int*)(skey + 256);                      // [8] by rank
    float* sLf = (float*)(sE + 8);                     // [8]
    float* sLo = sLf + 8;                              // [8]
    float* sHi = sLo + 8;                              // [8]
    uint32_t* smu = (uint32_t*)(sHi + 8);              // max key of the unselected upper bounds
    const bool valid = tid < NE;
    const double lv = pre.lv, bv = pre.bv;
    const float lf = (float)lv;
    const uint32_t key = valid ? ((float_key(lf) & 0xFFFFFF00u) | (uint32_t)(255 - tid)) : 0u;
    if (tid < ((NE + 31) & ~31)) skey[tid] = key;      // zero keys (never larger) pad to a multiple of 32
    if (tid == 0) *smu = float_key(-__builtin_inff());
    if (valid && logits_out) logits_out[tid] = lf;
    __syncthreads();
    // rank: with at least twice as many threads as experts, thread e + NE
    // counts the larger keys among the second half of the (32-padded) keys
    // and thread e the first half; else thread e counts all
    const int NEp = (NE + 31) & ~31;
    const bool split = (int)blockDim.x >= 2 * NE && NEp >= 64;
    const int half = (NEp / 2 + 31) & ~31;
    int* srank = (int*)(smu + 1);                      // [NE] second-half counts
    int rank = 0;
    if (tid < (split ? 2 * NE : NE)) {
        const int ee = tid < NE ? tid : tid - NE;
        const uint32_t kk = tid < NE ? key : skey[ee];
        const int j0 = split && tid >= NE ? half : 0, j1 = split && tid < NE ? half : NEp;
        // 32 keys per round: eight 16-byte LDS reads in flight, then the compares
        for (int j = j0; j < j1; j += 32) {
            u32x4 k4[8];
#pragma unroll
            for (int u = 0; u < 8; u++) k4[u] = *(const u32x4*)(skey + j + 4 * u);
#pragma unroll
            for (int u = 0; u < 8; u++) rank += (k4[u][0] > kk) + (k4[u][1] > kk) + (k4[u][2] > kk) + (k4[u][3] > kk);
        }
        if (split && tid >= NE) srank[ee] = rank;
    }
    if (split) __syncthreads();
    uint32_t mu_key = 0u;                              // this thread's unselected upper bound (0: none)
    if (valid) {
        if (split) rank += srank[tid];
        const float hi = f32_up(lv + bv);
        if (rank < K) { sE[rank] = tid; sLf[rank] = lf; sLo[rank] = f32_down(lv - bv); sHi[rank] = hi; }
        else mu_key = float_key(hi);
    }
    // one LDS atomic per wavefront (same-address LDS atomics serialise)
    const uint32_t wm = wave_max_u32(mu_key);
    if ((tid & 63) == 0 && wm) atomicMax(smu, wm);
    __syncthreads();
}

// EXACT_CAND / EXACT_CHUNK: router rows (and 16-byte loads per lane of each)
// in flight on the exact path; EXACT_CAND > 1 also streams the serial chains'
// LDS reads ahead (registers: the decode kernels keep both small)
// ranked: select_rank_wg ran first (the logits were published there); the
// wave certifies its LDS ranking and, on the rare exact path, reloads the
// intervals.
// defer: write only ids, logits and the fallback flag to *out (what the
// caller needs to start its weight loads); the softmax weights and the
// published ids / weights follow from select_publish, which workgroup 0 runs
// once its loads are in flight.
CPB_DEV void select_publish(const SelectIn& s, const Selection* out);
template <int EXACT_CAND = 1, int EXACT_CHUNK = 1>
CPB_DEV void select_topk_wave(const SelectIn& s, unsigned char* lds, Selection* out, bool publish_logits = false,
                              const SelectPre* pre = nullptr, bool ranked = false,
                              bool defer = false) {
    const int lane = threadIdx.x & 63;
    const int NE = s.ne, K = s.k;
    double lv[4] = {0.0, 0.0, 0.0, 0.0}, bv[4] = {0.0, 0.0, 0.0, 0.0};
    float lf[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int my_e = 0;
    float my_l = 0.0f;
    bool bad;
    if (ranked) {
        const int* sE = (const int*)(lds + 256 * 4);
        const float* sLf = (const float*)(sE + 8);
        const float* sLo = sLf + 8;
        const float* sHi = sLo + 8;
        const uint32_t mu = *(const uint32_t*)(sHi + 8);
        float later = key_float(mu), my_lo = 0.0f;
        const f32x4 h0 = *(const f32x4*)sHi, h1 = *(const f32x4*)(sHi + 4);
        const float hs[8] = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
#pragma unroll
        for (int j = 1; j < 8; j++)
            if (j > lane && j < K) later = fmaxf(later, hs[j]);
        if (lane < K) {
            my_e = sE[lane];
            my_l = sLf[lane];
            my_lo = sLo[lane];
        }
        bad = __any(lane < K && !(my_lo > later));
        wave_lds_order();
        if (bad) {
            // the exact path needs every interval (LDS state above is consumed)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = lane + 64 * j;
                lv[j] = e < NE ? s.lstar[e] : 0.0;
                bv[j] = e < NE ? s.lbound[e] : 0.0;
            }
        }
    } else if (NE <= 64) {
        // one expert per lane; rank = number of larger keys, read back from
        // LDS (no serial rounds); rank r < K is selection slot r
        const bool valid = lane < NE;
        lv[0] = pre ? pre->lv : valid ? s.lstar[lane] : 0.0;
        bv[0] = pre ? pre->bv : valid ? s.lbound[lane] : 0.0;
        lv[1] = lv[2] = lv[3] = bv[1] = bv[2] = bv[3] = 0.0;
        lf[0] = (float)lv[0];
        lf[1] = lf[2] = lf[3] = 0.0f;
        const uint32_t key = valid ? ((float_key(lf[0]) & 0xFFFFFF00u) | (uint32_t)(255 - lane)) : 0u;
        const float lo = f32_down(lv[0] - bv[0]);
        const float hi = valid ? f32_up(lv[0] + bv[0]) : -__builtin_inff();
        uint32_t* skey = (uint32_t*)lds;                  // [64]
        int* sE = (int*)(skey + 64);                      // [8] by rank
        float* sLf = (float*)(sE + 8);                    // [8]
        float* sHi = sLf + 8;                             // [8]
        skey[lane] = key;
        wave_lds_order();
        // 32 keys per round: eight 16-byte LDS reads in flight, then the compares
        int rank = 0;
        for (int j = 0; j < NE; j += 32) {
            u32x4 k4[8];
#pragma unroll
            for (int u = 0; u < 8; u++) k4[u] = *(const u32x4*)(skey + j + 4 * u);
#pragma unroll
            for (int u = 0; u < 8; u++) rank += (k4[u][0] > key) + (k4[u][1] > key) + (k4[u][2] > key) + (k4[u][3] > key);
        }
        const bool sel = valid && rank < K;
        if (sel) { sE[rank] = lane; sLf[rank] = lf[0]; sHi[rank] = hi; }
        // upper bound of every unselected expert
        const float mu = key_float(wave_max_u32(float_key(sel ? -__builtin_inff() : hi)));
        wave_lds_order();
        float later = mu;
        {
            // the later ranks' upper bounds in two 16-byte reads
            const f32x4 h0 = *(const f32x4*)sHi, h1 = *(const f32x4*)(sHi + 4);
            const float hs[8] = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
#pragma unroll
            for (int j = 1; j < 8; j++)
                if (sel && j > rank && j < K) later = fmaxf(later, hs[j]);
        }
        bad = __any(sel && !(lo > later));
        if (lane < K) { my_e = sE[lane]; my_l = sLf[lane]; }
        wave_lds_order();
    } else {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = lane + 64 * j;
        lv[j] = e < NE ? s.lstar[e] : 0.0;
        bv[j] = e < NE ? s.lbound[e] : 0.0;
    }
    uint32_t key[4];
    float lo[4], hi[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = lane + 64 * j;
        lf[j] = (float)lv[j];
        key[j] = e < NE ? ((float_key(lf[j]) & 0xFFFFFF00u) | (uint32_t)(255 - e)) : 0u;
        lo[j] = f32_down(lv[j] - bv[j]);
        hi[j] = e < NE ? f32_up(lv[j] + bv[j]) : -__builtin_inff();
    }
    float my_lo = 0.0f, my_hi = -__builtin_inff();
    for (int i = 0; i < K; i++) {
        const uint32_t m = wave_max_u32(max(max(key[0], key[1]), max(key[2], key[3])));
        const int bi = 255 - (int)(m & 0xFFu);
        const int src = bi & 63, jj = bi >> 6;
        // the chosen expert's values, read from its lane
        const float vl = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
            __builtin_bit_cast(int, jj == 0 ? lf[0] : jj == 1 ? lf[1] : jj == 2 ? lf[2] : lf[3]), src));
        const float vlo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
            __builtin_bit_cast(int, jj == 0 ? lo[0] : jj == 1 ? lo[1] : jj == 2 ? lo[2] : lo[3]), src));
        const float vhi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
            __builtin_bit_cast(int, jj == 0 ? hi[0] : jj == 1 ? hi[1] : jj == 2 ? hi[2] : hi[3]), src));
        if (lane == i) { my_e = bi; my_l = vl; my_lo = vlo; my_hi = vhi; }
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (lane + 64 * j == bi) { key[j] = 0u; hi[j] = -__builtin_inff(); }
    }
    // upper bound of every unselected expert (selected ones were set to -inf)
    const float mu = key_float(wave_max_u32(float_key(fmaxf(fmaxf(hi[0], hi[1]), fmaxf(hi[2], hi[3])))));
    float later = mu;
    for (int j = 0; j < K; j++) {
        const float hj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_hi), j));
        if (j > lane) later = fmaxf(later, hj);
    }
    bad = __any(lane < K && !(my_lo > later));
    }
    if (bad) {
        double* sL = (double*)lds;
        double* sH = sL + NE;
        int* sSel = (int*)(sH + NE);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = lane + 64 * j;
            if (e < NE) { sL[e] = lv[j]; sH[e] = lv[j] + bv[j]; }
        }
        if (lane < K) sSel[lane] = my_e;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        select_exact_path<EXACT_CAND, EXACT_CHUNK>(lds, NE, K, s.router_w, s.router_b, s.xn, s.d);
        if (lane < K) { my_e = sSel[lane]; my_l = (float)sL[my_e]; }
    }
    if (defer) {
        if (lane < K) {
            out->ids[lane] = my_e;
            out->logit[lane] = my_l;
        }
        if (lane == 0) out->fallback = bad ? 1 : 0;
        if (blockIdx.x == 0 && blockIdx.y == 0 && s.logits && !ranked) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = lane + 64 * j;
                if (e < NE) s.logits[e] = lf[j];
            }
        }
        return;
    }
    // softmax over the k selected, reference order: ex_i = exp(l_i - l_0)
    // (lane i), then the serial sum ex_0 + ex_1 + ...
    const float l0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_l), 0));
    const float ex = expf(my_l - l0);
    float wsum = 0.0f;
    for (int i = 0; i < K; i++) wsum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), i));
    const float wt = ex / wsum;
    if (lane < K) {
        out->ids[lane] = my_e;
        out->logit[lane] = my_l;
        out->wts[lane] = wt;
    }
    if (lane == 0) out->fallback = bad ? 1 : 0;
    // trace outputs and the routed ids / weights for later launches (by one
    // workgroup, or by this one when it alone selects for its token)
    if (publish_logits) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = lane + 64 * j;
            if (e < NE) s.logits[e] = lf[j];
        }
        __builtin_amdgcn_wave_barrier();
        if (lane < K) s.logits[my_e] = my_l;
    } else if (blockIdx.x == 0 && blockIdx.y == 0) {
        if (!ranked) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = lane + 64 * j;
                if (e < NE && s.logits) s.logits[e] = lf[j];
            }
        }
        __builtin_amdgcn_wave_barrier();
        if (lane < K) {
            s.ids[lane] = my_e;
            s.wts[lane] = wt;
            if (s.logits) s.logits[my_e] = my_l;     // as used (exact serial value after a fallback)
        }
        if (lane == 0 && s.fallback) s.fallback[0] = bad ? 1 : 0;
    }
}

// Softmax over the k experts of a deferred selection (reference order, as in
// select_topk_wave) and the routed ids / weights / used logits for later
// launches.  One wavefront of workgroup 0.
CPB_DEV void select_publish(const SelectIn& s, const Selection* out) {
    const int lane = threadIdx.x & 63, K = s.k;
    const int my_e = lane < K ? out->ids[lane] : 0;
    const float my_l = lane < K ? out->logit[lane] : 0.0f;
    const float l0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_l), 0));
    const float ex = expf(my_l - l0);
    float wsum = 0.0f;
    for (int i = 0; i < K; i++) wsum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), i));
    const float wt = ex / wsum;
    if (lane < K) {
        s.ids[lane] = my_e;
        s.wts[lane] = wt;
        if (s.logits) s.logits[my_e] = my_l;     // as used (exact serial value after a fallback)
    }
    if (lane == 0 && s.fallback) s.fallback[0] = out->fallback;
}

}  // namespace cpb
