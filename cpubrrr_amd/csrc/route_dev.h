// route_dev.h -- device body of the per-token routing step (see route.hip).
#pragma once
#include "moe_common.h"
#include "route.h"

#ifndef CPB_DEV_HOST
#define CPB_DEV_HOST __host__ __device__
#endif

namespace cpb {

// Per-token rmsnorm into LDS (xn) in the reference's summation order.
// gpt-oss: ssq() with 4 NEON accumulators x 4 lanes of fma over 16-wide steps
// (engine_gpt2.rs:710-726): lane q (0..15) of wave 0 runs chain q over
// x[16m + q]; Qwen: nt serial slices, then a serial sum of the partials
// (engine_qwen2.rs:457-467).
CPB_DEV void norm_into(const float* __restrict__ xg, const float* __restrict__ nw, int d, float eps,
                       int norm, int nt, int apply, float* xs, float* xn, float* scratch) {
    const int tid = threadIdx.x, nth = blockDim.x;
    // x may have been written by other workgroups of the same launch:
    // coherent 16-byte loads.  Thread tid owns float4 slots tid + k*nth
    // (nth * 16 >= d for every launch: d <= 4096, nth >= 256); the norm
    // weights of the same slots are fetched alongside, before the first wait.
    u32x4 wn[4];
    {
        const __amdgpu_buffer_rsrc_t r = buf_rsrc(xg, (uint32_t)d * 4);
        const __amdgpu_buffer_rsrc_t rw = buf_rsrc(nw, nw && apply ? (uint32_t)d * 4 : 0u);
        u32x4 v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = ld_dev16(r, (uint32_t)(tid + k * nth) * 16);
#pragma unroll
        for (int k = 0; k < 4; k++) wn[k] = __builtin_amdgcn_raw_buffer_load_b128(rw, (uint32_t)(tid + k * nth) * 16, 0, 0);
#pragma unroll
        for (int k = 0; k < 4; k++)
            if ((tid + k * nth) * 4 < d) ((u32x4*)xs)[tid + k * nth] = v[k];
    }
    __syncthreads();
    if (!apply) {
        for (int i = tid; i < d / 4; i += nth) ((float4*)xn)[i] = ((const float4*)xs)[i];
        __syncthreads();
        return;
    }
    if (norm == 0) {
        if (tid < 16) {
            float a = 0.0f;
            const int n16 = d / 16;
            int m = 0;
            for (; m + 16 <= n16; m += 16) {
                float t[16];
#pragma unroll
                for (int u = 0; u < 16; u++) t[u] = xs[(m + u) * 16 + tid];
#pragma unroll
                for (int u = 0; u < 16; u++) a = fmaf(t[u], t[u], a);
            }
            for (; m < n16; m++) { float t = xs[m * 16 + tid]; a = fmaf(t, t, a); }
            scratch[tid] = a;                  // chain q = 4v + l  ->  a[v][l]
        }
        __syncthreads();
        if (tid == 0) {
            float L[4];
            for (int l = 0; l < 4; l++) L[l] = (scratch[l] + scratch[4 + l]) + (scratch[8 + l] + scratch[12 + l]);
            float s = (L[0] + L[1]) + (L[2] + L[3]);
            for (int i = d - d % 16; i < d; i++) s += xs[i] * xs[i];
            scratch[16] = 1.0f / sqrtf(s / (float)d + eps);
        }
    } else {
        const int base = d / nt, rem = d % nt;
        if (tid < nt) {
            const int a = tid * base + (tid < rem ? tid : rem), sz = base + (tid < rem ? 1 : 0);
            float ps = 0.0f;
            int i = 0;
            for (; i + 16 <= sz; i += 16) {
                float t[16];
#pragma unroll
                for (int u = 0; u < 16; u++) t[u] = xs[a + i + u];
#pragma unroll
                for (int u = 0; u < 16; u++) ps += t[u] * t[u];
            }
            for (; i < sz; i++) { float v = xs[a + i]; ps += v * v; }
            scratch[tid] = ps;
        }
        __syncthreads();
        if (tid == 0) {
            float tot = 0.0f;
            for (int k = 0; k < nt; k++) tot += scratch[k];
            scratch[16] = 1.0f / sqrtf(tot / (float)d + eps);
        }
    }
    __syncthreads();
    const float inv = scratch[16];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i4 = tid + k * nth;
        if (i4 * 4 < d) {
            const float4 xv = ((const float4*)xs)[i4];
            float4 o;
            if (nw) {
                o.x = xv.x * inv * __uint_as_float(wn[k][0]);
                o.y = xv.y * inv * __uint_as_float(wn[k][1]);
                o.z = xv.z * inv * __uint_as_float(wn[k][2]);
                o.w = xv.w * inv * __uint_as_float(wn[k][3]);
            } else {
                o.x = xv.x * inv; o.y = xv.y * inv; o.z = xv.z * inv; o.w = xv.w * inv;
            }
            ((float4*)xn)[i4] = o;
        }
    }
    __syncthreads();
}



// ---- wavefront DPP helpers on doubles (no LDS round trips) ----
// v from the DPP source lane; lanes whose source is out of the row, or whose
// row is masked off, read 0.0
template <int CTRL, int ROWMASK>
CPB_DEV double dpp_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROWMASK, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROWMASK, 0xF, true);
    return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
// inclusive prefix sum over the 64 lanes (row_shr 1,2,4,8, then row_bcast 15, 31)
CPB_DEV double wave_scan_f64(double v) {
    v += dpp_f64<0x111, 0xF>(v);
    v += dpp_f64<0x112, 0xF>(v);
    v += dpp_f64<0x114, 0xF>(v);
    v += dpp_f64<0x118, 0xF>(v);
    v += dpp_f64<0x142, 0xA>(v);
    v += dpp_f64<0x143, 0xC>(v);
    return v;
}
// sum over the 64 lanes, valid in lane 63 (quad swaps, half-row and row
// mirrors, then row_bcast 15, 31)
CPB_DEV double wave_total63_f64(double v) {
    v += dpp_f64<0xB1, 0xF>(v);
    v += dpp_f64<0x4E, 0xF>(v);
    v += dpp_f64<0x141, 0xF>(v);
    v += dpp_f64<0x140, 0xF>(v);
    v += dpp_f64<0x142, 0xA>(v);
    v += dpp_f64<0x143, 0xC>(v);
    return v;
}
// max over each aligned group of 16 lanes (a DPP row), in every lane of it
CPB_DEV float row_max_f32(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
    return v;
}
// value of the neighbouring lane (lane ^ 1)
CPB_DEV float pair_f32(float v) { return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)); }
CPB_DEV int pair_i32(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }

// 16-byte store with the cache policy of st_dev (sc1: visible across XCDs)
CPB_DEV void st_dev16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, byte_off, 0, 16);
}

CPB_DEV float sumsq_chain(const f32x4 (&g)[8], float acc) {
#pragma unroll
    for (int u = 0; u < 8; u++) {
        acc = fmaf(g[u][0], g[u][0], acc);
        acc = fmaf(g[u][1], g[u][1], acc);
        acc = fmaf(g[u][2], g[u][2], acc);
        acc = fmaf(g[u][3], g[u][3], acc);
    }
    return acc;
}


constexpr int kRouteC = 16;         // consecutive elements per thread in route_expert

// LDS bytes route_expert needs (any block size; d <= 4096)
// transposed x: 16 rows of d/16 values, zero padded to at least d/16 + 32
// (whole 32-value groups of the chain read zeros past d/16) and offset so
// the 16 lanes' 16-byte reads spread over the banks; the chain's one-group
// look-ahead past the last row lands in the reduction area behind it
CPB_DEV_HOST inline int route_xt_stride(int d) { return (d / 16 + 32 + 63) / 64 * 64 + 4; }
// Qwen: slice q of the nt serial slices in row q (the same padding and bank
// offset for the longest slice, ceil(d / nt))
CPB_DEV_HOST inline int route_slice_stride(int d, int nt) { return ((d + nt - 1) / nt + 32 + 63) / 64 * 64 + 4; }
// slices of the Qwen sum of squares, 1 for the gpt-oss order
CPB_DEV_HOST inline int route_slices(const RouteArgs& a) { return a.norm == 0 ? 1 : a.norm_nt; }
CPB_DEV_HOST inline size_t route_lds_bytes(int d, int nt) {
    const size_t xt = sizeof(float) * 16 * (size_t)route_xt_stride(d);
    const size_t xs = sizeof(float) * (size_t)nt * route_slice_stride(d, nt);
    return (xt > xs ? xt : xs) + sizeof(double) * 64 + 64;
}
// s + p for the 32 values of g in order (the Qwen slice chain over squares
// already rounded to fp32: the reference's multiply then add, with the
// multiplies off the dependent chain)
CPB_DEV float sum_serial32(const f32x4 (&g)[8], float s) {
#pragma unroll
    for (int u = 0; u < 8; u++) {
#pragma unroll
        for (int c = 0; c < 4; c++) s = s + g[u][c];
    }
    return s;
}

// ---- router logit from unscaled products, shared by the decode route and
// the batched router so both produce the same bits ----
// Each thread of an element wave owns 16 consecutive elements; element wave
// ws covers elements 1024*ws .. 1024*ws + 1023.  Phase 1: P_j = W_j * x_j *
// g_j in fp64, this thread's sum, the wave's inclusive scan (wave total to
// dred[ws]).  Phase 2 (no barrier needed): the wave-local prefix sums for the
// bound, sum |prefix| to dred[16 + ws] and sum |P_j| to dred[32 + ws].  Final
// (after a barrier, one thread): logit and bound for the norm scale inv.
struct LogitThread {
    double P[16];
    double loc, absp, incl;
};
CPB_DEV void logit_phase1(const float* wf, const float* xf, const float* gf, LogitThread& L, double* dred, int ws) {
    const int lane = threadIdx.x & 63;
    L.loc = 0.0;
    L.absp = 0.0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        L.P[i] = (double)wf[i] * ((double)xf[i] * (double)gf[i]);
        L.loc += L.P[i];
        L.absp += fabs(L.P[i]);
    }
    L.incl = wave_scan_f64(L.loc);
    if (lane == 63) dred[ws] = L.incl;
}
CPB_DEV void logit_phase2(const LogitThread& L, bool act, double* dred, int ws) {
    const int lane = threadIdx.x & 63;
    double run = L.incl - L.loc;
    double sabs = 0.0;
#pragma unroll
    for (int i = 0; i < 16; i++) { run += L.P[i]; sabs += act ? fabs(run) : 0.0; }
    const double s1 = wave_total63_f64(sabs);
    const double s2 = wave_total63_f64(L.absp);
    if (lane == 63) { dred[16 + ws] = s1; dred[32 + ws] = s2; }
}
// The reference computes xn_j = fl(fl(x_j * inv) * g_j), p_j = fl(W_j * xn_j)
// and the serial fp32 chain acc = b; acc += p_j.  With t_j = inv * P_j
// (exact), |p_j - t_j| <= g3 |t_j|, and the chain lies within
// u/(1-u) (sum_k |S_k| + n gamma_n A) of b + sum p_j (Higham, Accuracy and
// Stability of Numerical Algorithms, 2nd ed., 4.2), where sum_k |S_k| <=
// n|b| + inv sum_k |P-prefix_k| + n g3 inv A' and A <= |b| + (1 + g3) inv A',
// A' = sum |P_j|.  n = d elements.  A prefix inside element wave w is the
// wave's offset O_w (the earlier waves' totals) plus a wave-local prefix, so
// sum_k |P-prefix_k| <= sum_w (n_w |O_w| + sum_wave-local |prefix|), n_w =
// the wave's element count.  gamma_n = nu/(1-nu) <= nu (1 + 2nu) (nu <= 1/2).
CPB_DEV void logit_final(const double* dred, int nws, int d, double b, float inv, double* lstar, double* lbound) {
    double wtot = 0.0, SS = 0.0, AP = 0.0;
    for (int w2 = 0; w2 < nws; w2++) {
        const int nw2 = min(max(d - 1024 * w2, 0), 1024);
        SS += (double)nw2 * fabs(wtot) + dred[16 + w2];
        wtot += dred[w2];
        AP += dred[32 + w2];
    }
    const double u = 5.9604644775390625e-08;  // 2^-24
    const double n = (double)d;
    const double g3 = 3.0 * u / (1.0 - 3.0 * u);
    const double gam = n * u * (1.0 + 2.0 * n * u);
    const double sc = (double)inv;
    const double IA = sc * AP;
    const double ab = fabs(b);
    const double bound = u / (1.0 - u) * (n * ab + sc * SS + n * g3 * IA + n * gam * (ab + (1.0 + g3) * IA)) + g3 * IA;
    *lstar = b + sc * wtot;
    *lbound = bound * 1.0001 + 1e-10 * (ab + IA) + 1e-30;
}

// Workgroup-level body: expert e's logit + bound, and this workgroup's share
// (blocks b with b % NEg == e) of the activation quantisation.  Wave 0 runs
// the rmsnorm sum of squares; waves 1.. are element waves (route_threads(d)
// threads in all).
//
// Thread 64 + t owns x[16t .. 16t+16): its x, norm weights and router weights
// arrive in registers from one round of loads and x goes to LDS.  The gpt-oss
// sum of squares (16 fma chains, chain q over x[16m + q],
// engine_gpt2.rs:710-726) runs in 16 lanes of wave 0 over a transposed copy
// (chain q's elements contiguous); the Qwen one (nt serial slices,
// engine_qwen2.rs:457-467) over the squares, in slice rows.  Meanwhile the
// element waves compute the router logit as the fp64 sum of the unscaled products W_j * x_j
// * g_j (scaled by the norm scale once that is known; its bound covers every
// rounding of the reference's fp32 path, see logit_final).
CPB_DEV_HOST_INLINE int route_threads(int d) { return 64 + (d / 16 + 63) / 64 * 64; }
CPB_DEV void route_expert(const RouteArgs& a, int e, int NEg, unsigned char* smem) {
    const int tid = threadIdx.x, nth = blockDim.x, lane = tid & 63, wv = tid >> 6;
    const int d = a.d;
    const int et = tid - 64, ws = wv - 1, nws = (nth >> 6) - 1;     // element thread / wave
    float* xl = (float*)smem;                                  // transposed (gpt-oss) or plain (Qwen) x
    double* dred = (double*)(smem + route_lds_bytes(d, route_slices(a)) - sizeof(double) * 64 - 64);   // [64]
    float* sinv = (float*)(dred + 64);

    const int j0 = et * kRouteC;
    const bool act = et >= 0 && j0 < d;
    const uint32_t off = (uint32_t)(act ? j0 : 0) * 4;
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.x, (uint32_t)d * 4);
    const __amdgpu_buffer_rsrc_t rW = buf_rsrc(a.router_w + (size_t)e * d, (uint32_t)d * 4);
    const bool use_g = a.norm_w && a.apply_norm;
    const __amdgpu_buffer_rsrc_t rg = buf_rsrc(a.norm_w, use_g ? (uint32_t)d * 4 : 0u);
    // the raw loads; converted where used (after x is in LDS), so that the
    // LDS copy of x waits for x only, not for the router and norm weights
    float xf[16], gf[16], wf[16];
    u32x4 xv[4] = {}, wq[4] = {}, gq[4] = {};
    if (wv > 0) {
#pragma unroll
        for (int k = 0; k < 4; k++) xv[k] = ld_dev16(rx, off + 16 * k);     // may come from this launch
#pragma unroll
        for (int k = 0; k < 4; k++) wq[k] = __builtin_amdgcn_raw_buffer_load_b128(rW, off + 16 * k, 0, 0);
#pragma unroll
        for (int k = 0; k < 4; k++) gq[k] = __builtin_amdgcn_raw_buffer_load_b128(rg, off + 16 * k, 0, 0);
    }
    const double b = a.router_b ? (double)a.router_b[e] : 0.0;
    // Q8 (qk == 0): element thread et quantises element et % 32 of this
    // workgroup's block slot et / 32 (the blocks b with b % NEg == e); its
    // x and norm weight are fetched now
    const int nbq = d / 32, qslots = (nth - 64) / 32;
    const int qb0 = et >> 5, qj = et & 31;
    float qx = 0.0f, qg = 1.0f;
    if (a.qk == 0 && wv > 0 && e + NEg * qb0 < nbq) {
        const int j = (e + NEg * qb0) * 32 + qj;
        qx = ld_dev(a.x + j);
        if (use_g) qg = a.norm_w[j];
    }

    // ---- x into LDS for the sum of squares ----
    const int S = route_xt_stride(d);
    if (a.apply_norm && wv > 0) {
        if (a.norm == 0) {
            // chain q's element m = x[16m + q] lives in element thread m,
            // register q: transposed (chain q's elements contiguous)
            // (from the loaded registers: the writes wait for x only, not
            // for the router and norm weights loaded beside it)
            if (act) {
#pragma unroll
                for (int i = 0; i < 16; i++) xl[i * S + et] = __uint_as_float(xv[i >> 2][i & 3]);
            }
            // zero padding past d/16: fma(0, 0, acc) leaves acc (>= 0) unchanged
            for (int c = d / 16 + et; c < S; c += nth - 64) {
#pragma unroll
                for (int i = 0; i < 16; i++) xl[i * S + c] = 0.0f;
            }
        } else {
            // the squares x_j * x_j (rounded to fp32, as the reference's
            // multiply) of slice q (the first d % nt slices one element
            // longer) in row q of stride SQ; zeros past each slice: p + 0
            // leaves p (>= 0)
            const int nt = a.norm_nt, base = d / nt, rem = d % nt, SQ = route_slice_stride(d, nt);
            const int big = rem * (base + 1);                 // elements of the longer slices
            if (act) {
                // this thread's 16 elements start at (q, i) and cross into
                // row q + 1 at most once (slices are >= 16 long: d >= 16 nt)
                const int q = j0 < big ? j0 / (base + 1) : rem + (j0 - big) / base;
                const int i = j0 - (q < rem ? q * (base + 1) : big + (q - rem) * base);
                const int cross = base + (q < rem ? 1 : 0) - i;          // elements left in row q
                const int a0 = q * SQ + i, a1 = (q + 1) * SQ - cross;
#pragma unroll
                for (int u = 0; u < 16; u++) {
                    const float v = __uint_as_float(xv[u >> 2][u & 3]);
                    xl[(u < cross ? a0 : a1) + u] = v * v;
                }
            }
            for (int q = 0; q < nt; q++)
                for (int i = base + (q < rem ? 1 : 0) + et; i < SQ; i += nth - 64) xl[q * SQ + i] = 0.0f;
        }
    }
    __syncthreads();
    if (wv == 0) {
        if (a.apply_norm && a.norm == 0) {
            // lane q streams its row: the next group's reads are issued before
            // the current group's fmas (software pipelined; the scheduling
            // barriers keep the compiler from regrouping them).  The zero
            // padding past d/16 leaves acc unchanged (fma(0, 0, acc) = acc,
            // acc >= 0), so whole groups run without a bound check.
            const int nm = d / 16;                   // <= 256
            float acc = 0.0f;
            uint32_t ra = lds_addr(xl + (lane & 15) * S);
            f32x4 ga[8], gb[8];                      // ping-pong groups of 32 values
            lds_read8(ga, ra);
            for (int m = 0;; m += 64) {
                lds_read8(gb, ra + 128);
                lds_wait_older8(ga);
                acc = sumsq_chain(ga, acc);
                if (m + 32 >= nm) break;
                lds_read8(ga, ra + 256);
                lds_wait_older8(gb);
                acc = sumsq_chain(gb, acc);
                if (m + 64 >= nm) break;
                ra += 256;
            }
            lds_wait_all();
            // chain q = 4v + l -> acc[v][l]; L[l] = (a0 + a1) + (a2 + a3); s = (L0 + L1) + (L2 + L3)
            float c16[16];
#pragma unroll
            for (int q = 0; q < 16; q++) c16[q] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), q));
            float L[4];
#pragma unroll
            for (int l = 0; l < 4; l++) L[l] = (c16[l] + c16[4 + l]) + (c16[8 + l] + c16[12 + l]);
            const float ssq = (L[0] + L[1]) + (L[2] + L[3]);
            if (lane == 0) *sinv = 1.0f / sqrtf(ssq / (float)d + a.eps);
        } else if (a.apply_norm) {
            // nt serial slices, then a serial sum of the partials (nt <= 64)
            // lane q streams row q of squares (lanes past nt repeat row 0,
            // unused) with the next 32 values' reads issued before the
            // current 32 adds: one dependent add per element
            const int nt = a.norm_nt, SQ = route_slice_stride(d, nt), nm = (d + nt - 1) / nt;
            float ps = 0.0f;
            uint32_t ra = lds_addr(xl + (lane < nt ? lane : 0) * SQ);
            f32x4 ga[8], gb[8];
            lds_read8(ga, ra);
            for (int m = 0;; m += 64) {
                lds_read8(gb, ra + 128);
                lds_wait_older8(ga);
                ps = sum_serial32(ga, ps);
                if (m + 32 >= nm) break;
                lds_read8(ga, ra + 256);
                lds_wait_older8(gb);
                ps = sum_serial32(gb, ps);
                if (m + 64 >= nm) break;
                ra += 256;
            }
            lds_wait_all();
            float tot = 0.0f;
            for (int k = 0; k < nt; k++) tot += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ps), k));
            if (lane == 0) *sinv = 1.0f / sqrtf(tot / (float)d + a.eps);
        }
    } else {
        // ---- router logit, unscaled, beside the sum-of-squares chain ----
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            xf[i] = act ? __uint_as_float(xv[i >> 2][i & 3]) : 0.0f;
            gf[i] = use_g ? __uint_as_float(gq[i >> 2][i & 3]) : 1.0f;
            wf[i] = act ? __uint_as_float(wq[i >> 2][i & 3]) : 0.0f;
        }
        LogitThread lt;
        logit_phase1(wf, xf, gf, lt, dred, ws);
        logit_phase2(lt, act, dred, ws);
    }
    __syncthreads();
    const float inv = a.apply_norm ? *sinv : 1.0f;
    if (tid == 0) {
        double ls = 0.0, lb = 0.0;
        logit_final(dred, nws, d, b, inv, &ls, &lb);
        st_dev(a.lstar + e, ls);
        st_dev(a.lbound + e, lb);
    }
    if (wv == 0) {
        return;
    }

    // ---- xn = (x * inv) * w, and this workgroup's share of the activation
    // quantisation ----
    if (a.qk == 0) {
        // Q8 per 32-block (engine_gpt2.rs:691-699): 32 lanes per block, the
        // block maximum over the lane group, then each lane's xq byte, its two
        // image bytes (K offset 2j or 2(j - 16) + 1 for element j) and xn
        for (int qb = qb0; e + NEg * qb < nbq; qb += qslots) {
            const int blk = e + NEg * qb, j = blk * 32 + qj;
            if (qb != qb0) {
                qx = ld_dev(a.x + j);
                qg = use_g ? a.norm_w[j] : 1.0f;
            }
            const float xnv = !a.apply_norm ? qx : use_g ? (qx * inv) * qg : qx * inv;
            float m = row_max_f32(fabsf(xnv));
            m = fmaxf(m, __shfl_xor(m, 16));
            const float sc = fmaxf(1e-12f, m) / 127.0f;
            const int8_t qv = q8_round(xnv, sc);
            a.xn[j] = xnv;
            a.xq[j] = qv;
            const int kpos = qj < 16 ? 2 * qj : 2 * (qj - 16) + 1;
            const uint32_t qb8 = (uint32_t)(uint8_t)qv;
            a.ximg[blk * 64 + kpos] = (uint8_t)img_hi(qb8);
            a.ximg[blk * 64 + 32 + kpos] = (uint8_t)img_lo(qb8);
            if (qj == 0) a.xsb[blk] = sc;
        }
    } else {
        // Q8_K per 256 (engine_qwen2.rs:288-300): the 16 threads of a DPP row
        // hold one superblock; per-32 sums from thread pairs
        float xn[16];
#pragma unroll
        for (int i = 0; i < 16; i++) xn[i] = !a.apply_norm ? xf[i] : use_g ? (xf[i] * inv) * gf[i] : xf[i] * inv;
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(xn[i]));
        m = row_max_f32(m);
        const int sb = et >> 4;
        const float sc = fmaxf(1e-12f, m) / 127.0f;
        uint32_t qp[4];
        q8_round16(xn, sc, qp);
        int s32 = 0;
#pragma unroll
        for (int i = 0; i < 16; i++) s32 += (int)(int8_t)(qp[i >> 2] >> (8 * (i & 3)));
        s32 += pair_i32(s32);
        if (act && sb % NEg == e) {
            const __amdgpu_buffer_rsrc_t rn = buf_rsrc(a.xn, (uint32_t)d * 4);
#pragma unroll
            for (int k = 0; k < 4; k++)
                st_dev16(rn, off + 16 * k, u32x4{__float_as_uint(xn[4 * k]), __float_as_uint(xn[4 * k + 1]),
                                                 __float_as_uint(xn[4 * k + 2]), __float_as_uint(xn[4 * k + 3])});
            st_dev16(buf_rsrc(a.xq, (uint32_t)d), (uint32_t)j0, u32x4{qp[0], qp[1], qp[2], qp[3]});
            if ((et & 15) == 0) st_dev(a.xsb + sb, sc);
            if ((et & 1) == 0) st_dev(a.xsum + (et >> 1), s32);
        }
    }
}



}  // namespace cpb
